// wir_splitk.hip -- split-K GEMM through the C ABI: the host side of one
// product (kernel arguments and the two launches) in one call.
//
// wir_gemm_splitk takes the fp32 workspace of splits * M * N partial sums
// from the caller (warpir_amd.api.gemm_split_k allocates it when the caller
// does not).  wir_gemm_splitk_noalloc runs the same two kernels -- the
// generated split-K GEMM and wir_splitk_reduce -- with that workspace in
// `scratch`, a file-scope device array of WIR_NOALLOC_SCRATCH_FLOATS floats
// that every device holds from the library's first use until the process
// ends.  Host code never passes `scratch` itself to a kernel: the name is a
// host-side stand-in.  The device address comes from hipGetSymbolAddress,
// looked up once per device with that device current and kept in
// g_scratch[device].
//
// Every call on one device shares that device's array.  The GEMM writes every
// partial element [split][row < M][col < N] before the reduction reads it, so
// nothing needs clearing between calls; two calls that overlap on one device
// (different streams or threads without ordering between them) race on it.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <mutex>

#include "warpir_rt.h"

static __device__ __align__(256) float scratch[WIR_NOALLOC_SCRATCH_FLOATS];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<float*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (looked up on the first
// call per device).
int scratch_on_current_device(float** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  float* p = g_scratch[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (!p) {
      void* addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return (int)e;
      if (!addr) return (int)hipErrorInvalidSymbol;
      p = (float*)addr;
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return 0;
}

// Host mirror of the generated kernel's wir::gl<T>: data pointer, four dims
// (b, d, r, c) and three element strides (sb, sd, sr).
struct GlobalView {
  const void* data;
  int b, d, r, c;
  long long sb, sd, sr;
};

// Kernel arguments of the split-K GEMM variants (128x128 output tiles, four
// wavefronts: gemm_128_splitk*), laid out as their emitted globals struct
// (inputs then outputs in IR order: A, B, N, C_global).
struct SplitKGemmArgs {
  GlobalView A;   // [1][splits][M][K/splits], K-slice s starts at column s*K/splits
  GlobalView B;   // [1][splits][K/splits][N]
  int N;          // K/splits: the loop bound of one slice
  GlobalView C;   // fp32 partials [1][splits][M][N]
};
static_assert(sizeof(GlobalView) == 48, "wir::gl layout");
static_assert(offsetof(SplitKGemmArgs, B) == 48 && offsetof(SplitKGemmArgs, N) == 96 &&
                  offsetof(SplitKGemmArgs, C) == 104 && sizeof(SplitKGemmArgs) == 152,
              "split-K GEMM globals layout");

// Kernel arguments of the fused split-K variants (gemm_128_splitk_fused): the
// same A, B, N and fp32 partials, then the bf16 result and the per-tile
// arrival counters the kernel's reduce_slices uses.
struct SplitKFusedArgs {
  SplitKGemmArgs g;
  GlobalView C;          // bf16 [1][1][M][N]
  GlobalView arrivals;   // u32 [1][1][1][tiles]
};
static_assert(offsetof(SplitKFusedArgs, C) == 152 && offsetof(SplitKFusedArgs, arrivals) == 200 &&
                  sizeof(SplitKFusedArgs) == 248,
              "fused split-K GEMM globals layout");

// Kernel arguments of wir_splitk_reduce (splitk_reduce.hip).
struct SplitKReduceArgs {
  const float* partials;
  void* out;
  long long n;
  long long split_stride;
  int splits;
};

constexpr int kTile = 128;       // split-K GEMM output tile (rows and columns)
constexpr int kThreads = 256;    // split-K GEMM workgroup size
constexpr int kKStep = 64;       // K per pipeline step
constexpr int kMaxSplits = 16;

int launch(hipFunction_t f, unsigned gx, unsigned gy, unsigned gz, unsigned bx, void* stream,
           void* args, size_t size) {
  void* config[] = {HIP_LAUNCH_PARAM_BUFFER_POINTER, args, HIP_LAUNCH_PARAM_BUFFER_SIZE, &size,
                    HIP_LAUNCH_PARAM_END};
  return (int)hipModuleLaunchKernel(f, gx, gy, gz, bx, 1, 1, 0, (hipStream_t)stream, nullptr, config);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// The GEMM arguments of one split-K product (A and B as K slices, the partials in `ws`).
SplitKGemmArgs splitk_args(const void* a, const void* b, float* ws, int m, int n, int k, int splits) {
  const long long split_elems = (long long)m * n;
  const int kc = k / splits;
  SplitKGemmArgs g;
  g.A = {a, 1, splits, m, kc, 0, kc, k};
  g.B = {b, 1, splits, kc, n, (long long)k * n, (long long)kc * n, n};
  g.N = kc;
  g.C = {ws, 1, splits, m, n, (long long)splits * split_elems, split_elems, n};
  return g;
}

// The two launches of a split-K product with its fp32 partials in `ws`
// (splits * m * n floats); arguments already validated.
int splitk_launch(hipFunction_t gemm, hipFunction_t reduce, const void* a, const void* b, void* out, float* ws,
                  int m, int n, int k, int splits, void* stream) {
  const long long split_elems = (long long)m * n;
  SplitKGemmArgs g = splitk_args(a, b, ws, m, n, k, splits);
  int e = launch(gemm, (unsigned)((n + kTile - 1) / kTile), (unsigned)((m + kTile - 1) / kTile), (unsigned)splits,
                 kThreads, stream, &g, sizeof(g));
  if (e) return e;
  SplitKReduceArgs r = {ws, out, split_elems, split_elems, splits};
  return launch(reduce, (unsigned)((split_elems / 8 + 255) / 256), 1, 1, 256, stream, &r, sizeof(r));
}

int splitk_check(wir_function_t gemm, wir_function_t reduce, const void* a, const void* b, void* out, int m, int n,
                 int k, int splits) {
  if (!gemm || !reduce || !a || !b || !out) return (int)hipErrorInvalidValue;
  if (m <= 0 || n <= 0 || k <= 0 || splits <= 0 || splits > kMaxSplits) return (int)hipErrorInvalidValue;
  if (k % (kKStep * splits) || n % 8 || !aligned16(a) || !aligned16(b) || !aligned16(out))
    return (int)hipErrorInvalidValue;
  return 0;
}

}  // namespace

extern "C" int wir_gemm_splitk(wir_function_t gemm, wir_function_t reduce, const void* a, const void* b, void* out,
                               void* workspace, size_t workspace_floats, int m, int n, int k, int splits,
                               void* stream) {
  int e = splitk_check(gemm, reduce, a, b, out, m, n, k, splits);
  if (e) return e;
  if (!workspace || !aligned16(workspace) || (unsigned long long)splits * m * n > workspace_floats)
    return (int)hipErrorInvalidValue;
  return splitk_launch((hipFunction_t)gemm, (hipFunction_t)reduce, a, b, out, (float*)workspace, m, n, k, splits,
                       stream);
}

extern "C" int wir_gemm_splitk_fused(wir_function_t gemm, const void* a, const void* b, void* out, void* workspace,
                                     size_t workspace_floats, void* arrivals, size_t arrival_count, int m, int n,
                                     int k, int splits, void* stream) {
  // the fused kernel has no separate reduction: pass the GEMM as both functions to the common checks
  int e = splitk_check(gemm, gemm, a, b, out, m, n, k, splits);
  if (e) return e;
  if (!workspace || !aligned16(workspace) || (unsigned long long)splits * m * n > workspace_floats)
    return (int)hipErrorInvalidValue;
  const long long tiles = (long long)((m + kTile - 1) / kTile) * ((n + kTile - 1) / kTile);
  if (!arrivals || ((uintptr_t)arrivals & 3) || (unsigned long long)tiles > arrival_count)
    return (int)hipErrorInvalidValue;
  SplitKFusedArgs f;
  f.g = splitk_args(a, b, (float*)workspace, m, n, k, splits);
  f.C = {out, 1, 1, m, n, (long long)m * n, (long long)m * n, n};
  f.arrivals = {arrivals, 1, 1, 1, (int)tiles, tiles, tiles, tiles};
  return launch((hipFunction_t)gemm, (unsigned)((n + kTile - 1) / kTile), (unsigned)((m + kTile - 1) / kTile),
                (unsigned)splits, kThreads, stream, &f, sizeof(f));
}

extern "C" int wir_gemm_splitk_noalloc(wir_function_t gemm, wir_function_t reduce, const void* a,
                                       const void* b, void* out, int m, int n, int k, int splits,
                                       void* stream) {
  int e = splitk_check(gemm, reduce, a, b, out, m, n, k, splits);
  if (e) return e;
  if ((long long)splits * m * n > (long long)WIR_NOALLOC_SCRATCH_FLOATS) return WIR_ERROR_SCRATCH_LIMIT;
  float* ws = nullptr;
  e = scratch_on_current_device(&ws);
  if (e) return e;
  return splitk_launch((hipFunction_t)gemm, (hipFunction_t)reduce, a, b, out, ws, m, n, k, splits, stream);
}
