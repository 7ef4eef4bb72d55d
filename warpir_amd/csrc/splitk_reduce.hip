// splitk_reduce.hip -- the reduction step of split-K GEMM.
//
// The split-K GEMM kernel (warpir_amd.workloads.build_gemm_kernel with
// split_k=True) writes S fp32 partial products [S][M][N]; this kernel sums
// them in fp32, in split order, and rounds once to bf16 (round to nearest
// even), the same final rounding as the unsplit kernel's store.  Each
// thread owns 8 consecutive elements: two 16-byte loads per split and one
// 16-byte store.  n (= M * N) must be a multiple of 8.
#include <hip/hip_runtime.h>

typedef float wr_f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 wr_bf16x8 __attribute__((ext_vector_type(8)));

struct wr_args {
  const float* partials;   // [splits][n]
  __bf16* out;             // [n]
  long long n;
  long long split_stride;  // elements between consecutive splits
  int splits;
};

extern "C" __global__ void __launch_bounds__(256) wir_splitk_reduce(const wr_args args) {
  const long long e = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e >= args.n) return;
  wr_f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < args.splits; ++s) {
    const float* p = args.partials + s * args.split_stride + e;
    lo += *(const wr_f32x4*)p;
    hi += *(const wr_f32x4*)(p + 4);
  }
  wr_bf16x8 v;
  for (int j = 0; j < 4; ++j) {
    v[j] = (__bf16)lo[j];
    v[4 + j] = (__bf16)hi[j];
  }
  *(wr_bf16x8*)(args.out + e) = v;
}
