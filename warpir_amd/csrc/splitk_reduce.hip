// splitk_reduce.hip -- fp32 partial sums rounded once to bf16: the reduction
// step of split-K GEMM (wir_splitk_reduce) and of the grouped-query
// attention backward (wir_group_reduce).
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

// lo/hi += the 8 floats of each of `count` partials at p, p + stride, ...
// in that order.  The loads of up to four partials are issued before their
// adds (the adds stay in partial order, so the sums are those of the
// one-at-a-time loop), so a thread waits for one memory round trip per four
// partials instead of one per partial.
__device__ __forceinline__ void wr_accumulate(wr_f32x4& lo, wr_f32x4& hi, const float* p, long long stride,
                                              int count) {
  int s = 0;
  for (; s + 4 <= count; s += 4) {
    wr_f32x4 a[4], b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] = *(const wr_f32x4*)(p + (s + j) * stride);
      b[j] = *(const wr_f32x4*)(p + (s + j) * stride + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo += a[j];
      hi += b[j];
    }
  }
  for (; s < count; ++s) {
    lo += *(const wr_f32x4*)(p + s * stride);
    hi += *(const wr_f32x4*)(p + s * stride + 4);
  }
}

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
  wr_accumulate(lo, hi, args.partials + e, args.split_stride, args.splits);
  wr_bf16x8 v;
  for (int j = 0; j < 4; ++j) {
    v[j] = (__bf16)lo[j];
    v[4 + j] = (__bf16)hi[j];
  }
  *(wr_bf16x8*)(args.out + e) = v;
}

// Grouped-query attention backward: the key-major dK / dV kernel writes one
// fp32 contribution per query head, [B, H, S, D] with H = G * splits heads
// grouped by key/value head (query head h belongs to key/value head
// h / splits).  out[g][e] = bf16(sum_r partials[(g * splits + r) * n + e]),
// summed in head order, for the G = B * H_kv groups of n = S * D elements.
// Each thread owns 8 consecutive elements of one group; n must be a multiple
// of 8.
struct wg_args {
  const float* partials;   // [groups][splits][n]
  __bf16* out;             // [groups][n]
  long long n;
  long long groups;
  int splits;
};

extern "C" __global__ void __launch_bounds__(256) wir_group_reduce(const wg_args args) {
  const long long e = ((long long)blockIdx.x * 256 + threadIdx.x) * 8;
  if (e >= args.n * args.groups) return;
  const long long g = e / args.n, off = e % args.n;
  wr_f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
  wr_accumulate(lo, hi, args.partials + g * args.splits * args.n + off, args.n, args.splits);
  wr_bf16x8 v;
  for (int j = 0; j < 4; ++j) {
    v[j] = (__bf16)lo[j];
    v[4 + j] = (__bf16)hi[j];
  }
  *(wr_bf16x8*)(args.out + e) = v;
}
