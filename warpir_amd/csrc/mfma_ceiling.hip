// mfma_ceiling.hip -- measurement kernel for the benchmark's roofline: the
// sustained bf16 MFMA rate of the whole chip with no memory traffic, and the
// shader clock it runs at.
//
// Every wavefront keeps 16 independent 32x32 fp32 accumulators (256 AGPRs at
// one wavefront per SIMD) and issues ITERS x 16 v_mfma_f32_32x32x16_bf16
// back to back.  Operands are either pseudo-random bf16 values of the
// benchmarks' magnitude (mode 0) or a few small constants (mode 1): MI355X's
// clock is power-limited, and the operand bit activity moves it by ~25%.
// Lane 0 of each wavefront stores the s_memtime (shader clock) and
// s_memrealtime (100 MHz) deltas of its loop with ordinary vector stores, so
// the host derives the clock as memtime / (realtime / 100 MHz).
#include <hip/hip_runtime.h>

typedef __bf16 wc_bf16x8 __attribute__((ext_vector_type(8)));
typedef float wc_f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ unsigned wc_hash(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

struct wc_args {
  float* sink;                 // written only if the accumulators hit a sentinel
  unsigned long long* clocks;  // [waves][2]: memtime delta, memrealtime delta
  int iters;
  int mode;                    // 0: random operands, 1: constant operands
};

extern "C" __global__ void __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1)))
wir_mfma_ceiling(const wc_args args) {
  const int lane = threadIdx.x & 63;
  wc_bf16x8 a[4], b[4];
  for (int j = 0; j < 4; ++j)
    for (int e = 0; e < 8; ++e) {
      float va = 0.01f * e, vb = 0.02f * j;
      if (args.mode == 0) {
        va = ((wc_hash(lane * 131 + j * 17 + e + 7) & 0xffff) / 65536.f - 0.5f) * 0.2f;
        vb = ((wc_hash(lane * 137 + j * 19 + e + 99) & 0xffff) / 65536.f - 0.5f) * 0.2f;
      }
      a[j][e] = (__bf16)va;
      b[j][e] = (__bf16)vb;
    }
  wc_f32x16 acc[16];
  for (int q = 0; q < 16; ++q) acc[q] = (wc_f32x16){};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < args.iters; ++it) {
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[q / 4], b[q % 4], acc[q], 0, 0, 0);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
  for (int q = 0; q < 16; ++q) s += acc[q][0] + acc[q][15];
  if (s == 12345.f) args.sink[threadIdx.x] = s;
  if (lane == 0) {
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    args.clocks[2 * w] = t1 - t0;
    args.clocks[2 * w + 1] = r1 - r0;
  }
}
