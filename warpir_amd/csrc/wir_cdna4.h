// wir_cdna4.h -- device tile library of the WarpIR gfx950 (CDNA4) lowering.
//
// Every kernel emitted by warpir_amd.lowering.CDNA4Lowerer is this header
// followed by one `extern "C" __global__` function whose body is a sequence
// of calls into the templates below, one group per IR op.  The header is
// pasted into the emitted source, so a generated .hip file is
// self-contained (no other include than the HIP runtime header).
//
// Execution model (wave64):
//   * A workgroup is NW wavefronts of 64 lanes.  Block-level tiles live in
//     LDS; register tiles are per-wavefront slices.
//   * Register tiles use the "lane = row" layout: the fp32 result of
//     v_mfma_f32_{32x32x16,16x16x32}_bf16 is computed for the transposed
//     product, so lane l owns logical row (l % MS) of each MS-row block and
//     the accumulator registers run along the columns.  Row reductions of
//     the online softmax are then lane-local plus one cross-lane step, and
//     4 consecutive registers hold 4 consecutive columns (8-byte stores).
//   * MFMA lane layouts on gfx950 (measured on the device):
//       32x32x16: operand lane l -> row/col l%32, k = 8*(l/32) + j (j<8);
//                 C reg i -> row 8*(i/4) + 4*(l/32) + i%4, col l%32.
//       16x16x32: operand lane l -> row/col l%16, k = 8*(l/16) + j;
//                 C reg i -> row 4*(l/16) + i, col l%16.
//   * global_load_lds_dwordx4 writes lane l's 16 bytes at M0 + 16*l, so a
//     tile load is 64 physical 16-byte LDS chunks per instruction and the
//     LDS swizzle is expressed by choosing each lane's global address.
//   * ds_read_b64_tr_b16: in each 16-lane group, lane s supplies row
//     (s/4) and columns 4*(s%4)..+3 of a 4x16 bf16 block; afterwards lane s
//     holds column s, rows 0..3.  It feeds MFMA operands from row-major
//     [K][N] tiles without a transpose pass.
#pragma once
#include <hip/hip_runtime.h>

namespace wir {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;

// A 4-D row-major tensor [b, d, r, c] in HBM; the column stride is 1.
// Mirrors the host-side ctypes structure of warpir_amd.runtime.
template <typename T>
struct gl {
  T* data;
  int b, d, r, c;
  long long sb, sd, sr;
};

// Zero-filled source for out-of-bounds tile chunks (TMA zero-fill semantics).
__device__ __attribute__((aligned(256))) unsigned int zero_page[64] = {0};

__device__ __forceinline__ int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

__device__ __forceinline__ lds_char* lds(char* generic) { return (lds_char*)(generic); }

// ---------------------------------------------------------------------------
// MFMA shape traits.
template <int MS> struct MF;
template <> struct MF<32> {
  static constexpr int LG = 2;      // lane groups (64 / MS)
  static constexpr int CREGS = 16;  // fp32 C registers per lane
  static constexpr int KSTEP = 16;  // k per MFMA
  typedef f32x16 cvec;
  static __device__ __forceinline__ cvec mma(bf16x8 a, bf16x8 b, cvec c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct MF<16> {
  static constexpr int LG = 4;
  static constexpr int CREGS = 4;
  static constexpr int KSTEP = 32;
  typedef f32x4 cvec;
  static __device__ __forceinline__ cvec mma(bf16x8 a, bf16x8 b, cvec c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// Column (within an MS-column block) held by C register i of a lane in
// lane group lh, in the lane = row layout.
template <int MS>
__device__ __forceinline__ int ccol(int i, int lh) {
  return (i / 4) * (4 * MF<MS>::LG) + 4 * lh + (i % 4);
}

// ---------------------------------------------------------------------------
// LDS tiles.  ROWS x COLS bf16, row-major, in 16-byte chunks (CPR per row)
// with an XOR swizzle of the chunk index chosen by how the tile is read.
// gfx950's LDS serves 256 bytes per cycle (64 banks of 4 bytes), so a
// ds_read_b128 is processed 16 lanes at a time and a ds_read_b64 32 lanes
// at a time (measured with SQ_LDS_BANK_CONFLICT: swizzles built for 128-byte
// banks showed 2-way conflicts).  The swizzles are
// conflict-free for the MFMA operand patterns under both a 256-byte and a
// 128-byte bank space:
//   ROWREAD -- ds_read_b128 of one row per lane, 16 consecutive rows per
//              phase: the 16 rows land in 16 distinct 16-byte bank slots;
//   TRREAD  -- ds_read_b64_tr_b16, per 32 lanes 4 rows x 64 bytes: the 4
//              rows' 64-byte runs land in 4 disjoint bank ranges.
//   BOTH    -- a tile read both ways (K in the dQ kernel, Q and dO in the
//              dK/dV kernel): the row bits that separate the 4 rows of a
//              transposed read pick the 64-byte run, and the others permute
//              the 16-byte chunks inside it, so 16 consecutive rows still take
//              16 distinct chunk slots.  Conflict-free for both patterns in the
//              256-byte bank space (TRREAD would leave the row reads 4-way
//              conflicted).
enum Role { ROWREAD = 0, TRREAD = 1, BOTH = 2 };

template <int CPR, int ROLE>
__device__ __forceinline__ int swz(int row) {
  if (ROLE == ROWREAD) {
    if (CPR >= 16) return row & 15;
    if (CPR == 8) return (row & 7) ^ ((row >> 3) & 1);
    if (CPR == 4) return ((row >> 1) ^ (row >> 2)) & 3;
    if (CPR == 2) return (row >> 2) & 1;
    return 0;
  } else if (ROLE == BOTH && CPR >= 8) {
    if (CPR >= 16) return ((row & 3) << 2) | ((row >> 2) & 3);
    return (((row >> 1) & 1) << 2) | ((row >> 2) & 3);
  } else {
    if (CPR >= 16) return ((row & 3) << 2) | (row & 2);
    if (CPR == 8) return (row & 3) << 1;
    if (CPR == 4) return ((row >> 1) & 1) << 1;
    return 0;
  }
}

template <int ROWS_, int COLS_, int ROLE_>
struct STile {
  static constexpr int ROWS = ROWS_, COLS = COLS_, ROLE = ROLE_;
  static constexpr int CPR = COLS / 8;
  static constexpr int BYTES = ROWS * COLS * 2;
  static_assert(COLS % 8 == 0, "tile columns must be a multiple of 8 bf16");
  // Byte offset of the 16-byte chunk holding columns 8*chunk..8*chunk+7 of `row`.
  static __device__ __forceinline__ int chunk_off(int row, int chunk) {
    return (row * CPR + (chunk ^ swz<CPR, ROLE>(row))) * 16;
  }
  // Byte offset of element (row, col) (col need not be chunk aligned).
  static __device__ __forceinline__ int elem_off(int row, int col) {
    return chunk_off(row, col >> 3) + (col & 7) * 2;
  }
};

// ---------------------------------------------------------------------------
// Asynchronous global -> LDS tile load (the IR's tma_load / tma_load_buf).
//
// The DMA instruction is issued from inline assembly on purpose: when LLVM
// sees global_load_lds it must assume the LDS write may alias any later
// ds_read and inserts s_waitcnt vmcnt(0) in front of it, which would
// serialise every ring stage.  Completion is instead tracked by the
// lowering itself (wait_vm_barrier<N> with N from its schedule analysis).
//
// WIR_DMA_CPOL: cache-policy modifiers appended to the tile DMAs (" sc0",
// " sc1", " nt" or a combination; empty for the default policy).
#ifndef WIR_DMA_CPOL
#define WIR_DMA_CPOL ""
#endif
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Uniform 64-bit base + per-lane 32-bit byte offset (the saddr form).
__device__ __forceinline__ void dma16_s(const void* gbase, unsigned voff, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" WIR_DMA_CPOL
               :: "v"(voff), "s"(gbase), "s"(lds_addr) : "memory", "m0");
}
// Per-lane 64-bit address.
__device__ __forceinline__ void dma16_v(const void* gaddr, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" WIR_DMA_CPOL
               :: "v"(gaddr), "s"(lds_addr) : "memory", "m0");
}
#pragma clang diagnostic pop

// 4 bytes per lane, per-lane 64-bit address (lane l writes M0 + 4*l).
__device__ __forceinline__ void dma4_v(const void* gaddr, unsigned lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(gaddr), "s"(lds_addr) : "memory", "m0");
}

__device__ __forceinline__ unsigned lds_addr(char* p) {
  return (unsigned)(size_t)(lds_char*)p;
}

// The tile's rows start at global row `row0`, its columns at `col0`
// (elements).  Chunks outside [0, r) x [0, c) or an out-of-range (b, d)
// read the zero page.  Every wave issues exactly INSTR_PER_WAVE DMA
// instructions, the count the lowering uses for its vmcnt waits.  Tiles
// that lie wholly inside the tensor take the fast path: one uniform base
// address plus loop-invariant per-lane offsets.
template <class Tile, int NW>
struct Loader {
  static constexpr int CHUNKS = Tile::ROWS * Tile::CPR;
  static constexpr int INSTR = CHUNKS / 64;
  static_assert(CHUNKS % 64 == 0, "tile must be a multiple of 1 KiB");
  static_assert(INSTR % NW == 0, "tile chunks must split evenly over the wavefronts");
  static constexpr int INSTR_PER_WAVE = INSTR / NW;

  // Row and logical chunk of the 16-byte chunk this lane moves in
  // instruction j of wave `wave`.
  static __device__ __forceinline__ void place(int wave, int j, int& row, int& c) {
    const int p = (wave + j * NW) * 64 + lane_id();
    row = p / Tile::CPR;
    c = (p % Tile::CPR) ^ swz<Tile::CPR, Tile::ROLE>(row);
  }

  // Source of one tile load, resolved once per tile.
  struct Src {
    const bf16* base;  // tile origin (ALIGNED, in bounds) or tensor origin
    bool inb;          // ALIGNED: tile inside the tensor; else: tile wholly inside (fast path)
    int row0, col0;
  };

  // ALIGNED (the tensor's extents are multiples of the tile and its row
  // pitch fits the 32-bit offset form): a tile is either wholly inside or
  // wholly outside the tensor, so issue() is branch-free -- outside tiles
  // read the zero page at offset 0.  Otherwise tiles straddling an edge are
  // loaded lane by lane with bounds checks.  INB (with ALIGNED): the kernel
  // has proved that every tile it loads lies inside the tensor, so neither
  // the tile base nor a lane's offset selects the zero page.
  template <bool ALIGNED, bool INB = false>
  static __device__ __forceinline__ Src prep(const gl<bf16>& g, int b, int d, int row0, int col0) {
    static_assert(ALIGNED || !INB, "the in-bounds form is a case of the aligned one");
    const bool bd_ok = (unsigned)b < (unsigned)g.b && (unsigned)d < (unsigned)g.d;
    const bf16* bd = g.data + (long long)b * g.sb + (long long)d * g.sd;
    if (ALIGNED) {
      const bool inb = INB || (bd_ok && (unsigned)row0 < (unsigned)g.r && (unsigned)col0 < (unsigned)g.c);
      const bf16* t = inb ? bd + (long long)row0 * g.sr + col0 : (const bf16*)zero_page;
      return Src{t, inb, row0, col0};
    }
    const bool fast = bd_ok && row0 >= 0 && col0 >= 0 && row0 + Tile::ROWS <= g.r && col0 + Tile::COLS <= g.c &&
                      (long long)Tile::ROWS * g.sr < (1ll << 30);
    return Src{bd_ok ? bd : (const bf16*)zero_page, fast, bd_ok ? row0 : -(1 << 30), col0};
  }

  // Issue this wave's j-th DMA instruction of the tile.
  template <bool ALIGNED, bool INB = false>
  static __device__ __forceinline__ void issue(int j, char* tile_base, const gl<bf16>& g, const Src& s, int wave) {
    int row, c;
    place(wave, j, row, c);
    const unsigned dst = lds_addr(tile_base + (wave + j * NW) * 1024);
    if (ALIGNED) {
      const unsigned voff = (INB || s.inb) ? (unsigned)(row * (int)g.sr + c * 8) * 2u : 0u;
      dma16_s(s.base, voff, dst);
      return;
    }
    if (s.inb) {
      dma16_s(s.base + (long long)s.row0 * g.sr + s.col0, (unsigned)(row * (int)g.sr + c * 8) * 2u, dst);
    } else {
      const int gr = s.row0 + row, gc = s.col0 + c * 8;
      const bool ok = (unsigned)gr < (unsigned)g.r && (unsigned)gc < (unsigned)g.c;
      const void* src = ok ? (const void*)(s.base + (long long)gr * g.sr + gc) : (const void*)zero_page;
      dma16_v(src, dst);
    }
  }

  template <bool ALIGNED, bool INB = false>
  static __device__ __forceinline__ void load(char* tile_base, const gl<bf16>& g, int b, int d, int row0,
                                              int col0, int wave) {
    const Src src = prep<ALIGNED, INB>(g, b, d, row0, col0);
#pragma unroll
    for (int j = 0; j < INSTR_PER_WAVE; ++j) issue<ALIGNED, INB>(j, tile_base, g, src, wave);
  }

  // Whether `g` qualifies for the kernel's ALIGNED specialisation.
  static __device__ __forceinline__ bool aligned(const gl<bf16>& g) {
    return g.r % Tile::ROWS == 0 && g.c % Tile::COLS == 0 && (long long)Tile::ROWS * g.sr < (1ll << 30);
  }
};

// fp32 vector tile of N elements in LDS (a per-row statistic such as the
// log-sum-exp), loaded asynchronously like the bf16 tiles: each of the NW
// wavefronts issues one global_load_lds_dword moving N / NW elements
// (lanes beyond that are masked off).  Elements outside the tensor read the
// zero page.  One DMA instruction per wavefront, the count the lowering
// uses for its vmcnt waits.
template <int N, int NW>
struct VecLoader {
  static constexpr int PER = N / NW;
  static_assert(N % NW == 0 && PER <= 64, "vector must split into at most 64 elements per wavefront");

  template <bool ALIGNED, bool INB = false>   // (every vector load checks its rows)
  static __device__ __forceinline__ void load(char* tile_base, const gl<float>& g, int b, int d, int row0, int wave) {
    const int lane = lane_id();
    const int r = row0 + wave * PER + lane;
    const bool ok = (unsigned)b < (unsigned)g.b && (unsigned)d < (unsigned)g.d && (unsigned)r < (unsigned)g.r;
    const float* src = ok ? g.data + (long long)b * g.sb + (long long)d * g.sd + (long long)r * g.sr
                          : (const float*)zero_page;
    const unsigned dst = lds_addr(tile_base + wave * PER * 4);
    if (PER == 64 || lane < PER) dma4_v(src, dst);
  }
};

template <bool B>
struct bool_tag {
  static constexpr bool value = B;
};

// Wait until at most N of this wave's vector-memory instructions are
// outstanding and its LDS reads have returned, then synchronise the
// workgroup: every wave's LDS-DMA writes up to that point are visible and
// no wave still reads a slot that the next loads overwrite.  The empty asm
// statements keep the compiler from moving memory accesses across.
template <int N>
__device__ __forceinline__ void wait_vm_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" :: "n"(N) : "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// wait_vm_barrier<N> after a wave's latest batch of N loads was issued;
// when that batch was skipped (a tile past the loop's end) the batch before
// it is the newest and must land too: wait_vm_barrier<0>.  One barrier on
// either branch (the condition is wave-uniform).
template <int N>
__device__ __forceinline__ void wait_vm_barrier_after(bool issued) {
  if (issued)
    wait_vm_barrier<N>();
  else
    wait_vm_barrier<0>();
}

__device__ __forceinline__ void barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------------------
// Register tiles (per wave), lane = row layout.
//   RTile<MS, R, C>: logical R x C fp32; f[cb][rb] is the MFMA C fragment
//   of column block cb and row block rb.  Lane l owns row rb*MS + l%MS and,
//   in register i, column cb*MS + ccol<MS>(i, l/MS).
template <int MS, int R, int C>
struct RTile {
  static constexpr int RB = R / MS, CB = C / MS;
  static_assert(R % MS == 0 && C % MS == 0, "register tile must be a multiple of the MFMA shape");
  typename MF<MS>::cvec f[CB][RB];
};

// bf16 copy of an RTile: each group of 4 C registers packed as bf16x4.
template <int MS, int R, int C>
struct BTile {
  static constexpr int RB = R / MS, CB = C / MS;
  static constexpr int G = MF<MS>::CREGS / 4;
  bf16x4 f[CB][RB][G];
};

// Column vector of a lane = row tile: one value per row block.
template <int MS, int R>
struct RVec {
  static constexpr int RB = R / MS;
  float v[RB];
};

// Row vector of a lane = row tile (one value per column, shared by all rows):
// v[cb][i] is the value of the column that C register i of column block cb
// holds in this lane, i.e. column cb*MS + ccol<MS>(i, lane / MS).
template <int MS, int C>
struct CVec {
  static constexpr int CB = C / MS;
  float v[CB][MF<MS>::CREGS];
};

template <int MS, int R, int C>
__device__ __forceinline__ void fill(RTile<MS, R, C>& t, float x) {
#pragma unroll
  for (int cb = 0; cb < t.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < t.RB; ++rb)
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) t.f[cb][rb][i] = x;
}

template <int MS, int R>
__device__ __forceinline__ void fill(RVec<MS, R>& t, float x) {
#pragma unroll
  for (int rb = 0; rb < t.RB; ++rb) t.v[rb] = x;
}

// ---------------------------------------------------------------------------
// MFMA operands.
//
// "Row operand": 8 bf16 along k of one row per lane, from a ROWREAD LDS
// tile (ds_read_b128).  Used for the IR's `a` operand of every MMA and for
// `b` of a transpose_b MMA.
template <class Tile, int MS>
__device__ __forceinline__ bf16x8 row_operand(char* tile_base, int row_base, int kstep) {
  const int lane = lane_id();
  const int row = row_base + lane % MS;
  const int chunk = kstep * MF<MS>::LG + lane / MS;
  return *(const __attribute__((address_space(3))) bf16x8*)(lds(tile_base) + Tile::chunk_off(row, chunk));
}

// 4 consecutive k of one column per lane from a TRREAD [K][N] LDS tile via
// ds_read_b64_tr_b16.  `k0` is this lane's first k (uniform per 16-lane
// group), `n0` the group's first column.
template <class Tile>
__device__ __forceinline__ bf16x4 tr_operand4(char* tile_base, int k0, int n0) {
  const int s = lane_id() & 15;
  const int row = k0 + (s >> 2);
  const int col = n0 + 4 * (s & 3);
  i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(lds(tile_base) + Tile::elem_off(row, col)));
  return __builtin_bit_cast(bf16x4, v);
}

__device__ __forceinline__ bf16x8 cat(bf16x4 lo, bf16x4 hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// 4 consecutive k of one row per lane from a ROWREAD tile (ds_read_b64).
template <class Tile>
__device__ __forceinline__ bf16x4 row_operand4(char* tile_base, int row, int k0) {
  return *(const __attribute__((address_space(3))) bf16x4*)(lds(tile_base) + Tile::elem_off(row, k0));
}

// Hoisted row operands of a loop-invariant LDS tile (e.g. the resident Q
// tile): RB row blocks x KS k-steps per wave.
template <int MS, int RB, int KS>
struct RowFrags {
  bf16x8 f[RB][KS];
};

template <class Tile, int MS, int RB, int KS>
__device__ __forceinline__ void load_row_frags(RowFrags<MS, RB, KS>& fr, char* tile_base, int row0) {
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) fr.f[rb][ks] = row_operand<Tile, MS>(tile_base, row0 + rb * MS, ks);
}

// Row operands of a tile read straight from global memory into registers,
// for a tile whose only use is as hoisted MFMA fragments (so it needs no
// LDS): rows row0 + rb*MS + lane%MS, 8 columns at col0 + 8*(ks*LG +
// lane/MS).  Out-of-range rows or columns give zeros.
template <int MS, int RB, int KS>
__device__ __forceinline__ void load_row_frags_global(RowFrags<MS, RB, KS>& fr, const gl<bf16>& g, int b, int d,
                                                      int row0, int col0) {
  const int lane = lane_id();
  const bool bd_ok = (unsigned)b < (unsigned)g.b && (unsigned)d < (unsigned)g.d;
  const bf16* base = g.data + (long long)b * g.sb + (long long)d * g.sd;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = row0 + rb * MS + lane % MS;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int col = col0 + 8 * (ks * MF<MS>::LG + lane / MS);
      const bool ok = bd_ok && (unsigned)row < (unsigned)g.r && (unsigned)col < (unsigned)g.c;
      fr.f[rb][ks] = ok ? *(const bf16x8*)(base + (long long)row * g.sr + col) : bf16x8{};
    }
  }
}

// ---------------------------------------------------------------------------
// MMA, lane = row result layout.  Result rows = the IR operand `a`'s rows
// [a_row0, a_row0 + R), result cols = `b`'s columns (or rows when
// transposed) [b_col0, b_col0 + C).  The MFMA computes result^T =
// b^T a^T: its A operand comes from `b`, its B operand from `a`.

// acc += a @ b; a: ROWREAD LDS [.][K]; b: TRREAD LDS [K][.].
//
// Software-pipelined over the K/KSTEP MFMA k-steps: the fragments of step
// ks+1 are read from LDS while the RB*CB MFMAs of step ks run, and a
// scheduling-group pattern interleaves one LDS read after each MFMA so the
// reads' latency hides under the matrix core.
template <int MS, int R, int C, class TA, class TB>
__device__ __forceinline__ void mma_AB(RTile<MS, R, C>& acc, char* a_base, int a_row0, char* b_base,
                                       int b_col0) {
  static_assert(TA::COLS == TB::ROWS, "inner dimensions differ");
  constexpr int K = TA::COLS;
  constexpr int KS = K / MF<MS>::KSTEP;
  constexpr int RB = RTile<MS, R, C>::RB, CB = RTile<MS, R, C>::CB;
  static_assert(K % MF<MS>::KSTEP == 0, "k tile must be a multiple of the MFMA k");
  const int lane = lane_id();
  const int lh = lane / MS;
  const int ngrp = (lane % MS) & ~15;
  bf16x8 bop[2][RB];
  bf16x8 aop[2][CB];
  auto read = [&](int ks, int buf) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) bop[buf][rb] = row_operand<TA, MS>(a_base, a_row0 + rb * MS, ks);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int k0 = ks * MF<MS>::KSTEP + 8 * lh;
      const int n0 = b_col0 + cb * MS + ngrp;
      aop[buf][cb] = cat(tr_operand4<TB>(b_base, k0, n0), tr_operand4<TB>(b_base, k0 + 4, n0));
    }
  };
  read(0, 0);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    __builtin_amdgcn_sched_barrier(0);
    if (ks + 1 < KS) read(ks + 1, (ks + 1) & 1);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc.f[cb][rb] = MF<MS>::mma(aop[ks & 1][cb], bop[ks & 1][rb], acc.f[cb][rb]);
    if (ks + 1 < KS) {
      constexpr int NREAD = RB + 2 * CB;
      constexpr int NMMA = RB * CB;
      constexpr int PAIRS = NREAD < NMMA ? NREAD : NMMA;
#pragma unroll
      for (int q = 0; q < PAIRS; ++q) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one LDS read
      }
      if (NMMA > PAIRS) __builtin_amdgcn_sched_group_barrier(0x008, NMMA - PAIRS, 0);
      if (NREAD > PAIRS) __builtin_amdgcn_sched_group_barrier(0x100, NREAD - PAIRS, 0);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Rotated form of mma_AB for the steady state of a pipelined ring loop
// (wait on slot -> loads -> MMA on that slot).  run() first issues the
// MFMAs of the previous call's last k-step from registers -- so the matrix
// core has work right after the wait's barrier -- interleaved with the LDS
// reads of this tile's first k-step, then k-steps 0..KS-2, and leaves the
// last k-step's fragments pending.  finish() issues the pending MFMAs.
// The order of MFMAs into every accumulator is exactly mma_AB's.  The
// pending fragments start as zeros, whose MFMAs add nothing.
template <int MS, int R, int C, class TA, class TB>
struct MMAPipeAB {
  static constexpr int K = TA::COLS;
  static constexpr int KS = K / MF<MS>::KSTEP;
  static constexpr int RB = RTile<MS, R, C>::RB, CB = RTile<MS, R, C>::CB;
  static constexpr int NREAD = RB + 2 * CB;
  static constexpr int NMMA = RB * CB;
  static_assert(TA::COLS == TB::ROWS, "inner dimensions differ");
  static_assert(K % MF<MS>::KSTEP == 0, "k tile must be a multiple of the MFMA k");
  static_assert(KS % 2 == 0, "the rotated pipeline alternates two fragment buffers");
  bf16x8 bop[2][RB];
  bf16x4 aop[2][CB][2];

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) bop[(KS - 1) & 1][rb] = bf16x8{};
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) aop[(KS - 1) & 1][cb][0] = aop[(KS - 1) & 1][cb][1] = bf16x4{};
  }

  __device__ __forceinline__ void read(char* a_base, int a_row0, char* b_base, int b_col0, int ks, int buf) {
    const int lane = lane_id();
    const int lh = lane / MS;
    const int ngrp = (lane % MS) & ~15;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) bop[buf][rb] = row_operand<TA, MS>(a_base, a_row0 + rb * MS, ks);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) {
      const int k0 = ks * MF<MS>::KSTEP + 8 * lh;
      const int n0 = b_col0 + cb * MS + ngrp;
      aop[buf][cb][0] = tr_operand4<TB>(b_base, k0, n0);
      aop[buf][cb][1] = tr_operand4<TB>(b_base, k0 + 4, n0);
    }
  }

  __device__ __forceinline__ void mfmas(RTile<MS, R, C>& acc, int buf) {
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc.f[cb][rb] = MF<MS>::mma(cat(aop[buf][cb][0], aop[buf][cb][1]), bop[buf][rb], acc.f[cb][rb]);
  }

  // Read item q (0 <= q < NREAD) of k-step ks into buffer buf: the RB row
  // operands first, then the 2*CB transposed half-operands.
  __device__ __forceinline__ void read_item(char* a_base, int a_row0, char* b_base, int b_col0, int ks, int buf,
                                            int q) {
    const int lane = lane_id();
    const int lh = lane / MS;
    if (q < RB) {
      bop[buf][q] = row_operand<TA, MS>(a_base, a_row0 + q * MS, ks);
      return;
    }
    const int cb = (q - RB) / 2, half = (q - RB) % 2;
    const int k0 = ks * MF<MS>::KSTEP + 8 * lh + 4 * half;
    const int n0 = b_col0 + cb * MS + ((lane % MS) & ~15);
    aop[buf][cb][half] = tr_operand4<TB>(b_base, k0, n0);
  }

  // One steady-state step.  The previous tile's pending k-step MFMAs are
  // issued first, each followed by one LDS read of this tile's first
  // k-step; then k-steps 0..KS-2, each MFMA followed by one read of the
  // next k-step.  The NLOAD DMA instructions of this iteration (`loads(q)`)
  // go after every EVERY-th MFMA from the start, i.e. spread over the first
  // half of the tile's MFMAs: bunched DMA issue stalls the issuing wave
  // (measured: 2764 -> 2416 cycles per 256x256x64 step with one DMA every
  // second MFMA), and issuing them later leaves too little time for them to
  // land before the next barrier.  With WHOLE the loads spread over all the
  // tile's MFMAs instead: for rings whose later loads have a step more to
  // land (a deeper ring on the operand issued last), so the CU's address
  // unit sees half the DMA rate.  sched_barrier fences pin the order.
  template <int NLOAD, bool WHOLE = false, class LoadFn>
  __device__ __forceinline__ void run(RTile<MS, R, C>& acc, char* a_base, int a_row0, char* b_base, int b_col0,
                                      LoadFn loads) {
    constexpr int PEND = (KS - 1) & 1;
    constexpr int HALF = WHOLE ? NMMA * KS : (NMMA * KS) / 2;
    constexpr int EVERY = NLOAD > 0 && HALF / NLOAD > 1 ? HALF / NLOAD : 1;
    int nl = 0;
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < NMMA; ++q) {
      const int cb = q / RB, rb = q % RB;
      acc.f[cb][rb] = MF<MS>::mma(cat(aop[PEND][cb][0], aop[PEND][cb][1]), bop[PEND][rb], acc.f[cb][rb]);
      __builtin_amdgcn_sched_barrier(0);
      if (q % EVERY == 0 && nl < NLOAD) loads(nl++);
      if (q < NREAD) read_item(a_base, a_row0, b_base, b_col0, 0, 0, q);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = NMMA; q < NREAD; ++q) read_item(a_base, a_row0, b_base, b_col0, 0, 0, q);
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
#pragma unroll
      for (int q = 0; q < NMMA; ++q) {
        const int cb = q / RB, rb = q % RB;
        acc.f[cb][rb] = MF<MS>::mma(cat(aop[ks & 1][cb][0], aop[ks & 1][cb][1]), bop[ks & 1][rb], acc.f[cb][rb]);
        __builtin_amdgcn_sched_barrier(0);
        if (q % EVERY == 0 && nl < NLOAD) loads(nl++);
        if (q < NREAD) read_item(a_base, a_row0, b_base, b_col0, ks + 1, (ks + 1) & 1, q);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int q = NMMA; q < NREAD; ++q) read_item(a_base, a_row0, b_base, b_col0, ks + 1, (ks + 1) & 1, q);
    }
    while (nl < NLOAD) loads(nl++);
    __builtin_amdgcn_sched_barrier(0);
  }

  __device__ __forceinline__ void finish(RTile<MS, R, C>& acc) {
    mfmas(acc, (KS - 1) & 1);
    init();
  }
};

// 8-wave ping-pong form of the ring-pipelined MMA (a 256x256 block tile as
// 8 wavefronts, two per SIMD).  Every wavefront runs the same step per
// tile -- a memory phase (the LDS reads of the tile's MFMA fragments and,
// in group 0 = wavefronts 0-3, the LDS-DMA of the tile the IR loads this
// iteration), a barrier, then a compute phase of MFMAs from registers, and
// the barrier that opens the next memory phase -- but group 1 (wavefronts
// 4-7) starts one barrier later and group 0 ends one barrier later.  The
// groups are therefore one phase apart: on every SIMD one wavefront feeds
// the matrix core while its partner moves data.  Both groups execute the
// same number of barriers.  A slot is refilled (by group 0's DMA in the
// memory phase of tile t) only after both groups have read its previous
// tile t-1 in the two phases before; group 0 waits for its own DMAs of
// tile t before the barrier that opens the first phase reading it.
// MFMAs into each accumulator run in k order, exactly as mma_AB.
template <int MS, int R, int C, class TA, class TB>
struct PingPongAB {
  static constexpr int K = TA::COLS;
  static constexpr int KS = K / MF<MS>::KSTEP;
  static constexpr int RB = RTile<MS, R, C>::RB, CB = RTile<MS, R, C>::CB;
  static_assert(TA::COLS == TB::ROWS, "inner dimensions differ");
  static_assert(K % MF<MS>::KSTEP == 0, "k tile must be a multiple of the MFMA k");
  int group;

  // Drain the prologue's DMAs (issued by all eight wavefronts), then put
  // group 1 one barrier behind group 0.
  __device__ __forceinline__ void init(int wave) {
    group = wave >> 2;
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (group != 0) barrier();
  }

  // One step on tile t (slot pointers a_t, b_t).  Group 0 also issues NLOAD
  // DMAs via loads(q) and, first, waits until at most VM of its DMAs (those
  // of tiles newer than t) are in flight.
  template <int VM, int NLOAD, class LoadFn>
  __device__ __forceinline__ void step(RTile<MS, R, C>& acc, char* a_t, int a_row0, char* b_t, int b_col0,
                                       LoadFn loads) {
    if (group == 0) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" :: "n"(VM) : "memory");
    else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const int lane = lane_id();
    const int lh = lane / MS;
    const int ngrp = (lane % MS) & ~15;
    bf16x8 bop[KS][RB];
    bf16x4 aop[KS][CB][2];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) bop[ks][rb] = row_operand<TA, MS>(a_t, a_row0 + rb * MS, ks);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int k0 = ks * MF<MS>::KSTEP + 8 * lh;
        const int n0 = b_col0 + cb * MS + ngrp;
        aop[ks][cb][0] = tr_operand4<TB>(b_t, k0, n0);
        aop[ks][cb][1] = tr_operand4<TB>(b_t, k0 + 4, n0);
      }
    }
    if (group == 0) {
#pragma unroll
      for (int q = 0; q < NLOAD; ++q) loads(q);
    }
    barrier();
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc.f[cb][rb] = MF<MS>::mma(cat(aop[ks][cb][0], aop[ks][cb][1]), bop[ks][rb], acc.f[cb][rb]);
    __builtin_amdgcn_s_setprio(0);
  }

  // Group 0 matches group 1's extra barrier.
  __device__ __forceinline__ void finish(RTile<MS, R, C>&) {
    if (group == 0) barrier();
  }
};

// acc = a @ b^T with `a` from hoisted register fragments or LDS; b: ROWREAD LDS [.][K].
// The LDS reads of b run LOOK k-steps ahead of the MFMAs that use them
// (explicit ring of fragment registers, order pinned by sched_barrier):
// left to itself the compiler issues each read right before its MFMA at
// two wavefronts per SIMD, exposing the LDS latency once per k-step.
template <int MS, int R, int C, class TB, int KS>
__device__ __forceinline__ void mma_ABt_frags(RTile<MS, R, C>& acc, const RowFrags<MS, R / MS, KS>& a,
                                              char* b_base, int b_row0) {
  static_assert(TB::COLS == KS * MF<MS>::KSTEP, "inner dimensions differ");
  constexpr int CB = RTile<MS, R, C>::CB, RB = RTile<MS, R, C>::RB;
  constexpr int LOOK = KS < 2 ? KS : 2;
  bf16x8 ring[LOOK + 1][CB];
  __builtin_amdgcn_s_setprio(1);  // MFMA run first; a co-resident wave's VALU fills the gaps
#pragma unroll
  for (int p = 0; p < LOOK; ++p)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) ring[p][cb] = row_operand<TB, MS>(b_base, b_row0 + cb * MS, p);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (ks + LOOK < KS) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        ring[(ks + LOOK) % (LOOK + 1)][cb] = row_operand<TB, MS>(b_base, b_row0 + cb * MS, ks + LOOK);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const typename MF<MS>::cvec c0 = ks == 0 ? typename MF<MS>::cvec{} : acc.f[cb][rb];
        acc.f[cb][rb] = MF<MS>::mma(ring[ks % (LOOK + 1)][cb], a.f[rb][ks], c0);
      }
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);
}

template <int MS, int R, int C, class TA, class TB>
__device__ __forceinline__ void mma_ABt(RTile<MS, R, C>& acc, char* a_base, int a_row0, char* b_base,
                                        int b_row0) {
  static_assert(TA::COLS == TB::COLS, "inner dimensions differ");
  constexpr int KS = TA::COLS / MF<MS>::KSTEP;
  fill(acc, 0.f);
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    bf16x8 bop[RTile<MS, R, C>::RB];
#pragma unroll
    for (int rb = 0; rb < acc.RB; ++rb) bop[rb] = row_operand<TA, MS>(a_base, a_row0 + rb * MS, ks);
#pragma unroll
    for (int cb = 0; cb < acc.CB; ++cb) {
      const bf16x8 aop = row_operand<TB, MS>(b_base, b_row0 + cb * MS, ks);
#pragma unroll
      for (int rb = 0; rb < acc.RB; ++rb) acc.f[cb][rb] = MF<MS>::mma(aop, bop[rb], acc.f[cb][rb]);
    }
  }
}

// acc += a @ b with `a` a bf16 register tile (lane = row, k along its
// columns) and b: TRREAD LDS [K][.].  The k order inside each MFMA follows
// the register layout of `a`: its 4-register group g of column block kb
// covers k = kb*MS + g*4*LG + 4*lh + (0..3).  The transposed LDS reads of b
// run LOOK MFMAs ahead of their use (see mma_ABt_frags).
template <int MS, int R, int K, int C, class TB>
__device__ __forceinline__ void mma_rAB(RTile<MS, R, C>& acc, const BTile<MS, R, K>& a, char* b_base,
                                        int b_col0) {
  static_assert(TB::ROWS == K, "inner dimensions differ");
  constexpr int G = BTile<MS, R, K>::G;      // 4-register groups per C fragment
  constexpr int NG = (K / MS) * G;            // groups along k
  static_assert(NG % 2 == 0, "k extent must fill whole MFMAs");
  constexpr int CB = RTile<MS, R, C>::CB, RB = RTile<MS, R, C>::RB;
  constexpr int ITEMS = (NG / 2) * CB;        // one B operand (two half reads) per item
  constexpr int LOOK = ITEMS < 4 ? ITEMS : 4;
  const int lane = lane_id();
  const int lh = lane / MS;
  const int ngrp = (lane % MS) & ~15;
  auto read = [&](int t) {
    const int q = 2 * (t / CB), cb = t % CB;
    const int kb0 = q / G, g0 = q % G, kb1 = (q + 1) / G, g1 = (q + 1) % G;
    const int k0 = kb0 * MS + g0 * 4 * MF<MS>::LG + 4 * lh;
    const int k1 = kb1 * MS + g1 * 4 * MF<MS>::LG + 4 * lh;
    const int n0 = b_col0 + cb * MS + ngrp;
    return cat(tr_operand4<TB>(b_base, k0, n0), tr_operand4<TB>(b_base, k1, n0));
  };
  bf16x8 ring[LOOK + 1];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int p = 0; p < LOOK; ++p) ring[p] = read(p);
#pragma unroll
  for (int t = 0; t < ITEMS; ++t) {
    if (t + LOOK < ITEMS) ring[(t + LOOK) % (LOOK + 1)] = read(t + LOOK);
    __builtin_amdgcn_sched_barrier(0);
    const int q = 2 * (t / CB), cb = t % CB;
    const int kb0 = q / G, g0 = q % G, kb1 = (q + 1) / G, g1 = (q + 1) % G;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      acc.f[cb][rb] = MF<MS>::mma(ring[t % (LOOK + 1)], cat(a.f[kb0][rb][g0], a.f[kb1][rb][g1]), acc.f[cb][rb]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);
}

// The first NPRE B operands of an mma_rAB, read ahead of it: the 8-wave
// attention ping-pong reads part of the next PV's V tile in its VALU phase,
// when the wave's own LDS reads have nothing else to do, so its next MFMA
// phase reads that much less.  Item t is the t-th MFMA's B operand in
// mma_rAB's order (k groups in pairs, column blocks inner).
template <int NPRE>
struct RABPre {
  bf16x8 f[NPRE > 0 ? NPRE : 1];
};

template <int MS, int R, int K, int C, class TB>
__device__ __forceinline__ bf16x8 rab_item(char* b_base, int b_col0, int t) {
  constexpr int G = BTile<MS, R, K>::G;
  constexpr int CB = RTile<MS, R, C>::CB;
  const int lane = lane_id();
  const int lh = lane / MS;
  const int ngrp = (lane % MS) & ~15;
  const int q = 2 * (t / CB), cb = t % CB;
  const int kb0 = q / G, g0 = q % G, kb1 = (q + 1) / G, g1 = (q + 1) % G;
  const int k0 = kb0 * MS + g0 * 4 * MF<MS>::LG + 4 * lh;
  const int k1 = kb1 * MS + g1 * 4 * MF<MS>::LG + 4 * lh;
  const int n0 = b_col0 + cb * MS + ngrp;
  return cat(tr_operand4<TB>(b_base, k0, n0), tr_operand4<TB>(b_base, k1, n0));
}

template <int MS, int R, int K, int C, class TB, int NPRE>
__device__ __forceinline__ void prefetch_rAB(RABPre<NPRE>& pre, char* b_base, int b_col0) {
#pragma unroll
  for (int t = 0; t < NPRE; ++t) pre.f[t] = rab_item<MS, R, K, C, TB>(b_base, b_col0, t);
}

// mma_rAB whose first NPRE B operands come from `pre` (prefetch_rAB of the
// same tile); the others are read LOOK MFMAs ahead as in mma_rAB.
template <int MS, int R, int K, int C, class TB, int NPRE>
__device__ __forceinline__ void mma_rAB_pre(RTile<MS, R, C>& acc, const BTile<MS, R, K>& a, const RABPre<NPRE>& pre,
                                            char* b_base, int b_col0) {
  static_assert(TB::ROWS == K, "inner dimensions differ");
  constexpr int G = BTile<MS, R, K>::G;
  constexpr int NG = (K / MS) * G;
  constexpr int CB = RTile<MS, R, C>::CB, RB = RTile<MS, R, C>::RB;
  constexpr int ITEMS = (NG / 2) * CB;
  static_assert(NPRE >= 0 && NPRE <= ITEMS, "prefetched operands must be items of this product");
  constexpr int REST = ITEMS - NPRE;
  constexpr int LOOK = REST < 4 ? REST : 4;
  bf16x8 ring[LOOK + 1];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int p = 0; p < LOOK; ++p) ring[p] = rab_item<MS, R, K, C, TB>(b_base, b_col0, NPRE + p);
#pragma unroll
  for (int t = 0; t < ITEMS; ++t) {
    const int u = t - NPRE;
    if (u >= 0 && u + LOOK < REST) ring[(u + LOOK) % (LOOK + 1)] = rab_item<MS, R, K, C, TB>(b_base, b_col0, t + LOOK);
    __builtin_amdgcn_sched_barrier(0);
    const int q = 2 * (t / CB), cb = t % CB;
    const int kb0 = q / G, g0 = q % G, kb1 = (q + 1) / G, g1 = (q + 1) % G;
    const bf16x8 bop = u < 0 ? pre.f[t < NPRE ? t : 0] : ring[(u < 0 ? 0 : u) % (LOOK + 1)];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      acc.f[cb][rb] = MF<MS>::mma(bop, cat(a.f[kb0][rb][g0], a.f[kb1][rb][g1]), acc.f[cb][rb]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);
}

// ---------------------------------------------------------------------------
// Software-pipelined attention (the lowering's overlapped form).
//
// Per KV tile i the lowering emits S_{i+1} = Q K_{i+1}^T through
// mma_ABt_frags_slots and O += P_i V_i through mma_rAB_slots, and passes
// each a `slot` functor.  After every MFMA (group) the functor is called
// with the group's index as a compile-time constant and issues that slot's
// share of the work that does not depend on the MFMAs in flight: the
// softmax of tile i, the running-max update of tile i+1, the DMAs of the
// next tiles.  sched_barrier pins "MFMA, then its slot's VALU": a wave
// keeps issuing independent VALU instructions while its MFMA runs (measured
// on gfx950: up to ~5 per 32-cycle 32x32x16 MFMA at no cost to the MFMA
// rate), where the unpipelined loop leaves the MFMA pipe idle during the
// softmax unless the other wave on the SIMD happens to be in its MFMA phase.
template <int N>
struct ic {
  static constexpr int value = N;
};

template <int T, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (T < N) {
    f(ic<T>{});
    static_for<T + 1, N>(f);
  }
}

template <int MS, int R, int C, class TB, int KS, class SlotF>
__device__ __forceinline__ void mma_ABt_frags_slots(RTile<MS, R, C>& acc, const RowFrags<MS, R / MS, KS>& a,
                                                    char* b_base, int b_row0, SlotF&& slot) {
  static_assert(TB::COLS == KS * MF<MS>::KSTEP, "inner dimensions differ");
  constexpr int CB = RTile<MS, R, C>::CB, RB = RTile<MS, R, C>::RB;
  constexpr int LOOK = KS < 2 ? KS : 2;
  bf16x8 ring[LOOK + 1][CB];
#pragma unroll
  for (int p = 0; p < LOOK; ++p)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) ring[p][cb] = row_operand<TB, MS>(b_base, b_row0 + cb * MS, p);
  static_for<0, KS>([&](auto ksc) {
    constexpr int ks = decltype(ksc)::value;
    if constexpr (ks + LOOK < KS) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        ring[(ks + LOOK) % (LOOK + 1)][cb] = row_operand<TB, MS>(b_base, b_row0 + cb * MS, ks + LOOK);
    }
    static_for<0, CB>([&](auto cbc) {
      constexpr int cb = decltype(cbc)::value;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const typename MF<MS>::cvec c0 = ks == 0 ? typename MF<MS>::cvec{} : acc.f[cb][rb];
        acc.f[cb][rb] = MF<MS>::mma(ring[ks % (LOOK + 1)][cb], a.f[rb][ks], c0);
      }
      __builtin_amdgcn_sched_barrier(0);
      slot(ic<ks * CB + cb>{});
      __builtin_amdgcn_sched_barrier(0);
    });
  });
}

template <int MS, int R, int K, int C, class TB, class SlotF>
__device__ __forceinline__ void mma_rAB_slots(RTile<MS, R, C>& acc, const BTile<MS, R, K>& a, char* b_base,
                                              int b_col0, SlotF&& slot) {
  static_assert(TB::ROWS == K, "inner dimensions differ");
  constexpr int G = BTile<MS, R, K>::G;
  constexpr int NG = (K / MS) * G;
  static_assert(NG % 2 == 0, "k extent must fill whole MFMAs");
  constexpr int CB = RTile<MS, R, C>::CB, RB = RTile<MS, R, C>::RB;
  constexpr int ITEMS = (NG / 2) * CB;
  constexpr int LOOK = ITEMS < 4 ? ITEMS : 4;
  const int lane = lane_id();
  const int lh = lane / MS;
  const int ngrp = (lane % MS) & ~15;
  auto read = [&](int t) {
    const int q = 2 * (t / CB), cb = t % CB;
    const int kb0 = q / G, g0 = q % G, kb1 = (q + 1) / G, g1 = (q + 1) % G;
    const int k0 = kb0 * MS + g0 * 4 * MF<MS>::LG + 4 * lh;
    const int k1 = kb1 * MS + g1 * 4 * MF<MS>::LG + 4 * lh;
    const int n0 = b_col0 + cb * MS + ngrp;
    return cat(tr_operand4<TB>(b_base, k0, n0), tr_operand4<TB>(b_base, k1, n0));
  };
  bf16x8 ring[LOOK + 1];
#pragma unroll
  for (int p = 0; p < LOOK; ++p) ring[p] = read(p);
  static_for<0, ITEMS>([&](auto tc) {
    constexpr int t = decltype(tc)::value;
    if constexpr (t + LOOK < ITEMS) ring[(t + LOOK) % (LOOK + 1)] = read(t + LOOK);
    constexpr int q = 2 * (t / CB), cb = t % CB;
    constexpr int kb0 = q / G, g0 = q % G, kb1 = (q + 1) / G, g1 = (q + 1) % G;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      acc.f[cb][rb] = MF<MS>::mma(ring[t % (LOOK + 1)], cat(a.f[kb0][rb][g0], a.f[kb1][rb][g1]), acc.f[cb][rb]);
    __builtin_amdgcn_sched_barrier(0);
    slot(ic<t>{});
    __builtin_amdgcn_sched_barrier(0);
  });
}

// ---------------------------------------------------------------------------
// Element-wise tile ops restricted to register groups [G0, G1): group q is
// the 4 C registers 4g..4g+3 of block (cb, rb), numbered (cb, rb, g).  A
// chain of element-wise ops may run group by group, each MFMA slot of an
// independent MMA (mma_*_slots) carrying its share, since every element of
// the chain depends only on the same element of its inputs (and on its row
// or column value).
template <int G0, int G1, int MS, int R, int C, class F>
__device__ __forceinline__ void each_group(F&& f) {
  constexpr int RB = R / MS, GPB = MF<MS>::CREGS / 4;
  static_assert(0 <= G0 && G0 <= G1 && G1 <= (C / MS) * RB * GPB, "register group range out of the tile");
#pragma unroll
  for (int q = G0; q < G1; ++q) f(q / (RB * GPB), (q / GPB) % RB, q % GPB);
}

template <int G0, int G1, int MS, int R, int C, class F>
__device__ __forceinline__ void map_part(RTile<MS, R, C>& out, const RTile<MS, R, C>& in, F fn) {
  each_group<G0, G1, MS, R, C>([&](int cb, int rb, int g) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out.f[cb][rb][4 * g + j] = fn(in.f[cb][rb][4 * g + j], rb);
  });
}

template <int G0, int G1, int MS, int R, int C, class F>
__device__ __forceinline__ void map2_part(RTile<MS, R, C>& out, const RTile<MS, R, C>& a, const RTile<MS, R, C>& b,
                                          F fn) {
  each_group<G0, G1, MS, R, C>([&](int cb, int rb, int g) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out.f[cb][rb][4 * g + j] = fn(a.f[cb][rb][4 * g + j], b.f[cb][rb][4 * g + j]);
  });
}

template <int G0, int G1, int MS, int R, int C, class F>
__device__ __forceinline__ void col_apply_part(RTile<MS, R, C>& out, const RTile<MS, R, C>& t, const CVec<MS, C>& v,
                                               F fn) {
  each_group<G0, G1, MS, R, C>([&](int cb, int rb, int g) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out.f[cb][rb][4 * g + j] = fn(t.f[cb][rb][4 * g + j], v.v[cb][4 * g + j]);
  });
}

template <int G0, int G1, int MS, int R, int C, class F>
__device__ __forceinline__ void row_apply_part(RTile<MS, R, C>& out, const RTile<MS, R, C>& t, const RVec<MS, R>& v,
                                               F fn) {
  each_group<G0, G1, MS, R, C>([&](int cb, int rb, int g) {
#pragma unroll
    for (int j = 0; j < 4; ++j) out.f[cb][rb][4 * g + j] = fn(t.f[cb][rb][4 * g + j], v.v[rb]);
  });
}

template <int G0, int G1, int MS, int R, int C>
__device__ __forceinline__ void to_bf16_part(BTile<MS, R, C>& out, const RTile<MS, R, C>& in) {
  each_group<G0, G1, MS, R, C>([&](int cb, int rb, int g) {
    bf16x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (bf16)in.f[cb][rb][4 * g + j];
    out.f[cb][rb][g] = v;
  });
}

// Element pairs [P0, P1) of a lane = row tile (pair p = registers 2p, 2p+1
// in (cb, rb, i) order): p = fn(s, rb) in fp32, added to the lane's partial
// row sums and packed to bf16 into `pb`.
template <int P0, int P1, int MS, int R, int C, class F>
__device__ __forceinline__ void e_pairs(const RTile<MS, R, C>& s, BTile<MS, R, C>& pb, float (&rsum)[R / MS],
                                        F fn) {
  constexpr int RB = R / MS, CR = MF<MS>::CREGS;
#pragma unroll
  for (int p = P0; p < P1; ++p) {
    const int e = 2 * p;
    const int cb = e / (RB * CR), rb = (e / CR) % RB, i = e % CR;
    const float x0 = fn(s.f[cb][rb][i], rb), x1 = fn(s.f[cb][rb][i + 1], rb);
    rsum[rb] += x0;
    rsum[rb] += x1;
    pb.f[cb][rb][i / 4][i % 4] = (bf16)x0;
    pb.f[cb][rb][i / 4][i % 4 + 1] = (bf16)x1;
  }
}

// Partial row reduction over elements [E0, E1) (in (cb, rb, i) order) into
// lane-local accumulators; row_finish completes it across the lane groups.
template <int E0, int E1, int MS, int R, int C, class F>
__device__ __forceinline__ void row_partial(float (&acc)[R / MS], const RTile<MS, R, C>& t, F op) {
  constexpr int RB = R / MS, CR = MF<MS>::CREGS;
#pragma unroll
  for (int e = E0; e < E1; ++e) {
    const int cb = e / (RB * CR), rb = (e / CR) % RB, i = e % CR;
    acc[rb] = op(acc[rb], t.f[cb][rb][i]);
  }
}

// ---------------------------------------------------------------------------
// Element-wise and row operations on lane = row tiles.
template <int MS, int R, int C, class F>
__device__ __forceinline__ void map(RTile<MS, R, C>& out, const RTile<MS, R, C>& in, F fn) {
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < out.RB; ++rb)
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) out.f[cb][rb][i] = fn(in.f[cb][rb][i], rb);
}

template <int MS, int R, int C, class F>
__device__ __forceinline__ void map2(RTile<MS, R, C>& out, const RTile<MS, R, C>& a,
                                     const RTile<MS, R, C>& b, F fn) {
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < out.RB; ++rb)
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) out.f[cb][rb][i] = fn(a.f[cb][rb][i], b.f[cb][rb][i]);
}

template <int MS, int C, class F>
__device__ __forceinline__ void cvmap(CVec<MS, C>& out, const CVec<MS, C>& in, F fn) {
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int i = 0; i < MF<MS>::CREGS; ++i) out.v[cb][i] = fn(in.v[cb][i]);
}

template <int MS, int C, class F>
__device__ __forceinline__ void cvmap2(CVec<MS, C>& out, const CVec<MS, C>& a, const CVec<MS, C>& b, F fn) {
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int i = 0; i < MF<MS>::CREGS; ++i) out.v[cb][i] = fn(a.v[cb][i], b.v[cb][i]);
}

// out[r, c] = fn(t[r, c], v[c]).
template <int MS, int R, int C, class F>
__device__ __forceinline__ void col_apply(RTile<MS, R, C>& out, const RTile<MS, R, C>& t, const CVec<MS, C>& v, F fn) {
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < out.RB; ++rb)
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) out.f[cb][rb][i] = fn(t.f[cb][rb][i], v.v[cb][i]);
}

// Per-column values from an fp32 vector global [b, d, n] (unit column):
// columns col0.. of this wavefront's tile; indices >= n read 0.
template <int MS, int C>
__device__ __forceinline__ void load_cvec(CVec<MS, C>& out, const gl<float>& g, int b, int d, int col0) {
  const int lh = lane_id() / MS;
  const bool bd_ok = (unsigned)b < (unsigned)g.b && (unsigned)d < (unsigned)g.d;
  const float* base = g.data + (long long)b * g.sb + (long long)d * g.sd;
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int q = 0; q < MF<MS>::CREGS / 4; ++q) {
      const int c = col0 + cb * MS + ccol<MS>(4 * q, lh);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        out.v[cb][4 * q + j] = (bd_ok && c + j < g.r) ? base[(long long)(c + j) * g.sr] : 0.f;
    }
}

// Per-row values from an fp32 vector global [b, d, n]: rows row0.. of this
// wavefront's tile (one per row block and lane); indices >= n read 0.
template <int MS, int R>
__device__ __forceinline__ void load_rvec(RVec<MS, R>& out, const gl<float>& g, int b, int d, int row0) {
  const bool bd_ok = (unsigned)b < (unsigned)g.b && (unsigned)d < (unsigned)g.d;
  const float* base = g.data + (long long)b * g.sb + (long long)d * g.sd;
#pragma unroll
  for (int rb = 0; rb < out.RB; ++rb) {
    const int r = row0 + rb * MS + lane_id() % MS;
    out.v[rb] = (bd_ok && r < g.r) ? base[(long long)r * g.sr] : 0.f;
  }
}

// Per-column / per-row values from an fp32 vector tile in LDS (see load_cvec
// and load_rvec for the register layout).
template <int MS, int C>
__device__ __forceinline__ void load_cvec_lds(CVec<MS, C>& out, char* vec_base, int col0) {
  const int lh = lane_id() / MS;
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int q = 0; q < MF<MS>::CREGS / 4; ++q) {
      const int c = col0 + cb * MS + ccol<MS>(4 * q, lh);
      const f32x4 v = *(__attribute__((address_space(3))) f32x4*)(lds(vec_base) + c * 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) out.v[cb][4 * q + j] = v[j];
    }
}

template <int MS, int R>
__device__ __forceinline__ void load_rvec_lds(RVec<MS, R>& out, char* vec_base, int row0) {
#pragma unroll
  for (int rb = 0; rb < out.RB; ++rb)
    out.v[rb] = *(__attribute__((address_space(3))) float*)(lds(vec_base) + (row0 + rb * MS + lane_id() % MS) * 4);
}

// bf16 LDS tile -> fp32 register tile (lane = row layout): rows row0..,
// columns col0.. of the tile.
template <class Tile, int MS, int R, int C>
__device__ __forceinline__ void load_tile(RTile<MS, R, C>& out, char* tile_base, int row0, int col0) {
  const int lane = lane_id();
  const int lr = lane % MS, lh = lane / MS;
#pragma unroll
  for (int rb = 0; rb < out.RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
      for (int q = 0; q < MF<MS>::CREGS / 4; ++q) {
        const bf16x4 v = row_operand4<Tile>(tile_base, row0 + rb * MS + lr, col0 + cb * MS + ccol<MS>(4 * q, lh));
#pragma unroll
        for (int j = 0; j < 4; ++j) out.f[cb][rb][4 * q + j] = (float)v[j];
      }
}

template <int MS, int R, class F>
__device__ __forceinline__ void vmap(RVec<MS, R>& out, const RVec<MS, R>& in, F fn) {
#pragma unroll
  for (int rb = 0; rb < out.RB; ++rb) out.v[rb] = fn(in.v[rb]);
}

template <int MS, int R, class F>
__device__ __forceinline__ void vmap2(RVec<MS, R>& out, const RVec<MS, R>& a, const RVec<MS, R>& b, F fn) {
#pragma unroll
  for (int rb = 0; rb < out.RB; ++rb) out.v[rb] = fn(a.v[rb], b.v[rb]);
}

// Combine a value across the lanes that hold the same row (lane groups).
template <int MS, class F>
__device__ __forceinline__ float lane_group_reduce(float x, F op) {
  if (MS == 32) {
    auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
  } else {
    x = op(x, __shfl_xor(x, 16));
    return op(x, __shfl_xor(x, 32));
  }
}

struct OpMax { __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpAdd { __device__ __forceinline__ float operator()(float a, float b) const { return a + b; } };

// out[r] = op(op_c tile[r, c], prev[r]).
template <int MS, int R, int C, class F>
__device__ __forceinline__ void row_reduce(RVec<MS, R>& out, const RTile<MS, R, C>& t, const RVec<MS, R>& prev,
                                           F op) {
#pragma unroll
  for (int rb = 0; rb < out.RB; ++rb) {
    float x = t.f[0][rb][0];
#pragma unroll
    for (int cb = 0; cb < t.CB; ++cb)
#pragma unroll
      for (int i = (cb == 0 ? 1 : 0); i < MF<MS>::CREGS; ++i) x = op(x, t.f[cb][rb][i]);
    x = lane_group_reduce<MS>(x, op);
    out.v[rb] = op(x, prev.v[rb]);
  }
}

// out[r] = op(reduced lane partials of row r, prev[r]) (see row_partial).
template <int MS, int R, class F>
__device__ __forceinline__ void row_finish(RVec<MS, R>& out, const float (&part)[R / MS], const RVec<MS, R>& prev,
                                           F op) {
#pragma unroll
  for (int rb = 0; rb < R / MS; ++rb) out.v[rb] = op(lane_group_reduce<MS>(part[rb], op), prev.v[rb]);
}

template <int MS, int R, int C, class F>
__device__ __forceinline__ void row_apply(RTile<MS, R, C>& out, const RTile<MS, R, C>& t, const RVec<MS, R>& v,
                                          F fn) {
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < out.RB; ++rb) {
      const float s = v.v[rb];
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) out.f[cb][rb][i] = fn(t.f[cb][rb][i], s);
    }
}

// out = t * v[row], skipping the multiplies when every v is exactly 1.0
// (the online-softmax correction once the running maximum has settled):
// x * 1.0f == x bit for bit, so the result is the same either way.
template <int MS, int R, int C>
__device__ __forceinline__ void row_scale(RTile<MS, R, C>& out, const RTile<MS, R, C>& t, const RVec<MS, R>& v) {
  bool ones = true;
#pragma unroll
  for (int rb = 0; rb < out.RB; ++rb) ones = ones && (v.v[rb] == 1.0f);
  if (__builtin_amdgcn_ballot_w64(!ones) == 0) {
    out = t;
    return;
  }
  row_apply(out, t, v, [](float x, float s) { return x * s; });
}

template <int MS, int R, int C>
__device__ __forceinline__ void to_bf16(BTile<MS, R, C>& out, const RTile<MS, R, C>& in) {
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < out.RB; ++rb)
#pragma unroll
      for (int g = 0; g < out.G; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (bf16)in.f[cb][rb][4 * g + j];
        out.f[cb][rb][g] = v;
      }
}

// The speculative half of lazy_softmax on its own: computes pb and updates l
// and returns true when no score exceeds m + slack; returns false (pb written,
// m and l untouched) when the step needs lazy_softmax's exact path.  A loop
// that calls this and leaves for the exact path keeps every access to o in
// its MFMAs, so o keeps one register assignment around the loop.
template <int MS, int R, int C>
__device__ __forceinline__ bool lazy_softmax_fast(const RTile<MS, R, C>& s, const RVec<MS, R>& m, RVec<MS, R>& l,
                                                  BTile<MS, R, C>& pb, float c, float slack) {
  constexpr int RB = R / MS, CB = C / MS, G = BTile<MS, R, C>::G;
  const float guard = __builtin_amdgcn_exp2f(slack * c);
  float part[RB][4], sum[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j) part[rb][j] = 0.f;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s.f[cb][rb][4 * g + j], c, -m.v[rb] * c));
          part[rb][j] += e;
          v[j] = (bf16)e;
        }
        pb.f[cb][rb][g] = v;
      }
  bool ok = true;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    sum[rb] = (part[rb][0] + part[rb][1]) + (part[rb][2] + part[rb][3]);
    ok = ok && (sum[rb] <= guard);  // false for inf and NaN
  }
  if (__builtin_amdgcn_ballot_w64(!ok) != 0) return false;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) l.v[rb] = lane_group_reduce<MS>(sum[rb], OpAdd()) + l.v[rb];
  return true;
}

// One online-softmax step with a lazy running maximum (the IR ops
//   cand = row_max(s, m); m' = lazy_max(m, cand, slack);
//   p = exp2(s*c - m'*c); corr = exp2(m*c - m'*c);
//   l' = row_sum(p, l*corr); o' = o*corr; pb = bf16(p)
// with m, l, o updated in place), evaluated speculatively.  The step is
// first computed with m' = m.  Every p is at most its lane's partial row
// sum, so when no partial sum exceeds 2^(slack*c) no score exceeds
// m + slack: lazy_max keeps m on every row, corr is exactly 1 and o, l are
// not rescaled, and the speculation is the IR's result.  Otherwise (the
// first tile, where m = -inf, or a tile whose scores rise above m + slack)
// the step is recomputed row by row with the exact lazy maximum
// (lazy_softmax_exact, which a loop that already ran lazy_softmax_fast on
// the tile calls directly).  The fast path is one fma, one exp2, one add and
// half a bf16 pack per score: no row maximum, no rescale.
template <int MS, int R, int C, int DO>
__device__ __forceinline__ void lazy_softmax_exact(const RTile<MS, R, C>& s, RVec<MS, R>& m, RVec<MS, R>& l,
                                                   RTile<MS, R, DO>& o, BTile<MS, R, C>& pb, float c, float slack) {
  constexpr int RB = R / MS, CB = C / MS, G = BTile<MS, R, C>::G;
  float corr[RB], sum[RB], part[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float x = s.f[0][rb][0];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int i = (cb == 0 ? 1 : 0); i < MF<MS>::CREGS; ++i) x = __builtin_fmaxf(x, s.f[cb][rb][i]);
    const float cand = __builtin_fmaxf(lane_group_reduce<MS>(x, OpMax()), m.v[rb]);
    const float mn = cand > m.v[rb] + slack ? cand : m.v[rb];
    corr[rb] = __builtin_amdgcn_exp2f(m.v[rb] * c - mn * c);
    m.v[rb] = mn;
#pragma unroll
    for (int j = 0; j < 4; ++j) part[rb][j] = 0.f;
  }
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s.f[cb][rb][4 * g + j], c, -m.v[rb] * c));
          part[rb][j] += e;
          v[j] = (bf16)e;
        }
        pb.f[cb][rb][g] = v;
      }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    sum[rb] = (part[rb][0] + part[rb][1]) + (part[rb][2] + part[rb][3]);
    l.v[rb] = lane_group_reduce<MS>(sum[rb], OpAdd()) + l.v[rb] * corr[rb];
  }
#pragma unroll
  for (int cb = 0; cb < o.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) o.f[cb][rb][i] *= corr[rb];
}

template <int MS, int R, int C, int DO>
__device__ __forceinline__ void lazy_softmax(const RTile<MS, R, C>& s, RVec<MS, R>& m, RVec<MS, R>& l,
                                             RTile<MS, R, DO>& o, BTile<MS, R, C>& pb, float c, float slack) {
  if (lazy_softmax_fast(s, m, l, pb, c, slack)) return;
  lazy_softmax_exact(s, m, l, o, pb, c, slack);
}

// ---------------------------------------------------------------------------
// Row sums on the matrix core.  A 32-row P tile (lane = row: lane l holds
// row l%32, lanes l and l+32 complementary keys) is summed per row by
// 16x16x32 MFMAs that take two of its 4-element groups (8 bf16 per lane)
// as the B operand, against a 0/1 A operand.  The MFMA reads B lane L as
// column L%16 of k block L/16; with A[m][k] = 1 exactly when the parities
// of m/4 and k/8 agree, C row m sums the k blocks of its parity, so C
// register i of lane l (row 4*(l/16)+i, column l%16) is the sum over
// lanes {l%32, l%32+32}: every C register of a lane holds its own row's sum
// of the 16 probabilities in those two groups.  Four such MFMAs cover a
// 64-key tile, in place of 32 fp32 adds and a cross-lane reduction per lane.
__device__ __forceinline__ bf16x8 rowsum_selector() {
  const int l = lane_id();
  const bf16 e = ((((l & 15) >> 2) ^ (l >> 4)) & 1) == 0 ? (bf16)1.0f : (bf16)0.0f;
  bf16x8 v;
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = e;
  return v;
}

// lazy_softmax_fast with the row sums of the bf16 probabilities from the
// matrix core (rowsum_selector).  The guard is checked on those sums: all
// terms are non-negative and the MFMA adds them exactly from bf16 products,
// so each bf16(p) is at most its row's sum, and a sum at most
// 2^(slack*c) * (1 - 2^-8) bounds every p (at most 2^-9 above its bf16) below
// 2^(slack*c): no score exceeds m + slack, exactly as in lazy_softmax_fast.
// A full-row sum is at least a lane's partial sum, so the guard passes less
// often than lazy_softmax_fast's (the exact half then runs, which computes
// the same step).  l accumulates sums of the rounded probabilities that the
// PV MFMAs multiply, in place of the fp32 ones (at most 2^-9 relative per
// term).  32-row fragments (MS = 32) only.
template <int MS, int R, int C>
__device__ __forceinline__ bool lazy_softmax_fast_mr(const RTile<MS, R, C>& s, const RVec<MS, R>& m, RVec<MS, R>& l,
                                                     BTile<MS, R, C>& pb, float c, float slack) {
  static_assert(MS == 32, "matrix-core row sums take the 32x32 fragment layout");
  constexpr int RB = R / MS, CB = C / MS, G = BTile<MS, R, C>::G;
  static_assert((CB * G) % 2 == 0, "the key tile must fill whole 16x16x32 MFMAs");
  const float guard = __builtin_amdgcn_exp2f(slack * c) * (1.0f - 1.0f / 256.0f);
  const bf16x8 sel = rowsum_selector();
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (bf16)__builtin_amdgcn_exp2f(__builtin_fmaf(s.f[cb][rb][4 * g + j], c, -m.v[rb] * c));
        pb.f[cb][rb][g] = v;
      }
  float sum[RB];
  bool ok = true;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < CB * G; t += 2)
      acc = MF<16>::mma(sel, cat(pb.f[t / G][rb][t % G], pb.f[(t + 1) / G][rb][(t + 1) % G]), acc);
    sum[rb] = acc[0];
    ok = ok && (sum[rb] <= guard);  // false for inf and NaN
  }
  if (__builtin_amdgcn_ballot_w64(!ok) != 0) return false;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) l.v[rb] += sum[rb];
  return true;
}

template <int MS, int R, int C, int DO>
__device__ __forceinline__ void lazy_softmax_mr(const RTile<MS, R, C>& s, RVec<MS, R>& m, RVec<MS, R>& l,
                                                RTile<MS, R, DO>& o, BTile<MS, R, C>& pb, float c, float slack) {
  if (lazy_softmax_fast_mr(s, m, l, pb, c, slack)) return;
  lazy_softmax_exact(s, m, l, o, pb, c, slack);
}

// ---------------------------------------------------------------------------
// Lazy softmax with the scale folded into Q and the running max into the
// score MFMAs.  The hoisted Q fragments are scaled by c once (bf16 of c*q),
// and every column block of S = Q K^T starts with one extra MFMA whose
// operands are (1, 1, 0...) on the key side and (-b_hi, -b_lo, 0...) on the
// query side, b = the running max in scaled units split into two bf16 words
// (b_hi = bf16(b), b_lo = bf16(b - b_hi), exact to ~2^-16 relative).  The
// MFMAs then deliver s = c*S - b directly, and the speculative half is one
// exp2, one add and half a bf16 pack per score, without the fma.  Only
// lanes 0-31 carry operand values: k = 8*(lane/32) + j, so the bias sits in
// k = 0, 1.
template <int RB>
struct ScoreBias {
  float b[RB];       // the bias in the MFMAs, c * running max (0 while the max is -inf)
  bf16x8 q[RB];      // query-side operand per row block
  bf16x8 k;          // key-side operand (the same for every block)
  __device__ __forceinline__ static bf16x8 query_operand(float b) {
    bf16x8 v = {};
    const bf16 hi = (bf16)b;
    const bf16 lo = (bf16)(b - (float)hi);
    if (lane_id() < 32) {
      v[0] = -hi;
      v[1] = -lo;
    }
    return v;
  }
  __device__ __forceinline__ void init() {
    k = bf16x8{};
    if (lane_id() < 32) k[0] = k[1] = (bf16)1.0f;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      b[rb] = 0.f;
      q[rb] = query_operand(0.f);
    }
  }
};

// q *= c in place, bf16 -> fp32 -> bf16 (the scale folded into Q).
template <int MS, int RB, int KS>
__device__ __forceinline__ void scale_frags(RowFrags<MS, RB, KS>& fr, float c) {
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int j = 0; j < 8; ++j) fr.f[rb][ks][j] = (bf16)((float)fr.f[rb][ks][j] * c);
}

// mma_ABt_frags with every accumulator started by the bias MFMA: acc = a b^T - bias.
template <int MS, int R, int C, class TB, int KS>
__device__ __forceinline__ void mma_ABt_frags_bias(RTile<MS, R, C>& acc, const RowFrags<MS, R / MS, KS>& a,
                                                   const ScoreBias<R / MS>& sb, char* b_base, int b_row0) {
  static_assert(MS == 32, "the bias operands follow the 32x32x16 lane layout");
  constexpr int CB = RTile<MS, R, C>::CB, RB = RTile<MS, R, C>::RB;
  constexpr int LOOK = KS < 2 ? KS : 2;
  bf16x8 ring[LOOK + 1][CB];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int p = 0; p < LOOK; ++p)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) ring[p][cb] = row_operand<TB, MS>(b_base, b_row0 + cb * MS, p);
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc.f[cb][rb] = MF<MS>::mma(sb.k, sb.q[rb], typename MF<MS>::cvec{});
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    if (ks + LOOK < KS) {
#pragma unroll
      for (int cb = 0; cb < CB; ++cb)
        ring[(ks + LOOK) % (LOOK + 1)][cb] = row_operand<TB, MS>(b_base, b_row0 + cb * MS, ks + LOOK);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc.f[cb][rb] = MF<MS>::mma(ring[ks % (LOOK + 1)][cb], a.f[rb][ks], acc.f[cb][rb]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);
}

// lazy_softmax_fast on biased scores s = c*S - b: valid while b is the scaled
// running max, i.e. after the step that first set it (lazy_softmax_exact_b).
// `guard` = 2^(slack*c).
template <int MS, int R, int C>
__device__ __forceinline__ bool lazy_softmax_fast_b(const RTile<MS, R, C>& s, RVec<MS, R>& l,
                                                    BTile<MS, R, C>& pb, float guard) {
  constexpr int RB = R / MS, CB = C / MS, G = BTile<MS, R, C>::G;
  float part[RB][4], sum[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j) part[rb][j] = 0.f;
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(s.f[cb][rb][4 * g + j]);
          part[rb][j] += e;
          v[j] = (bf16)e;
        }
        pb.f[cb][rb][g] = v;
      }
  bool ok = true;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    sum[rb] = (part[rb][0] + part[rb][1]) + (part[rb][2] + part[rb][3]);
    ok = ok && (sum[rb] <= guard);  // false for inf and NaN
  }
  if (__builtin_amdgcn_ballot_w64(!ok) != 0) return false;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) l.v[rb] = lane_group_reduce<MS>(sum[rb], OpAdd()) + l.v[rb];
  return true;
}

// lazy_softmax_exact on biased scores s = c*S - b.  m stays in unscaled units
// (the IR's running max); the scaled max is sb.b once m is finite.  With
// cand = max(s) + b: the max moves to cand when cand > c*m + c*slack, then
// p = exp2(s - (m'c - b)), corr = exp2(c*m - m'c), l' = rowsum(p) + l*corr,
// o' = o*corr, and the bias becomes m'c.
template <int MS, int R, int C, int DO>
__device__ __forceinline__ void lazy_softmax_exact_b(const RTile<MS, R, C>& s, RVec<MS, R>& m, RVec<MS, R>& l,
                                                     RTile<MS, R, DO>& o, BTile<MS, R, C>& pb, float c,
                                                     float slack, ScoreBias<R / MS>& sb) {
  constexpr int RB = R / MS, CB = C / MS, G = BTile<MS, R, C>::G;
  float corr[RB], delta[RB], sum[RB], part[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    float x = s.f[0][rb][0];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int i = (cb == 0 ? 1 : 0); i < MF<MS>::CREGS; ++i) x = __builtin_fmaxf(x, s.f[cb][rb][i]);
    const float cand = lane_group_reduce<MS>(x, OpMax()) + sb.b[rb];
    const float old = m.v[rb] == -__builtin_inff() ? -__builtin_inff() : sb.b[rb];
    const bool take = cand > old + slack * c;
    const float mn = take ? cand : old;
    corr[rb] = __builtin_amdgcn_exp2f(old - mn);
    delta[rb] = mn - sb.b[rb];
    if (take) {
      m.v[rb] = cand / c;
      sb.b[rb] = cand;
      sb.q[rb] = ScoreBias<RB>::query_operand(cand);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) part[rb][j] = 0.f;
  }
#pragma unroll
  for (int cb = 0; cb < CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float e = __builtin_amdgcn_exp2f(s.f[cb][rb][4 * g + j] - delta[rb]);
          part[rb][j] += e;
          v[j] = (bf16)e;
        }
        pb.f[cb][rb][g] = v;
      }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    sum[rb] = (part[rb][0] + part[rb][1]) + (part[rb][2] + part[rb][3]);
    l.v[rb] = lane_group_reduce<MS>(sum[rb], OpAdd()) + l.v[rb] * corr[rb];
  }
#pragma unroll
  for (int cb = 0; cb < o.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) o.f[cb][rb][i] *= corr[rb];
}

template <int MS, int R, int C, int DO>
__device__ __forceinline__ void lazy_softmax_b(const RTile<MS, R, C>& s, RVec<MS, R>& m, RVec<MS, R>& l,
                                               RTile<MS, R, DO>& o, BTile<MS, R, C>& pb, float c, float slack,
                                               ScoreBias<R / MS>& sb) {
  // rows whose max is still -inf have no bias yet: the exact half sets it
  bool fresh = false;
#pragma unroll
  for (int rb = 0; rb < R / MS; ++rb) fresh = fresh || m.v[rb] == -__builtin_inff();
  if (__builtin_amdgcn_ballot_w64(fresh) == 0 && lazy_softmax_fast_b(s, l, pb, __builtin_amdgcn_exp2f(slack * c)))
    return;
  lazy_softmax_exact_b(s, m, l, o, pb, c, slack, sb);
}

// Lower-triangular mask: keep (row, col) when col_g <= row_g with
// row_g = row_tile*BR + row0 + r and col_g = col_tile*BC + c.
template <bool TRANSPOSED, int MS, int R, int C>
__device__ __forceinline__ void causal_mask(RTile<MS, R, C>& out, const RTile<MS, R, C>& t, int row_g0,
                                            int col_g0) {
  // every element kept (a wave-uniform test on the tile's corners)
  if (TRANSPOSED ? row_g0 + R - 1 <= col_g0 : col_g0 + C - 1 <= row_g0) {
    out = t;
    return;
  }
  const int lane = lane_id();
  const int lr = lane % MS, lh = lane / MS;
  const float ninf = -__builtin_inff();
#pragma unroll
  for (int cb = 0; cb < out.CB; ++cb)
#pragma unroll
    for (int rb = 0; rb < out.RB; ++rb) {
      const int row = row_g0 + rb * MS + lr;
#pragma unroll
      for (int i = 0; i < MF<MS>::CREGS; ++i) {
        const int col = col_g0 + cb * MS + ccol<MS>(i, lh);
        const bool keep = TRANSPOSED ? row <= col : col <= row;
        out.f[cb][rb][i] = keep ? t.f[cb][rb][i] : ninf;
      }
    }
}

// ---------------------------------------------------------------------------
// Stores (the IR's tma_store) with TMA bounds semantics: elements outside
// the tensor are dropped.

// Register tile -> bf16 or fp32 global; rows from row0, cols from col0.
template <typename T, int MS, int R, int C>
__device__ __forceinline__ void store_tile(const gl<T>& g, const RTile<MS, R, C>& t, int b, int d, int row0,
                                           int col0) {
  if ((unsigned)b >= (unsigned)g.b || (unsigned)d >= (unsigned)g.d) return;
  const int lane = lane_id();
  const int lr = lane % MS, lh = lane / MS;
  T* base = g.data + (long long)b * g.sb + (long long)d * g.sd;
  const bool full_cols = (col0 + C <= g.c) && ((g.c & 3) == 0);
#pragma unroll
  for (int rb = 0; rb < t.RB; ++rb) {
    const int row = row0 + rb * MS + lr;
    if (row >= g.r) continue;
    T* prow = base + (long long)row * g.sr;
#pragma unroll
    for (int cb = 0; cb < t.CB; ++cb)
#pragma unroll
      for (int q = 0; q < MF<MS>::CREGS / 4; ++q) {
        const int col = col0 + cb * MS + ccol<MS>(4 * q, lh);
        if (full_cols) {
          if constexpr (sizeof(T) == 2) {
            bf16x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = (bf16)t.f[cb][rb][4 * q + j];
            *(bf16x4*)(prow + col) = v;
          } else {
            f32x4 v;
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = t.f[cb][rb][4 * q + j];
            *(f32x4*)(prow + col) = v;
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (col + j < g.c) prow[col + j] = (T)t.f[cb][rb][4 * q + j];
        }
      }
  }
}

// Split-K fix-up (the IR's reduce_slices).  Every workgroup calls this, all
// its threads, after storing its fp32 partial tile [row0, row0 + TR) x
// [col0, col0 + TC) of slice blockIdx.z into `part` ([b][slice][row][col]).
// arrivals[idx] counts the slices that have stored the tile.  The release
// fence makes this workgroup's partial stores visible to every XCD before it
// counts itself; the last of the part.d slices to arrive (the counter's old
// value is part.d - 1) takes the acquire fence, sums the slices in slice
// order in fp32 (from 0, as the separate reduction kernel does), writes the
// bf16 tile with the usual bounds (N a multiple of 8) and puts the counter
// back to zero, so a zeroed counter array stays zeroed across launches.  No
// workgroup waits for another.  `flag` is one word of LDS that nothing else
// uses here (the ring is drained by the loop's last wait).
template <int TR, int TC, int NT>
__device__ __forceinline__ void reduce_slices(const gl<float>& part, const gl<bf16>& dst, const gl<unsigned>& arrivals,
                                              int b, int row0, int col0, int idx, char* flag) {
  volatile unsigned* last = (volatile unsigned*)flag;
  // The barrier makes every wave's stores visible within the workgroup; one
  // wave's device-scope fence then releases them all (the fence writes back
  // the XCD's whole L2, so one per workgroup is enough), and the same wave
  // takes the acquire side for the workgroup.
  __syncthreads();
  if (threadIdx.x < 64) {
    __threadfence();
    if (threadIdx.x == 0) *last = atomicAdd(arrivals.data + idx, 1u) == (unsigned)(part.d - 1) ? 1u : 0u;
  }
  __syncthreads();
  if (!*last) return;
  if (threadIdx.x < 64) __threadfence();
  __syncthreads();
  const float* pb = part.data + (long long)b * part.sb;
  bf16* db = dst.data + (long long)b * dst.sb;
  for (int e = threadIdx.x * 8; e < TR * TC; e += NT * 8) {
    const int r = row0 + e / TC, c = col0 + e % TC;
    if (r >= dst.r || c >= dst.c) continue;
    const float* p = pb + (long long)r * part.sr + c;
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
    for (int sl = 0; sl < part.d; ++sl) {
      lo += *(const f32x4*)(p + sl * part.sd);
      hi += *(const f32x4*)(p + sl * part.sd + 4);
    }
    bf16x8 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = (bf16)lo[j];
      v[4 + j] = (bf16)hi[j];
    }
    *(bf16x8*)(db + (long long)r * dst.sr + c) = v;
  }
  if (threadIdx.x == 0) arrivals.data[idx] = 0u;
}

// Register tile -> bf16 global through this wave's private LDS area `stage`
// (R * C * 2 bytes, free for the rest of the kernel).  In the lane = row
// layout one store instruction would touch MS rows with 8 bytes each; the
// staged form writes the bf16 tile to LDS row-major (16-byte chunks XOR-
// swizzled by row) and reads it back as whole rows, so each store
// instruction writes C*2 contiguous bytes per row and 16 bytes per lane.
// NT: the 16-byte stores carry the non-temporal hint.  The kernel never
// reads its output back, and when every workgroup stores its tile at the
// same time (equal-work grids), streaming the writes past the caches
// shortens that burst.
template <bool NT = false, int MS, int R, int C>
__device__ __forceinline__ void store_tile_staged(const gl<bf16>& g, const RTile<MS, R, C>& t, int b, int d,
                                                  int row0, int col0, char* stage) {
  constexpr int CPR = C / 8;   // 16-byte chunks per row
  static_assert(C % 8 == 0 && (CPR & (CPR - 1)) == 0, "staged store needs a power-of-two count of 16-byte chunks");
  constexpr int SW = CPR < 16 ? CPR - 1 : 15;
  if ((unsigned)b >= (unsigned)g.b || (unsigned)d >= (unsigned)g.d) return;
  const int lane = lane_id();
  const int lr = lane % MS, lh = lane / MS;
  lds_char* s = lds(stage);
#pragma unroll
  for (int rb = 0; rb < t.RB; ++rb) {
    const int row = rb * MS + lr;
#pragma unroll
    for (int cb = 0; cb < t.CB; ++cb)
#pragma unroll
      for (int q = 0; q < MF<MS>::CREGS / 4; ++q) {
        const int col = cb * MS + ccol<MS>(4 * q, lh);
        bf16x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] = (bf16)t.f[cb][rb][4 * q + j];
        *(__attribute__((address_space(3))) bf16x4*)(s + row * (C * 2) + (((col >> 3) ^ (row & SW)) << 4) +
                                                      (col & 7) * 2) = v;
      }
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  bf16* base = g.data + (long long)b * g.sb + (long long)d * g.sd;
  const bool vec_ok = ((g.sr & 7) == 0) && ((col0 & 7) == 0) && ((((size_t)base) & 15) == 0);
#pragma unroll
  for (int it = 0; it < R * CPR / 64; ++it) {
    const int idx = it * 64 + lane;
    const int row = idx / CPR, ch = idx % CPR;
    const bf16x8 v = *(__attribute__((address_space(3))) bf16x8*)(s + row * (C * 2) + ((ch ^ (row & SW)) << 4));
    const int grow = row0 + row, gcol = col0 + ch * 8;
    if (grow >= g.r) continue;
    bf16* p = base + (long long)grow * g.sr + gcol;
    if (vec_ok && gcol + 8 <= g.c) {
      if (NT)
        __builtin_nontemporal_store(v, (bf16x8*)p);
      else
        *(bf16x8*)p = v;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (gcol + j < g.c) p[j] = v[j];
    }
  }
}

// Column vector -> global column `col0` of rows row0.. (one writer lane per row).
template <typename T, int MS, int R>
__device__ __forceinline__ void store_vec(const gl<T>& g, const RVec<MS, R>& v, int b, int d, int row0, int col0) {
  if ((unsigned)b >= (unsigned)g.b || (unsigned)d >= (unsigned)g.d || col0 >= g.c) return;
  const int lane = lane_id();
  if (lane >= MS) return;
  T* base = g.data + (long long)b * g.sb + (long long)d * g.sd;
#pragma unroll
  for (int rb = 0; rb < v.RB; ++rb) {
    const int row = row0 + rb * MS + lane;
    if (row < g.r) base[(long long)row * g.sr + col0] = (T)v.v[rb];
  }
}

// ---------------------------------------------------------------------------
// Program-id remapping.  Workgroups are dispatched round-robin over the 8
// XCDs (each with its own L2).  remap_xcd turns the hardware linear id into
// a logical one such that each XCD walks a contiguous range of logical ids,
// so neighbouring tiles (same A row panel / same attention head) share an
// L2.  Any bijection is valid because programs are independent.
__device__ __forceinline__ int remap_xcd(int hw_id, int total) {
  constexpr int NXCD = 8;
  const int per = total / NXCD;  // ids that split evenly
  if (hw_id >= per * NXCD) return hw_id;
  return (hw_id % NXCD) * per + hw_id / NXCD;
}

// Grouped tile order over a (tiles_y x tiles_x) grid: GROUP rows of tiles
// are walked column by column, so consecutive ids reuse B column panels
// while A row panels stay hot.
template <int GROUP>
__device__ __forceinline__ void grouped_tile(int id, int tiles_x, int tiles_y, int& tx, int& ty) {
  const int per_group = GROUP * tiles_x;
  const int grp = id / per_group;
  const int first_y = grp * GROUP;
  const int gsize = min(tiles_y - first_y, GROUP);
  const int in = id % per_group;
  ty = first_y + in % gsize;
  tx = in / gsize;
}

}  // namespace wir
