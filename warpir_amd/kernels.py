"""Named kernel variants used by the tests, the benchmark and the smoke check.

Each entry builds a WarpIR ``Kernel`` (through the front end and, where
named, ``kernel_pass``).  ``__graft_entry__.build()`` lowers and compiles
every entry into the code-object cache, so GPU runs load prebuilt
``.hsaco`` files and never invoke hipcc.
"""
from __future__ import annotations

import threading
from typing import Callable, Dict, Optional

from warpir_amd.ir import Kernel
from warpir_amd.passes.modulo_scheduler import gfx950_attention_cost_model, gfx950_cost_model, kernel_pass
from warpir_amd.workloads import (build_attention_kernel, build_gemm_kernel, build_mha_bwd_dkdv_kernel,
                                  build_mha_bwd_dq_kernel, build_mha_bwd_prep_kernel, build_mha_forward_kernel)


def _gemm_mi355x(block_k: int = 32, block_m: int = 256, block_n: int = 256, wave_m: int = 128,
                 wave_n: int = 128, load_units: int = 8, lds_budget: int = 160 * 1024,
                 split_k: bool = False, hbm_sources=(), fused_reduce: bool = False) -> Kernel:
    return kernel_pass(build_gemm_kernel(block_m=block_m, block_n=block_n, block_k=block_k, wave_m=wave_m,
                                         wave_n=wave_n, name="gemm_splitk" if split_k else "gemm",
                                         split_k=split_k, fused_reduce=fused_reduce),
                       cost_model=gfx950_cost_model(block_m, block_n, block_k, load_units=load_units,
                                                    lds_budget=lds_budget, hbm_sources=tuple(hbm_sources)))


VARIANTS: Dict[str, Callable[[], Kernel]] = {
    # The reference's own GEMM IR (tests/gemm_baseline_v2.py:31-88): SSA and pipelined.
    "gemm_ref_ssa": lambda: build_gemm_kernel(),
    "gemm_ref_piped": lambda: kernel_pass(build_gemm_kernel()),
    # MI355X GEMM: 256x256 block tile, 4 wavefronts of 128x128, 3-stage LDS ring.
    "gemm_256_k32": lambda: _gemm_mi355x(32),
    "gemm_256_k64_g4": lambda: _gemm_mi355x(64),
    "gemm_256_k64_g16": lambda: _gemm_mi355x(64),
    "gemm_256_k64_g32": lambda: _gemm_mi355x(64),
    "gemm_256_k64_noxcd": lambda: _gemm_mi355x(64),
    # Same tile with a 64-deep K step: MMA twice as long per stage, 2-slot ring.
    "gemm_256_k64": lambda: _gemm_mi355x(64),
    # 128x128 block tile (4 wavefronts of 64x64): more workgroups for short M (skinny GEMM).
    "gemm_128_k64": lambda: _gemm_mi355x(64, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                         lds_budget=80 * 1024),
    # Narrow-N tiles for short M (skinny GEMM): 128 and 256 workgroups at M=128, N=8192,
    # two workgroups per CU (LDS <= 80 KiB).
    "gemm_128x64_k64": lambda: _gemm_mi355x(64, block_m=128, block_n=64, wave_m=64, wave_n=32,
                                            lds_budget=80 * 1024),
    "gemm_128x32_k64": lambda: _gemm_mi355x(64, block_m=128, block_n=32, wave_m=32, wave_n=32,
                                            lds_budget=80 * 1024),
    "gemm_128x32_k64_s8": lambda: _gemm_mi355x(64, block_m=128, block_n=32, wave_m=32, wave_n=32,
                                               lds_budget=160 * 1024),
    "gemm_128x32_k128": lambda: _gemm_mi355x(128, block_m=128, block_n=32, wave_m=32, wave_n=32,
                                             lds_budget=160 * 1024),
    # Split-K form of the 128x128 tile: K slices along blockIdx.z, fp32 partials
    # summed by the split-K reduction (short M, long K).
    "gemm_128_splitk": lambda: _gemm_mi355x(64, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                            lds_budget=80 * 1024, split_k=True),
    "gemm_128_splitk_k128": lambda: _gemm_mi355x(128, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                 lds_budget=160 * 1024, split_k=True),
    # the same with B streaming from HBM and A L2-resident in the cost model: kernel_pass sizes the
    # rings per operand (B three slots, loaded two tiles ahead; A two slots, one tile ahead)
    "gemm_128_splitk_k128_b3": lambda: _gemm_mi355x(128, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                    lds_budget=160 * 1024, split_k=True, hbm_sources=("B",)),
    # shallower K steps, so kernel_pass's per-operand rings go deeper in the same 160 KiB (K=64:
    # B 7 slots, A 3; K=32: B 14, A 6); _sw spreads each step's DMAs over all its MFMAs
    "gemm_128_splitk_k64_b7": lambda: _gemm_mi355x(64, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                   lds_budget=160 * 1024, split_k=True, hbm_sources=("B",)),
    "gemm_128_splitk_k64_b7sw": lambda: _gemm_mi355x(64, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                     lds_budget=160 * 1024, split_k=True, hbm_sources=("B",)),
    "gemm_128_splitk_k32_b14": lambda: _gemm_mi355x(32, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                    lds_budget=160 * 1024, split_k=True, hbm_sources=("B",)),
    "gemm_128_splitk_k32_b14sw": lambda: _gemm_mi355x(32, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                      lds_budget=160 * 1024, split_k=True, hbm_sources=("B",)),
    # the same rings with the slices summed in the kernel: the last slice to store an output tile
    # adds the fp32 partials in slice order and writes the bf16 tile (reduce_slices)
    "gemm_128_splitk_fused": lambda: _gemm_mi355x(128, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                  lds_budget=160 * 1024, split_k=True, hbm_sources=("B",),
                                                  fused_reduce=True),
    "gemm_128x64_splitk": lambda: _gemm_mi355x(64, block_m=128, block_n=64, wave_m=64, wave_n=32,
                                               lds_budget=80 * 1024, split_k=True),
    "gemm_128_splitk_s5": lambda: _gemm_mi355x(64, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                               lds_budget=160 * 1024, split_k=True),
    "gemm_128_splitk_k32": lambda: _gemm_mi355x(32, block_m=128, block_n=128, wave_m=64, wave_n=64,
                                                lds_budget=160 * 1024, split_k=True, load_units=12),
    # 8 wavefronts (2 per SIMD) of 128x64 in the ping-pong form, K=32 with a 4-slot ring.
    "gemm_256_pp": lambda: _gemm_mi355x(32, wave_m=128, wave_n=64, load_units=12),
    # warp-specialised: 4 MFMA wavefronts of 128x64 plus 4 DMA-only wavefronts (2 per SIMD)
    "gemm_256x128_ws": lambda: _gemm_mi355x(64, block_n=128, wave_n=64),
    "gemm_256x128_ws_ab": lambda: _gemm_mi355x(64, block_n=128, wave_n=64),
    "gemm_256x128_ws_k32": lambda: _gemm_mi355x(32, block_n=128, wave_n=64, load_units=12),
    "gemm_256x128_ws_all": lambda: _gemm_mi355x(64, block_n=128, wave_n=64),
    "gemm_256x128": lambda: _gemm_mi355x(64, block_n=128, wave_n=64),
    # 256x256x64 with rings per operand from kernel_pass (B priced as the long stream: B 3 slots
    # loaded two steps ahead, A 2 slots, 160 KiB); _sw with B's DMAs in each step's second half
    "gemm_256_k64_b3": lambda: _gemm_mi355x(64, lds_budget=160 * 1024, hbm_sources=("B",)),
    "gemm_256_k64_b3sw": lambda: _gemm_mi355x(64, lds_budget=160 * 1024, hbm_sources=("B",)),
    # The reference's single-head attention IR (tests/attention_baseline.py:46-186).
    "attn_ref_ssa": lambda: build_attention_kernel(),
    # Multi-head FlashAttention forward, [B, H, S, D] with LSE: SSA form (loads
    # waited every KV step) and the pipelined prefetch form of kernel_pass.
    "mha_d128_ssa": lambda: build_mha_forward_kernel(d=128, block_q=128, block_kv=64, wave_rows=32),
    # The config-4 kernel: 256 query rows (8 wavefronts of 32) in the ping-pong form (one wave
    # group's MFMAs beside the other's softmax, one barrier per iteration), a 4-slot K/V ring
    # loaded two tiles ahead, and the online softmax with a lazy running max (lowered
    # speculatively: no row max, no rescale unless a tile rises above the slack).
    "mha_d128": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                             rescale_slack=LAZY_SLACK),
    # the same with the softmax scale folded into Q and the running max into the score MFMAs
    # (CDNA4Target.fold_softmax_scale: no fma per score, a second bf16 rounding of Q)
    "mha_d128_fold": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                    rescale_slack=LAZY_SLACK),
    # the same with a barrier at the end of every phase (the groups in lock-step)
    "mha_d128_pp2b": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                  rescale_slack=LAZY_SLACK),
    # the same with a 5-slot ring (the whole 160 KB of LDS), loaded three tiles ahead
    "mha_d128_s5": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=160 * 1024, min_stages=5,
                                rescale_slack=LAZY_SLACK),
    # the 5-slot ring with a workgroup barrier every second iteration only (K and V both loaded
    # three tiles ahead)
    "mha_d128_u2": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=160 * 1024, min_stages=5,
                                rescale_slack=LAZY_SLACK),
    # persistent programs: 256 workgroups walking the (query block, head) tiles
    "mha_d128_pers": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                  rescale_slack=LAZY_SLACK),
    # the same with one K/V ring stream across each program's tiles (persistent_stream)
    "mha_d128_stream": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                    rescale_slack=LAZY_SLACK),
    # the same with group B's barrier between its PV and QK (groups a third of an iteration apart)
    "mha_d128_sb": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                rescale_slack=LAZY_SLACK),
    # the same with part of the next PV's V operands read at the end of each VALU phase (4 or 8 of its 16)
    "mha_d128_vp4": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                 rescale_slack=LAZY_SLACK),
    "mha_d128_vp8": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                 rescale_slack=LAZY_SLACK),
    # the same with the K and V load streams on the opposite wave groups from the warp assigner's answer
    "mha_d128_pp_swapped": lambda: _mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                                        rescale_slack=LAZY_SLACK),
    # 4 wavefronts of 32 rows (two workgroups per CU), 2-slot ring: with the lazy softmax, and
    # with the reference IR's exact online softmax (the previous config-4 kernel)
    "mha_d128_w4": lambda: _mha(128, 128, 64, 32, causal=False, rescale_slack=LAZY_SLACK),
    "mha_d128_online": lambda: _mha(128, 128, 64, 32, causal=False),
    # 256 query rows per workgroup (8 wavefronts) in the plain loop (2-slot ring, no ping-pong)
    "mha_d128_q256": lambda: _mha(128, 256, 64, 32, causal=False),
    "mha_d64_causal_ssa": lambda: build_mha_forward_kernel(d=64, block_q=128, block_kv=64, wave_rows=32,
                                                           causal=True, name="mha_fwd_causal"),
    # The config-5 kernel: 128 query rows (4 wavefronts of 32, three workgroups per CU), a 3-slot
    # ring, the lazy-max softmax; and the same with the reference IR's exact online softmax.
    "mha_d64_causal": lambda: _mha(64, 128, 64, 32, causal=True, rescale_slack=LAZY_SLACK),
    "mha_d64_causal_online": lambda: _mha(64, 128, 64, 32, causal=True),
    # the config-5 kernel with the folded softmax scale and running max
    "mha_d64_causal_fold": lambda: _mha(64, 128, 64, 32, causal=True, rescale_slack=LAZY_SLACK),
    "mha_d128_causal": lambda: _mha(128, 128, 64, 32, causal=True),
    "mha_d64": lambda: _mha(64, 128, 64, 32, causal=False),
    # Eight wavefronts in ping-pong (256 query rows, 4-slot K/V rings) with the lazy-max softmax.
    "mha_d64_causal_pp": lambda: _mha(64, 256, 64, 32, causal=True, lds_budget=128 * 1024, min_stages=4,
                                      rescale_slack=LAZY_SLACK),
    # software-pipelined attention loop (QK of tile i+1 and PV of tile i carry tile i's softmax)
    "mha_d128_ovl": lambda: _mha(128, 128, 64, 32, causal=False, rescale_slack=8.0, phases="mixed"),
    "mha_d64_causal_ovl": lambda: _mha(64, 128, 64, 32, causal=True, rescale_slack=8.0, lds_budget=32 * 1024,
                                       phases="mixed"),
    # FlashAttention backward: Dv = rowsum(dO * O); query-major dQ; key-major dK, dV.
    "mha_bwd_prep_d128": lambda: build_mha_bwd_prep_kernel(d=128, block_q=128, wave_rows=32),
    "mha_bwd_dq_d128": lambda: _bwd_dq(128, causal=False),
    # the previous dQ schedule (64-row key tiles, one wave per SIMD), kept for the schedule comparison
    "mha_bwd_dq_d128_kv64": lambda: kernel_pass(build_mha_bwd_dq_kernel(d=128, block_q=128, block_kv=64,
                                                                        wave_rows=32),
                                                cost_model=gfx950_attention_cost_model(128, 64, 128)),
    "mha_bwd_dkdv_d128": lambda: _bwd(build_mha_bwd_dkdv_kernel(d=128, block_kv=128, block_q=64, wave_rows=32), 128),
    "mha_bwd_prep_d64": lambda: build_mha_bwd_prep_kernel(d=64, block_q=128, wave_rows=32),
    "mha_bwd_dq_d64": lambda: _bwd_dq(64, causal=False),
    "mha_bwd_dkdv_d64": lambda: _bwd(_BWD_BUILDERS["dkdv"](64, False, False), 64),
    # grouped-query attention (K / V with H / HR heads): forward, and backward with per-query-head
    # fp32 dK / dV contributions that api.attention_backward sums per key/value head
    "mha_d128_gqa": lambda: _mha(128, 128, 64, 32, causal=False, gqa=True),
    "mha_d128_causal_gqa": lambda: _mha(128, 128, 64, 32, causal=True, gqa=True),
    "mha_d64_causal_gqa": lambda: _mha(64, 128, 64, 32, causal=True, gqa=True),
    "mha_d64_gqa": lambda: _mha(64, 128, 64, 32, causal=False, gqa=True),
    **{f"mha_bwd_{part}_d{d}{'_causal' if c else ''}_gqa": (
        lambda part=part, d=d, c=c: _bwd(_BWD_BUILDERS[part](d, c, True), d))
       for part in ("dq", "dkdv") for d in (128, 64) for c in (False, True)},
    # causal backward: dq stops at the diagonal; dkdv starts at it (transposed mask)
    "mha_bwd_dq_d128_causal": lambda: _bwd_dq(128, causal=True),
    "mha_bwd_dkdv_d128_causal": lambda: _bwd(build_mha_bwd_dkdv_kernel(d=128, block_kv=128, block_q=64, wave_rows=32,
                                                                       causal=True, name="mha_bwd_dkdv_causal"), 128),
    "mha_bwd_dq_d64_causal": lambda: _bwd_dq(64, causal=True),
    "mha_bwd_dkdv_d64_causal": lambda: _bwd(_BWD_BUILDERS["dkdv"](64, True, False), 64),
}


# Slack (in exp2 units) of the lazy running max of the forward kernels: the softmax
# exponentials stay below 2**LAZY_SLACK, and a tile's row maximum is computed only when
# some exponential would exceed it.
LAZY_SLACK = 16.0

# The query-major dQ kernel steps over 32-row key tiles: its score, dP and dS tiles are then
# 32 x 32 per wavefront, which leaves D=128 at two waves per SIMD (254 VGPRs, 32 KiB ring) and
# D=64 at three, where 64-row key tiles needed the whole register file at D=128.
DQ_BLOCK_KV = 32
# The key-major dK/dV kernel steps over 32-row query tiles at D=64: its transposed score and
# gradient tiles are then 32 x 32 per wavefront and it fits two waves per SIMD (190-206 VGPRs,
# where 64-row steps needed the whole file).  At D=128 the dK and dV accumulators keep it at
# one wave either way, and 64-row steps measured faster.
DKDV_BLOCK_Q = {128: 64, 64: 32}

_BWD_BUILDERS = {
    "dq": lambda d, causal, gqa: build_mha_bwd_dq_kernel(
        d=d, block_q=128, block_kv=DQ_BLOCK_KV, wave_rows=32, causal=causal, gqa=gqa,
        name="mha_bwd_dq" + ("_causal" if causal else "") + ("_gqa" if gqa else "")),
    "dkdv": lambda d, causal, gqa: build_mha_bwd_dkdv_kernel(
        d=d, block_kv=128, block_q=DKDV_BLOCK_Q[d], wave_rows=32, causal=causal, gqa=gqa,
        name="mha_bwd_dkdv" + ("_causal" if causal else "") + ("_gqa" if gqa else "")),
}


def _bwd(kernel: Kernel, d: int) -> Kernel:
    if kernel.name.startswith("mha_bwd_dq"):
        # two-slot ring of 32-row K and V tiles (32 KiB at D=128)
        return kernel_pass(kernel, cost_model=gfx950_attention_cost_model(128, DQ_BLOCK_KV, d,
                                                                          lds_budget=32 * 1024))
    # dK / dV: the 128-row key tile stays resident, query tiles of DKDV_BLOCK_Q[d] rows stream
    return kernel_pass(kernel, cost_model=gfx950_attention_cost_model(128, DKDV_BLOCK_Q[d], d))


def _bwd_dq(d: int, causal: bool) -> Kernel:
    return _bwd(_BWD_BUILDERS["dq"](d, causal, False), d)


def _mha(d: int, block_q: int, block_kv: int, wave_rows: int, causal: bool, lds_budget: int = 64 * 1024,
         min_stages: int = 2, rescale_slack: Optional[float] = None, gqa: bool = False,
         phases: Optional[str] = None) -> Kernel:
    """Forward FlashAttention through kernel_pass.  The lazy-max kernels have
    their softmax chain placed by the pass's phase schedule (``phases``,
    default "auto": the MFMA / VALU phase alternation at their waves per
    SIMD); the exact online-softmax kernels keep program order."""
    name = ("mha_fwd_causal" if causal else "mha_fwd") + ("_gqa" if gqa else "")
    k = build_mha_forward_kernel(d=d, block_q=block_q, block_kv=block_kv, wave_rows=wave_rows, causal=causal,
                                 name=name, rescale_slack=rescale_slack, gqa=gqa)
    if phases is None and rescale_slack == LAZY_SLACK:
        phases = "auto"
    return kernel_pass(k, cost_model=gfx950_attention_cost_model(block_q, block_kv, d, lds_budget=lds_budget,
                                                                 min_stages=min_stages, phase_schedule=phases))

# Lowering options of variants that differ from the defaults.
TARGETS: Dict[str, dict] = {
    "mha_d128_ovl": {"lazy_softmax": False},
    "mha_d128_pp_swapped": {"wave_groups": {"k": 1, "v": 0}},
    "mha_d128_pp2b": {"pingpong_one_barrier": False},
    "mha_d128_u2": {"pingpong_barrier_every": 2},
    "mha_d128_sb": {"pingpong_split_barrier": True},
    "mha_d128_pers": {"persistent": 256},
    "mha_d128_stream": {"persistent": 256, "persistent_stream": True},
    "mha_d128_vp4": {"pingpong_v_prefetch": 4},
    "mha_d128_vp8": {"pingpong_v_prefetch": 8},
    "mha_d128_fold": {"fold_softmax_scale": True},
    "mha_d64_causal_fold": {"fold_softmax_scale": True},
    # tile orders of the 8192^3 GEMM: GROUP_M rows of tiles per group, and without the XCD remap
    "gemm_256_k64_g4": {"group_m": 4},
    "gemm_256_k64_g16": {"group_m": 16},
    "gemm_256_k64_g32": {"group_m": 32},
    "gemm_256_k64_noxcd": {"xcd_remap": False},
    # (the rotated pipeline's extra fragment registers do not fit two waves per SIMD)
    # A / B load streams split between the wave sets as the warp assigner's steady-state
    # assignment with the gfx950 costs places them (both on the DMA waves); _all forces that
    # split, _ab the one the reference demo's constants gave (A with the MFMA waves, B on the
    # DMA waves; measured 9% slower)
    "gemm_256x128_ws": {"warp_specialize": True, "rotate_mma": False, "mve": False},
    "gemm_256x128_ws_ab": {"warp_specialize": True, "rotate_mma": False, "mve": False,
                           "wave_groups": {"a": 0, "b": 1}},
    "gemm_256x128_ws_k32": {"warp_specialize": True, "rotate_mma": False},
    "gemm_256x128_ws_all": {"warp_specialize": True, "rotate_mma": False, "mve": False,
                            "wave_groups": {"a": 1, "b": 1}},
    "mha_d64_causal_ovl": {"lazy_softmax": False},
    "gemm_256_k64_b3sw": {"dma_spread_whole": True},
    "gemm_128_splitk_k64_b7sw": {"dma_spread_whole": True},
    "gemm_128_splitk_k32_b14sw": {"dma_spread_whole": True},
}
# the lazy softmax's row sums on the matrix core (CDNA4Target.rowsum_mfma; config 5 within 0.3-0.7%
# of the default, the config-4 ping-pong 5% slower)
for _base in ("mha_d128", "mha_d64_causal"):
    VARIANTS[f"{_base}_mr"] = VARIANTS[_base]
    TARGETS[f"{_base}_mr"] = {"rowsum_mfma": True}
# device-scope cache policy on the tile DMAs (CDNA4Target.dma_cache_policy) of the two headline
# kernels (measured equal to the default policy; "nt" slower)
for _base in ("gemm_256_k64", "mha_d128"):
    VARIANTS[f"{_base}_dma_sc1"] = VARIANTS[_base]
    TARGETS[f"{_base}_dma_sc1"] = {"dma_cache_policy": "sc1"}

# The D=128 dK/dV kernels hold dK, dV and the score tiles in more than 256 registers.  With
# the MFMAs' VGPR form the S and dP tiles stay in arch VGPRs (no v_accvgpr_read per score
# before the softmax algebra) and dK, dV take the AGPRs: 4.21-4.24 against 4.38-4.51 ms at
# B16 H16 S4096, bitwise the same gradients.  (The GEMM does not compile in that form.)
for _name in ("mha_bwd_dkdv_d128", "mha_bwd_dkdv_d128_causal", "mha_bwd_dkdv_d128_gqa",
              "mha_bwd_dkdv_d128_causal_gqa"):
    TARGETS[_name] = {"mfma_vgpr_form": True}
# the D=128 dK/dV kernel with its element-wise chains in the MFMA slots of the MMAs after them
# (CDNA4Target.slot_fusion: P^T in dP^T's MFMAs, dS^T in dV's)
VARIANTS["mha_bwd_dkdv_d128_sf"] = VARIANTS["mha_bwd_dkdv_d128"]
TARGETS["mha_bwd_dkdv_d128_sf"] = {"mfma_vgpr_form": True, "slot_fusion": True}


def lowerer(name: str):
    """The ``CDNA4Lowerer`` variant *name* is built with."""
    from warpir_amd.lowering import CDNA4Lowerer, CDNA4Target

    return CDNA4Lowerer(CDNA4Target(**TARGETS.get(name, {})))


_handles: Dict[str, object] = {}
_handles_lock = threading.Lock()


def kernel(name: str) -> Kernel:
    return VARIANTS[name]()


def handle(name: str):
    """A compiled, launchable ``KernelHandle`` for variant *name* (memoised;
    safe to call from several threads: each variant is built once)."""
    from warpir_amd.runtime import compile_kernel

    h = _handles.get(name)
    if h is not None:
        return h
    with _handles_lock:
        if name not in _handles:
            _handles[name] = compile_kernel(VARIANTS[name](), lowerer(name))
        return _handles[name]


def build_all(verbose: bool = False, prune: bool = True) -> Dict[str, str]:
    """Lower and compile every variant; returns name -> code-object path.

    With ``prune`` the cache keeps only the files of the current variants.
    """
    import os

    from warpir_amd.runtime import CACHE_DIR, compile_source, resource_usage

    out = {}
    for name, make in VARIANTS.items():
        src = lowerer(name).lower(make())
        out[name] = compile_source(src, force=True)
        if verbose:
            u = resource_usage(src)
            print(f"built {name}: {os.path.basename(out[name])} vgpr={u.get('vgpr')} agpr={u.get('agpr')} "
                  f"spill={u.get('vgpr_spill')} lds={u.get('lds')}", flush=True)
    if prune and os.path.isdir(CACHE_DIR):
        keep = {os.path.basename(p)[: -len(".hsaco")] for p in out.values()}
        for f in os.listdir(CACHE_DIR):
            if f.split(".")[0] not in keep:
                os.remove(os.path.join(CACHE_DIR, f))
    return out
