"""IR builders for the GEMM and FlashAttention-forward workloads.

``build_gemm_kernel`` and ``build_attention_kernel`` with their default
arguments construct the same IR as the reference's builder scripts
(``tests/gemm_baseline_v2.py:31-88`` and
``tests/attention_baseline.py:46-186``): same value names, types and op
order (checked against the reference printer's text in the tests).  The
keyword arguments widen them to the MI355X configurations -- block tiles
of 256x256x64, per-wavefront accumulator slices, multi-head
``[B, H, S, D]`` attention with a log-sum-exp output and causal block
skipping -- using only additive ops.
"""
from __future__ import annotations

import math
from typing import Optional

from warpir_amd.ir import (
    AddOp,
    CausalMaskOp,
    ColVecType,
    CopyOp,
    DivRowOp,
    Exp2Op,
    ForOp,
    GPUType,
    GlobalType,
    IntAffineOp,
    IntDivOp,
    IntType,
    IterArg,
    Kernel,
    LazyMaxOp,
    LoadVecOp,
    Log2Op,
    MMAOp,
    MulOp,
    MulRowOp,
    MulScalarOp,
    NegInftyOp,
    RegTileType,
    ReduceSlicesOp,
    RowMaxOp,
    RowSumOp,
    RowVecType,
    SharedTileType,
    SubColOp,
    SubOp,
    SubRowOp,
    TMALoadOp,
    TMAStoreOp,
    Value,
    WaitOp,
    YieldOp,
    ZeroOp,
)

LOG2E = math.log2(math.e)
LN2 = math.log(2.0)

# The reference attention builder's exp2 scale for D=64 (tests/attention_baseline.py:42-43).
REFERENCE_ATTENTION_SCALE = 0.125 * 1.44269504089


def _bf16_global(tile: SharedTileType, batch: int = 1, depth: int = 1) -> GlobalType:
    return GlobalType(data_type=GPUType.bf16, sub_tile_type=tile, batch=batch, depth=depth,
                      rows=-1, cols=-1)


def build_gemm_kernel(block_m: int = 64, block_n: int = 64, block_k: int = 64,
                      wave_m: int = 16, wave_n: int = 64, name: str = "gemm",
                      split_k: bool = False, fused_reduce: bool = False) -> Kernel:
    """``C[M, N] = A[M, K] @ B[K, N]``, bf16 in, fp32 accumulate, bf16 out.

    One program per ``block_m x block_n`` tile of C at
    ``(blockIdx.y, blockIdx.x)``; the loop walks ``ceil(N / block_k)``
    K-tiles, where the loop bound input is named ``N`` as in the
    reference (it is the reduction extent).  The accumulator type is the
    per-wavefront slice ``wave_m x wave_n``, so a block runs
    ``(block_m / wave_m) * (block_n / wave_n)`` wavefronts.

    Defaults reproduce ``tests/gemm_baseline_v2.py:31-88``.

    ``split_k`` (additive): the globals get a depth dimension indexed by
    ``blockIdx.z``, one K slice per depth -- A as ``[1, S, M, K/S]``, B as
    ``[1, S, K/S, N]`` -- and C_global becomes an fp32 ``[1, S, M, N]`` of
    partial products, which the host sums (``warpir_amd.api.gemm``).  ``N``
    is then the slice's reduction extent.

    ``fused_reduce`` (additive, with ``split_k``): the kernel sums the slices
    itself -- a ``reduce_slices`` after the partial store writes the bf16
    ``C`` ``[1, 1, M, N]`` once every slice of a tile has stored, counting
    arrivals in ``Arrivals`` (u32, one counter per output tile, zero before
    the first launch and left zero).  Outputs: ``C_global``, ``C``,
    ``Arrivals``.
    """
    if fused_reduce and not split_k:
        raise ValueError("fused_reduce needs split_k")
    a_tile = SharedTileType(GPUType.bf16, block_m, block_k)
    b_tile = SharedTileType(GPUType.bf16, block_k, block_n)
    if split_k:
        c_tile = SharedTileType(GPUType.fp32, block_m, block_n)
        a_glob, b_glob = _bf16_global(a_tile, depth=-1), _bf16_global(b_tile, depth=-1)
        c_glob = GlobalType(data_type=GPUType.fp32, sub_tile_type=c_tile, batch=1, depth=-1, rows=-1, cols=-1)
        depth = Value("blockIdx.z", IntType())
    else:
        c_tile = SharedTileType(GPUType.bf16, block_m, block_n)
        a_glob, b_glob, c_glob = _bf16_global(a_tile), _bf16_global(b_tile), _bf16_global(c_tile)
        depth = 0
    acc = RegTileType(GPUType.fp32, wave_m, wave_n)

    A, B, C = Value("A", a_glob), Value("B", b_glob), Value("C_global", c_glob)
    n_red = Value("N", IntType())
    row, col = Value("blockIdx.y", IntType()), Value("blockIdx.x", IntType())
    i = Value("i", IntType())
    c_init, c_accum, c_final, c_new = (Value(n, acc) for n in ("c_init", "c_accum", "c_final", "c_new"))
    a_sh, b_sh = Value("a_shared", a_tile), Value("b_shared", b_tile)

    loop = ForOp(
        induction_var=i, start=0, stop=n_red, step=1, tile_size=block_k,
        iter_args=(IterArg(block_arg=c_accum, init=c_init),),
        body=(
            TMALoadOp(result=a_sh, source=A, coords=(0, depth, row, i)),
            TMALoadOp(result=b_sh, source=B, coords=(0, depth, i, col)),
            WaitOp(values=(a_sh, b_sh)),
            MMAOp(result=c_new, a=a_sh, b=b_sh, accum=c_accum),
            YieldOp(values=(c_new,)),
        ),
        results=(c_final,),
    )
    body = (ZeroOp(result=c_init), loop, TMAStoreOp(source=c_final, dest=C, coords=(0, depth, row, col)))
    outputs = (C,)
    if fused_reduce:
        out = Value("C", _bf16_global(SharedTileType(GPUType.bf16, block_m, block_n)))
        arrivals = Value("Arrivals", GlobalType(data_type=GPUType.u32, sub_tile_type=SharedTileType(GPUType.u32, 1, 1),
                                                batch=1, depth=1, rows=1, cols=-1))
        body += (ReduceSlicesOp(partials=C, dest=out, arrivals=arrivals, coords=(0, depth, row, col)),)
        outputs = (C, out, arrivals)
    return Kernel(name=name, inputs=(A, B, n_red), outputs=outputs, body=body)


def build_attention_kernel(d: int = 64, block: int = 64, warp_rows: int = 16,
                           scale: float = REFERENCE_ATTENTION_SCALE) -> Kernel:
    """Single-head FlashAttention forward in exp2 form.

    Defaults reproduce ``tests/attention_baseline.py:46-186``: Q tile
    resident, loop over K/V tiles with ``S = Q K^T``, online softmax in the
    exp2 domain with ``scale = log2(e) / sqrt(d)``, ``O += bf16(P) V``,
    final ``O / l``.
    """
    return _attention(name="attention_fwd", d=d, block_q=block, block_kv=block,
                      wave_rows=warp_rows, scale=scale, multi_head=False, causal=False,
                      with_lse=False, rescale_slack=None, gqa=False)


def build_mha_forward_kernel(d: int = 128, block_q: int = 128, block_kv: int = 64,
                             wave_rows: int = 32, causal: bool = False, with_lse: bool = True,
                             name: str = "mha_fwd", rescale_slack: Optional[float] = None,
                             gqa: bool = False) -> Kernel:
    """Multi-head FlashAttention forward over ``[B, H, S, D]`` tensors.

    Program ``(blockIdx.x, blockIdx.y, blockIdx.z)`` = (query tile, head,
    batch).  Outputs O ``[B, H, S, D]`` bf16 and, with ``with_lse``, the
    natural-log log-sum-exp ``L[B, H, S]`` fp32 (as the plain
    ``logsumexp(S * scale)``; the reference TK kernel stores a
    ``-sqrt(D)``-scaled variant, ``mha_h100.cu:216-221``).  With ``causal``
    the KV loop stops at the query tile's last row
    (``IntAffineOp``) and the score tile is masked (``CausalMaskOp``).

    ``rescale_slack`` (additive, in exp2 units, e.g. 8.0): the running max
    only moves when a tile's maximum exceeds it by more than that
    (``LazyMaxOp``), so the O / l rescale is skipped on most steps and
    ``P <= 2**slack``.  ``None`` builds the plain online softmax.

    ``gqa`` (additive): grouped-query attention.  K and V have ``H / HR``
    heads (an extra int input ``HR`` after ``N``); query head ``h`` reads
    key/value head ``h // HR`` (``mha_h100.cu:74``).
    """
    return _attention(name=name, d=d, block_q=block_q, block_kv=block_kv, wave_rows=wave_rows,
                      scale=LOG2E / math.sqrt(d), multi_head=True, causal=causal,
                      with_lse=with_lse, rescale_slack=rescale_slack, gqa=gqa)


def _attention(*, name, d, block_q, block_kv, wave_rows, scale, multi_head, causal, with_lse,
               rescale_slack, gqa):
    q_tile = SharedTileType(GPUType.bf16, block_q, d)
    kv_tile = SharedTileType(GPUType.bf16, block_kv, d)
    if multi_head:
        q_glob = GlobalType(GPUType.bf16, q_tile)
        kv_glob = GlobalType(GPUType.bf16, kv_tile)
    else:
        q_glob = kv_glob = _bf16_global(q_tile)
    att_f = RegTileType(GPUType.fp32, wave_rows, block_kv)
    att_b = RegTileType(GPUType.bf16, wave_rows, block_kv)
    o_reg = RegTileType(GPUType.fp32, wave_rows, d)
    cvec = ColVecType(GPUType.fp32, wave_rows, block_kv)

    Q, K, V, O = Value("Q", q_glob), Value("K", kv_glob), Value("V", kv_glob), Value("O", q_glob)
    n_kv = Value("N", IntType())
    q_idx = Value("blockIdx.x", IntType())
    if multi_head:
        head, batch = Value("blockIdx.y", IntType()), Value("blockIdx.z", IntType())
        bh = (batch, head)
    else:
        bh = (0, 0)
    head_map, bh_kv, extra_inputs = [], bh, ()
    if gqa:
        hr, kv_head = Value("HR", IntType()), Value("kv_head", IntType())
        head_map = [IntDivOp(result=kv_head, input=head, divisor=hr)]
        bh_kv, extra_inputs = (batch, kv_head), (hr,)

    def v(n, t):
        return Value(n, t)

    q_sh = v("q_shared", q_tile)
    o_init, max_init, norm_init = v("o_init", o_reg), v("max_init", cvec), v("norm_init", cvec)
    i = v("i", IntType())
    o_acc, max_vec, norm_vec = v("o_accum", o_reg), v("max_vec", cvec), v("norm_vec", cvec)
    k_sh, v_sh = v("k_shared", kv_tile), v("v_shared", kv_tile)
    att_zero, att = v("att_zero", att_f), v("att", att_f)
    max_prev, max_new = v("max_prev", cvec), v("max_new", cvec)
    att_scaled, max_new_sc, max_prev_sc = v("att_scaled", att_f), v("max_new_sc", cvec), v("max_prev_sc", cvec)
    att_shifted, p_f = v("att_shifted", att_f), v("P_fp32", att_f)
    corr_diff, corr = v("corr_diff", cvec), v("correction", cvec)
    norm_rescaled, norm_new = v("norm_rescaled", cvec), v("norm_new", cvec)
    o_rescaled, p_b, o_new = v("o_rescaled", o_reg), v("P_bf16", att_b), v("o_new", o_reg)
    o_final, max_final, norm_final, o_norm = (v("o_final", o_reg), v("max_final", cvec),
                                              v("norm_final", cvec), v("o_norm", o_reg))

    scores = att
    body = [
        TMALoadOp(result=k_sh, source=K, coords=(*bh_kv, i, 0)),
        TMALoadOp(result=v_sh, source=V, coords=(*bh_kv, i, 0)),
        WaitOp(values=(k_sh, v_sh)),
        ZeroOp(result=att_zero),
        MMAOp(result=att, a=q_sh, b=k_sh, accum=att_zero, transpose_b=True),
    ]
    if causal:
        scores = v("att_masked", att_f)
        body.append(CausalMaskOp(result=scores, tile=att, row_tile=q_idx, col_tile=i))
    body.append(CopyOp(result=max_prev, input=max_vec))
    if rescale_slack is None:
        body.append(RowMaxOp(result=max_new, tile=scores, prev=max_vec))
    else:
        max_cand = v("max_cand", cvec)
        body += [RowMaxOp(result=max_cand, tile=scores, prev=max_vec),
                 LazyMaxOp(result=max_new, prev=max_vec, cand=max_cand, slack=rescale_slack / scale)]
    body += [
        MulScalarOp(result=att_scaled, input=scores, scalar=scale),
        MulScalarOp(result=max_new_sc, input=max_new, scalar=scale),
        MulScalarOp(result=max_prev_sc, input=max_prev, scalar=scale),
        SubRowOp(result=att_shifted, tile=att_scaled, vec=max_new_sc),
        Exp2Op(result=p_f, input=att_shifted),
        SubOp(result=corr_diff, a=max_prev_sc, b=max_new_sc),
        Exp2Op(result=corr, input=corr_diff),
        MulOp(result=norm_rescaled, a=norm_vec, b=corr),
        RowSumOp(result=norm_new, tile=p_f, prev=norm_rescaled),
        MulRowOp(result=o_rescaled, tile=o_acc, vec=corr),
        CopyOp(result=p_b, input=p_f),
        MMAOp(result=o_new, a=p_b, b=v_sh, accum=o_rescaled),
        YieldOp(values=(o_new, max_new, norm_new)),
    ]

    prologue = []
    stop = n_kv
    if causal:
        stop = v("kv_stop", IntType())
        prologue.append(IntAffineOp(result=stop, input=q_idx, mul=block_q, add=block_q))

    loop = ForOp(
        induction_var=i, start=0, stop=stop, step=1, tile_size=block_kv,
        iter_args=(IterArg(block_arg=o_acc, init=o_init),
                   IterArg(block_arg=max_vec, init=max_init),
                   IterArg(block_arg=norm_vec, init=norm_init)),
        body=tuple(body),
        results=(o_final, max_final, norm_final),
    )
    kernel_body = [
        *head_map,
        TMALoadOp(result=q_sh, source=Q, coords=(*bh, q_idx, 0)),
        WaitOp(values=(q_sh,)),
        ZeroOp(result=o_init),
        NegInftyOp(result=max_init),
        ZeroOp(result=norm_init),
        *prologue,
        loop,
        DivRowOp(result=o_norm, tile=o_final, vec=norm_final),
        TMAStoreOp(source=o_norm, dest=O, coords=(*bh, q_idx, 0)),
    ]
    outputs = [O]
    if with_lse:
        lse_tile = SharedTileType(GPUType.fp32, block_q, 1)
        L = Value("L", GlobalType(GPUType.fp32, lse_tile, cols=1))
        m_sc, l2, lse2, lse = (v("max_final_sc", cvec), v("norm_log2", cvec),
                               v("lse_log2", cvec), v("lse", cvec))
        kernel_body += [
            MulScalarOp(result=m_sc, input=max_final, scalar=scale),
            Log2Op(result=l2, input=norm_final),
            AddOp(result=lse2, a=m_sc, b=l2),
            MulScalarOp(result=lse, input=lse2, scalar=LN2),
            TMAStoreOp(source=lse, dest=L, coords=(*bh, q_idx, 0)),
        ]
        outputs.append(L)
    return Kernel(name=name, inputs=(Q, K, V, n_kv, *extra_inputs), outputs=tuple(outputs), body=tuple(kernel_body))


# ---------------------------------------------------------------------------
# FlashAttention backward (additive): three kernels over the forward's O and
# LSE, following the structure of the reference's TK backward
# (kernel_examples/attention/mha_h100.cu:253-303 prep, :482-642 main) with
# dQ computed by its own query-major kernel instead of atomic adds:
#   prep:  Dv[q]   = sum_d dO[q, d] * O[q, d]
#   dq:    per query tile, over key tiles: P = exp(Q K^T s - LSE),
#          dS = P * (dO V^T - Dv),  dQ = s * sum dS K
#   dkdv:  per key tile, over query tiles (key-major, so P^T and dS^T come
#          straight out of the MMAs): dV = sum P^T dO,  dK = s * sum dS^T Q
# with s = 1/sqrt(D).  Exponentials run in the exp2 domain.
# ---------------------------------------------------------------------------

def _bwd_globals(d: int, rows: int):
    tile = SharedTileType(GPUType.bf16, rows, d)
    vec_tile = SharedTileType(GPUType.fp32, rows, 1)
    return GlobalType(GPUType.bf16, tile), GlobalType(GPUType.fp32, vec_tile, cols=1), tile


def build_mha_bwd_prep_kernel(d: int = 128, block_q: int = 128, wave_rows: int = 32,
                              name: str = "mha_bwd_prep", lse_log2: bool = True) -> Kernel:
    """``Dv[b, h, q] = sum_d dO * O`` over ``[B, H, S, D]`` (bwd prep, ``mha_h100.cu:253-303``).

    With ``lse_log2`` it also writes ``L2 = L * log2(e)`` from the forward's
    natural-log ``L``: the key-major dK/dV kernel reads the LSE of every
    query column at every step, and taking it in log2 units there saves one
    multiply per column per step (the same fp32 product, computed once)."""
    g_bf, g_vec, tile = _bwd_globals(d, block_q)
    O, dO, Dv = Value("O", g_bf), Value("dO", g_bf), Value("Dv", g_vec)
    L, L2 = Value("L", g_vec), Value("L2", g_vec)
    q_idx, head, batch = (Value(n, IntType()) for n in ("blockIdx.x", "blockIdx.y", "blockIdx.z"))
    reg = RegTileType(GPUType.fp32, wave_rows, d)
    cvec = ColVecType(GPUType.fp32, wave_rows, d)
    o_sh, do_sh = Value("o_shared", tile), Value("do_shared", tile)
    o_r, do_r, prod = Value("o_reg", reg), Value("do_reg", reg), Value("prod", reg)
    zero, dvec = Value("d_zero", cvec), Value("d_vec", cvec)
    body = (
        TMALoadOp(result=o_sh, source=O, coords=(batch, head, q_idx, 0)),
        TMALoadOp(result=do_sh, source=dO, coords=(batch, head, q_idx, 0)),
        WaitOp(values=(o_sh, do_sh)),
        CopyOp(result=o_r, input=o_sh),
        CopyOp(result=do_r, input=do_sh),
        MulOp(result=prod, a=o_r, b=do_r),
        ZeroOp(result=zero),
        RowSumOp(result=dvec, tile=prod, prev=zero),
        TMAStoreOp(source=dvec, dest=Dv, coords=(batch, head, q_idx, 0)),
    )
    if not lse_log2:
        return Kernel(name=name, inputs=(O, dO), outputs=(Dv,), body=body)
    lse, lse2 = Value("lse", cvec), Value("lse_log2", cvec)
    body += (
        LoadVecOp(result=lse, source=L, coords=(batch, head, q_idx, 0)),
        MulScalarOp(result=lse2, input=lse, scalar=LOG2E),
        TMAStoreOp(source=lse2, dest=L2, coords=(batch, head, q_idx, 0)),
    )
    return Kernel(name=name, inputs=(O, dO, L), outputs=(Dv, L2), body=body)


def build_mha_bwd_dq_kernel(d: int = 128, block_q: int = 128, block_kv: int = 64, wave_rows: int = 32,
                            name: str = "mha_bwd_dq", causal: bool = False, gqa: bool = False) -> Kernel:
    """``dQ`` of attention forward, query-major: one program per query tile
    ``(blockIdx.x, head, batch)``; the loop walks key tiles.  With
    ``causal`` it stops at the query tile's last row and masks the scores
    as the causal forward does; with ``gqa`` K and V come from key/value
    head ``head // HR`` (an extra int input)."""
    scale = 1.0 / math.sqrt(d)
    q_glob, vec_glob, q_tile = _bwd_globals(d, block_q)
    kv_glob, _, kv_tile = _bwd_globals(d, block_kv)
    Q, K, V, dO = Value("Q", q_glob), Value("K", kv_glob), Value("V", kv_glob), Value("dO", q_glob)
    L, Dv, dQ = Value("L", vec_glob), Value("Dv", vec_glob), Value("dQ", q_glob)
    n_kv = Value("N", IntType())
    q_idx, head, batch = (Value(n, IntType()) for n in ("blockIdx.x", "blockIdx.y", "blockIdx.z"))
    bh = (batch, head)
    head_map, bh_kv, extra_inputs = [], bh, ()
    if gqa:
        hr, kv_head = Value("HR", IntType()), Value("kv_head", IntType())
        head_map = [IntDivOp(result=kv_head, input=head, divisor=hr)]
        bh_kv, extra_inputs = (batch, kv_head), (hr,)
    att_f = RegTileType(GPUType.fp32, wave_rows, block_kv)
    att_b = RegTileType(GPUType.bf16, wave_rows, block_kv)
    acc = RegTileType(GPUType.fp32, wave_rows, d)
    cvec = ColVecType(GPUType.fp32, wave_rows, block_kv)

    def v(n, t):
        return Value(n, t)

    q_sh, do_sh, k_sh, v_sh = v("q_shared", q_tile), v("do_shared", q_tile), v("k_shared", kv_tile), v("v_shared", kv_tile)
    lse, dvec, lse2 = v("lse", cvec), v("d_vec", cvec), v("lse_log2", cvec)
    i = v("i", IntType())
    dq_init, dq_acc, dq_new, dq_final, dq_out = (v(n, acc) for n in ("dq_init", "dq_accum", "dq_new", "dq_final", "dq_out"))
    zero, s_t, s_sc, s_sh, p = (v(n, att_f) for n in ("s_zero", "s", "s_scaled", "s_shifted", "p"))
    dp_zero, dp, dp_sub, ds = (v(n, att_f) for n in ("dp_zero", "dp", "dp_minus_d", "ds"))
    ds_b = v("ds_bf16", att_b)
    stop, prologue, scores, mask = n_kv, [], s_t, []
    if causal:
        stop = v("kv_stop", IntType())
        prologue = [IntAffineOp(result=stop, input=q_idx, mul=block_q, add=block_q)]
        scores = v("s_masked", att_f)
        mask = [CausalMaskOp(result=scores, tile=s_t, row_tile=q_idx, col_tile=i)]
    loop = ForOp(
        induction_var=i, start=0, stop=stop, step=1, tile_size=block_kv,
        iter_args=(IterArg(block_arg=dq_acc, init=dq_init),),
        body=(
            TMALoadOp(result=k_sh, source=K, coords=(*bh_kv, i, 0)),
            TMALoadOp(result=v_sh, source=V, coords=(*bh_kv, i, 0)),
            WaitOp(values=(k_sh, v_sh)),
            ZeroOp(result=zero),
            MMAOp(result=s_t, a=q_sh, b=k_sh, accum=zero, transpose_b=True),
            *mask,
            MulScalarOp(result=s_sc, input=scores, scalar=scale * LOG2E),
            SubRowOp(result=s_sh, tile=s_sc, vec=lse2),
            Exp2Op(result=p, input=s_sh),
            ZeroOp(result=dp_zero),
            MMAOp(result=dp, a=do_sh, b=v_sh, accum=dp_zero, transpose_b=True),
            SubRowOp(result=dp_sub, tile=dp, vec=dvec),
            MulOp(result=ds, a=p, b=dp_sub),
            CopyOp(result=ds_b, input=ds),
            MMAOp(result=dq_new, a=ds_b, b=k_sh, accum=dq_acc),
            YieldOp(values=(dq_new,)),
        ),
        results=(dq_final,),
    )
    body = (
        *head_map,
        TMALoadOp(result=q_sh, source=Q, coords=(*bh, q_idx, 0)),
        TMALoadOp(result=do_sh, source=dO, coords=(*bh, q_idx, 0)),
        WaitOp(values=(q_sh, do_sh)),
        LoadVecOp(result=lse, source=L, coords=(*bh, q_idx, 0)),
        LoadVecOp(result=dvec, source=Dv, coords=(*bh, q_idx, 0)),
        MulScalarOp(result=lse2, input=lse, scalar=LOG2E),
        ZeroOp(result=dq_init),
        *prologue,
        loop,
        MulScalarOp(result=dq_out, input=dq_final, scalar=scale),
        TMAStoreOp(source=dq_out, dest=dQ, coords=(*bh, q_idx, 0)),
    )
    return Kernel(name=name, inputs=(Q, K, V, dO, L, Dv, n_kv, *extra_inputs), outputs=(dQ,), body=body)


def build_mha_bwd_dkdv_kernel(d: int = 128, block_kv: int = 128, block_q: int = 64, wave_rows: int = 32,
                              name: str = "mha_bwd_dkdv", causal: bool = False, gqa: bool = False,
                              lse_log2: bool = True) -> Kernel:
    """``dK`` and ``dV`` of attention forward, key-major: one program per key
    tile ``(blockIdx.x, head, batch)``; the loop walks query tiles.  Scores
    are computed transposed (``S^T = K Q^T``), so the per-query LSE and Dv
    are row_vecs, read from fp32 ``block_q x 1`` shared tiles that are loaded
    (and pipelined) with the query tile.  With ``causal`` the loop starts at
    the first query tile that sees the key tile (``mha_h100.cu:525``) and the
    transposed scores are masked (``CausalMaskOp(transposed=True)``).

    With ``gqa`` one program runs per (key tile, *query* head): K and V come
    from key/value head ``head // HR`` (an extra int input) and the outputs
    are that query head's fp32 contributions ``dK_part`` / ``dV_part``
    ``[B, H, S, D]``; the ``HR`` contributions of a key/value head are then
    summed (the reference adds them with TMA reduce-add stores,
    ``mha_h100.cu:456-479``).

    With ``lse_log2`` the LSE input is ``L2``, already in log2 units
    (``build_mha_bwd_prep_kernel`` writes it); otherwise ``L`` is scaled by
    log2(e) in the loop."""
    scale = 1.0 / math.sqrt(d)
    kv_glob, vec_glob, kv_tile = _bwd_globals(d, block_kv)
    q_glob, qvec_glob, q_tile = _bwd_globals(d, block_q)
    Q, K, V, dO = Value("Q", q_glob), Value("K", kv_glob), Value("V", kv_glob), Value("dO", q_glob)
    L, Dv = Value("L2" if lse_log2 else "L", qvec_glob), Value("Dv", qvec_glob)
    if gqa:
        part_glob = GlobalType(GPUType.fp32, kv_tile)
        dK, dV = Value("dK_part", part_glob), Value("dV_part", part_glob)
    else:
        dK, dV = Value("dK", kv_glob), Value("dV", kv_glob)
    n_q = Value("N", IntType())
    kv_idx, head, batch = (Value(n, IntType()) for n in ("blockIdx.x", "blockIdx.y", "blockIdx.z"))
    bh = (batch, head)
    head_map, bh_kv, extra_inputs = [], bh, ()
    if gqa:
        hr, kv_head = Value("HR", IntType()), Value("kv_head", IntType())
        head_map = [IntDivOp(result=kv_head, input=head, divisor=hr)]
        bh_kv, extra_inputs = (batch, kv_head), (hr,)
    st_f = RegTileType(GPUType.fp32, wave_rows, block_q)
    st_b = RegTileType(GPUType.bf16, wave_rows, block_q)
    acc = RegTileType(GPUType.fp32, wave_rows, d)
    rvec = RowVecType(GPUType.fp32, wave_rows, block_q)

    def v(n, t):
        return Value(n, t)

    k_sh, v_sh, q_sh, do_sh = v("k_shared", kv_tile), v("v_shared", kv_tile), v("q_shared", q_tile), v("do_shared", q_tile)
    qvec_tile = qvec_glob.sub_tile_type
    lse_sh, dv_sh = v("lse_shared", qvec_tile), v("dvec_shared", qvec_tile)
    i = v("i", IntType())
    lse, lse2, dvec = v("lse", rvec), v("lse_log2", rvec), v("d_vec", rvec)
    dk_init, dk_acc, dk_new, dk_final, dk_out = (v(n, acc) for n in ("dk_init", "dk_accum", "dk_new", "dk_final", "dk_out"))
    dv_init, dv_acc, dv_new, dv_final = (v(n, acc) for n in ("dv_init", "dv_accum", "dv_new", "dv_final"))
    zero, st, st_sc, st_sh, pt = (v(n, st_f) for n in ("st_zero", "st", "st_scaled", "st_shifted", "pt"))
    dpt_zero, dpt, dpt_sub, dst = (v(n, st_f) for n in ("dpt_zero", "dpt", "dpt_minus_d", "dst"))
    pt_b, dst_b = v("pt_bf16", st_b), v("dst_bf16", st_b)
    start, prologue, scores, mask = 0, [], st, []
    if causal:
        if block_kv % block_q:
            raise ValueError("causal key-major loop needs block_kv to be a multiple of block_q")
        start = v("q_start", IntType())
        prologue = [IntAffineOp(result=start, input=kv_idx, mul=block_kv // block_q, add=0)]
        scores = v("st_masked", st_f)
        mask = [CausalMaskOp(result=scores, tile=st, row_tile=kv_idx, col_tile=i, transposed=True)]
    loop = ForOp(
        induction_var=i, start=start, stop=n_q, step=1, tile_size=block_q,
        iter_args=(IterArg(block_arg=dk_acc, init=dk_init), IterArg(block_arg=dv_acc, init=dv_init)),
        body=(
            TMALoadOp(result=q_sh, source=Q, coords=(*bh, i, 0)),
            TMALoadOp(result=do_sh, source=dO, coords=(*bh, i, 0)),
            TMALoadOp(result=lse_sh, source=L, coords=(*bh, i, 0)),
            TMALoadOp(result=dv_sh, source=Dv, coords=(*bh, i, 0)),
            WaitOp(values=(q_sh, do_sh, lse_sh, dv_sh)),
            LoadVecOp(result=lse, source=lse_sh, coords=()),
            LoadVecOp(result=dvec, source=dv_sh, coords=()),
            ZeroOp(result=zero),
            MMAOp(result=st, a=k_sh, b=q_sh, accum=zero, transpose_b=True),
            *mask,
            MulScalarOp(result=st_sc, input=scores, scalar=scale * LOG2E),
            *([] if lse_log2 else [MulScalarOp(result=lse2, input=lse, scalar=LOG2E)]),
            SubColOp(result=st_sh, tile=st_sc, vec=lse if lse_log2 else lse2),
            Exp2Op(result=pt, input=st_sh),
            ZeroOp(result=dpt_zero),
            MMAOp(result=dpt, a=v_sh, b=do_sh, accum=dpt_zero, transpose_b=True),
            SubColOp(result=dpt_sub, tile=dpt, vec=dvec),
            MulOp(result=dst, a=pt, b=dpt_sub),
            CopyOp(result=pt_b, input=pt),
            CopyOp(result=dst_b, input=dst),
            MMAOp(result=dv_new, a=pt_b, b=do_sh, accum=dv_acc),
            MMAOp(result=dk_new, a=dst_b, b=q_sh, accum=dk_acc),
            YieldOp(values=(dk_new, dv_new)),
        ),
        results=(dk_final, dv_final),
    )
    body = (
        *head_map,
        TMALoadOp(result=k_sh, source=K, coords=(*bh_kv, kv_idx, 0)),
        TMALoadOp(result=v_sh, source=V, coords=(*bh_kv, kv_idx, 0)),
        WaitOp(values=(k_sh, v_sh)),
        ZeroOp(result=dk_init),
        ZeroOp(result=dv_init),
        *prologue,
        loop,
        MulScalarOp(result=dk_out, input=dk_final, scalar=scale),
        TMAStoreOp(source=dk_out, dest=dK, coords=(*bh, kv_idx, 0)),
        TMAStoreOp(source=dv_final, dest=dV, coords=(*bh, kv_idx, 0)),
    )
    return Kernel(name=name, inputs=(Q, K, V, dO, L, Dv, n_q, *extra_inputs), outputs=(dK, dV), body=body)
