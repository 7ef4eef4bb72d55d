"""FlashAttention backward as WarpIR kernels, checked on the CPU interpreter.

The three kernels (``workloads.build_mha_bwd_*``) are run by the oracle's
IR interpreter -- in SSA form and after ``kernel_pass`` -- and compared
with torch autograd of the fp32 forward.  The autograd oracle itself is
pinned by closed forms: with uniform attention (identical key rows) dV is the
column sum of dO divided by S, dQ vanishes and dK has a closed form; Dv = rowsum(dO * O) is
checked against the identity sum(dP * P) = Dv row by row.
"""
import math

import pytest
import torch

from oracle.ir_interp import run_kernel
from oracle.torch_ref import attention_bwd_ref, attention_ref, rel_err, seeded_normal
from warpir_amd.passes.modulo_scheduler import gfx950_attention_cost_model, kernel_pass
from warpir_amd.workloads import (build_mha_bwd_dkdv_kernel, build_mha_bwd_dq_kernel,
                                  build_mha_bwd_prep_kernel)

TOL = 1e-2


def _inputs(b, h, s, d, seed=0, causal=False):
    q, k, v, do = (seeded_normal((b, h, s, d), seed + j) for j in range(4))
    o, lse = attention_ref(q, k, v, causal=causal)
    return q, k, v, do, o.to(torch.bfloat16), lse


def _bwd_via_ir(q, k, v, do, o, lse, pipelined: bool, d: int, causal: bool = False):
    b, h, s, _ = q.shape
    prep = build_mha_bwd_prep_kernel(d=d, block_q=128, wave_rows=32)
    dq_k = build_mha_bwd_dq_kernel(d=d, block_q=128, block_kv=64, wave_rows=32, causal=causal)
    dkdv_k = build_mha_bwd_dkdv_kernel(d=d, block_kv=128, block_q=64, wave_rows=32, causal=causal)
    if pipelined:
        dq_k = kernel_pass(dq_k, cost_model=gfx950_attention_cost_model(128, 64, d))
        dkdv_k = kernel_pass(dkdv_k, cost_model=gfx950_attention_cost_model(128, 64, d))
    dv_vec, lse2 = torch.zeros(b, h, s), torch.zeros(b, h, s)
    run_kernel(prep, {"O": o, "dO": do, "L": lse, "Dv": dv_vec, "L2": lse2}, {})
    assert torch.equal(lse2, lse * math.log2(math.e))   # the same fp32 product as the dq kernel's
    dq = torch.zeros(b, h, s, d, dtype=torch.bfloat16)
    dk, dv = torch.zeros_like(dq), torch.zeros_like(dq)
    run_kernel(dq_k, {"Q": q, "K": k, "V": v, "dO": do, "L": lse, "Dv": dv_vec, "dQ": dq}, {"N": s})
    run_kernel(dkdv_k, {"Q": q, "K": k, "V": v, "dO": do, "L2": lse2, "Dv": dv_vec, "dK": dk, "dV": dv}, {"N": s})
    return dv_vec, dq, dk, dv


@pytest.mark.parametrize("pipelined", [False, True])
def test_attention_backward_ir_matches_autograd(pipelined):
    q, k, v, do, o, lse = _inputs(1, 2, 256, 64)
    dv_vec, dq, dk, dv = _bwd_via_ir(q, k, v, do, o, lse, pipelined, d=64)
    rq, rk, rv = attention_bwd_ref(q, k, v, do)
    assert torch.allclose(dv_vec, (do.float() * o.float()).sum(-1), rtol=1e-5, atol=1e-5)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert rel_err(got.float(), ref) <= TOL


@pytest.mark.parametrize("pipelined", [False, True])
@pytest.mark.parametrize("s", [256, 192])
def test_causal_attention_backward_ir_matches_autograd(pipelined, s):
    q, k, v, do, o, lse = _inputs(1, 2, s, 64, seed=3, causal=True)
    _, dq, dk, dv = _bwd_via_ir(q, k, v, do, o, lse, pipelined, d=64, causal=True)
    rq, rk, rv = attention_bwd_ref(q, k, v, do, causal=True)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert rel_err(got.float(), ref) <= TOL


def test_causal_backward_closed_forms():
    # The first query sees only the first key: P[0, 0] = 1 and Dv[0] = dO[0].V[0] = dP[0, 0],
    # so dS[0, 0] = 0 and dQ[0] = 0.  The last key is seen only by the last query, so
    # dV[-1] = P[-1, -1] dO[-1] and dK[-1] is a multiple of Q[-1].
    q, k, v, do, o, lse = _inputs(1, 1, 128, 64, seed=5, causal=True)
    _, dq, dk, dv = _bwd_via_ir(q, k, v, do, o, lse, True, d=64, causal=True)
    rq, rk, rv = attention_bwd_ref(q, k, v, do, causal=True)
    s_last = (q[0, 0, -1].double() @ k[0, 0].double().t()) / 8.0
    p_last = torch.softmax(s_last, dim=0)[-1].item()
    for dq_, dk_, dv_ in ((dq.float(), dk.float(), dv.float()), (rq, rk, rv)):
        assert dq_[0, 0, 0].abs().max().item() <= 1e-2 * dq_.abs().max().item()
        assert torch.allclose(dv_[0, 0, -1], p_last * do[0, 0, -1].float(), rtol=2e-2, atol=2e-3)
        cos = torch.nn.functional.cosine_similarity(dk_[0, 0, -1], q[0, 0, -1].float(), dim=0).abs()
        assert cos.item() > 0.99


@pytest.mark.parametrize("causal", [False, True])
def test_grouped_query_attention_ir_matches_autograd(causal):
    """H = 4 query heads over 2 key/value heads: forward and backward IR (pipelined) against
    autograd through the head expansion; dK / dV are the per-query-head contributions summed
    over each group."""
    import math as _m
    from warpir_amd.workloads import build_mha_forward_kernel
    b, hq, hkv, s, d = 1, 4, 2, 256, 64
    hr = hq // hkv
    q, do = seeded_normal((b, hq, s, d), 21), seeded_normal((b, hq, s, d), 24)
    k, v = seeded_normal((b, hkv, s, d), 22), seeded_normal((b, hkv, s, d), 23)
    cost = gfx950_attention_cost_model(128, 64, d)
    fwd = kernel_pass(build_mha_forward_kernel(d=d, causal=causal, gqa=True), cost_model=cost)
    o = torch.zeros(b, hq, s, d, dtype=torch.bfloat16)
    lse = torch.zeros(b, hq, s)
    run_kernel(fwd, {"Q": q, "K": k, "V": v, "O": o, "L": lse}, {"N": s, "HR": hr})
    ref_o, ref_lse = attention_ref(q, k.repeat_interleave(hr, 1), v.repeat_interleave(hr, 1), causal=causal)
    assert rel_err(o, ref_o) <= TOL and (lse - ref_lse).abs().max().item() <= 1e-3
    dv_vec, lse2 = torch.zeros(b, hq, s), torch.zeros(b, hq, s)
    run_kernel(build_mha_bwd_prep_kernel(d=d), {"O": o, "dO": do, "L": lse, "Dv": dv_vec, "L2": lse2}, {})
    dq = torch.zeros(b, hq, s, d, dtype=torch.bfloat16)
    dq_k = kernel_pass(build_mha_bwd_dq_kernel(d=d, causal=causal, gqa=True), cost_model=cost)
    run_kernel(dq_k, {"Q": q, "K": k, "V": v, "dO": do, "L": lse, "Dv": dv_vec, "dQ": dq}, {"N": s, "HR": hr})
    dk_part, dv_part = torch.zeros(b, hq, s, d), torch.zeros(b, hq, s, d)
    dkdv_k = kernel_pass(build_mha_bwd_dkdv_kernel(d=d, causal=causal, gqa=True), cost_model=cost)
    run_kernel(dkdv_k, {"Q": q, "K": k, "V": v, "dO": do, "L2": lse2, "Dv": dv_vec, "dK_part": dk_part,
                        "dV_part": dv_part}, {"N": s, "HR": hr})
    dk, dv = dk_part.view(b, hkv, hr, s, d).sum(2), dv_part.view(b, hkv, hr, s, d).sum(2)
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    sc = qf @ kf.repeat_interleave(hr, 1).transpose(-1, -2) / _m.sqrt(d)
    if causal:
        sc = sc.masked_fill(torch.ones(s, s, dtype=torch.bool).triu(1), float("-inf"))
    (torch.softmax(sc, -1) @ vf.repeat_interleave(hr, 1)).backward(do.float())
    for got, ref in ((dq.float(), qf.grad), (dk, kf.grad), (dv, vf.grad)):
        assert rel_err(got, ref) <= TOL
    # with HR = 1 the grouped kernels are the plain ones
    o1 = torch.zeros(b, hkv, s, d, dtype=torch.bfloat16)
    l1 = torch.zeros(b, hkv, s)
    run_kernel(fwd, {"Q": q[:, :hkv].contiguous(), "K": k, "V": v, "O": o1, "L": l1}, {"N": s, "HR": 1})
    o2 = torch.zeros_like(o1)
    l2 = torch.zeros_like(l1)
    plain = kernel_pass(build_mha_forward_kernel(d=d, causal=causal), cost_model=cost)
    run_kernel(plain, {"Q": q[:, :hkv].contiguous(), "K": k, "V": v, "O": o2, "L": l2}, {"N": s})
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_attention_backward_ir_d128_ragged_kv_blocks():
    # S = 192: the key-major kernel's 128-row key tiles are partial
    q, k, v, do, o, lse = _inputs(1, 1, 192, 128, seed=7)
    _, dq, dk, dv = _bwd_via_ir(q, k, v, do, o, lse, True, d=128)
    rq, rk, rv = attention_bwd_ref(q, k, v, do)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        assert rel_err(got.float(), ref) <= TOL


def test_autograd_oracle_closed_forms():
    s, d = 64, 32
    q = seeded_normal((1, s, d), 1)
    k = torch.ones(1, s, d, dtype=torch.bfloat16)          # every score equal -> uniform softmax
    v, do = seeded_normal((1, s, d), 2), seeded_normal((1, s, d), 3)
    dq, dk, dv = attention_bwd_ref(q, k, v, do)
    assert torch.allclose(dv, do.float().sum(1, keepdim=True).expand(1, s, d) / s, atol=1e-5)
    # identical key rows: each row of dS = P * (dP - rowsum(P dP)) sums to 0, so dQ = dS K = 0;
    # dK_j = scale * sum_i dS_ij q_i  (a textbook restatement with P = 1/S)
    assert dq.abs().max().item() < 1e-5
    p_u = torch.full((s, s), 1.0 / s)
    dp = do[0].float() @ v[0].float().t()
    ds = p_u * (dp - (p_u * dp).sum(-1, keepdim=True))
    assert torch.allclose(dk[0], ds.t() @ q[0].float() / math.sqrt(d), atol=1e-5)
    # Dv identity: rowsum(dO * O) == rowsum(P * dP)
    q2, k2, v2 = (seeded_normal((s, d), j) for j in (4, 5, 6))
    sc = (q2.float() @ k2.float().t()) / math.sqrt(d)
    p = torch.softmax(sc, -1)
    o = p @ v2.float()
    dp = do[0].float() @ v2.float().t()
    assert torch.allclose((do[0].float() * o).sum(-1), (p * dp).sum(-1), rtol=1e-4, atol=1e-5)
