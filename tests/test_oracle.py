"""The CPU oracle itself (CPU): interpreter vs torch closed forms.

Config 1 of the benchmark set: the reference GEMM IR at M=N=K=1024,
through ``kernel_pass``, printed, interpreted on the CPU and checked
against ``torch.matmul`` (no GPU).  The interpreter follows the
reference lowering's storage semantics (aliasing, in-place MMA
accumulation, drain counter), so SSA and buffer forms must agree bit for
bit.  Closed forms pin ``oracle.torch_ref``: identity B, one-hot V,
constant K, and the log-sum-exp of constant scores.
"""
import math

import pytest
import torch

from oracle.ir_interp import run_kernel
from oracle.torch_ref import attention_ref, gemm_ref, rel_err, seeded_normal
from warpir_amd.passes.modulo_scheduler import GFX950_COST_MODEL, kernel_pass
from warpir_amd.printing import format_kernel
from warpir_amd.workloads import build_attention_kernel, build_gemm_kernel, build_mha_forward_kernel


def _gemm(kernel, a, b):
    c = torch.zeros(a.shape[0], b.shape[1], dtype=torch.bfloat16)
    run_kernel(kernel, {"A": a, "B": b, "C_global": c}, {"N": a.shape[1]})
    return c


def test_config1_gemm_1024_through_pass_and_printer():
    a = seeded_normal((1024, 1024), 0, 0.1)
    b = seeded_normal((1024, 1024), 1, 0.1)
    piped = kernel_pass(build_gemm_kernel())
    assert "mma_buf" in format_kernel(piped)
    c = _gemm(piped, a, b)
    assert rel_err(c, gemm_ref(a, b)) <= 1e-2


@pytest.mark.parametrize("m,n,k", [(64, 64, 64), (128, 192, 64), (100, 72, 136), (64, 64, 200)])
def test_ssa_and_buffer_forms_agree_bitwise(m, n, k):
    a = seeded_normal((m, k), 5, 0.1)
    b = seeded_normal((k, n), 6, 0.1)
    ssa = _gemm(build_gemm_kernel(), a, b)
    piped = _gemm(kernel_pass(build_gemm_kernel()), a, b)
    assert torch.equal(ssa, piped)
    assert rel_err(ssa, gemm_ref(a, b)) <= 1e-2


def test_mi355x_gemm_ir_interpreted():
    a = seeded_normal((300, 520), 2, 0.1)
    b = seeded_normal((520, 264), 3, 0.1)
    k = kernel_pass(build_gemm_kernel(256, 256, 32, 128, 128), cost_model=GFX950_COST_MODEL)
    assert rel_err(_gemm(k, a, b), gemm_ref(a, b)) <= 1e-2


@pytest.mark.parametrize("variant", ["gemm_256_k64", "gemm_128x32_k64", "gemm_128_k64"])
@pytest.mark.parametrize("k", [0, 8])
def test_pipelined_gemm_with_fewer_steps_than_stages(variant, k):
    """K = 0 and K = 8 (no loop trip after the prologue): the pipelined IR's
    drain reads only ring slots its prologue loaded (an unloaded slot is None
    here and would raise), and the product is A @ B (zeros for K = 0)."""
    from warpir_amd import kernels

    a = seeded_normal((256, k), 11, 0.1)
    b = seeded_normal((k, 96), 12, 0.1)
    c = _gemm(kernels.VARIANTS[variant](), a, b)
    if k == 0:
        assert torch.equal(c, torch.zeros_like(c))
    else:
        assert rel_err(c, gemm_ref(a, b)) <= 1e-2


def test_gemm_ref_identity_closed_form():
    a = seeded_normal((64, 64), 9, 0.1)
    assert torch.equal(gemm_ref(a, torch.eye(64, dtype=torch.bfloat16)), a.float())


@pytest.mark.parametrize("n", [64, 256])
def test_reference_attention_ir_interpreted(n):
    q, k, v = (seeded_normal((n, 64), s) for s in (0, 1, 2))
    o = torch.zeros(n, 64, dtype=torch.bfloat16)
    run_kernel(build_attention_kernel(), {"Q": q, "K": k, "V": v, "O": o}, {"N": n})
    ref, _ = attention_ref(q, k, v, scale=1 / math.sqrt(64))
    assert rel_err(o, ref) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
def test_mha_ir_interpreted_with_lse(causal):
    b, h, s, d = 1, 2, 256, 64
    q, k, v = (seeded_normal((b, h, s, d), sd) for sd in (3, 4, 5))
    o = torch.zeros(b, h, s, d, dtype=torch.bfloat16)
    lse = torch.zeros(b, h, s, dtype=torch.float32)
    kern = build_mha_forward_kernel(d=d, block_q=128, block_kv=64, wave_rows=32, causal=causal)
    run_kernel(kern, {"Q": q, "K": k, "V": v, "O": o, "L": lse}, {"N": s})
    ref, ref_lse = attention_ref(q, k, v, causal=causal)
    assert rel_err(o, ref) <= 1e-2
    assert (lse - ref_lse).abs().max().item() <= 1e-3


def _mha_interp(q, k, v, causal, slack):
    b, h, s, d = q.shape
    o = torch.zeros(b, h, s, d, dtype=torch.bfloat16)
    lse = torch.zeros(b, h, s, dtype=torch.float32)
    kern = build_mha_forward_kernel(d=d, block_q=128, block_kv=64, wave_rows=32, causal=causal,
                                    rescale_slack=slack)
    run_kernel(kern, {"Q": q, "K": k, "V": v, "O": o, "L": lse}, {"N": s})
    return o, lse


@pytest.mark.parametrize("causal", [False, True])
def test_mha_lazy_rescale_interpreted(causal):
    b, h, s, d = 1, 2, 256, 64
    q, k, v = (seeded_normal((b, h, s, d), sd) for sd in (3, 4, 5))
    # keys grow along the sequence, so later tiles raise the row maxima by
    # more than the slack and the rescale path runs too
    k = (k.float() * torch.linspace(0.5, 6.0, s).view(1, 1, s, 1)).to(torch.bfloat16)
    o, lse = _mha_interp(q, k, v, causal, 8.0)
    ref, ref_lse = attention_ref(q, k, v, causal=causal)
    assert rel_err(o, ref) <= 1e-2
    assert (lse - ref_lse).abs().max().item() <= 1e-3


def test_lazy_max_with_zero_slack_is_the_plain_max():
    # cand = max(prev, rowmax) >= prev, so slack 0 selects exactly the running max
    q, k, v = (seeded_normal((1, 1, 256, 64), sd) for sd in (6, 7, 8))
    o0, l0 = _mha_interp(q, k, v, False, 0.0)
    o1, l1 = _mha_interp(q, k, v, False, None)
    assert torch.equal(o0, o1) and torch.equal(l0, l1)


def test_attention_ref_closed_forms():
    s, d = 64, 64
    q = seeded_normal((s, d), 1)
    k = torch.zeros(s, d, dtype=torch.bfloat16)  # constant scores -> uniform softmax
    v = seeded_normal((s, d), 2)
    o, lse = attention_ref(q, k, v)
    assert torch.allclose(o, v.float().mean(0, keepdim=True).expand(s, d), atol=1e-6)
    assert torch.allclose(lse, torch.full((s,), math.log(s)), atol=1e-6)
    # one-hot V columns return the probability matrix itself
    v1 = torch.eye(s, dtype=torch.bfloat16)
    k1 = seeded_normal((s, d), 3)
    o1, _ = attention_ref(q, k1, v1)
    p = torch.softmax((q.float() @ k1.float().t()) / math.sqrt(d), dim=-1)
    assert torch.allclose(o1, p, atol=1e-6)


def test_causal_first_row_attends_only_to_first_key():
    q, k, v = (seeded_normal((1, 1, 64, 64), s) for s in (7, 8, 9))
    o, _ = attention_ref(q, k, v, causal=True)
    assert torch.allclose(o[0, 0, 0], v[0, 0, 0].float(), atol=1e-6)


def test_fused_split_k_interprets_as_the_slice_sum():
    """reduce_slices: after all slices of a ragged 200 x 384 product (2 x 3 tiles, 3 slices),
    C holds bf16 of the partials summed in slice order from 0 -- what the two-launch
    reduction computes -- and every arrival counter is back at zero."""
    from warpir_amd.passes.modulo_scheduler import gfx950_cost_model
    from warpir_amd.printing import format_kernel
    from warpir_amd.workloads import build_gemm_kernel
    k = kernel_pass(build_gemm_kernel(block_m=128, block_n=128, block_k=128, wave_m=64, wave_n=64, name="gemm_splitk",
                                      split_k=True, fused_reduce=True),
                    cost_model=gfx950_cost_model(128, 128, 128, lds_budget=160 * 1024, hbm_sources=("B",)))
    assert "reduce_slices(%C_global" in format_kernel(k)
    s, m, n, kc = 3, 200, 384, 256
    a = seeded_normal((m, kc * s), 31, 0.1)
    b = seeded_normal((kc * s, n), 32, 0.1)
    part = torch.zeros(1, s, m, n)
    out = torch.full((1, 1, m, n), float("nan"), dtype=torch.bfloat16)
    arrivals = torch.zeros(6, dtype=torch.int64)
    run_kernel(k, {"A": a.view(m, s, kc).permute(1, 0, 2).unsqueeze(0), "B": b.view(s, kc, n).unsqueeze(0),
                   "C_global": part, "C": out, "Arrivals": arrivals}, {"N": kc})
    total = torch.zeros(m, n)
    for j in range(s):
        total = total + part[0, j]
    assert torch.equal(out[0, 0], total.bfloat16())
    assert int(arrivals.abs().sum()) == 0
    assert rel_err(out[0, 0], gemm_ref(a, b)) <= 1e-2


@pytest.mark.parametrize("causal", [False, True])
def test_bf16_operand_backward_reference_is_autograd_without_rounding(causal):
    """The hand-written gradient of ``attention_bwd_ref_bf16`` (dV = P^T dO,
    dS = P (dP - D) * scale, dQ = dS K, dK = dS^T Q) equals torch autograd when
    its bf16 roundings are off and D comes from the exact output; with them on
    it moves by about the bf16 rounding of P and dS (well under 1e-2 here)."""
    from oracle.torch_ref import attention_bwd_ref, attention_bwd_ref_bf16

    q, k, v, do = (seeded_normal((2, 96, 64), sd) for sd in (21, 22, 23, 24))
    o, _ = attention_ref(q, k, v, causal=causal)
    exact = attention_bwd_ref(q, k, v, do, causal=causal)
    plain = attention_bwd_ref_bf16(q, k, v, o, do, causal=causal, round_operands=False)
    for a, b in zip(plain, exact):
        assert rel_err(a, b) <= 1e-5
    rounded = attention_bwd_ref_bf16(q, k, v, o, do, causal=causal)
    errs = [rel_err(a, b) for a, b in zip(rounded, exact)]
    assert all(1e-5 < e <= 1e-2 for e in errs), errs
