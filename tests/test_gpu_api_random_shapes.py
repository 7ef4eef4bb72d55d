"""GPU parity of the public entry points (``warpir_amd.api``) over seeded
random shapes: every routing decision (256x256 / 128x128 / 128x64 /
128x32 tiles, split-K; the four attention variants, grouped-query heads)
meets the shapes a caller may pass, including M = 1, ragged M and short K.

Oracle: ``oracle/torch_ref.py`` (fp32 ``A @ B``, naive fp32 attention and
its autograd backward; reference ``tests/test_modal_gpu.py:115``,
``tests/test_modal_attention.py:92-98``), evaluated on the GPU with torch's
own fp32 matmuls, at ``max|out - ref| / max|ref| <= 1e-2``.
"""
import random

import pytest
import torch

from oracle.torch_ref import attention_bwd_ref, attention_ref, gemm_ref, rel_err, seeded_normal
from tests.conftest import announce
from warpir_amd import api

TOL = 1e-2
pytestmark = pytest.mark.gpu


def _gemm_shapes():
    rng = random.Random(2026)
    shapes = [(1, 8, 8), (1, 4096, 8192), (3, 264, 4104), (17, 1024, 64), (128, 8192, 8192),
              (129, 520, 1032), (255, 8, 2048), (256, 768, 136), (300, 4096, 512),
              (4096, 4096, 520), (4100, 4104, 136), (5000, 3336, 1000)]
    while len(shapes) < 43:
        m = rng.choice([rng.randint(1, 128), rng.randint(129, 256), rng.randint(257, 1500)])
        n = 8 * rng.randint(1, 400)
        k = 8 * rng.choice([rng.randint(1, 64), rng.randint(65, 1200)])
        shapes.append((m, n, k))
    return shapes


@pytest.mark.parametrize("m,n,k", _gemm_shapes())
def test_gemm_random_shapes(gpu, m, n, k):
    announce(f"api.gemm {m}x{n}x{k} -> {api.gemm_variant(m, n, k)}")
    seed = m * 1_000_003 + n * 1009 + k
    a = seeded_normal((m, k), seed % 100_000, 0.1).cuda()
    b = seeded_normal((k, n), (seed + 1) % 100_000, 0.1).cuda()
    c = api.gemm(a, b)
    err = rel_err(c, gemm_ref(a, b))
    torch.cuda.synchronize()
    assert err <= TOL, err
    assert not torch.isnan(c.float()).any()


def _attention_shapes():
    rng = random.Random(4242)
    cases = []
    while len(cases) < 16:
        d = rng.choice([64, 128])
        hkv = rng.randint(1, 3)
        cases.append((rng.randint(1, 3), hkv * rng.choice([1, 1, 2, 3]), hkv, 64 * rng.randint(1, 24), d,
                      rng.random() < 0.5))
    return cases


@pytest.mark.parametrize("b,hq,hkv,s,d,causal", _attention_shapes())
def test_attention_forward_random_shapes(gpu, b, hq, hkv, s, d, causal):
    announce(f"api.attention_forward B={b} Hq={hq} Hkv={hkv} S={s} D={d} causal={causal}")
    seed = (b * 7 + hq * 11 + hkv * 13 + s * 17 + d) % 100_000
    q = seeded_normal((b, hq, s, d), seed).cuda()
    k = seeded_normal((b, hkv, s, d), seed + 1).cuda()
    v = seeded_normal((b, hkv, s, d), seed + 2).cuda()
    o, lse = api.attention_forward(q, k, v, causal=causal)
    hr = hq // hkv
    for bi in range(b):
        for hi in range(hq):
            ref, ref_lse = attention_ref(q[bi, hi], k[bi, hi // hr], v[bi, hi // hr], causal=causal)
            assert rel_err(o[bi, hi], ref) <= TOL, (bi, hi)
            assert (lse[bi, hi] - ref_lse).abs().max().item() <= 1e-3 * ref_lse.abs().max().item() + 1e-3


@pytest.mark.parametrize("b,hq,hkv,s,d,causal", _attention_shapes()[:8])
def test_attention_backward_random_shapes(gpu, b, hq, hkv, s, d, causal):
    announce(f"api.attention_backward B={b} Hq={hq} Hkv={hkv} S={s} D={d} causal={causal}")
    seed = (b * 5 + hq * 3 + hkv * 19 + s * 23 + d) % 100_000
    q = seeded_normal((b, hq, s, d), seed).cuda()
    k = seeded_normal((b, hkv, s, d), seed + 1).cuda()
    v = seeded_normal((b, hkv, s, d), seed + 2).cuda()
    do = seeded_normal((b, hq, s, d), seed + 3).cuda()
    o, lse = api.attention_forward(q, k, v, causal=causal)
    dq, dk, dv = api.attention_backward(q, k, v, o, lse, do, causal=causal)
    hr = hq // hkv
    # grouped-query: expand K/V to the query heads, then sum the expanded gradients per K/V head
    ke = k.repeat_interleave(hr, dim=1)
    ve = v.repeat_interleave(hr, dim=1)
    rq, rk, rv = attention_bwd_ref(q, ke, ve, do, causal=causal)
    rk = rk.reshape(b, hkv, hr, s, d).sum(2)
    rv = rv.reshape(b, hkv, hr, s, d).sum(2)
    for name, out, ref in (("dq", dq, rq), ("dk", dk, rk), ("dv", dv, rv)):
        err = rel_err(out, ref)
        assert err <= TOL, (name, err)


@pytest.mark.parametrize("m,n,k", [(0, 64, 64), (64, 0, 64), (0, 0, 0), (64, 64, 0), (128, 8192, 0),
                                   (300, 4096, 0), (1024, 1024, 0)])
def test_gemm_empty_products(gpu, m, n, k):
    """M or N = 0 launches nothing; K = 0 runs the kernel with no loop step and
    its tile loads reading the zero page, so every output element is 0 (the
    output starts as NaN to show that the kernel wrote it)."""
    announce(f"api.gemm empty {m}x{n}x{k} -> {api.gemm_variant(m, n, k)}")
    a = torch.randn(m, k).to(torch.bfloat16).cuda()
    b = torch.randn(k, n).to(torch.bfloat16).cuda()
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    c = api.gemm(a, b, out=out)
    torch.cuda.synchronize()
    assert c is out and tuple(c.shape) == (m, n)
    assert torch.equal(c.float().cpu(), torch.zeros(m, n))


@pytest.mark.parametrize("b,hq,hkv,s,d,causal", [(1, 2, 2, 0, 128, False), (0, 2, 2, 128, 128, False),
                                                 (1, 2, 2, 0, 64, True), (1, 4, 2, 0, 128, False)])
def test_attention_empty_shapes(gpu, b, hq, hkv, s, d, causal):
    """No queries (S = 0) or no batch: the forward and backward return empty
    tensors of the right shapes and launch nothing."""
    announce(f"api.attention empty B={b} Hq={hq} Hkv={hkv} S={s} D={d} causal={causal}")
    q = torch.randn(b, hq, s, d).to(torch.bfloat16).cuda()
    k = torch.randn(b, hkv, s, d).to(torch.bfloat16).cuda()
    v = torch.randn(b, hkv, s, d).to(torch.bfloat16).cuda()
    o, lse = api.attention_forward(q, k, v, causal=causal)
    dq, dk, dv = api.attention_backward(q, k, v, o, lse, torch.zeros_like(o), causal=causal)
    torch.cuda.synchronize()
    assert o.shape == q.shape and tuple(lse.shape) == (b, hq, s)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape


@pytest.mark.parametrize("b,s,h,d,causal", [(2, 256, 4, 128, False), (1, 384, 3, 64, True), (2, 192, 2, 128, True)])
def test_attention_on_transposed_views_of_packed_qkv(gpu, b, s, h, d, causal):
    """Q, K, V as ``[B, H, S, D]`` views of one packed ``[B, S, 3, H, D]`` tensor
    (the layout a QKV projection produces): the kernels take the row, head and
    batch strides as given, forward and backward, and O comes out in the same
    dimension order."""
    announce(f"api.attention packed-QKV views B={b} S={s} H={h} D={d} causal={causal}")
    torch.manual_seed(b * 100 + s + h + d)
    base = torch.randn(b, s, 3, h, d, device="cuda").to(torch.bfloat16)
    q, k, v = (base[:, :, i].transpose(1, 2) for i in range(3))
    assert not q.is_contiguous()
    o, lse = api.attention_forward(q, k, v, causal=causal)
    do = torch.randn(b, s, h, d, device="cuda").to(torch.bfloat16).transpose(1, 2)
    dq, dk, dv = api.attention_backward(q, k, v, o, lse, do, causal=causal)
    torch.cuda.synchronize()
    ref, ref_lse = attention_ref(q.contiguous(), k.contiguous(), v.contiguous(), causal=causal)
    assert o.stride() == (s * h * d, d, h * d, 1)   # empty_like keeps the [B, S, H, D] order, compacted
    assert rel_err(o, ref) <= TOL
    assert (lse - ref_lse).abs().max().item() <= 1e-3 * ref_lse.abs().max().item() + 1e-3
    refs = attention_bwd_ref(q.contiguous(), k.contiguous(), v.contiguous(), do.contiguous(), causal=causal)
    for name, got, r in zip(("dQ", "dK", "dV"), (dq, dk, dv), refs):
        assert rel_err(got, r) <= TOL, (name, rel_err(got, r))
