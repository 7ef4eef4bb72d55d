"""Full-size parity: every output element of the headline configurations
against the fp32 oracle, evaluated on the GPU.

The sampled tests in ``test_gpu_gemm.py`` / ``test_gpu_attention.py`` run
the oracle on the CPU over a few rows or heads.  Here the same oracle
functions (``oracle/torch_ref.py``: fp32 ``A @ B``; naive fp32 attention
and its autograd backward, reference ``tests/test_modal_gpu.py:115`` and
``tests/test_modal_attention.py:92-98``) run on the GPU with torch's own
fp32 matmuls, which share no code with the generated kernels, so every
head and every output row is checked at ``max|out - ref| / max|ref| <=
1e-2`` (per head for attention).
"""
import pytest
import torch

from oracle.torch_ref import attention_bwd_ref, attention_ref, gemm_ref, rel_err, seeded_normal
from tests.conftest import announce
from warpir_amd import api, kernels

TOL = 1e-2
pytestmark = pytest.mark.gpu


def test_gemm_8192_every_element(gpu):
    """Config 1 (GEMM 8192^3, the default kernel), all 8192 x 8192 outputs."""
    n = 8192
    announce(f"gemm full {n}^3 against the GPU fp32 oracle")
    a = seeded_normal((n, n), 51, 0.1).cuda()
    b = seeded_normal((n, n), 52, 0.1).cuda()
    c = torch.full((n, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    kernels.handle("gemm_256_k64")(A=a, B=b, N=n, C_global=c)
    ref = gemm_ref(a, b)
    assert ref.is_cuda
    err = rel_err(c, ref)
    torch.cuda.synchronize()
    assert err <= TOL, err
    assert not torch.isnan(c.float()).any()


@pytest.mark.parametrize("causal,shape", [(False, (16, 16, 4096, 128)), (True, (8, 32, 8192, 64))])
def test_attention_forward_every_head(gpu, causal, shape):
    """Config 4 (B16 H16 S4096 D128) and config 5 (causal B8 H32 S8192 D64), default kernels:
    O and LSE of all 256 (b, h) heads."""
    announce(f"attention forward full causal={causal} {shape}, every head against the GPU fp32 oracle")
    q, k, v = (seeded_normal(shape, sd).cuda() for sd in (53, 54, 55))
    o, lse = api.attention_forward(q, k, v, causal=causal)
    worst, worst_lse, worst_at = 0.0, 0.0, None
    for bi in range(shape[0]):
        for hi in range(shape[1]):
            ref, ref_lse = attention_ref(q[bi, hi], k[bi, hi], v[bi, hi], causal=causal)
            e = rel_err(o[bi, hi], ref)
            if e > worst:
                worst, worst_at = e, (bi, hi)
            worst_lse = max(worst_lse, (lse[bi, hi] - ref_lse).abs().max().item())
    assert worst <= TOL, (worst, worst_at)
    assert worst_lse <= 1e-2, worst_lse


@pytest.mark.parametrize("causal", [False, True])
def test_attention_backward_every_head(gpu, causal):
    """Backward at the config-4 shape (prep + dQ + dK/dV kernels): dQ, dK, dV of all 256 heads
    against autograd of the fp32 forward."""
    shape = (16, 16, 4096, 128)
    announce(f"attention backward full causal={causal} {shape}, every head against the GPU fp32 oracle")
    q, k, v, do = (seeded_normal(shape, sd).cuda() for sd in (56, 57, 58, 59))
    o, lse = api.attention_forward(q, k, v, causal=causal)
    dq, dk, dv = api.attention_backward(q, k, v, o, lse, do, causal=causal)
    worst = {}
    for bi in range(shape[0]):
        for hi in range(shape[1]):
            refs = attention_bwd_ref(q[bi, hi], k[bi, hi], v[bi, hi], do[bi, hi], causal=causal)
            for name, out, ref in zip(("dq", "dk", "dv"), (dq, dk, dv), refs):
                e = rel_err(out[bi, hi], ref)
                if e > worst.get(name, (0.0, None))[0]:
                    worst[name] = (e, (bi, hi))
    for name, (e, at) in worst.items():
        assert e <= TOL, (name, e, at)
