"""The no-allocation split-K entry point (wir_gemm_splitk_noalloc) against
the allocating one (api.gemm_split_k): same kernels, same summation order,
so the results must be bitwise equal -- on two calls in a row, the second
smaller, sharing the library's device scratch."""
import pytest
import torch

from oracle.torch_ref import gemm_ref, rel_err, seeded_normal
from warpir_amd import api
from warpir_amd.runtime import HipError

from tests.conftest import announce


@pytest.mark.gpu
def test_noalloc_split_k_matches_the_allocating_entry_point(gpu):
    for m, n, k, splits, seed in ((64, 8192, 8192, 4, 0), (32, 2048, 4096, 8, 1)):
        announce(f"noalloc split-K M={m} N={n} K={k} splits={splits}")
        a = seeded_normal((m, k), seed, 0.1).cuda()
        b = seeded_normal((k, n), seed + 100, 0.1).cuda()
        ref = api.gemm_split_k(a, b, splits=splits)
        out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
        api.gemm_split_k_noalloc(a, b, out, splits=splits)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), (m, n, k, splits)
        cols = torch.arange(0, n, 16)
        assert rel_err(out[:, cols].cpu(), gemm_ref(a.cpu(), b.cpu()[:, cols])) <= 1e-2


@pytest.mark.gpu
def test_noalloc_split_k_rejects_inputs_beyond_its_scratch(gpu):
    m, n, k, splits = 512, 8192, 8192, 4          # 16 Mi partials > 8 Mi floats of scratch
    a = torch.zeros(m, k, dtype=torch.bfloat16, device="cuda")
    b = torch.zeros(k, n, dtype=torch.bfloat16, device="cuda")
    out = torch.zeros(m, n, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(HipError, match="device scratch"):
        api.gemm_split_k_noalloc(a, b, out, splits=splits)
