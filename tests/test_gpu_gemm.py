"""GPU parity of WarpIR-generated GEMM kernels against the torch oracle.

Oracle: ``torch.matmul(A.float(), B.float())`` on the CPU from the same
seeded bf16 inputs (reference ``tests/test_modal_gpu.py:115``), compared
at ``max|out - ref| / max|ref| <= 1e-2`` (the
reference itself checks only max-abs < 1.0, ``:118``).
"""
import pytest
import torch

from oracle.torch_ref import gemm_ref, rel_err, seeded_normal
from tests.conftest import announce
from warpir_amd import kernels

TOL = 1e-2
pytestmark = pytest.mark.gpu


def _run(variant, m, n, k, seed=0):
    announce(f"gemm {variant} M={m} N={n} K={k} seed={seed}")
    a = seeded_normal((m, k), seed, 0.1)
    b = seeded_normal((k, n), seed + 1, 0.1)
    c = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    kernels.handle(variant)(A=a.cuda(), B=b.cuda(), N=k, C_global=c)
    torch.cuda.synchronize()
    return a, b, c.cpu()


@pytest.mark.parametrize("variant", ["gemm_ref_ssa", "gemm_ref_piped"])
@pytest.mark.parametrize("n", [64, 128, 256, 512, 1024])
def test_reference_ir_square(gpu, variant, n):
    a, b, c = _run(variant, n, n, n)
    err = rel_err(c, gemm_ref(a, b))
    assert err <= TOL, err


MI355X_VARIANTS = sorted(v for v in kernels.VARIANTS
                         if v.startswith(("gemm_256", "gemm_128")) and "splitk" not in v)


@pytest.mark.parametrize("variant", MI355X_VARIANTS)
@pytest.mark.parametrize("m,n,k", [(256, 256, 32), (256, 256, 64), (512, 512, 512), (1024, 1024, 1024),
                                   (300, 520, 264), (1000, 776, 1032), (128, 8192, 512)])
def test_mi355x_gemm(gpu, variant, m, n, k):
    a, b, c = _run(variant, m, n, k)
    err = rel_err(c, gemm_ref(a, b))
    assert err <= TOL, err
    assert not torch.isnan(c.float()).any()


@pytest.mark.parametrize("variant", MI355X_VARIANTS)
@pytest.mark.parametrize("size", [4096, 8192])
def test_mi355x_gemm_large_sampled(gpu, variant, size):
    """Full-size run; the oracle is evaluated on 256 sampled rows."""
    a, b, c = _run(variant, size, size, size, seed=3)
    rows = torch.randperm(size, generator=torch.Generator().manual_seed(7))[:256]
    ref = gemm_ref(a[rows], b)
    err = rel_err(c[rows], ref)
    assert err <= TOL, err
    assert not torch.isnan(c.float()).any()


def test_identity_returns_a(gpu):
    """Closed form: A @ I == A exactly (bf16 products with 1.0, fp32 sums of one term)."""
    n = 512
    a = seeded_normal((n, n), 11, 0.1)
    eye = torch.eye(n, dtype=torch.bfloat16)
    c = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
    announce("gemm identity 512")
    kernels.handle("gemm_256_k64")(A=a.cuda(), B=eye.cuda(), N=n, C_global=c)
    torch.cuda.synchronize()
    assert torch.equal(c.cpu(), a)


@pytest.mark.parametrize("m,n,k,splits", [(128, 8192, 8192, None), (128, 1024, 2048, 4), (64, 512, 1024, 2),
                                          (300, 520, 2048, 4), (128, 256, 4096, 8),
                                          # K slices that are not a whole number of the kernel's 128-deep steps
                                          (96, 384, 384, 2), (128, 256, 8256, 3)])
def test_split_k_gemm(gpu, m, n, k, splits):
    """Split-K form (K slices on blockIdx.z, fp32 partials, HIP reduction) vs the fp32 oracle."""
    from warpir_amd import api

    announce(f"gemm_split_k {m}x{n}x{k} splits={splits}")
    a = seeded_normal((m, k), 21, 0.1)
    b = seeded_normal((k, n), 22, 0.1)
    c = api.gemm_split_k(a.cuda(), b.cuda(), splits=splits)
    torch.cuda.synchronize()
    err = rel_err(c.cpu(), gemm_ref(a, b))
    assert err <= TOL, err
    assert not torch.isnan(c.float()).any()


def test_api_gemm_routes_short_m_to_split_k(gpu):
    from warpir_amd import api

    m, n, k = 64, 1024, 4096
    assert api.gemm_variant(m, n, k) == api.SPLITK_GEMM_VARIANT
    announce(f"api.gemm {m}x{n}x{k} (split-K route)")
    a = seeded_normal((m, k), 23, 0.1)
    b = seeded_normal((k, n), 24, 0.1)
    c = api.gemm(a.cuda(), b.cuda())
    torch.cuda.synchronize()
    assert rel_err(c.cpu(), gemm_ref(a, b)) <= TOL


def test_api_gemm_row_strided_short_m(gpu):
    """M=128 with long K and row-strided A and out: api.gemm takes the tiled kernel (split-K
    needs dense operands) and reads and writes through the row strides."""
    from warpir_amd import api

    m, n, k = 128, 1024, 8192
    announce(f"api.gemm {m}x{n}x{k} row-strided A and out")
    a_full = seeded_normal((m, k + 64), 25, 0.1)
    b = seeded_normal((k, n), 26, 0.1)
    out_full = torch.full((m, n + 64), float("nan"), dtype=torch.bfloat16, device="cuda")
    a_dev = a_full.cuda()[:, :k]
    out = out_full[:, :n]
    api.gemm(a_dev, b.cuda(), out=out)
    torch.cuda.synchronize()
    assert rel_err(out.cpu(), gemm_ref(a_full[:, :k].contiguous(), b)) <= TOL
    assert torch.isnan(out_full[:, n:].float()).all()   # the padding columns stay untouched


def test_gemm_repeated_launches_bitwise_stable(gpu):
    """GEMM 8192^3 (the headline kernel), 6 launches into the same C: no atomics and a fixed
    accumulation order, so every launch reproduces the first bit for bit."""
    n = 8192
    announce(f"gemm_256_k64 repeated launches {n}^3")
    a = seeded_normal((n, n), 50, 0.1).cuda()
    b = seeded_normal((n, n), 51, 0.1).cuda()
    h = kernels.handle("gemm_256_k64")
    c = torch.empty(n, n, dtype=torch.bfloat16, device="cuda")
    h(A=a, B=b, N=n, C_global=c)
    first = c.clone()
    for it in range(5):
        c.fill_(float("nan"))
        h(A=a, B=b, N=n, C_global=c)
        assert torch.equal(c, first), it


def test_split_k_repeated_launches_bitwise_stable(gpu):
    """Split-K GEMM (fp32 partials per K slice, HIP reduction in slice order), 4 launches into the
    same output and workspace: bitwise identical each time."""
    from warpir_amd import api

    m, n, k, splits = 128, 8192, 8192, 4
    announce(f"gemm_split_k repeated launches {m}x{n}x{k} splits={splits}")
    a = seeded_normal((m, k), 80, 0.1).cuda()
    b = seeded_normal((k, n), 81, 0.1).cuda()
    ws = torch.empty(splits * m * n, dtype=torch.float32, device="cuda")
    c = api.gemm_split_k(a, b, splits=splits, workspace=ws)
    first = c.clone()
    for it in range(3):
        c.fill_(float("nan"))
        api.gemm_split_k(a, b, out=c, splits=splits, workspace=ws)
        assert torch.equal(c, first), it


def test_skinny_benchmark_kernel_at_its_exact_shape(gpu):
    """The kernel bench.py times for config 3' (gemm_128x32_k64) at exactly
    M=128, N=K=8192; the oracle runs on 512 sampled output columns."""
    a, b, c = _run("gemm_128x32_k64", 128, 8192, 8192, seed=11)
    cols = torch.randperm(8192, generator=torch.Generator().manual_seed(5))[:512]
    ref = gemm_ref(a, b[:, cols])
    err = rel_err(c[:, cols], ref)
    assert err <= TOL, err
    assert not torch.isnan(c.float()).any()


def test_split_k_kernel_variants_agree(gpu):
    """The 64-deep-step split-K kernel against the default 128-deep one on the same slices: both
    accumulate every output's k in order, 16 per MFMA, so the results are bitwise equal."""
    from warpir_amd import api

    m, n, k, splits = 128, 1024, 4096, 4
    announce(f"split-K variants {m}x{n}x{k} splits={splits}")
    a = seeded_normal((m, k), 90, 0.1).cuda()
    b = seeded_normal((k, n), 91, 0.1).cuda()
    c64 = api.gemm_split_k(a, b, splits=splits, variant="gemm_128_splitk")
    c128 = api.gemm_split_k(a, b, splits=splits, variant="gemm_128_splitk_k128")
    torch.cuda.synchronize()
    assert torch.equal(c64, c128)
    assert rel_err(c128.cpu(), gemm_ref(a.cpu(), b.cpu())) <= TOL


@pytest.mark.parametrize("variant", ["gemm_128_splitk_k128_b3", "gemm_128_splitk_k64_b7", "gemm_128_splitk_k64_b7sw",
                                     "gemm_128_splitk_k32_b14", "gemm_128_splitk_k32_b14sw"])
@pytest.mark.parametrize("m,n,k,splits", [(128, 8192, 8192, 4), (128, 1024, 512, 4), (128, 1024, 1024, 4),
                                          (96, 384, 384, 2), (128, 256, 8256, 3), (300, 520, 2048, 4)])
def test_split_k_per_ring_depth_agrees(gpu, m, n, k, splits, variant):
    """The per-operand ring forms (kernel_pass with B as the HBM stream: B three slots loaded two
    tiles ahead and A two at K=128, B 7 / A 3 at K=64, B 14 / A 6 at K=32, with and without the
    whole-step DMA spread) against the uniform two-slot kernel: the same MFMAs in the same k order,
    so bitwise equal -- also for slices of one or two 128-deep steps,
    where the drain consumes prologue slots and its drain_index load reads past the slice."""
    from warpir_amd import api

    announce(f"split-K per-ring depths {variant} {m}x{n}x{k} splits={splits}")
    a = seeded_normal((m, k), 92, 0.1).cuda()
    b = seeded_normal((k, n), 93, 0.1).cuda()
    ref = api.gemm_split_k(a, b, splits=splits, variant="gemm_128_splitk_k128")
    c = api.gemm_split_k(a, b, splits=splits, variant=variant)
    torch.cuda.synchronize()
    assert torch.equal(c, ref)
    assert rel_err(c.cpu(), gemm_ref(a.cpu(), b.cpu())) <= TOL


@pytest.mark.parametrize("m,n,k,splits", [(128, 8192, 8192, 4), (128, 1024, 512, 4), (96, 384, 384, 2),
                                          (128, 256, 8256, 3), (300, 520, 2048, 4), (64, 512, 1024, 16)])
def test_split_k_fused_reduction_agrees(gpu, m, n, k, splits):
    """One launch, the last slice of each output tile summing the partials (reduce_slices),
    against the two-launch form (same GEMM, separate reduction kernel): both add the fp32
    partials in slice order from 0, so bitwise equal.  Three products in a row on the same
    counters, which the kernel leaves at zero."""
    from warpir_amd import api

    announce(f"split-K fused reduction {m}x{n}x{k} splits={splits}")
    a = seeded_normal((m, k), 94, 0.1).cuda()
    b = seeded_normal((k, n), 95, 0.1).cuda()
    ref = api.gemm_split_k(a, b, splits=splits, variant=api.SPLITK_TWO_LAUNCH_VARIANT)
    for it in range(3):
        c = api.gemm_split_k(a, b, splits=splits, variant=api.SPLITK_FUSED_VARIANT)
        torch.cuda.synchronize()
        assert torch.equal(c, ref), it
    stream = torch.cuda.current_stream().cuda_stream
    arr = api._arrivals[(a.device.index, stream)]
    assert int(arr.abs().sum()) == 0
    assert rel_err(c.cpu(), gemm_ref(a.cpu(), b.cpu())) <= TOL


def test_split_k_fused_on_two_streams(gpu):
    """Products on two streams keep separate arrival counters; each matches the two-launch form."""
    from warpir_amd import api

    m, n, k, splits = 128, 2048, 4096, 4
    announce(f"split-K fused on two streams {m}x{n}x{k}")
    a = seeded_normal((m, k), 96, 0.1).cuda()
    b = seeded_normal((k, n), 97, 0.1).cuda()
    ref = api.gemm_split_k(a, b, splits=splits, variant=api.SPLITK_TWO_LAUNCH_VARIANT)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = []
    for s in (s1, s2):
        with torch.cuda.stream(s):
            outs.append(api.gemm_split_k(a, b, splits=splits, variant=api.SPLITK_FUSED_VARIANT))
    torch.cuda.synchronize()
    assert all(torch.equal(o, ref) for o in outs)
    assert (a.device.index, s1.cuda_stream) in api._arrivals and (a.device.index, s2.cuda_stream) in api._arrivals


def test_grid_outrunning_an_operand_reads_zeros(gpu):
    """A launch whose C tile grid is taller than A: the in-bounds
    specialisation's run-time conditions fail, so the kernel takes the
    checked body and A's missing rows read as zeros (C's lower half is 0).
    A is a view of the first half of a taller buffer, so even a wrong proof
    would read valid memory; it would show as nonzero rows."""
    announce("gemm_256_k64 grid taller than A")
    k, n = 512, 256
    big = seeded_normal((512, k), 51, 0.1).cuda()
    a = big[:256]
    b = seeded_normal((k, n), 52, 0.1).cuda()
    c = torch.full((512, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    kernels.handle("gemm_256_k64")(A=a, B=b, N=k, C_global=c)
    torch.cuda.synchronize()
    assert rel_err(c[:256], gemm_ref(a, b)) <= TOL
    assert torch.equal(c[256:].float().cpu(), torch.zeros(256, n))
