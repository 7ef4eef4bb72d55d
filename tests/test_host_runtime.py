"""Host-side runtime behaviour that needs no GPU: the variant-handle cache is
safe under threads, packed kernel arguments are reused per argument
signature, and the split-K entry point rejects an ``out`` it would scramble."""
import threading

import pytest
import torch

from warpir_amd import api, kernels


def test_handle_cache_builds_each_variant_once_across_threads():
    name = "gemm_ref_ssa"
    kernels._handles.pop(name, None)
    got, barrier = [], threading.Barrier(4)

    def worker():
        barrier.wait()
        got.append(kernels.handle(name))

    threads = [threading.Thread(target=worker) for _ in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(got) == 4 and all(h is got[0] for h in got)


def test_kernarg_signature_distinguishes_buffers_and_ints():
    h = kernels.handle("gemm_ref_ssa")
    a = torch.zeros(64, 64, dtype=torch.bfloat16)
    b = torch.zeros(64, 64, dtype=torch.bfloat16)
    c = torch.zeros(64, 64, dtype=torch.bfloat16)
    s1 = h._signature(dict(A=a, B=b, N=64, C_global=c))
    s2 = h._signature(dict(A=a, B=b, N=64, C_global=c))
    s3 = h._signature(dict(A=a, B=c, N=64, C_global=b))
    s4 = h._signature(dict(A=a, B=b, N=32, C_global=c))
    assert s1 == s2 and s1 != s3 and s1 != s4
    assert h._signature(dict(A=a, B=b, N=64)) is None           # a missing argument is not cached
    assert h._signature(dict(A=a, B=b, N=64.0, C_global=c)) is None


@pytest.mark.parametrize("bad", ["shape", "dtype", "strided"])
def test_split_k_rejects_an_out_it_would_scramble(bad):
    a = torch.zeros(64, 1024, dtype=torch.bfloat16)
    b = torch.zeros(1024, 256, dtype=torch.bfloat16)
    out = {"shape": torch.zeros(64, 128, dtype=torch.bfloat16),
           "dtype": torch.zeros(64, 256, dtype=torch.float32),
           "strided": torch.zeros(256, 64, dtype=torch.bfloat16).t()}[bad]
    with pytest.raises(ValueError, match="out must be a contiguous bf16"):
        api.gemm_split_k(a, b, out=out, splits=4)


def test_noalloc_entry_point_rejects_oversize_inputs_before_touching_a_device():
    import ctypes

    from warpir_amd.runtime import LIB_PATH, library
    import os
    if not os.path.exists(LIB_PATH):
        pytest.skip("libwarpir_rt.so not built")
    lib = library()
    fake = ctypes.c_void_p(256)   # never dereferenced: validation fails first
    code = lib.wir_gemm_splitk_noalloc(fake, fake, fake, fake, fake, 1024, 8192, 8192, 4, None)
    assert code == 20001
    assert b"device scratch" in lib.wir_error_string(code)
    assert lib.wir_gemm_splitk_noalloc(fake, fake, fake, fake, fake, 64, 8192, 8000, 4, None) != 0  # K % 256


def test_noalloc_split_k_validates_operands_on_the_host():
    a = torch.zeros(64, 1024, dtype=torch.bfloat16)
    b = torch.zeros(1024, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="gemm_split_k_noalloc: out"):
        api.gemm_split_k_noalloc(a, b, torch.zeros(64, 128, dtype=torch.bfloat16), splits=4)
    with pytest.raises(ValueError, match="must be on one GPU"):
        api.gemm_split_k_noalloc(a, b, torch.zeros(64, 256, dtype=torch.bfloat16), splits=4)


def test_source_flag_marker_is_parsed_and_restricted():
    """A generated source's first line may ask for the MFMA VGPR form; nothing else passes."""
    from warpir_amd.lowering.cdna4 import HIPCC_FLAGS_MARKER
    from warpir_amd.runtime import CompileError, hsaco_path, source_flags

    body = "// Generated\nextern \"C\" __global__ void k() {}\n"
    assert source_flags(body) == ()
    marked = f"{HIPCC_FLAGS_MARKER} -mllvm -amdgpu-mfma-vgpr-form=1\n" + body
    assert source_flags(marked) == ("-mllvm", "-amdgpu-mfma-vgpr-form=1")
    assert hsaco_path(marked) != hsaco_path(body)   # the flags are part of the cache key
    for bad in ("-O0", "-mllvm -amdgpu-mfma-vgpr-form=1 -fsanitize=address", "-mllvm"):
        with pytest.raises(CompileError):
            source_flags(f"{HIPCC_FLAGS_MARKER} {bad}\n" + body)


def test_dkdv_d128_kernels_ask_for_the_vgpr_form_and_others_do_not():
    from warpir_amd.runtime import source_flags

    for name in ("mha_bwd_dkdv_d128", "mha_bwd_dkdv_d128_causal", "mha_bwd_dkdv_d128_gqa"):
        src = kernels.lowerer(name).lower(kernels.kernel(name))
        assert source_flags(src) == ("-mllvm", "-amdgpu-mfma-vgpr-form=1"), name
    for name in ("gemm_256_k64", "mha_d128", "mha_bwd_dq_d128", "mha_bwd_dkdv_d64"):
        src = kernels.lowerer(name).lower(kernels.kernel(name))
        assert source_flags(src) == (), name


@pytest.mark.parametrize("m,n,k", [(0, 8192, 8192), (128, 0, 8192), (128, 8192, 0), (64, 1024, 0)])
def test_empty_products_stay_off_the_split_k_route(m, n, k):
    """An empty product has no slices to split: splitk_count is 1 and api.gemm
    routes it to the tiled kernels (which launch nothing for an empty output
    and store zeros for K = 0)."""
    assert api.splitk_count(m, n, k) == 1
    assert api.gemm_variant(m, n, k) != api.SPLITK_GEMM_VARIANT


def test_split_k_rejects_an_empty_k_before_touching_a_device():
    a = torch.zeros(64, 0, dtype=torch.bfloat16)
    b = torch.zeros(0, 256, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="K must be positive"):
        api.gemm_split_k(a, b)
    with pytest.raises(ValueError, match="K must be positive"):
        api.gemm_split_k_noalloc(a, b, torch.zeros(64, 256, dtype=torch.bfloat16))
