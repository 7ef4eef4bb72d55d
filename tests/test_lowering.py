"""CDNA4 lowering and the C-ABI boundary (CPU only: no kernel is launched).

Checks the emitted HIP's structure (self-contained, one extern "C"
kernel named after the IR kernel, globals struct in IR argument order),
the wait/barrier analysis that replaces the reference's semaphores, the
kernel-argument layout seen from the host, the error paths, and that
``libwarpir_rt.so`` loads and exports every entry point that
``include/warpir_rt.h`` declares.
"""
import ctypes
import os
import re
import shutil

import pytest
import torch

from warpir_amd import kernels
from warpir_amd.lowering import CDNA4Lowerer, CDNA4Target, LoweringError
from warpir_amd.passes.modulo_scheduler import GFX950_COST_MODEL, kernel_pass
from warpir_amd.runtime import GL, LIB_PATH, kernarg_struct
from warpir_amd.workloads import build_gemm_kernel, build_mha_forward_kernel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.parametrize("name", sorted(kernels.VARIANTS))
def test_every_variant_lowers_to_self_contained_hip(name):
    k = kernels.kernel(name)
    src = CDNA4Lowerer().lower(k)
    assert f'extern "C" __global__' in src and f"\n{k.name}(const {k.name}_globals globals)" in src
    includes = re.findall(r"#include\s*[<\"]([^>\"]+)", src)
    assert includes == ["hip/hip_runtime.h"]
    for banned in ("kittens", "cuda_runtime", "__nv_", "HIP_PLATFORM", "hipify"):
        assert banned not in src


def _waits(src):
    body = src[src.rindex('extern "C" __global__'):]   # the kernel, not the tile library
    return [int(x) for x in re.findall(r"wait_vm_barrier<(\d+)>", body)]


def test_pipelined_gemm_waits_keep_one_stage_in_flight():
    src = CDNA4Lowerer(CDNA4Target(mve=False)).lower(kernels.kernel("gemm_256_k32"))
    # 256x32 A tile and 32x256 B tile: 16 KiB each = 16 DMA instructions / 4 waves = 4 + 4 per stage;
    # the last wait is the drain before the staged store
    assert _waits(src) == [8, 8, 0, 0]


def test_modulo_variable_expansion_unrolls_by_ring_size():
    src = CDNA4Lowerer().lower(kernels.kernel("gemm_256_k32"))
    # 3-slot ring: 3 unrolled copies with constant slots + the run-time remainder loop, then 2 drains,
    # then the drain before the staged store
    assert _waits(src) == [8, 8, 8, 8, 8, 0, 0]
    loop = src[src.index("int wir_base_i"):]
    assert "(smem + 0 + 2 * 16384)" in loop and "% 3) * 16384" in loop
    # the ring's waits already order every slot reuse: the only other barrier is the drain before
    # the staged store
    assert src.count("wir::barrier()") == 0
    assert src.rindex("wir::wait_vm_barrier<0>()") > src.index("pipe0.finish")


def test_final_store_is_staged_through_lds():
    src = CDNA4Lowerer().lower(kernels.kernel("gemm_256_k64"))
    tail = src[src.index("pipe0.finish"):]
    assert tail.index("wir::wait_vm_barrier<0>()") < tail.index("store_tile_staged") and "wir::store_tile(" not in tail
    assert "smem + wir_wave * 32768" in tail        # 128x128 bf16 per wavefront
    plain = CDNA4Lowerer(CDNA4Target(staged_stores=False)).lower(kernels.kernel("gemm_256_k64"))
    plain = plain[plain.rindex('extern "C" __global__'):]
    assert "store_tile_staged" not in plain and "wir::store_tile(" in plain
    # the attention output is staged; its fp32 LSE column vector is stored directly
    fa = CDNA4Lowerer().lower(kernels.kernel("mha_d128"))
    assert "store_tile_staged<true>(globals.O" in fa and "store_vec(globals.L" in fa
    # the staged stores carry the non-temporal hint unless the target turns it off
    assert "store_tile_staged<true>(" in tail
    cached = CDNA4Lowerer(CDNA4Target(nontemporal_stores=False)).lower(kernels.kernel("gemm_256_k64"))
    cached = cached[cached.rindex('extern "C" __global__'):]
    assert "wir::store_tile_staged(" in cached and "store_tile_staged<true>" not in cached
    # the staging area is the K/V ring, into which the loop's last prefetch may still be landing:
    # every wave drains its DMAs (vmcnt 0) before the barrier that hands the LDS over
    for name in ("mha_d128", "mha_d64_causal", "mha_d128_w4", "mha_d128_ovl", "mha_bwd_dq_d128", "mha_bwd_dkdv_d128"):
        src = kernels.lowerer(name).lower(kernels.kernel(name))
        body = src[src.rindex('extern "C" __global__'):]
        pre = body[: body.index("wir::store_tile_staged")]
        last_sync = max(pre.rfind("wir::barrier()"), pre.rfind("wir::wait_vm_barrier<"))
        assert pre[last_sync:].startswith("wir::wait_vm_barrier<0>();  // ring buffers dead"), name


def test_ssa_gemm_waits_for_everything_and_guards_reuse():
    src = CDNA4Lowerer().lower(build_gemm_kernel())
    assert _waits(src) == [0, 0]        # every k-step, and the drain before the staged store
    body = src[src.index("for (int v_i"):]
    assert body.index("wir::barrier()") < body.index("Loader")


def test_attention_hoists_resident_q_fragments():
    src = CDNA4Lowerer().lower(kernels.kernel("mha_d128"))
    loop = src.index("for (int v_i")
    assert src.index("load_row_frags") < loop
    assert "mma_ABt_frags" in src and "mma_rAB" in src


def test_attention_overlap_form():
    from warpir_amd.lowering.cdna4 import CDNA4Target
    plain = CDNA4Lowerer().lower(kernels.kernel("mha_d128"))
    assert "mma_ABt_frags_slots" not in plain.split('extern "C"')[-1]
    for name in ("mha_d128_ovl", "mha_d64_causal_ovl"):
        src = kernels.lowerer(name).lower(kernels.kernel(name))
        body = src[src.rindex('extern "C" __global__'):]
        # unaligned tensors keep the plain loop; aligned ones take the pipeline
        assert "if constexpr (!WIR_AL)" in body
        assert body.count("wir::mma_ABt_frags_slots") == 3     # unrolled pair + remainder step
        assert body.count("wir::mma_rAB_slots") == 3
        assert "wir::e_pairs<0, 16>" in body                   # the peeled last tile
        assert ("causal_mask" in body) == ("causal" in name)
    # eight-wave kernels are not matched, even with the overlapped placement
    eight = kernels._mha(128, 256, 64, 32, causal=False, lds_budget=128 * 1024, min_stages=4,
                         rescale_slack=kernels.LAZY_SLACK, phases="mixed")
    src = CDNA4Lowerer(CDNA4Target(lazy_softmax=False)).lower(eight)
    assert "mma_ABt_frags_slots" not in src[src.rindex('extern "C" __global__'):]


def test_attention_pingpong_groups_follow_the_warp_assignment():
    from warpir_amd.lowering.cdna4 import CDNA4Target
    from warpir_amd.passes.modulo_scheduler import gfx950_attention_cost_model, kernel_pass
    from warpir_amd.passes.warp_assigner import assign_waves
    from warpir_amd.lowering.cdna4 import ASSIGN_ITERATIONS
    from warpir_amd.workloads import build_mha_forward_kernel
    # the short unroll the lowering uses places the streams as a longer one does (checked on the
    # 3-slot ring, where the exact search over 4 unrolled iterations stays small)
    k3 = kernel_pass(build_mha_forward_kernel(d=128, block_q=256, block_kv=64, wave_rows=32),
                     cost_model=gfx950_attention_cost_model(256, 64, 128, lds_budget=96 * 1024, min_stages=3))
    sol3 = assign_waves(k3, num_warps=2, iterations=ASSIGN_ITERATIONS)
    assert sol3.type_warp["v_load"] == 1 - sol3.type_warp["k_load"]
    assert assign_waves(k3, num_warps=2, iterations=4).type_warp == sol3.type_warp
    k = kernels.kernel("mha_d128")
    sol = assign_waves(k, num_warps=2, iterations=ASSIGN_ITERATIONS)
    k_group = sol.type_warp["k_load"]
    assert sol.type_warp["v_load"] == 1 - k_group

    def group_line(target):
        src = CDNA4Lowerer(target).lower(k)
        return [l.strip() for l in src.split("\n") if "const int wir_grp =" in l]

    assert group_line(CDNA4Target()) == [f"const int wir_grp = (wir_wave >> 2) ^ {k_group}, wir_gw = wir_wave & 3;"
                                         f"  // group A (K loads) = physical wave group {k_group}"]
    assert "^ 1," in group_line(CDNA4Target(wave_groups={"k": 1, "v": 0}))[0]
    # both streams on one group cannot be realised by the ping-pong form
    assert group_line(CDNA4Target(wave_groups={"k": 0, "v": 0})) == []


def test_attention_pingpong_one_barrier_per_iteration():
    """Group A passes its barrier after each V phase, group B after each M
    phase: one barrier per iteration per wave (the peeled first iteration,
    the inner loop and the lazy softmax's exact path included), and the same
    count in front of the loop, so the groups' barrier sequences pair up."""
    from warpir_amd.lowering.cdna4 import CDNA4Target
    k = kernels.kernel("mha_d128")
    src = CDNA4Lowerer(CDNA4Target()).lower(k)
    pp = src[src.index("const int wir_grp ="):src.index("ring buffers dead")]
    lines = [l.strip() for l in pp.split("\n")]
    stop = "((globals.N) + 63) / 64"
    after = f"wir::wait_vm_barrier_after<4>((v_i) + 2 < {stop});"   # drains fully once past the end
    assert lines.count("wir::wait_vm_barrier<4>();") == 1                      # after the prologue loads
    assert lines.count(f"if (wir_grp == 1) {after}") == 2    # after M: peeled, loop
    assert lines.count(f"if (wir_grp == 0) {after}") == 3    # after V: peeled, loop, exact
    assert "pairs with group B" not in pp
    # ring loads of tiles past the end are skipped
    assert lines.count(f"if ((v_i) + 2 < {stop})") == 2 and lines.count(f"if ((v_i) + 3 < {stop})") == 2
    two = CDNA4Lowerer(CDNA4Target(pingpong_one_barrier=False)).lower(k)
    pp2 = two[two.index("const int wir_grp ="):two.index("ring buffers dead")]
    assert "if (wir_grp == 0) wir::wait_vm_barrier<0>();   // pairs with group B's extra V phase" in pp2
    assert "if (wir_grp == 1) wir::wait_vm_barrier" not in pp2 and "wir_grp == 0 ? 1 : 0" in pp2


def test_lazy_softmax_fusion_needs_its_inputs_defined_first():
    """The lazy-softmax group is emitted as one call at its first member.  With the copy of the
    running max moved ahead of the QK MMA (still valid IR: it reads only the max), that call would
    read the scores before the MMA defines them, so the fusion is skipped and the ops are lowered
    one by one instead."""
    import copy

    from warpir_amd.ir.ops import CopyOp, ForOp, MMAOp
    k = copy.deepcopy(kernels.kernel("mha_d64_causal"))
    low = kernels.lowerer("mha_d64_causal")
    assert "wir::lazy_softmax_fast(" in low.lower(k)
    loop = next(op for op in k.body if isinstance(op, ForOp))
    cp = next(o for o in loop.body if isinstance(o, CopyOp) and o.result.name == "max_prev")
    qk = next(o for o in loop.body if isinstance(o, MMAOp))
    body = [o for o in loop.body if o is not cp]
    body.insert(body.index(qk), cp)
    object.__setattr__(loop, "body", tuple(body))   # the IR dataclasses are frozen
    src = kernels.lowerer("mha_d64_causal").lower(k)
    body = src[src.rindex('extern "C" __global__'):]
    assert "wir::lazy_softmax_fast(" not in body and "wir::lazy_softmax_exact(" not in body


def test_lazy_softmax_folds_scale_into_q_and_max_into_the_score_mfmas():
    """``fold_softmax_scale`` (opt-in): with the lazy softmax on hoisted Q, the fused loop scales
    the fragments once, declares the score bias, starts each QK MMA with the bias MFMA and calls
    the _b softmax halves (no fma per score).  The ping-pong kernel's plain loop for unaligned
    tensors keeps the unfolded math; the defaults and the exact online softmax are not folded."""
    from warpir_amd.lowering.cdna4 import CDNA4Target

    def body(src):
        return src[src.rindex('extern "C" __global__'):]

    fold = CDNA4Target(fold_softmax_scale=True)
    for name in ("mha_d128", "mha_d64_causal", "mha_d128_w4", "mha_d64_causal_pp"):
        b = body(CDNA4Lowerer(fold).lower(kernels.kernel(name)))
        assert b.count("wir::scale_frags(hf_q_shared, ") == 1, name
        assert b.count("wir_sb.init();") == 1, name
        assert "wir::lazy_softmax_fast(" not in b and "wir::lazy_softmax_exact(" not in b, name
        assert b.count("wir::lazy_softmax_fast_b(") == 1 and b.count("wir::lazy_softmax_exact_b(") == 2, name
        assert b.count("wir::mma_ABt_frags_bias<") == 2, name   # the peeled first tile and the loop
        # the scale is applied before any folded MMA reads the fragments
        assert b.index("wir::scale_frags(") < b.index("wir::mma_ABt_frags_bias<"), name
    pp = body(CDNA4Lowerer(fold).lower(kernels.kernel("mha_d128")))
    plain, aligned = pp.split("} else {", 1)
    assert "wir::mma_ABt_frags<" in plain and "scale_frags" not in plain and "wir_sb" not in plain
    assert "wir::mma_ABt_frags<" not in aligned.split("ring buffers dead")[0]
    for name in ("mha_d128_fold", "mha_d64_causal_fold"):
        assert kernels.TARGETS[name] == {"fold_softmax_scale": True}
        assert "wir::mma_ABt_frags_bias<" in body(kernels.lowerer(name).lower(kernels.kernel(name)))
    default = body(kernels.lowerer("mha_d128").lower(kernels.kernel("mha_d128")))
    assert "scale_frags" not in default and "wir::lazy_softmax_fast(" in default and "_b(" not in default
    online = body(CDNA4Lowerer(fold).lower(kernels.kernel("mha_d128_online")))
    assert "scale_frags" not in online and "mma_ABt_frags_bias" not in online


def test_warp_specialized_gemm_form():
    k = kernels.kernel("gemm_256x128_ws")
    low = kernels.lowerer("gemm_256x128_ws")
    src = low.lower(k)
    body = src[src.rindex('extern "C" __global__'):]
    assert low.num_threads == 512 and "amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2)" in body
    assert "const bool wir_producer = wir_wave_hw >= 4;" in body
    # every DMA is issued by a producer wave, every MFMA helper and store by a consumer wave
    for line in body.split("\n"):
        if "::load<WIR_AL>(" in line:
            assert line.strip().startswith(("if (wir_producer)", "if (!wir_producer)")), line
    assert body.count("if (!wir_producer) {") >= 3
    assert low.launch_config(k, {"A": (512, 512), "B": (512, 512), "C_global": (512, 512)}).block == (512, 1, 1)
    # the warp assigner's steady-state assignment with the gfx950 costs puts both streams on the
    # DMA waves: the same kernel as the forced _all split
    allp = kernels.lowerer("gemm_256x128_ws_all").lower(kernels.kernel("gemm_256x128_ws_all"))
    assert "if (!wir_producer) wir::Loader" not in allp and "wir::wait_vm_barrier<12>();" in allp
    assert src == allp
    # the split the reference demo's constants give (_ab): the MFMA waves issue A, the DMA waves
    # B, and each set waits on its own share of the in-flight DMAs
    ab = kernels.lowerer("gemm_256x128_ws_ab").lower(kernels.kernel("gemm_256x128_ws_ab"))
    ab = ab[ab.rindex('extern "C" __global__'):]
    assert "if (!wir_producer) wir::Loader<wir::STile<256, 64, 0>, 4>::load" in ab
    assert "if (wir_producer) wir::Loader<wir::STile<64, 128, 1>, 4>::load" in ab
    assert "if (wir_producer) wir::wait_vm_barrier<4>(); else wir::wait_vm_barrier<8>();" in ab
    # the same kernel without the option is the plain 4-wave form
    plain = kernels.lowerer("gemm_256x128").lower(kernels.kernel("gemm_256x128"))
    assert "wir_producer" not in plain


def test_kernarg_layout_matches_globals_struct():
    assert ctypes.sizeof(GL) == 48
    s = kernarg_struct(build_gemm_kernel())
    assert [f[0] for f in s._fields_] == ["A", "B", "N", "C_global"]
    assert s.C_global.offset == 104 and ctypes.sizeof(s) == 152


def test_lds_budget_is_enforced():
    k = kernel_pass(build_gemm_kernel(256, 256, 64, 128, 128), cost_model=GFX950_COST_MODEL)
    with pytest.raises(LoweringError, match="LDS"):
        CDNA4Lowerer().lower(k)


def test_uneven_wave_split_is_rejected():
    k = build_gemm_kernel(block_m=64, block_n=64, block_k=64, wave_m=16, wave_n=16)
    with pytest.raises(LoweringError):
        CDNA4Lowerer().lower(k)


def test_mfma_shape_choice():
    assert "wir::RTile<32, 128, 128>" in CDNA4Lowerer().lower(kernels.kernel("gemm_256_k32"))
    assert "wir::RTile<16, 16, 64>" in CDNA4Lowerer().lower(build_gemm_kernel())
    forced = CDNA4Lowerer(CDNA4Target(mfma=16)).lower(kernels.kernel("gemm_256_k32"))
    assert "wir::RTile<16, 128, 128>" in forced


def test_launch_config_from_output_shapes():
    low = CDNA4Lowerer()
    k = kernels.kernel("gemm_256_k32")
    cfg = low.launch_config(k, {"A": (1000, 264), "B": (264, 520), "C_global": (1000, 520)})
    assert cfg.grid == (3, 4, 1) and cfg.block == (256, 1, 1)
    m = build_mha_forward_kernel(d=128, block_q=128, block_kv=64, wave_rows=32)
    cfg = CDNA4Lowerer().launch_config(m, {"O": (2, 3, 512, 128), "L": (2, 3, 512, 1)})
    assert cfg.grid == (4, 3, 2)


def _declared_symbols():
    with open(os.path.join(ROOT, "include", "warpir_rt.h")) as f:
        text = f.read()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(wir_\w+)\(", text, re.M)))


def test_c_abi_library_exports_every_declared_symbol():
    if not os.path.exists(LIB_PATH):
        pytest.skip("libwarpir_rt.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    syms = _declared_symbols()
    assert len(syms) == 18
    for s in syms:
        assert hasattr(lib, s), s
    lib.wir_abi_version.restype = ctypes.c_int
    assert lib.wir_abi_version() == 4
    lib.wir_error_string.restype = ctypes.c_char_p
    assert lib.wir_error_string(0)


@pytest.mark.skipif(shutil.which("hipcc") is None and not os.path.exists("/opt/rocm/bin/hipcc"),
                    reason="hipcc not available")
def test_generated_source_compiles_for_gfx950(tmp_path, monkeypatch):
    import warpir_amd.runtime as rt
    monkeypatch.setattr(rt, "CACHE_DIR", str(tmp_path))
    src = CDNA4Lowerer().lower(build_gemm_kernel())
    path = rt.compile_source(src)
    with open(path, "rb") as f:
        assert f.read(24) == b"__CLANG_OFFLOAD_BUNDLE__"
    usage = rt.resource_usage(src)
    assert usage.get("scratch", 0) == 0


def test_gemm_variant_selection():
    from warpir_amd import api
    assert api.gemm_variant(8192, 8192) == "gemm_256_k64"
    assert api.gemm_variant(4096, 4096) == "gemm_256_k64"      # 256 tiles: one per CU
    assert api.gemm_variant(2048, 2048) == "gemm_128_k64"      # 64 tiles of 256x256
    assert api.gemm_variant(128, 8192) == "gemm_128x32_k64"          # K unknown: no split
    assert api.gemm_variant(256, 8192) == "gemm_128x64_k64"
    assert api.gemm_variant(64, 8192, 8192) == api.SPLITK_GEMM_VARIANT == "gemm_128_splitk_k64_b7"
    assert api.gemm_variant(128, 8192, 8192) == api.SPLITK_GEMM_VARIANT
    assert api.gemm_variant(64, 8192, 100) == "gemm_128x32_k64"   # K too short to split
    for v in ("gemm_256_k64", "gemm_128_k64", "gemm_128x32_k64"):
        assert v in kernels.VARIANTS


def test_gemm_routes_strided_short_m_away_from_split_k(monkeypatch):
    """api.gemm sends M <= 128, long-K products to split-K only when every tensor is dense:
    the split-K entry points address a, b and out as contiguous arrays, while the tiled
    kernel reads row-strided views through the globals' row stride."""
    from warpir_amd import api

    taken = []
    monkeypatch.setattr(api, "gemm_split_k", lambda a, b, out=None, workspace=None: taken.append("splitk") or out)

    class _Handle:
        def __init__(self, name):
            self.name = name

        def __call__(self, **kw):
            taken.append(self.name)

    monkeypatch.setattr(kernels, "handle", _Handle)
    a_full = torch.zeros(128, 8192 + 64, dtype=torch.bfloat16)
    b = torch.zeros(8192, 1024, dtype=torch.bfloat16)
    api.gemm(a_full[:, :8192].contiguous(), b)
    api.gemm(a_full[:, :8192], b)                       # row-strided A
    out_full = torch.zeros(128, 1024 + 64, dtype=torch.bfloat16)
    api.gemm(a_full[:, :8192].contiguous(), b, out=out_full[:, :1024])   # row-strided out
    assert taken == ["splitk", api.SKINNY_GEMM_VARIANT, api.SKINNY_GEMM_VARIANT]
    assert api._splitk_operands_ok(a_full[:, :8192].contiguous(), b, torch.zeros(128, 1024, dtype=torch.bfloat16))
    assert not api._splitk_operands_ok(a_full[:, :8192], b, torch.zeros(128, 1024, dtype=torch.bfloat16))


def test_dkdv_cost_model_follows_its_query_tile():
    """The dK/dV kernel's kernel_pass prices its real loop tile (DKDV_BLOCK_Q[d] query rows
    against the resident 128-row key tile): at D=64, two 32-row Q / dO slots plus the LSE and Dv
    vectors, 17 KiB of LDS."""
    from warpir_amd.kernels import DKDV_BLOCK_Q
    assert DKDV_BLOCK_Q == {128: 64, 64: 32}
    low = kernels.lowerer("mha_bwd_dkdv_d64")
    low.lower(kernels.kernel("mha_bwd_dkdv_d64"))
    off = low.lds_off
    assert [low.tile_type_of(k).rows for k in ("q_bufs", "do_bufs", "l2_bufs", "dv_bufs")] == [32] * 4
    assert off["do_bufs"] - off["q_bufs"] == off["l2_bufs"] - off["do_bufs"] == 2 * 32 * 64 * 2   # two slots
    assert low.lds_total == 17408   # + two 256-byte-aligned slots of each fp32 vector


def test_split_k_count_and_ir():
    from warpir_amd import api
    assert api.splitk_count(128, 8192, 8192) == 4        # 64 tiles x 4 slices = 256 workgroups
    assert api.splitk_count(8192, 8192, 8192) == 1
    assert api.splitk_count(128, 256, 4096) == 16        # 2 tiles: as many 64-deep slices as fit
    assert api.splitk_count(128, 8192, 8256) == 3        # 8256 = 3 * 2752 = 3 * 43 * 64
    src = CDNA4Lowerer().lower(kernels.kernel("gemm_128_splitk"))
    assert "wir::gl<float> C_global" in src and "pid_z, (pid_y) * 128" in src


def test_per_ring_gemm_lowering_merges_ring_waits():
    """Rings of two depths (A 2, B 3): the loop is unrolled by their period 6, the two ring
    waits of an iteration share one barrier that leaves B's newest tile (8 DMAs per wave) in
    flight, and the drain counter counts MMAs (a drain_index reads it) and is reduced per ring."""
    name = "gemm_128_splitk_k128_b3"
    src = kernels.lowerer(name).lower(kernels.kernel(name))
    loop = src[src.index("for (; WIR_AL && wir_base_i + 6 <="):src.index("pipe0.finish")]
    assert loop.count("const int v_i = wir_base_i + ") == 6
    assert loop.count("wir::wait_vm_barrier<8>();") == 7   # six copies and the remainder loop
    assert "wir::wait_vm_barrier<" not in loop.replace("wir::wait_vm_barrier<8>();", "")
    assert "wir_drain += 1;" in src and "(wir_drain % 2)" in src and "(wir_drain % 3)" in src
    assert "const int v_i_d0_1 = wir_drain + 1;" in src


@pytest.mark.parametrize("name", ["mha_d128", "mha_d64_causal"])
def test_lazy_attention_loop_sits_inside_the_first_tile_guard(name):
    """The peeled first tile, the loop and the last PV share one
    ``if (tiles > start)`` guard, so the loop is entered only through the
    peeled tile, whose MFMAs already wait for the register-hoisted Q: the
    compiler then puts no vmcnt(0) for Q inside the loop (it would also wait
    for the ring DMAs this wave has in flight)."""
    src = kernels.lowerer(name).lower(kernels.VARIANTS[name]())
    body = src[src.rindex('extern "C"'):].split("\n")
    guards = [i for i, l in enumerate(body) if l.strip().startswith("if (") and l.rstrip().endswith(") > 0) {")]
    loop = next(i for i, l in enumerate(body) if l.strip() == "for (;;) {")
    assert len(guards) == 1 and guards[0] < loop
    indent = len(body[guards[0]]) - len(body[guards[0]].lstrip())
    close = next(i for i in range(guards[0] + 1, len(body))
                 if body[i].strip() == "}" and len(body[i]) - len(body[i].lstrip()) == indent)
    assert close > loop
    assert any("mma_rAB" in l for l in body[loop:close] if "const int v_i" not in l)


def _in_bounds_conditions(name):
    src = kernels.lowerer(name).lower(kernels.kernel(name))
    body = src[src.rindex('extern "C" __global__'):]
    line = next(l for l in body.split("\n") if "const bool wir_aligned =" in l)
    conds = line.split("=", 1)[1].rstrip(";").split(" && ")
    return body, [c.strip() for c in conds if "Loader<" not in c]


def _holds(conds, extents, grid, n):
    env = dict(nx_=grid[0], ny_=grid[1], nz_=grid[2])
    ok = True
    for c in conds:
        expr = c.replace("globals.N", str(n)).replace("/", "//")
        for g, (b, d, r, col) in extents.items():
            for k, v in (("b", b), ("d", d), ("r", r), ("c", col)):
                expr = expr.replace(f"globals.{g}.{k}", str(v))
        ok = ok and eval(expr, {}, env)   # noqa: S307 - integers and comparisons only
    return ok


def test_in_bounds_specialisation_only_where_every_tile_load_is_proved_inside():
    """The reference buffer form with one ring depth drops the zero-page
    selects (WIR_INB) under run-time conditions that put every tile it loads
    inside its tensor: the grid's tile extent within each tensor, the loop's
    tile count within K, and the prologue's tiles present.  The lazy
    attention prefetch form (config 5's loop prefetches past its end) and
    per-ring depths keep the selects."""
    body, conds = _in_bounds_conditions("gemm_256_k64")
    assert "constexpr bool WIR_INB = WIR_AL && true;" in body
    other, _ = _in_bounds_conditions("mha_d64_causal")
    assert "constexpr bool WIR_INB = WIR_AL && false;" in other
    ext = lambda m, n, k: {"A": (1, 1, m, k), "B": (1, 1, k, n)}   # noqa: E731
    assert _holds(conds, ext(8192, 8192, 8192), (32, 32, 1), 8192)
    assert _holds(conds, ext(256, 256, 64), (1, 1, 1), 64)
    assert not _holds(conds, ext(256, 512, 8192), (2, 2, 1), 8192)    # C grid twice A's rows
    assert not _holds(conds, ext(512, 256, 8192), (2, 2, 1), 8192)    # ... or twice B's columns
    assert not _holds(conds, ext(256, 256, 4096), (1, 1, 1), 8192)    # loop longer than K
    assert not _holds(conds, ext(256, 256, 0), (1, 1, 1), 0)          # no prologue tile


def test_pingpong_attention_loads_its_own_prologue_and_proves_it_in_bounds():
    """The 8-wave ping-pong issues its first K and V tiles itself, split
    between its wave groups, so the aligned body skips the prefetch form's
    prologue loads (the plain loop of unaligned tensors still issues them).
    Its ring loads past the loop's end are skipped, so the in-bounds form
    holds when the grid fits Q's batch and heads in K and V, the loop's tiles
    fit K and V, and the unguarded prologue tiles (0 .. 2: K and V 0 .. 1,
    group B's first V tile 2) are there."""
    body, conds = _in_bounds_conditions("mha_d128")
    assert "constexpr bool WIR_INB = WIR_AL && true;" in body
    loads = [ln for ln in body.split("\n") if "::load<WIR_AL, WIR_INB>(" in ln]
    prologue = [ln for ln in loads if ln.lstrip().startswith("if constexpr (!WIR_AL)")]
    assert len(prologue) == 6                       # K and V tiles 0 .. 2 of the 4-slot rings
    assert all("Loader<wir::STile<64, 128, 0>, 8>" in ln or "Loader<wir::STile<64, 128, 1>, 8>" in ln
               for ln in prologue)
    assert any(", 4>::load<" in ln for ln in loads)  # the ping-pong's own, four waves a group
    ext = lambda b, h, s, d: {"K": (b, h, s, d), "V": (b, h, s, d)}   # noqa: E731
    assert _holds(conds, ext(16, 16, 4096, 128), (16, 16, 16), 4096)
    assert _holds(conds, ext(1, 1, 192, 128), (1, 1, 1), 192)        # exactly the prologue's tiles
    assert not _holds(conds, ext(1, 1, 128, 128), (1, 1, 1), 128)    # the first V phase's tile 2 outside
    assert not _holds(conds, ext(16, 16, 2048, 128), (16, 16, 16), 4096)   # loop longer than K
    assert not _holds(conds, ext(8, 16, 4096, 128), (16, 16, 16), 4096)    # grid's batches past K's
    assert not _holds(conds, ext(16, 8, 4096, 128), (16, 16, 16), 4096)    # ... or its heads
    assert not _holds(conds, ext(16, 16, 4096, 64), (16, 16, 16), 4096)    # head dim below the tile


def _tile_loads(kernel, tiles, grid):
    """Every tile load of a buffer-form kernel as (tensor, coordinates, tile
    extents), interpreted from the IR for a loop of ``tiles`` tiles and the
    largest program index of ``grid``: the loop runs from its start to
    ``tiles - 1``, and a drain index is the count of buffered MMAs run so far
    plus its offset."""
    from warpir_amd.ir.ops import DrainIndexOp, ForOp, IntAffineOp, MMABufOp, TMALoadBufOp
    env = {"blockIdx.x": grid[0] - 1, "blockIdx.y": grid[1] - 1, "blockIdx.z": grid[2] - 1}
    mmas, loads = [0], []

    def val(x):
        return x if isinstance(x, int) else env[x.name]

    def run(ops):
        for op in ops:
            if isinstance(op, TMALoadBufOp):
                sub = op.source.type.sub_tile_type
                loads.append((op.source.name, tuple(val(c) for c in op.coords), (1, 1, sub.rows, sub.cols)))
            elif isinstance(op, MMABufOp):
                mmas[0] += 1
            elif isinstance(op, DrainIndexOp):
                env[op.result.name] = mmas[0] + op.offset
            elif isinstance(op, IntAffineOp):
                env[op.result.name] = val(op.input) * op.mul + op.add
            elif isinstance(op, ForOp):
                for i in range(op.start, tiles):
                    env[op.induction_var.name] = i
                    run(op.body)
    run(kernel.body)
    return loads


@pytest.mark.parametrize("name", ["gemm_256_k64", "gemm_128x32_k64", "gemm_128_splitk_k128_b3",
                                  "gemm_128_splitk_s5", "gemm_128_splitk_k64_b7", "gemm_256_k64_b3"])
def test_in_bounds_conditions_cover_every_tile_load(name):
    """Wherever the emitted conditions hold, every tile that the kernel's IR
    loads (prologue, loop, drain steps with their drain indices, per-ring
    shifts) lies inside its tensor; and the sweep does reach launches whose
    loads leave a tensor, each of which the conditions reject.  Extents are
    tile multiples (the aligned body's domain); the loop's tiles, the K
    extent, the grid and the slice count vary."""
    kernel = kernels.kernel(name)
    _, conds = _in_bounds_conditions(name)
    assert conds
    tm, tn = 256 if "256" in name else 128, {"gemm_256_k64": 256, "gemm_128x32_k64": 32}.get(name, 128)
    tk = kernels.lowerer(name).lower(kernel) and next(
        o.tile_size for o in kernel.body if type(o).__name__ == "ForOp")
    seen_outside = 0
    for tiles in range(0, 7):
        ks = sorted({max(tiles - 1, 0), tiles, tiles + 1})
        for ka, kb in ((ka, kb) for ka in ks for kb in ks):
            for slices in (1, 2):
                for grid in ((1, 1, 1), (2, 1, 1), (1, 2, 1), (1, 1, slices), (1, 1, slices + 1)):
                    ext = {"A": (1, slices, tm, ka * tk), "B": (1, slices, kb * tk, tn)}
                    outside = []
                    for src, coords, unit in _tile_loads(kernel, tiles, grid):
                        if any(c < 0 or (c + 1) * u > e for c, u, e in zip(coords, unit, ext[src])):
                            outside.append((src, coords))
                    holds = _holds(conds, ext, grid, tiles * tk)
                    assert not (holds and outside), (tiles, ka, kb, slices, grid, outside)
                    seen_outside += bool(outside)
    assert seen_outside


def api_splitk_variant():
    from warpir_amd import api
    return api.SPLITK_GEMM_VARIANT


def test_dma_cache_policy_option():
    """CDNA4Target.dma_cache_policy: the modifiers reach the tile DMAs through a define ahead of
    the tile library (canonical order), the default emits none, and unknown or repeated words
    are rejected."""
    k = kernels.kernel("gemm_256_k64")
    assert '#define WIR_DMA_CPOL " ' not in CDNA4Lowerer().lower(k)
    src = CDNA4Lowerer(CDNA4Target(dma_cache_policy="nt sc1")).lower(k)
    assert src.index('#define WIR_DMA_CPOL " sc1 nt"') < src.index("#ifndef WIR_DMA_CPOL")
    for bad in ("sc2", "nt nt", "glc"):
        with pytest.raises(ValueError):
            CDNA4Lowerer(CDNA4Target(dma_cache_policy=bad)).lower(k)


def test_rowsum_mfma_option_emits_matrix_core_sums():
    """CDNA4Target.rowsum_mfma: the speculative softmax half becomes lazy_softmax_fast_mr."""
    name = "mha_d64_causal"
    base = kernels.lowerer(name).lower(kernels.kernel(name))
    mr = CDNA4Lowerer(CDNA4Target(rowsum_mfma=True)).lower(kernels.kernel(name))
    body = lambda s: s[s.rindex('extern "C" __global__'):]  # noqa: E731
    assert "lazy_softmax_fast(" in body(base) and "lazy_softmax_fast_mr(" not in body(base)
    assert "lazy_softmax_fast_mr(" in body(mr) and "lazy_softmax_fast(" not in body(mr)


def test_rowsum_selector_sums_a_rows_two_half_lanes():
    """The layout argument of wir::rowsum_selector, checked on a model of v_mfma_f32_16x16x32_bf16
    (A lane l: row l%16, k 8*(l/16)+j; B lane l: column l%16, the same k; C register i of lane l:
    row 4*(l/16)+i, column l%16): with P's 8 values per lane as B, every C register of lane l is
    the sum of lanes l%32 and l%32+32, i.e. its own row's sum in the lane = row layout."""
    src = open(os.path.join(os.path.dirname(kernels.__file__), "csrc", "wir_cdna4.h")).read()
    expr = re.search(r"const bf16 e = (.*) \? \(bf16\)1\.0f", src).group(1)
    sel = [1.0 if eval(expr.replace("==", " == "), {"l": lane}) else 0.0 for lane in range(64)]
    g = torch.Generator().manual_seed(0)
    bvals = torch.rand(64, 8, generator=g, dtype=torch.float64)
    a = torch.zeros(16, 32, dtype=torch.float64)
    b = torch.zeros(32, 16, dtype=torch.float64)
    for lane in range(64):
        for j in range(8):
            a[lane % 16, 8 * (lane // 16) + j] = sel[lane]
            b[8 * (lane // 16) + j, lane % 16] = bvals[lane, j]
    c = a @ b
    for lane in range(64):
        want = bvals[lane % 32].sum() + bvals[lane % 32 + 32].sum()
        for i in range(4):
            assert abs(c[4 * (lane // 16) + i, lane % 16] - want) < 1e-12, (lane, i)


def test_persistent_programs_launch_and_tile_walk():
    """CDNA4Target.persistent: the grid is min(tiles, programs) on x, the kernel takes its tile
    counts from the output tensor, and each program walks tiles blockIdx.x + k * gridDim.x
    through the same XCD remap as the one-workgroup-per-tile form, a barrier between tiles."""
    k = kernels.kernel("mha_d128")
    shapes = {"Q": (16, 16, 4096, 128), "K": (16, 16, 4096, 128), "V": (16, 16, 4096, 128),
              "O": (16, 16, 4096, 128), "L": (16, 16, 4096)}
    assert CDNA4Lowerer().launch_config(k, shapes).grid == (16, 16, 16)
    lw = CDNA4Lowerer(CDNA4Target(persistent=256))
    assert lw.launch_config(k, shapes).grid == (256, 1, 1)
    small = {n: (1, 2, 512, 128) for n in "QKVO"}
    small["L"] = (1, 2, 512)
    assert lw.launch_config(k, small).grid == (4, 1, 1)
    src = lw.lower(k)
    body = src[src.rindex('extern "C" __global__'):]
    assert "const int nx_ = max(((globals.O.r) + 255) / 256, ((globals.L.r) + 255) / 256), ny_ = max(globals.O.d, globals.L.d)" in body
    assert "for (int wir_blk = blockIdx.x; wir_blk < wir_nblk; wir_blk += gridDim.x) {" in body
    assert "const int lid_ = wir::remap_xcd(wir_blk, wir_nblk);" in body
    assert body.count("wir::barrier();   // the tile's LDS") == 1


def test_persistent_stream_form():
    """CDNA4Target.persistent_stream on the config-4 kernel: the aligned body is one ring stream
    (loop end wir_T, loads through each wave's cursor, the tile's first key tile peeled, O stored
    from registers after the tile's last PV), the unaligned body walks tiles one by one; without
    persistent programs the option is refused."""
    k = kernels.kernel("mha_d128")
    src = CDNA4Lowerer(CDNA4Target(persistent=256, persistent_stream=True)).lower(k)
    body = src[src.rindex('extern "C" __global__'):]
    al = body[body.index("if constexpr (WIR_AL) {"):body.index("} else {\n  for (int wir_blk")]
    assert "const int wir_T = wir_cnt * wir_nt;" in al and "wir_adv();" in al
    assert "store_tile_staged" not in al and al.count("wir::store_tile(globals.O") == 1
    assert "wir::wait_vm_barrier_after<4>((v_i) + 2 < wir_T);" in al
    assert "for (; v_i < wir_nb; ++v_i)" in al and "if (v_i == wir_T) break;" in al
    assert "for (int wir_blk = blockIdx.x; wir_blk < wir_nblk; wir_blk += gridDim.x) {" in body
    with pytest.raises(LoweringError):
        CDNA4Lowerer(CDNA4Target(persistent_stream=True)).lower(k)
