"""IR API, printer and builders (CPU).

The printer golden files under tests/golden/ were produced by the
reference's own printer from the reference's builders
(tests/golden/make_printer_golden.py); they pin ``format_kernel`` byte
for byte and, through it, that ``build_gemm_kernel`` /
``build_attention_kernel`` construct the reference's IR.
"""
import os

import warpir
from warpir.ir import GlobalType, GPUType, Kernel, SharedTileType, TMALoadOp, Value, WaitOp, YieldOp, ZeroOp
from warpir.passes.modulo_scheduler import kernel_pass
from warpir.printing import format_kernel
from warpir_amd.workloads import build_attention_kernel, build_gemm_kernel, build_mha_forward_kernel

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return f.read()


def test_gemm_ssa_text_matches_reference_printer():
    assert format_kernel(build_gemm_kernel()) + "\n" == _golden("gemm_ssa.txt")


def test_attention_ssa_text_matches_reference_printer():
    assert format_kernel(build_attention_kernel()) + "\n" == _golden("attention_ssa.txt")


def test_pipelined_gemm_text_matches_reference_structure():
    """kernel_pass output for the reference GEMM (ii=6, 3 stages) printed like the reference."""
    assert format_kernel(kernel_pass(build_gemm_kernel())) + "\n" == _golden("gemm_pipelined.txt")


def test_alias_package_exposes_reference_module_paths():
    from warpir.lowering import CDNA4Lowerer  # noqa: F401
    from warpir.ir import ops, types  # noqa: F401
    assert warpir.ir.Kernel is Kernel


def test_substitute_rewrites_coords_and_keeps_other_fields():
    i = Value("i", warpir.ir.IntType())
    t = SharedTileType(GPUType.bf16, 64, 64)
    g = Value("A", GlobalType(GPUType.bf16, t, 1, 1))
    op = TMALoadOp(result=Value("a", t), source=g, coords=(0, 0, Value("blockIdx.y", warpir.ir.IntType()), i))
    sub = op.substitute({i: 3})
    assert sub.coords[3] == 3 and sub.coords[2] == op.coords[2] and sub.source is g


def test_mha_builder_shapes():
    k = build_mha_forward_kernel(d=128, block_q=128, block_kv=64, wave_rows=32)
    assert [v.name for v in k.inputs] == ["Q", "K", "V", "N"]
    assert [v.name for v in k.outputs] == ["O", "L"]
    text = format_kernel(k)
    assert "log2" in text and "transpose_b=True" in text
    kc = build_mha_forward_kernel(d=64, causal=True)
    assert "causal_mask" in format_kernel(kc) and "int_affine" in format_kernel(kc)


def test_printer_skips_unknown_ops():
    class Weird(warpir.ir.Op):
        pass
    k = Kernel(name="k", body=(Weird(),))
    assert format_kernel(k) == "kernel k() -> () {\n}"
