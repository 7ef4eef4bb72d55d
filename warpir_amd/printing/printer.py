"""Text form of a WarpIR kernel.

Produces the same text as the reference printer
(``warpir/printing/printer.py:33-191``) for every op the reference knows;
the additive ops print in the same ``%r = name(args)`` style.  The
rendering is table-driven: each op class maps to a function returning
its line without indentation.
"""
from __future__ import annotations

from typing import Callable, Dict, List

from warpir_amd.ir.ops import (
    AddOp,
    AllocSharedOp,
    CausalMaskOp,
    CopyOp,
    DivRowOp,
    DrainIndexOp,
    Exp2Op,
    ForOp,
    IntAffineOp,
    IntDivOp,
    LoadVecOp,
    Kernel,
    Log2Op,
    MMABufOp,
    MMAOp,
    MulOp,
    MulRowOp,
    MulScalarOp,
    NegInftyOp,
    Op,
    PipelineStageOp,
    ReduceSlicesOp,
    RowMaxOp,
    RowSumOp,
    SlotViewOp,
    SubOp,
    SubColOp,
    LazyMaxOp,
    SubRowOp,
    TMALoadBufOp,
    TMALoadOp,
    TMAStoreOp,
    Value,
    WaitBufOp,
    WaitOp,
    YieldOp,
    ZeroOp,
)


def print_kernel(kernel: Kernel) -> None:
    """Write ``format_kernel(kernel)`` to stdout (``printer.py:33-35``)."""
    print(format_kernel(kernel))


def format_kernel(kernel: Kernel) -> str:
    """Return the text form of *kernel* (``printer.py:38-46``)."""
    ins = ", ".join(repr(v) for v in kernel.inputs)
    outs = ", ".join(repr(v) for v in kernel.outputs)
    out: List[str] = [f"kernel {kernel.name}({ins}) -> ({outs}) {{"]
    _emit(kernel.body, 1, out)
    out.append("}")
    return "\n".join(out)


def _coord(c) -> str:
    return str(c) if isinstance(c, int) else repr(c)


def _coords(cs) -> str:
    return "[" + ", ".join(_coord(c) for c in cs) + "]"


def _slot(slot) -> str:
    """Ring-slot text (``printer.py:55-63``); the offset is printed raw."""
    if isinstance(slot, int):
        return str(slot)
    if slot.value is None:
        return f"drain(+{slot.offset}, %{slot.modulus})"
    if slot.offset == 0:
        return f"{slot.value!r} % {slot.modulus}"
    return f"({slot.value!r} + {slot.offset}) % {slot.modulus}"


def _call(op: Op, name: str, *args) -> str:
    return f"{op.result!r} = {name}(" + ", ".join(repr(a) for a in args) + ")"


_LINE: Dict[type, Callable[[Op], str]] = {
    ZeroOp: lambda op: f"{op.result!r} = zero",
    AllocSharedOp: lambda op: f"{op.result!r} = alloc_shared",
    NegInftyOp: lambda op: f"{op.result!r} = neg_infty",
    TMALoadOp: lambda op: f"{op.result!r} = tma_load({op.source!r}, {_coords(op.coords)})",
    TMALoadBufOp: lambda op: (
        f"tma_load_buf({op.buf.name}[{_slot(op.slot)}], {op.source!r}, {_coords(op.coords)})"
    ),
    WaitOp: lambda op: "wait(" + ", ".join(repr(v) for v in op.values) + ")",
    WaitBufOp: lambda op: (
        "wait_buf(" + ", ".join(b.name for b in op.bufs) + f", slot={_slot(op.slot)})"
    ),
    MMAOp: lambda op: (
        f"{op.result!r} = mma({op.a!r}, {op.b!r}, {op.accum!r}"
        + (", transpose_b=True" if op.transpose_b else "") + ")"
    ),
    CopyOp: lambda op: _call(op, "copy", op.input),
    MulScalarOp: lambda op: f"{op.result!r} = mul_scalar({op.input!r}, {op.scalar})",
    SubOp: lambda op: _call(op, "sub", op.a, op.b),
    MulOp: lambda op: _call(op, "mul", op.a, op.b),
    Exp2Op: lambda op: _call(op, "exp2", op.input),
    RowMaxOp: lambda op: _call(op, "row_max", op.tile, op.prev),
    RowSumOp: lambda op: _call(op, "row_sum", op.tile, op.prev),
    SubRowOp: lambda op: _call(op, "sub_row", op.tile, op.vec),
    MulRowOp: lambda op: _call(op, "mul_row", op.tile, op.vec),
    DivRowOp: lambda op: _call(op, "div_row", op.tile, op.vec),
    MMABufOp: lambda op: (
        f"{op.result!r} = mma_buf({op.a_buf.name}[{_slot(op.a_slot)}], "
        f"{op.b_buf.name}[{_slot(op.b_slot)}], {op.accum!r})"
    ),
    TMAStoreOp: lambda op: f"tma_store({op.source!r}, {op.dest!r}, {_coords(op.coords)})",
    YieldOp: lambda op: "yield(" + ", ".join(repr(v) for v in op.values) + ")",
    # additive ops
    AddOp: lambda op: _call(op, "add", op.a, op.b),
    Log2Op: lambda op: _call(op, "log2", op.input),
    CausalMaskOp: lambda op: (
        f"{op.result!r} = causal_mask({op.tile!r}, {_coord(op.row_tile)}, {_coord(op.col_tile)}"
        + (", transposed=True" if op.transposed else "") + ")"
    ),
    SlotViewOp: lambda op: f"{op.result!r} = slot_view({op.buf.name}[{_slot(op.slot)}])",
    IntAffineOp: lambda op: (
        f"{op.result!r} = int_affine({_coord(op.input)}, {op.mul}, {op.add})"
    ),
    SubColOp: lambda op: _call(op, "sub_col", op.tile, op.vec),
    LoadVecOp: lambda op: f"{op.result!r} = load_vec({op.source!r}, {_coords(op.coords)})",
    LazyMaxOp: lambda op: f"{op.result!r} = lazy_max({op.prev!r}, {op.cand!r}, {op.slack})",
    IntDivOp: lambda op: f"{op.result!r} = int_div({_coord(op.input)}, {_coord(op.divisor)})",
    DrainIndexOp: lambda op: f"{op.result!r} = drain_index(+{op.offset})",
    PipelineStageOp: lambda op: f"pipeline_stage({op.stage})",
    ReduceSlicesOp: lambda op: (
        f"reduce_slices({op.partials!r}, {op.dest!r}, {op.arrivals!r}, {_coords(op.coords)})"
    ),
}


def _emit(ops, indent: int, out: List[str]) -> None:
    pad = "  " * indent
    for op in ops:
        if isinstance(op, ForOp):
            _emit_for(op, indent, out)
            continue
        render = _LINE.get(type(op))
        if render is None:
            # Unknown ops are skipped, as the reference printer does.
            continue
        out.append(pad + render(op))


def _bound(x) -> str:
    # f-string formatting of an int or a Value (whose str() is its repr).
    return f"{x}"


def _emit_for(op: ForOp, indent: int, out: List[str]) -> None:
    """Loop header, iter_args line and body (``printer.py:178-191``)."""
    pad = "  " * indent
    results = ", ".join(repr(r) for r in op.results)
    tile = f" tile_size={op.tile_size}" if op.tile_size else ""
    out.append(
        f"{pad}({results}) = for {op.induction_var!r} = {_bound(op.start)} to "
        f"{_bound(op.stop)} step {_bound(op.step)}{tile}"
    )
    carried = ", ".join(f"{ia.block_arg!r} = {ia.init!r}" for ia in op.iter_args)
    out.append(f"{pad}    iter_args({carried}) {{")
    _emit(op.body, indent + 2, out)
    out.append(f"{pad}}}")


__all__ = ["print_kernel", "format_kernel"]
