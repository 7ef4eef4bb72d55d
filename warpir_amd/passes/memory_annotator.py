"""Waits for asynchronous loads (``warpir/passes/memory_annotator.py``).

The reference file states the pass's purpose -- take the asynchronous
memory operations and place the waits they need before their first use --
and stops at a stub (``process_memory_annotations`` breaks off at "where is
the first use of that operation?").  This is that pass for the pre-pipeline
IR: every ``tma_load`` result is asynchronous until a ``wait`` names it, so
before the first op that reads a pending tile (in the same block) one
``wait`` is inserted for all tiles pending at that point that the op reads.
Existing waits are kept and retire what they name.  Loops are processed
body by body: a tile loaded inside an iteration must be waited on inside it,
and a tile loaded before a loop and first read inside it is waited on right
before the loop.
"""
from __future__ import annotations

from typing import List, Set

from warpir_amd.ir import ForOp, Kernel, Op, TMALoadOp, Value, WaitOp


def _reads(op: Op) -> Set[str]:
    out: Set[str] = set()
    for name, v in vars(op).items():
        if name in ("result", "results", "induction_var", "iter_args", "body"):
            continue
        if isinstance(v, Value):
            out.add(v.name)
        elif isinstance(v, tuple):
            out |= {x.name for x in v if isinstance(x, Value)}
    if isinstance(op, ForOp):
        for inner in op.body:
            out |= _reads(inner)
        out |= {ia.init.name for ia in op.iter_args}
    return out


def _process(ops) -> List[Op]:
    out: List[Op] = []
    pending: List[Value] = []          # loaded, not yet waited, in load order
    for op in ops:
        if isinstance(op, WaitOp):
            names = {v.name for v in op.values}
            pending = [v for v in pending if v.name not in names]
            out.append(op)
            continue
        needed = [v for v in pending if v.name in _reads(op)]
        if needed:
            out.append(WaitOp(values=tuple(needed)))
            names = {v.name for v in needed}
            pending = [v for v in pending if v.name not in names]
        if isinstance(op, ForOp):
            op = ForOp(induction_var=op.induction_var, start=op.start, stop=op.stop, step=op.step,
                       iter_args=op.iter_args, body=tuple(_process(op.body)), results=op.results,
                       tile_size=op.tile_size)
        out.append(op)
        if isinstance(op, TMALoadOp):
            pending.append(op.result)
    return out


def process_memory_annotations(kernel: Kernel) -> Kernel:
    """*kernel* with a ``wait`` before the first read of every pending ``tma_load``."""
    return Kernel(name=kernel.name, inputs=kernel.inputs, outputs=kernel.outputs,
                  body=tuple(_process(kernel.body)))


class MissingWaitError(ValueError):
    """An op reads a ``tma_load`` result that no ``wait`` has completed."""


def _check(ops, pending: Set[str]) -> None:
    pending = set(pending)
    for op in ops:
        if isinstance(op, WaitOp):
            pending -= {v.name for v in op.values}
            continue
        early = sorted(pending & _reads(op))
        if early:
            raise MissingWaitError(f"{type(op).__name__} reads {', '.join(early)} before a wait completes it")
        if isinstance(op, ForOp):
            _check(op.body, pending)
        if isinstance(op, TMALoadOp):
            pending.add(op.result.name)


def check_memory_annotations(kernel: Kernel) -> None:
    """Raise ``MissingWaitError`` if any op reads a ``tma_load`` result before a ``wait`` for it."""
    _check(kernel.body, set())


__all__ = ["process_memory_annotations", "check_memory_annotations", "MissingWaitError"]
