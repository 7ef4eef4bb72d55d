"""Register footprint of a kernel's wavefront (``warpir/passes/register_counter.py``).

The reference file is a one-line intent ("count how many register tiles
are being used and come up with a value to increase / decrease registers
by"): on H100 that value would feed ``setmaxnreg``.  gfx950 has no such
instruction -- every wavefront of a kernel gets the same allocation, and
the allocation fixes how many wavefronts share a SIMD (512 registers per
lane per SIMD, VGPRs and AGPRs together).  So the CDNA4 reading of the
pass is: estimate the per-lane registers one wavefront needs at its
busiest program point, and from that pick the waves per SIMD the lowering
compiles for.

The estimate is a liveness analysis over the IR in the lowering's storage
model (loop iter_args, their inits, results and yields share storage):

* an fp32 register tile of ``R x C`` elements per wavefront takes
  ``R*C/64`` registers per lane, a bf16 one ``R*C/128``;
* a col_vec takes one register per 32 rows, a row_vec ``C/2`` (the lane =
  row layout keeps 16 of every 32 columns in each lane);
* a loop-invariant shared tile that is the row operand of a ``transpose_b``
  MMA is held as bf16 fragments for the whole loop (the lowering hoists it);
* values live into a loop (iter_args, loop-invariant operands) count at
  every point of its body.

Addresses, loop counters and MMA operand staging add a fixed allowance.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Set

from warpir_amd.ir import (
    ColVecType, ForOp, GPUType, Kernel, MMAOp, RegTileType, RowVecType, SharedTileType, TMALoadOp, Value,
    YieldOp,
)

# Registers per lane for addresses, loop state and MFMA operand staging.
OVERHEAD = 40
# Registers per lane per SIMD (VGPRs and AGPRs together) on gfx950.
FILE = 512


@dataclass
class RegisterReport:
    peak: int                       # live registers per lane at the busiest point (without OVERHEAD)
    peak_at: str                    # the op where the peak occurs
    hoisted: Dict[str, int] = field(default_factory=dict)   # hoisted fragment tiles -> registers

    @property
    def need(self) -> int:
        return self.peak + OVERHEAD

    @property
    def waves_per_simd(self) -> int:
        """Wavefronts of this kernel one SIMD can hold by registers, at most 3:
        the file is split evenly and allocated in blocks of 8, so 3 waves get
        168 registers per lane, 2 get 256 and 1 gets all 512.  (The lowering
        also caps this by how many workgroups the LDS holds.)"""
        for w in (3, 2):
            if self.need <= FILE // w // 8 * 8:
                return w
        return 1


def value_registers(t) -> int:
    """Per-lane registers of one wavefront's value of type *t* (0 if not a register value)."""
    if isinstance(t, RegTileType):
        per = 64 if t.data_type == GPUType.fp32 else 128
        return max(1, t.rows * t.cols // per)
    if isinstance(t, ColVecType):
        return max(1, t.rows // 32)
    if isinstance(t, RowVecType):
        return max(1, t.cols // 2)
    return 0


def _operands(op) -> List[Value]:
    out = []
    for name, v in vars(op).items():
        if name in ("result", "results", "body", "iter_args", "induction_var"):
            continue
        if isinstance(v, Value):
            out.append(v)
        elif isinstance(v, tuple):
            out.extend(x for x in v if isinstance(x, Value))
    return out


def _results(op) -> List[Value]:
    r = vars(op).get("result")
    return [r] if isinstance(r, Value) else []


class _Liveness:
    def __init__(self, kernel: Kernel):
        self.alias: Dict[str, str] = {}
        self._aliases(kernel.body)
        self.types: Dict[str, object] = {}
        self.hoisted: Dict[str, int] = {}
        self._collect(kernel.body)

    def _aliases(self, ops) -> None:
        for op in ops:
            if isinstance(op, ForOp):
                for k, ia in enumerate(op.iter_args):
                    self.alias[ia.init.name] = ia.block_arg.name
                    if k < len(op.results):
                        self.alias[op.results[k].name] = ia.block_arg.name
                for inner in op.body:
                    if isinstance(inner, YieldOp):
                        for k, y in enumerate(inner.values):
                            if k < len(op.iter_args):
                                self.alias[y.name] = op.iter_args[k].block_arg.name
                self._aliases(op.body)

    def key(self, v: Value) -> str:
        name, seen = v.name, set()
        while name in self.alias and name not in seen:
            seen.add(name)
            name = self.alias[name]
        return name

    def _collect(self, ops) -> None:
        for op in ops:
            for v in _results(op) + _operands(op):
                self.types.setdefault(self.key(v), v.type)
            if isinstance(op, ForOp):
                for ia in op.iter_args:
                    self.types.setdefault(self.key(ia.block_arg), ia.block_arg.type)
                loaded = {o.result.name for o in op.body if isinstance(o, TMALoadOp)}
                for o in op.body:
                    if isinstance(o, MMAOp) and o.transpose_b and isinstance(o.a.type, SharedTileType) \
                            and o.a.name not in loaded:
                        self.hoisted[self.key(o.a)] = o.result.type.rows * o.a.type.cols // 128
                self._collect(op.body)

    def regs(self, name: str) -> int:
        if name in self.hoisted:
            return self.hoisted[name]
        return value_registers(self.types.get(name))


def count_registers(kernel: Kernel) -> RegisterReport:
    """Peak per-lane register footprint of one wavefront of *kernel*."""
    lv = _Liveness(kernel)
    best = [0, ""]

    def uses_in(ops) -> Set[str]:
        out: Set[str] = set()
        for op in ops:
            out |= {lv.key(v) for v in _operands(op)}
            if isinstance(op, ForOp):
                out |= uses_in(op.body)
                out |= {lv.key(ia.init) for ia in op.iter_args}
        return out

    def walk(ops, live_out: Set[str]) -> Set[str]:
        """Backward liveness over *ops*; returns the live-in set and records the peak."""
        live = set(live_out)
        for op in reversed(ops):
            if isinstance(op, ForOp):
                carried = {lv.key(ia.block_arg) for ia in op.iter_args}
                inside = uses_in(op.body)
                # everything the body reads that is defined outside it stays live across the loop
                defined_inside = {lv.key(r) for o in op.body for r in _results(o)}
                loop_in = (inside - defined_inside) | carried
                body_live = walk(list(op.body), live | loop_in)
                live = (live - {lv.key(r) for r in op.results}) | body_live | loop_in
                continue
            res = {lv.key(r) for r in _results(op)}
            after = live
            live = (live - res) | {lv.key(v) for v in _operands(op)}
            here = sum(lv.regs(n) for n in (after | live))
            if here > best[0]:
                best[0], best[1] = here, type(op).__name__ + (f" -> {res.pop()}" if res else "")
        return live

    walk(list(kernel.body), set())
    return RegisterReport(peak=best[0], peak_at=best[1], hoisted=dict(lv.hoisted))


__all__ = ["RegisterReport", "count_registers", "value_registers", "OVERHEAD", "FILE"]
