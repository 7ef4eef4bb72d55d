"""TEST INFRASTRUCTURE -- block-granular CPU interpreter of the tile IR.

Runs a ``Kernel`` once per program of its grid with torch fp32 on CPU.
Storage follows the reference lowering, not pure SSA, because the
pipelined IR relies on it (``warpir/lowering/lowering.py``):

* a loop's iter_arg ``init``, its ``results`` and the yielded values all
  name the block argument's storage (``lowering.py:87-107``);
* ``MMAOp`` without ``transpose_b`` copies ``accum`` into ``result`` when
  they are different storages and accumulates ``a @ b`` into ``result``;
  with ``transpose_b`` it computes ``a @ b^T`` only (``lowering.py:454-470``);
* ``MMABufOp`` accumulates in place into ``accum`` and then advances the
  drain counter by one (``lowering.py:472-488``, which keeps it reduced by
  the single ring size; here it counts MMAs, and each read reduces it);
* a drain slot (``BufSlotExpr(value=None)``) reads the drain counter modulo
  its ring size, its offset is not used (``lowering.py:196-207``);
  ``DrainIndexOp`` (additive) reads the unreduced counter plus its offset;
* register values are block-level tiles (all wavefront slices together);
  ``zero`` / ``neg_infty`` are scalars that broadcast to the first shape
  they are combined with;
* tile loads read zeros outside the tensor and stores drop elements
  outside it (TMA's out-of-bounds behaviour);
* a ``CopyOp`` into a bf16 type, and every store to a bf16 global, round
  to bf16; a ``CopyOp`` of a shared tile into a register tile is a plain
  read (the tile is already fp32 here);
* ``LoadVecOp`` reads ``L`` consecutive rows of an ``L x 1``-tiled global
  (zeros outside), or with no coordinates the fp32 ``L x 1`` shared tile
  it names, as a block-level vector: a col_vec's length is its
  block's rows, a row_vec's its tile's columns; ``SubColOp`` subtracts a
  row_vec from every row.

Tile coordinates are ``(batch, depth, row_tile, col_tile)`` in units of
the global's ``sub_tile_type``.  The grid covers every store: a coordinate
that is ``blockIdx.{x,y,z}`` spans ``ceil(extent / unit)`` programs.
"""
from __future__ import annotations

import math
from typing import Dict, Tuple

import torch

from warpir_amd.ir import (
    AddOp, AllocSharedOp, BufSlotExpr, CausalMaskOp, ColVecType, CopyOp, DivRowOp, DrainIndexOp, Exp2Op,
    ForOp, GPUType, IntAffineOp, IntDivOp, Kernel, LoadVecOp, Log2Op, MMABufOp, MMAOp, MulOp, MulRowOp, MulScalarOp,
    NegInftyOp, PipelineStageOp, ReduceSlicesOp, RegTileType, RowMaxOp, RowSumOp, RowVecType, SlotViewOp, SubColOp, SubOp, SubRowOp, LazyMaxOp,
    TMALoadBufOp, TMALoadOp, TMAStoreOp, Value, WaitBufOp, WaitOp, YieldOp, ZeroOp,
)

BUILTINS = ("blockIdx.x", "blockIdx.y", "blockIdx.z")


def _as4d(t: torch.Tensor, gtype=None) -> torch.Tensor:
    """View a tensor as [batch, depth, rows, cols]; a global typed with
    ``cols == 1`` gets its unit column appended (e.g. LSE ``[B, H, S]``)."""
    if gtype is not None and getattr(gtype, "cols", -1) == 1 and t.shape[-1] != 1:
        t = t.unsqueeze(-1)
    while t.dim() < 4:
        t = t.unsqueeze(0)
    return t


def _aliases(ops, table: Dict[str, str]) -> None:
    for op in ops:
        if isinstance(op, ForOp):
            for k, ia in enumerate(op.iter_args):
                table[ia.init.name] = ia.block_arg.name
                if k < len(op.results):
                    table[op.results[k].name] = ia.block_arg.name
            for inner in op.body:
                if isinstance(inner, YieldOp):
                    for k, y in enumerate(inner.values):
                        if k < len(op.iter_args):
                            table[y.name] = op.iter_args[k].block_arg.name
            _aliases(op.body, table)


def grid_of(kernel: Kernel, tensors: Dict[str, torch.Tensor]) -> Tuple[int, int, int]:
    grid = [1, 1, 1]
    for op in kernel.body:
        if not isinstance(op, TMAStoreOp):
            continue
        t = _as4d(tensors[op.dest.name], op.dest.type)
        sub = op.dest.type.sub_tile_type
        units = (1, 1, sub.rows, sub.cols)
        for p, c in enumerate(op.coords):
            if isinstance(c, Value) and c.name in BUILTINS:
                axis = BUILTINS.index(c.name)
                grid[axis] = max(grid[axis], math.ceil(t.shape[p] / units[p]))
    return tuple(grid)


class Interpreter:
    def __init__(self, kernel: Kernel):
        self.kernel = kernel
        self.alias: Dict[str, str] = {}
        _aliases(kernel.body, self.alias)

    def _key(self, v: Value) -> str:
        name, seen = v.name, set()
        while name in self.alias and name not in seen:
            seen.add(name)
            name = self.alias[name]
        return name

    # -- evaluation helpers --------------------------------------------------
    def _int(self, x) -> int:
        if isinstance(x, int):
            return x
        return int(self.env[self._key(x)])

    def _get(self, v: Value):
        return self.env[self._key(v)]

    def _set(self, v: Value, x) -> None:
        self.env[self._key(v)] = x

    def _slot(self, slot) -> int:
        if isinstance(slot, int):
            return slot
        if slot.value is None:
            return self.drain % slot.modulus
        return (self._int(slot.value) + slot.offset) % slot.modulus

    def _load(self, src: Value, coords, rows: int, cols: int) -> torch.Tensor:
        g = _as4d(self.tensors[src.name], src.type)
        sub = src.type.sub_tile_type
        b, d, rt, ct = (self._int(c) for c in coords)
        r0, c0 = rt * sub.rows, ct * sub.cols
        tile = torch.zeros(rows, cols, dtype=torch.float32)
        if 0 <= b < g.shape[0] and 0 <= d < g.shape[1]:
            blk = g[b, d, r0:r0 + rows, c0:c0 + cols].float()
            tile[:blk.shape[0], :blk.shape[1]] = blk
        return tile

    def _store(self, val, dest: Value, coords) -> None:
        g = _as4d(self.tensors[dest.name], dest.type)
        sub = dest.type.sub_tile_type
        b, d, rt, ct = (self._int(c) for c in coords)
        tile = val if val.dim() == 2 else val.reshape(-1, 1)
        r0, c0 = rt * sub.rows, ct * sub.cols
        rows = max(0, min(tile.shape[0], g.shape[2] - r0))
        cols = max(0, min(tile.shape[1], g.shape[3] - c0))
        g[b, d, r0:r0 + rows, c0:c0 + cols] = tile[:rows, :cols].to(g.dtype)

    def _reduce_slices(self, op) -> None:
        """Split-K fix-up (``ReduceSlicesOp``): count this slice's arrival; the
        last of the S slices sums them in slice order and resets the count."""
        part = _as4d(self.tensors[op.partials.name], op.partials.type)
        dest = _as4d(self.tensors[op.dest.name], op.dest.type)
        arr = self.tensors[op.arrivals.name].view(-1)
        sub = op.dest.type.sub_tile_type
        b, _d, rt, ct = (self._int(c) for c in op.coords)
        idx = rt * math.ceil(dest.shape[3] / sub.cols) + ct
        arr[idx] += 1
        if int(arr[idx]) < part.shape[1]:
            return
        r0, c0 = rt * sub.rows, ct * sub.cols
        tile = torch.zeros_like(part[b, 0, r0:r0 + sub.rows, c0:c0 + sub.cols], dtype=torch.float32)
        for s in range(part.shape[1]):
            tile = tile + part[b, s, r0:r0 + sub.rows, c0:c0 + sub.cols].float()
        dest[b, 0, r0:r0 + tile.shape[0], c0:c0 + tile.shape[1]] = tile.to(dest.dtype)
        arr[idx] = 0

    # -- execution -----------------------------------------------------------
    def run(self, tensors: Dict[str, torch.Tensor], scalars: Dict[str, int], grid=None) -> None:
        self.tensors = tensors
        grid = grid or grid_of(self.kernel, tensors)
        for z in range(grid[2]):
            for y in range(grid[1]):
                for x in range(grid[0]):
                    self.env = dict(scalars)
                    self.env.update({"blockIdx.x": x, "blockIdx.y": y, "blockIdx.z": z})
                    self.drain = 0
                    self._ops(self.kernel.body)

    def _ops(self, ops) -> None:
        for op in ops:
            self._op(op)

    def _op(self, op) -> None:  # noqa: C901 - one branch per op kind
        g, s = self._get, self._set
        if isinstance(op, (WaitOp, WaitBufOp, YieldOp, PipelineStageOp)):
            return
        if isinstance(op, ZeroOp):
            s(op.result, torch.tensor(0.0))
        elif isinstance(op, NegInftyOp):
            s(op.result, torch.tensor(float("-inf")))
        elif isinstance(op, TMALoadOp):
            t = op.result.type
            s(op.result, self._load(op.source, op.coords, t.rows, t.cols))
        elif isinstance(op, ReduceSlicesOp):
            self._reduce_slices(op)
        elif isinstance(op, DrainIndexOp):
            s(op.result, self.drain + op.offset)
        elif isinstance(op, AllocSharedOp):
            s(op.result, [None] * op.result.type.count)
        elif isinstance(op, SlotViewOp):
            s(op.result, g(op.buf)[self._slot(op.slot)])
        elif isinstance(op, TMALoadBufOp):
            t = op.buf.type.tile_type
            g(op.buf)[self._slot(op.slot)] = self._load(op.source, op.coords, t.rows, t.cols)
        elif isinstance(op, MMAOp):
            a, b = g(op.a), g(op.b)
            if op.transpose_b:
                s(op.result, a @ b.t())
            else:
                s(op.result, g(op.accum) + a @ b)
        elif isinstance(op, MMABufOp):
            a = g(op.a_buf)[self._slot(op.a_slot)]
            b = g(op.b_buf)[self._slot(op.b_slot)]
            acc = g(op.accum) + a @ b
            s(op.accum, acc)
            s(op.result, acc)
            if isinstance(op.a_slot, BufSlotExpr):
                self.drain += 1
        elif isinstance(op, CopyOp):
            x = g(op.input).clone()
            rt = op.result.type
            if isinstance(rt, (RegTileType, ColVecType)) and rt.data_type == GPUType.bf16:
                x = x.to(torch.bfloat16).float()
            s(op.result, x)
        elif isinstance(op, MulScalarOp):
            s(op.result, g(op.input) * op.scalar)
        elif isinstance(op, SubOp):
            s(op.result, g(op.a) - g(op.b))
        elif isinstance(op, MulOp):
            s(op.result, g(op.a) * g(op.b))
        elif isinstance(op, AddOp):
            s(op.result, g(op.a) + g(op.b))
        elif isinstance(op, Exp2Op):
            s(op.result, torch.exp2(g(op.input)))
        elif isinstance(op, Log2Op):
            s(op.result, torch.log2(g(op.input)))
        elif isinstance(op, RowMaxOp):
            s(op.result, torch.maximum(g(op.tile).amax(dim=1), g(op.prev)))
        elif isinstance(op, RowSumOp):
            s(op.result, g(op.tile).sum(dim=1) + g(op.prev))
        elif isinstance(op, SubRowOp):
            s(op.result, g(op.tile) - _col(g(op.vec)))
        elif isinstance(op, MulRowOp):
            s(op.result, g(op.tile) * _col(g(op.vec)))
        elif isinstance(op, DivRowOp):
            s(op.result, g(op.tile) / _col(g(op.vec)))
        elif isinstance(op, CausalMaskOp):
            t = g(op.tile)
            rows, cols = t.shape
            r = torch.arange(rows).unsqueeze(1) + self._int(op.row_tile) * rows
            c = torch.arange(cols).unsqueeze(0) + self._int(op.col_tile) * cols
            s(op.result, t.masked_fill((r > c) if op.transposed else (c > r), float("-inf")))
        elif isinstance(op, IntDivOp):
            s(op.result, self._int(op.input) // self._int(op.divisor))
        elif isinstance(op, IntAffineOp):
            s(op.result, self._int(op.input) * op.mul + op.add)
        elif isinstance(op, SubColOp):
            s(op.result, g(op.tile) - g(op.vec).reshape(1, -1))
        elif isinstance(op, LazyMaxOp):
            prev, cand = g(op.prev), g(op.cand)
            s(op.result, torch.where(cand > prev + op.slack, cand, prev))
        elif isinstance(op, LoadVecOp) and not op.coords:
            s(op.result, g(op.source)[:, 0].clone())   # from an fp32 L x 1 shared tile
        elif isinstance(op, LoadVecOp):
            gl = _as4d(self.tensors[op.source.name], op.source.type)
            n = op.source.type.sub_tile_type.rows
            b, d, rt, _ct = (self._int(c) for c in op.coords)
            vec = torch.zeros(n, dtype=torch.float32)
            if 0 <= b < gl.shape[0] and 0 <= d < gl.shape[1]:
                blk = gl[b, d, rt * n:rt * n + n, 0].float()
                vec[:blk.shape[0]] = blk
            s(op.result, vec)
        elif isinstance(op, TMAStoreOp):
            self._store(g(op.source), op.dest, op.coords)
        elif isinstance(op, ForOp):
            self._for(op)
        else:
            raise NotImplementedError(type(op).__name__)

    def _for(self, op: ForOp) -> None:
        start, stop, step = self._int(op.start), self._int(op.stop), self._int(op.step)
        if op.tile_size is not None:
            stop = -(-stop // op.tile_size)
        i = start
        while i < stop:
            self.env[self._key(op.induction_var)] = i
            self._ops(op.body)
            i += step


def _col(v):
    return v.unsqueeze(1) if v.dim() == 1 else v


def run_kernel(kernel: Kernel, tensors: Dict[str, torch.Tensor], scalars: Dict[str, int], grid=None):
    """Interpret *kernel* over its grid; outputs are written into *tensors* in place."""
    Interpreter(kernel).run(tensors, scalars, grid)
    return tensors
