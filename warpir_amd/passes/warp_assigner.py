"""Warp (wavefront) assignment: which wave group issues each instruction.

Same API as the reference (``warpir/passes/warp_assigner.py``):
``WAInstruction``, ``WAInstructionManager.add_instruction`` and
``solve(max_cycles, num_warps, synchronization_cost, instruction_types,
use_verbose)``, which prints one table per warp.  The model is the
reference's CP-SAT model (``:31-119``), solved here by an exact
branch-and-bound search instead of OR-Tools:

* every instruction gets a start cycle in ``[0, max_cycles - 1 -
  max(cuda_latency, total_latency)]`` (``ValueError`` when that is empty)
  and exactly one warp; instructions whose name is listed in
  ``instruction_types`` share that type's warp (``:37-61``);
* a data dependence ``p -> i`` needs ``start_i >= start_p + sep`` with
  ``sep = max(gap, p.total_latency)`` if the modulo issue gap is positive,
  else ``p.total_latency``; a synchronous parent on another warp adds
  ``synchronization_cost`` (``:67-89``); ordering dependences never pay it
  (``:92-100``);
* the ``[start, start + cuda_latency)`` intervals of one warp do not
  overlap (``:103-113``);
* minimise ``makespan = max(start + total_latency)`` (``:116-119``).

``solve`` also returns the solution (the reference returns ``None``; a
caller that ignores the value sees the same behaviour) and prints
``INFEASIBLE!`` when no assignment fits (``:136-137``).

``assign_waves(kernel)`` is the IR-connected entry point the reference
leaves as a TODO (``:214``): it unrolls the steady state of a pipelined
loop into ``WAInstruction`` s (loads asynchronous, MMAs synchronous,
issue cycles from the modulo schedule) and solves it for a producer /
consumer split.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple


@dataclass
class WAInstruction:
    """One unrolled instruction (``warp_assigner.py:6-21``)."""

    name: str
    version: int
    parent_instructions: List["WAInstruction"]    # data deps: pay the sync cost across warps
    ordering_instructions: List["WAInstruction"]  # ordering deps: never pay it
    is_async: bool
    cuda_latency: int
    total_latency: int
    modulo_issue_cycle: int

    def __str__(self) -> str:
        return f"{self.name}_{self.version}"


@dataclass
class WASolution:
    """An optimal assignment: warp and start cycle per instruction key."""

    makespan: int
    warp_of: Dict[str, int]
    start_of: Dict[str, int]
    type_warp: Dict[str, int] = field(default_factory=dict)

    def table(self, instructions: Sequence[WAInstruction], num_warps: int) -> List[List[Tuple[str, int]]]:
        rows: List[List[Tuple[str, int]]] = [[] for _ in range(num_warps)]
        for t, w in self.type_warp.items():
            rows[w].append((f"[type: {t}]", -1))
        for ins in instructions:
            k = str(ins)
            rows[self.warp_of[k]].append((f"{ins.name}@{ins.version}", self.start_of[k]))
        for r in rows:
            r.sort(key=lambda x: x[1])
        return rows


def _separation(child: WAInstruction, parent: WAInstruction) -> int:
    gap = child.modulo_issue_cycle - parent.modulo_issue_cycle
    return max(gap, parent.total_latency) if gap > 0 else parent.total_latency


class WAInstructionManager:
    """Collects unrolled instructions and solves the warp assignment (``:23-143``)."""

    def __init__(self):
        self.instructions: List[WAInstruction] = []
        self.intervals: Dict[str, Tuple[int, int]] = {}

    def add_instruction(self, instruction: WAInstruction) -> None:
        self.instructions.append(instruction)

    def solve(self, max_cycles: int, num_warps: int, synchronization_cost: int,
              instruction_types: List[str], use_verbose: bool = False) -> Optional[WASolution]:
        for ins in self.instructions:
            if max_cycles - 1 - max(ins.cuda_latency, ins.total_latency) < 0:
                raise ValueError(f"max_cycles too small for {ins}")
        sol = _BranchAndBound(self.instructions, max_cycles, num_warps, synchronization_cost,
                              list(instruction_types)).run()
        if sol is None:
            print("INFEASIBLE!")
            for w in range(num_warps):
                print(f"warp {w}:")
            return None
        self.intervals = {k: (s, s + next(i.cuda_latency for i in self.instructions if str(i) == k))
                          for k, s in sol.start_of.items()}
        for w, rows in enumerate(sol.table(self.instructions, num_warps)):
            print(f"warp {w}:")
            for entry in rows:
                print("\t", entry)
        if use_verbose:
            print(f"makespan {sol.makespan}")
        return sol


class _BranchAndBound:
    """Exact search: type warps, then instructions in dependence order.

    Each instruction is placed on a warp at a start cycle; starts are tried
    from the earliest the placed parents allow, skipping cycles its warp
    already occupies, up to the bound the incumbent leaves.  The lower
    bound is ``max(start + tail)`` over placed and ``est + tail`` over
    unplaced instructions, where ``tail`` is the longest remaining chain
    (without synchronisation costs).
    """

    def __init__(self, instrs, max_cycles, num_warps, sync_cost, types):
        self.ins = list(instrs)
        self.n = len(self.ins)
        self.key = [str(i) for i in self.ins]
        idx = {id(i): k for k, i in enumerate(self.ins)}
        self.parents: List[List[Tuple[int, int, bool]]] = []  # (parent, sep, pays_sync)
        for i in self.ins:
            ps = []
            for p in i.parent_instructions:
                ps.append((idx[id(p)], _separation(i, p), not p.is_async))
            for p in i.ordering_instructions:
                ps.append((idx[id(p)], _separation(i, p), False))
            self.parents.append(ps)
        self.children: List[List[Tuple[int, int]]] = [[] for _ in range(self.n)]
        for c, ps in enumerate(self.parents):
            for p, sep, _ in ps:
                self.children[p].append((c, sep))
        self.ub = [max_cycles - 1 - max(i.cuda_latency, i.total_latency) for i in self.ins]
        self.max_cycles = max_cycles
        self.num_warps = num_warps
        self.sync = sync_cost
        self.types = types
        self.type_of = [types.index(i.name) if i.name in types else -1 for i in self.ins]
        self.order = self._topo()
        self.tail = self._tails()
        self.best: Optional[WASolution] = None
        self.best_span = max_cycles  # makespan must be <= max_cycles - 1

    def _topo(self) -> List[int]:
        indeg = [len(ps) for ps in self.parents]
        ready = [k for k in range(self.n) if indeg[k] == 0]
        out = []
        while ready:
            ready.sort(key=lambda k: (self.ins[k].modulo_issue_cycle, k))
            k = ready.pop(0)
            out.append(k)
            for c, _ in self.children[k]:
                indeg[c] -= 1
                if indeg[c] == 0:
                    ready.append(c)
        if len(out) != self.n:
            raise ValueError("dependence cycle among warp-assignment instructions")
        return out

    def _tails(self) -> List[int]:
        tail = [0] * self.n
        for k in reversed(self.order):
            t = self.ins[k].total_latency
            for c, sep in self.children[k]:
                t = max(t, sep + tail[c])
            tail[k] = t
        return tail

    def run(self) -> Optional[WASolution]:
        tw = [0] * len(self.types)
        self._types(0, tw)
        return self.best

    def _types(self, t: int, tw: List[int]) -> None:
        if t == len(self.types):
            self._search(tw)
            return
        # symmetry: a type's warp is at most one above the largest used so far
        top = max(tw[:t], default=-1)
        for w in range(min(self.num_warps, top + 2)):
            tw[t] = w
            self._types(t + 1, tw)

    def _search(self, tw: List[int]) -> None:
        start = [-1] * self.n
        warp = [-1] * self.n
        busy: List[set] = [set() for _ in range(self.num_warps)]

        def est(k: int, w: int) -> int:
            lo = 0
            for p, sep, pays in self.parents[k]:
                lo = max(lo, start[p] + sep + (self.sync if pays and warp[p] != w else 0))
            return lo

        def bound(pos: int, span: int) -> int:
            lb = span
            for k in self.order[pos:]:
                lo = 0
                for p, sep, _ in self.parents[k]:
                    if start[p] >= 0:
                        lo = max(lo, start[p] + sep)
                lb = max(lb, lo + self.tail[k])
            return lb

        def dfs(pos: int, span: int) -> None:
            if pos == self.n:
                if span < self.best_span:
                    self.best_span = span
                    self.best = WASolution(
                        makespan=span, warp_of={self.key[k]: warp[k] for k in range(self.n)},
                        start_of={self.key[k]: start[k] for k in range(self.n)},
                        type_warp={t: tw[j] for j, t in enumerate(self.types)})
                return
            if bound(pos, span) >= self.best_span:
                return
            k = self.order[pos]
            ins = self.ins[k]
            warps = [tw[self.type_of[k]]] if self.type_of[k] >= 0 else range(self.num_warps)
            for w in warps:
                s = est(k, w)
                limit = min(self.ub[k], self.best_span - 1 - self.tail[k])
                while s <= limit:
                    occ = range(s, s + ins.cuda_latency)
                    if any(t in busy[w] for t in occ):
                        s += 1
                        continue
                    start[k], warp[k] = s, w
                    busy[w].update(occ)
                    dfs(pos + 1, max(span, s + ins.total_latency))
                    busy[w].difference_update(occ)
                    start[k] = warp[k] = -1
                    s += 1
                    if self.best_span <= bound(pos, span):
                        break

        dfs(0, 0)


# ---------------------------------------------------------------------------
# IR-connected entry point
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class WaveCosts:
    """Costs of the unrolled instructions, in one time unit: how long an
    instruction keeps its warp busy (``cuda_latency``) and how long until its
    result is usable (``total_latency``), per load stream and for the MMAs,
    and the synchronisation cost of a dependence across warps."""

    load_issue: Dict[str, int]
    load_latency: int
    mma_issue: int
    mma_latency: int
    sync: int
    default_load_issue: int = 1


# The reference demo's constants (warp_assigner.py:147-152; load 12, MMA 4, sync 80), with
# every instruction holding its warp for one cycle.
REFERENCE_WAVE_COSTS = WaveCosts(load_issue={}, load_latency=12, mma_issue=1, mma_latency=4, sync=80)

# gfx950 measurements, in shader cycles: a global_load_lds_dwordx4 (1 KiB per wave) stalls the
# issuing wave ~20 cycles; a 32x32x16 bf16 MFMA occupies its SIMD 32 cycles; an LDS-DMA tile
# lands ~2048 cycles after issue under load; a workgroup barrier between two wave sets ~80.
DMA_ISSUE_CYCLES = 20
DMA_LANDING_CYCLES = 2048
BARRIER_CYCLES = 80


def gfx950_wave_costs(kernel, waves_per_group: int = 4, unit: int = 32) -> WaveCosts:
    """Costs of *kernel*'s pipelined loop on gfx950 in units of ``unit``
    cycles (one MFMA): each load stream keeps its issuing wave busy for its
    DMA instructions (tile bytes / 1 KiB spread over ``waves_per_group``
    waves, ~20 cycles each), and the MMA keeps its wave busy for its MFMAs
    (the per-wavefront result tile times the reduction depth)."""
    from warpir_amd.ir.ops import ForOp, MMABufOp, TMALoadBufOp

    loop = next((op for op in kernel.body if isinstance(op, ForOp)), None)
    if loop is None:
        raise ValueError("kernel has no loop")
    issue = {}
    for op in loop.body:
        if isinstance(op, TMALoadBufOp):
            t = op.buf.type.tile_type
            instr = max(1, t.rows * t.cols * 2 // 1024 // waves_per_group)
            issue[op.buf.name.replace("_bufs", "") + "_load"] = -(-instr * DMA_ISSUE_CYCLES // unit)
    mma = next(op for op in loop.body if isinstance(op, MMABufOp))
    acc = mma.accum.type
    k = mma.a_buf.type.tile_type.cols
    cycles = max(1, acc.rows * acc.cols * k // (32 * 32 * 16)) * 32
    mma_units = -(-cycles // unit)
    return WaveCosts(load_issue=issue, load_latency=-(-DMA_LANDING_CYCLES // unit), mma_issue=mma_units,
                     mma_latency=mma_units, sync=-(-BARRIER_CYCLES // unit))


def instructions_from_pipeline(kernel, iterations: int = 4, ii: Optional[int] = None,
                               load_latency: int = 12, mma_latency: int = 4,
                               costs: Optional[WaveCosts] = None) -> List[WAInstruction]:
    """Unroll the steady state of *kernel*'s pipelined loop into WAInstructions.

    Loads (``tma_load_buf``) are asynchronous with ``load_latency``; MMAs
    (``mma_buf``, ``mma``) are synchronous with ``mma_latency``.  The MMA of
    iteration ``k`` consumes the loads of the slot it waits on, as the
    buffer form's slot expressions say, and the accumulator chains MMA to
    MMA.  A load that refills a slot is ordered after the MMA that last
    read it (the buffer form's write-after-read rule).  ``costs`` (a
    ``WaveCosts``) replaces the latencies and sets how long each
    instruction keeps its warp busy (one cycle without it).
    """
    if costs is not None:
        load_latency, mma_latency = costs.load_latency, costs.mma_latency
    from warpir_amd.ir.ops import BufSlotExpr, ForOp, MMABufOp, MMAOp, TMALoadBufOp

    loop = next((op for op in kernel.body if isinstance(op, ForOp)), None)
    if loop is None:
        raise ValueError("kernel has no loop")
    loads = [op for op in loop.body if isinstance(op, TMALoadBufOp)]
    mmas = [op for op in loop.body if isinstance(op, (MMABufOp, MMAOp))]
    if not loads or not mmas:
        raise ValueError("loop is not in buffer form (run kernel_pass first)")
    stages = loads[0].buf.type.count
    ii = ii or max(mma_latency * len(mmas), 1)

    def lag(slot) -> int:
        # slot (i + off) % S of a load vs the MMA's slot: how many iterations ahead it loads
        return slot.offset % stages if isinstance(slot, BufSlotExpr) else 0

    mma_slot = getattr(mmas[0], "a_slot", None)
    distance = (lag(loads[0].slot) - lag(mma_slot)) % stages if mma_slot is not None else stages - 1
    out: List[WAInstruction] = []
    ld: Dict[Tuple[int, int], WAInstruction] = {}
    mm: Dict[Tuple[int, int], WAInstruction] = {}
    total = iterations + distance
    for t in range(total):
        for j, op in enumerate(loads):
            name = op.buf.name.replace("_bufs", "") + "_load"
            busy = costs.load_issue.get(name, costs.default_load_issue) if costs is not None else 1
            ld[(t, j)] = WAInstruction(name, t, [], [], True, busy, load_latency, t * ii)
    for t in range(total):
        for j, op in enumerate(mmas):
            tile = t  # logical tile consumed by this MMA copy
            if tile >= total:
                continue
            parents = [ld[(tile, q)] for q in range(len(loads))]
            if (t - 1, j) in mm:
                parents.append(mm[(t - 1, j)])
            if j > 0:
                parents.append(mm[(t, j - 1)])
            mm[(t, j)] = WAInstruction("mma" if len(mmas) == 1 else f"mma{j}", t, parents, [], False,
                                       costs.mma_issue if costs is not None else 1,
                                       mma_latency, (t + distance) * ii + j * mma_latency)
    for (t, j), ins in ld.items():
        if t - stages >= 0 and (t - stages, 0) in mm:
            ins.ordering_instructions.append(mm[(t - stages, len(mmas) - 1)])
    out = [ld[k] for k in sorted(ld)] + [mm[k] for k in sorted(mm)]
    return out


def assign_waves(kernel, num_warps: int = 2, synchronization_cost: int = 80, iterations: int = 4,
                 max_cycles: int = 500, verbose: bool = False,
                 costs: Optional[WaveCosts] = None) -> Optional[WASolution]:
    """Solve the warp assignment of *kernel*'s pipelined loop.

    Types are pinned as in the reference demo (every load stream and the
    MMA each get one warp), so the answer is a producer / consumer split:
    which wave group issues which load stream relative to the MMAs.
    ``costs`` (e.g. ``gfx950_wave_costs(kernel)``) replaces the reference
    demo's latencies and its ``synchronization_cost``.
    """
    if costs is not None:
        synchronization_cost = costs.sync
    instrs = instructions_from_pipeline(kernel, iterations=iterations, costs=costs)
    mgr = WAInstructionManager()
    for ins in instrs:
        mgr.add_instruction(ins)
    types = sorted({i.name for i in instrs})
    import contextlib
    import io
    buf = io.StringIO()
    with contextlib.redirect_stdout(buf):
        sol = mgr.solve(max_cycles, num_warps, synchronization_cost, types, use_verbose=verbose)
    if verbose:
        print(buf.getvalue())
    return sol


def steady_state_period(kernel, type_warp: Dict[str, int], costs: WaveCosts) -> float:
    """Cycles (in ``costs``' unit) per iteration of *kernel*'s pipelined loop
    in steady state with the load streams and the MMA on the warps
    ``type_warp`` names: the busiest warp's issue time per iteration (each
    stream's DMA issue plus the MMA's), the accumulator recurrence (one MMA
    per iteration), and each ring's recurrence -- the MMA frees a slot, the
    stream refills it (issue, landing, and the synchronisation when the
    stream is on another warp than the MMA), and the MMA reads it again
    ``slots`` iterations later."""
    from warpir_amd.ir.ops import ForOp, TMALoadBufOp

    loop = next(op for op in kernel.body if isinstance(op, ForOp))
    slots = {op.buf.name.replace("_bufs", "") + "_load": op.buf.type.count
             for op in loop.body if isinstance(op, TMALoadBufOp)}
    mma_warp = type_warp["mma"]
    busy: Dict[int, float] = {}
    busy[mma_warp] = float(costs.mma_issue)
    period = float(costs.mma_latency)
    for name, n in slots.items():
        issue = costs.load_issue.get(name, costs.default_load_issue)
        w = type_warp[name]
        busy[w] = busy.get(w, 0.0) + issue
        sync = costs.sync if w != mma_warp else 0
        period = max(period, (costs.mma_latency + issue + costs.load_latency + sync) / n)
    return max(period, max(busy.values()))


def assign_streams(kernel, costs: WaveCosts, num_warps: int = 2) -> WASolution:
    """Warp of every load stream and of the MMA that minimises the loop's
    steady-state period (``steady_state_period``), by enumeration (the MMA
    on warp 0; ties go to fewer streams off the MMA's warp).  The exact
    makespan search over an unrolled window (``assign_waves``) does not see
    a stream's per-iteration issue cost until the window spans a ring's
    refill, and that window is out of its reach for these loops; the
    period is what a loop's throughput follows.  ``makespan`` holds the
    period."""
    import itertools

    from warpir_amd.ir.ops import ForOp, TMALoadBufOp

    loop = next(op for op in kernel.body if isinstance(op, ForOp))
    streams = sorted({op.buf.name.replace("_bufs", "") + "_load" for op in loop.body
                      if isinstance(op, TMALoadBufOp)})
    best = None
    for warps in itertools.product(range(num_warps), repeat=len(streams)):
        tw = dict(zip(streams, warps), mma=0)
        key = (steady_state_period(kernel, tw, costs), sum(1 for w in warps if w != 0), warps)
        if best is None or key < best[0]:
            best = (key, tw)
    (period, _off, _w), tw = best
    return WASolution(makespan=period, warp_of={}, start_of={}, type_warp=tw)


__all__ = ["WAInstruction", "WAInstructionManager", "WASolution", "WaveCosts", "REFERENCE_WAVE_COSTS",
           "gfx950_wave_costs", "instructions_from_pipeline", "assign_waves", "steady_state_period",
           "assign_streams"]
