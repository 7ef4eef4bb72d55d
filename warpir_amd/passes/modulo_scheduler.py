"""Modulo scheduling of tile loops into a multi-buffered pipeline.

Public API as in the reference (``warpir/passes/modulo_scheduler.py``):
``MSInstructionEdge``, ``MSInstruction``, ``MSInstructionManager.solve``
and ``kernel_pass``.  The model is the same; the solver is this
package's own exact search (``_modsched_search``) instead of OR-Tools
CP-SAT, which is not available on MI355X hosts here.

``kernel_pass`` rewrites every top-level unit-step ``ForOp`` whose body
is made of loads and MMAs into the buffer form: a ring of
``num_stages`` shared slots per loaded tile, ``num_stages - 1`` prologue
load steps, a steady-state loop that waits on the slot the MMA reads,
refills the slot just freed and runs the MMA, and ``num_stages - 1``
drain steps (``modulo_scheduler.py:233-358``).  On CDNA4 the ring
becomes LDS slots filled by ``global_load_lds`` DMA and the waits become
``s_waitcnt vmcnt`` + ``s_barrier``; see ``warpir_amd.lowering``.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable, Dict, List, Optional, Tuple

from warpir_amd.ir.ops import (
    AddOp,
    AllocSharedOp,
    BufSlotExpr,
    CausalMaskOp,
    CopyOp,
    DivRowOp,
    DrainIndexOp,
    Exp2Op,
    ForOp,
    IntAffineOp,
    Kernel,
    LazyMaxOp,
    Log2Op,
    MMABufOp,
    MMAOp,
    MulOp,
    MulRowOp,
    MulScalarOp,
    Op,
    PipelineStageOp,
    RowMaxOp,
    RowSumOp,
    SlotViewOp,
    SubColOp,
    SubOp,
    SubRowOp,
    TMALoadBufOp,
    TMALoadOp,
    TMAStoreOp,
    Value,
    WaitBufOp,
    WaitOp,
    YieldOp,
)
from warpir_amd.ir.types import ColVecType, GPUType, RegTileType, RowVecType, SharedBufferType

from . import _modsched_search

# Cost model of the reference pass (modulo_scheduler.py:169-172, 186-190).
RESOURCE_COUNTS = {"tma": 4, "tc": 1}
MAX_CYCLES = 100
DEPTH = 5
LATENCY = {TMALoadOp: ("tma", 12), MMAOp: ("tc", 4), TMAStoreOp: ("tma", 12)}


@dataclass
class CostModel:
    """Latencies (resource, cycles) per op type, resource capacities and the
    solver horizon.  ``kernel_pass`` uses the reference's constants unless
    given another model."""

    latency: Dict[type, Tuple[str, int]]
    resources: Dict[str, int]
    max_cycles: int = MAX_CYCLES
    depth: int = DEPTH
    # Upper bound on ring slots (the LDS budget); None = no bound.
    max_stages: Optional[int] = None
    # Lower bound on ring slots of the prefetch form (a lowering that keeps
    # a tile resident one iteration longer asks for 3).
    min_stages: int = 2
    # Prefetch form only: issue the next tiles' loads after the first MMA of
    # the body instead of before it.  Issuing a wave's LDS-DMA instructions
    # can stall that wave for tens of cycles each; after the MMA they fall in
    # the shadow of its MFMAs, whose results the next op waits for anyway.
    loads_after_first_mma: bool = False
    # Load latency per source global (by name), overriding the op type's:
    # an operand that streams from HBM lands later than one that every
    # program re-reads from L2.
    source_latency: Dict[str, int] = field(default_factory=dict)
    # Reference form: give every ring its own depth, the distance from its
    # load's stage to the MMA's.  Loads are first moved as late as the
    # schedule allows (their MMA's start minus their latency, where the load
    # resource is free), so a ring holds only the tiles its latency needs;
    # rings over ``lds_budget`` lose slots where the least latency is then
    # exposed.  False keeps the reference's one depth for every ring.
    per_ring_depth: bool = False
    # LDS bytes per workgroup for the rings (per-ring depths).
    lds_budget: Optional[int] = None
    # Registers per lane the kernel may use, and an estimator of a rewritten
    # kernel's registers per lane.  A ring depth whose kernel the estimator
    # puts over the budget is not emitted; the pass takes the next shallower
    # one (down to two slots).
    register_budget: Optional[int] = None
    register_estimate: Optional[Callable[["Kernel"], int]] = None
    # Prefetch form: schedule the loop's compute ops -- the MMAs and the
    # softmax chain -- into MFMA and VALU phases (``_phase_stages``) and mark
    # the placement with ``pipeline_stage``.  "alternate": an iteration of a
    # wavefront is an MFMA phase then a VALU phase, the other wavefronts on
    # its SIMD filling each phase's idle unit; "mixed": one phase in which a
    # wavefront co-issues its VALU work beside its own MFMAs; "auto": the one
    # with the shorter estimated iteration (``phase_estimates``) at the
    # kernel's waves per SIMD.  None keeps the compute ops in program order.
    phase_schedule: Optional[str] = None

    def load_latency(self, op) -> Optional[Tuple[str, int]]:
        kind = self.latency.get(type(op))
        if kind is not None and isinstance(op, TMALoadOp) and op.source.name in self.source_latency:
            return kind[0], self.source_latency[op.source.name]
        return kind


REFERENCE_COST_MODEL = CostModel(latency=dict(LATENCY), resources=dict(RESOURCE_COUNTS))



def gfx950_cost_model(block_m: int, block_n: int, block_k: int, load_units: int = 8,
                      lds_budget: int = 160 * 1024, hbm_sources: Tuple[str, ...] = ()) -> CostModel:
    """Cost model of one K-step on an MI355X CU, in units of 256 cycles.

    The MMA's latency is the block tile's MFMA time spread over the CU's 4
    SIMDs at 1024 bf16 flop/clk each; an LDS-DMA tile load takes ~2048
    cycles from issue to landing under load (8 units).  For 256x256x32 the
    MMA is 4 units and the optimum is ii=4 with the MMA two stages behind
    its loads (a 3-slot ring); for 256x256x64 it is 8 units, ii=8 and a
    2-slot ring.  ``load_units`` raises the load latency for schedules that
    keep more tiles in flight (12 units: a 4-slot ring at K=32).  The ring
    depth is capped by ``lds_budget`` bytes per workgroup.

    ``hbm_sources`` names the operands that stream from HBM while the others
    stay in L2 (short-M GEMM: every program re-reads the one A row panel,
    and each B tile is read by one program).  Their loads take twice
    ``load_units``, the L2-resident ones ``load_units``, and each ring gets
    its own depth (``CostModel.per_ring_depth``).
    """
    mma_units = max(1, round(2 * block_m * block_n * block_k / (4 * 1024) / 256))
    stage_bytes = (block_m + block_n) * block_k * 2
    return CostModel(latency={TMALoadOp: ("tma", load_units), MMAOp: ("tc", mma_units),
                              TMAStoreOp: ("tma", load_units)},
                     resources={"tma": 8, "tc": 1}, max_stages=max(2, lds_budget // stage_bytes),
                     source_latency={name: 2 * load_units for name in hbm_sources},
                     per_ring_depth=bool(hbm_sources), lds_budget=lds_budget)


GFX950_COST_MODEL = gfx950_cost_model(256, 256, 32)


def gfx950_attention_cost_model(block_q: int, block_kv: int, d: int, lds_budget: int = 64 * 1024,
                                min_stages: int = 2, register_budget: Optional[int] = None,
                                register_estimate: Optional[Callable[[Kernel], int]] = None,
                                phase_schedule: Optional[str] = None) -> CostModel:
    """Cost model of one FlashAttention KV step on an MI355X CU.

    Each of the two MMAs (S = Q K^T and O += P V) is ``2*block_q*block_kv*d``
    flops; loads take ~8 units as for GEMM.  The ring depth is capped by an
    LDS budget per workgroup (64 KiB by default, so two workgroups share a
    CU and one's softmax overlaps the other's MFMAs).  ``min_stages`` = 3
    suits the 8-wavefront ping-pong lowering, which reads each V tile one
    iteration after its K tile.  ``register_budget`` / ``register_estimate``
    as in ``CostModel``: a ring too deep for the registers is not emitted.
    ``phase_schedule`` as in ``CostModel``: the softmax chain's placement.
    """
    mma_units = max(1, round(2 * block_q * block_kv * d / (4 * 1024) / 256))
    stage_bytes = 2 * block_kv * d * 2
    return CostModel(latency={TMALoadOp: ("tma", 8), MMAOp: ("tc", mma_units), TMAStoreOp: ("tma", 8)},
                     resources={"tma": 4, "tc": 1}, max_stages=max(2, lds_budget // stage_bytes),
                     min_stages=min_stages, loads_after_first_mma=True, register_budget=register_budget,
                     register_estimate=register_estimate, phase_schedule=phase_schedule)


@dataclass
class MSInstructionEdge:
    """Dependence ``source -> dest`` across ``distance`` iterations (``:25-29``)."""

    source: "MSInstruction"
    dest: "MSInstruction"
    distance: int


@dataclass
class MSInstruction:
    """One schedulable instruction of the loop body (``:31-37``)."""

    resource: str
    latency: int
    name: str
    parent_edges: List[MSInstructionEdge]


class PipelineError(KeyError):
    """The loop cannot be rewritten into buffer form.

    Raised where the reference pass fails with a ``KeyError``
    (``modulo_scheduler.py:309``): an MMA operand that is not produced by
    a load inside the loop, or a loop without an MMA.
    """


class MSInstructionManager:
    """Collects instructions and solves the modulo schedule (``:40-166``)."""

    def __init__(self) -> None:
        self.instructions: List[MSInstruction] = []
        self.child_edges: Dict[str, List[MSInstructionEdge]] = {}
        # (depth, name) -> (start, end) of the solved schedule.
        self.intervals: Dict[Tuple[int, str], Tuple[int, int]] = {}

    def add_instruction(self, instruction: MSInstruction) -> None:
        self.instructions.append(instruction)
        for edge in instruction.parent_edges:
            self.child_edges.setdefault(edge.source.name, []).append(edge)

    def solve(self, max_cycles: int, depth: int, resource_counts: Dict[str, int],
              use_verbose: bool = False):
        """Solve for the minimum-makespan schedule.

        Returns ``(prologue, steady_state, epilogue, ii, num_stages,
        stage_of)`` as the reference does (``:108-162``), or six ``None``
        when no schedule fits in ``max_cycles``:

        * ``prologue[i]``     -- ``(logical_iter, name)`` pairs issued in fill step ``i``;
        * ``steady_state[j]`` -- ``(name, buffer_offset)`` pairs of unrolled copy
          ``num_stages - 1 + j``;
        * ``epilogue[i]``     -- ``(name, stage - (i + 1))`` pairs of drain step ``i``;
        * ``stage_of[name]``  -- ``start // ii`` of the instruction's first copy.
        """
        index = {ins.name: k for k, ins in enumerate(self.instructions)}
        edges = []
        for k, ins in enumerate(self.instructions):
            for e in ins.parent_edges:
                if e.source.name not in index:
                    raise KeyError(e.source.name)
                edges.append((index[e.source.name], k, e.distance))
        problem = _modsched_search.Problem(
            latencies=[ins.latency for ins in self.instructions],
            resources=[ins.resource for ins in self.instructions],
            edges=edges, depth=depth, max_cycles=max_cycles, capacity=resource_counts,
        )
        found = _modsched_search.solve(problem)
        if found is None:
            if use_verbose:
                print("modulo schedule: no solution within", max_cycles, "cycles")
            return None, None, None, None, None, None
        ii, offsets, makespan = found
        self.intervals = {}
        for d in range(depth):
            for ins, s in zip(self.instructions, offsets):
                self.intervals[(d, ins.name)] = (s + d * ii, s + d * ii + ins.latency)
        if use_verbose:
            print(f"modulo schedule: ii={ii} makespan={makespan} offsets={offsets}")
        return _shape_schedule(self.instructions, offsets, ii, depth)


def _shape_schedule(instructions: List[MSInstruction], offsets: List[int], ii: int, depth: int):
    names = [ins.name for ins in instructions]
    # ii == 0 places every copy at the same cycle; everything is stage 0.
    stage_of = {n: (s // ii if ii else 0) for n, s in zip(names, offsets)}
    num_stages = max(stage_of.values()) + 1
    prologue = [[(i - stage_of[n], n) for n in names if stage_of[n] <= i]
                for i in range(num_stages - 1)]
    steady_state = [[(n, k - stage_of[n]) for n in names] for k in range(num_stages - 1, depth)]
    epilogue = [[(n, stage_of[n] - i) for n in names if stage_of[n] >= i]
                for i in range(1, num_stages)]
    return prologue, steady_state, epilogue, ii, num_stages, stage_of


def _shape_from_stages(names: List[str], stage_of: Dict[str, int], depth: int):
    """Prologue / steady-state / epilogue lists for given stages (as ``_shape_schedule``)."""
    num_stages = max(stage_of.values()) + 1
    prologue = [[(i - stage_of[n], n) for n in names if stage_of[n] <= i] for i in range(num_stages - 1)]
    steady_state = [[(n, k - stage_of[n]) for n in names] for k in range(num_stages - 1, depth)]
    epilogue = [[(n, stage_of[n] - i) for n in names if stage_of[n] >= i] for i in range(1, num_stages)]
    return prologue, steady_state, epilogue, num_stages


def _loop_instructions(loop: ForOp, cost: CostModel, transitive: bool = False) -> Dict[str, MSInstruction]:
    """One ``MSInstruction`` per load / MMA / store, keyed by the op's text (``:183-217``)."""
    instrs: Dict[str, MSInstruction] = {}
    for op in loop.body:
        kind = cost.load_latency(op)
        if kind is not None:
            instrs[str(op)] = MSInstruction(resource=kind[0], latency=kind[1], name=str(op),
                                            parent_edges=[])
    producer: Dict[Value, MSInstruction] = {
        op.result: instrs[str(op)] for op in loop.body if type(op) in (TMALoadOp, MMAOp)
    }
    if transitive:
        # Values computed by unscheduled ops (the softmax chain) inherit the
        # scheduled producers of their operands, so an MMA fed by them still
        # depends on the MMA that started the chain.
        chains: Dict[Value, List[MSInstruction]] = {}
        for op in loop.body:
            if str(op) in instrs or not hasattr(op, "result"):
                continue
            srcs: List[MSInstruction] = []
            for name, operand in vars(op).items():
                if name == "result" or not isinstance(operand, Value):
                    continue
                if operand in producer:
                    srcs.append(producer[operand])
                srcs.extend(chains.get(operand, []))
            chains[op.result] = srcs
    carried = {ia.block_arg for ia in loop.iter_args}
    yld = next(op for op in loop.body if isinstance(op, YieldOp))
    next_value = {ia.block_arg: yld.values[k] for k, ia in enumerate(loop.iter_args)}
    for op in loop.body:
        ins = instrs.get(str(op))
        if ins is None:
            continue
        # Only bare Value operands carry dependences; coordinate tuples do not.
        for name, operand in vars(op).items():
            if name == "result" or not isinstance(operand, Value):
                continue
            distance = 1 if operand in carried else 0
            src = producer.get(next_value.get(operand, operand))
            if src is not None:
                ins.parent_edges.append(MSInstructionEdge(source=src, dest=ins, distance=distance))
            if transitive and distance == 0:
                for s in chains.get(operand, []):
                    if s is not ins and all(e.source is not s for e in ins.parent_edges):
                        ins.parent_edges.append(MSInstructionEdge(source=s, dest=ins, distance=0))
    return instrs


def _reference_form_applies(loop: ForOp) -> bool:
    """The reference rewrite (``:239-358``) handles bodies of loads, waits and
    MMAs whose operands are all loaded inside the loop."""
    loaded = {op.result for op in loop.body if isinstance(op, TMALoadOp)}
    for op in loop.body:
        if isinstance(op, MMAOp):
            if op.transpose_b or op.a not in loaded or op.b not in loaded:
                return False
        elif not isinstance(op, (TMALoadOp, WaitOp, YieldOp)):
            return False
    return True


def _pipeline_loop(loop: ForOp, cost: CostModel,
                   rebuild: Optional[Callable[[List[Op]], Kernel]] = None) -> Optional[List[Op]]:
    if not _reference_form_applies(loop) and any(isinstance(op, TMALoadOp) for op in loop.body):
        return _prefetch_loop(loop, cost, rebuild)
    instrs = _loop_instructions(loop, cost)
    manager = MSInstructionManager()
    for ins in instrs.values():
        manager.add_instruction(ins)
    prologue, _steady, _epilogue, ii, stages, stage_of = manager.solve(
        max_cycles=cost.max_cycles, depth=cost.depth, resource_counts=cost.resources)
    if prologue is None:
        return None
    loads = [op for op in loop.body if isinstance(op, TMALoadOp)]
    mmas = [op for op in loop.body if isinstance(op, MMAOp)]
    if not mmas:
        raise PipelineError("loop has no MMA to pipeline")
    loaded = {ld.result for ld in loads}
    for mma in mmas:
        for operand in (mma.a, mma.b):
            if operand not in loaded:
                raise PipelineError(f"MMA operand {operand!r} is not loaded inside the loop")

    if cost.per_ring_depth and len(mmas) == 1:
        plans = _ring_depth_plans(loop, cost, manager, instrs, ii, loads, mmas[0])
    else:
        if cost.max_stages is not None and stages > cost.max_stages:
            # The LDS budget holds fewer slots than the schedule wants: pull the
            # late instructions forward to the last stage that fits.
            stage_of = {n: min(st, cost.max_stages - 1) for n, st in stage_of.items()}
        stages = max(stage_of.values()) + 1
        plans = [(stage_of, {str(ld): stages for ld in loads})]
        if cost.register_budget is not None:
            # shallower uniform rings for the register check: the loads keep
            # their stage, the MMAs move one stage earlier per step
            mma_names = {str(op) for op in mmas}
            for depth in range(stages - 1, 1, -1):
                st = {n: (min(v, depth - 1) if n in mma_names else v) for n, v in stage_of.items()}
                plans.append((st, {str(ld): depth for ld in loads}))
    out = None
    for stage_plan, depths in plans:
        out = _buffer_form(loop, stage_plan, depths, loads)
        if _fits_registers(cost, rebuild, out):
            return out
    return out


def _fits_registers(cost: CostModel, rebuild: Optional[Callable[[List[Op]], Kernel]], ops: List[Op]) -> bool:
    """Whether the kernel with this rewritten loop fits ``cost.register_budget``
    (always true without a budget and an estimator)."""
    if cost.register_budget is None or cost.register_estimate is None or rebuild is None:
        return True
    return cost.register_estimate(rebuild(ops)) <= cost.register_budget


def _modulo_fits(instrs: Dict[str, MSInstruction], offsets: Dict[str, int], ii: int, depth: int,
                 capacity: Dict[str, int]) -> bool:
    """The solver's cumulative resource limits, for given offsets."""
    usage: Dict[Tuple[str, int], int] = {}
    for name, ins in instrs.items():
        if ins.resource not in capacity:
            continue
        for d in range(depth):
            for t in range(offsets[name] + d * ii, offsets[name] + d * ii + ins.latency):
                usage[(ins.resource, t)] = usage.get((ins.resource, t), 0) + 1
                if usage[(ins.resource, t)] > capacity[ins.resource]:
                    return False
    return True


def _ring_depth_plans(loop: ForOp, cost: CostModel, manager: MSInstructionManager,
                      instrs: Dict[str, MSInstruction], ii: int, loads: List[TMALoadOp], mma: MMAOp):
    """Per-ring depths for the one-MMA reference form, deepest first.

    Every load is moved as late as its MMA allows (the MMA's start minus the
    load's latency, at the latest offset where the load resource is free),
    so its ring needs ``stage(MMA) - stage(load) + 1`` slots.  Rings over the
    LDS budget lose slots one at a time: each time the ring whose loss
    leaves the least load latency uncovered,
    ``max_r(latency_r - (slots_r - 1) * ii)``.  Further plans continue that
    order down to two slots per ring (the register check's candidates).
    Returns ``[(stage_of, slots_of_load)]``.
    """
    offsets = {name: manager.intervals[(0, name)][0] for name in instrs}
    m_name = str(mma)
    for ld in loads:
        n = str(ld)
        latest = offsets[m_name] - instrs[n].latency
        for t in range(latest, offsets[n], -1):
            trial = dict(offsets, **{n: t})
            if _modulo_fits(instrs, trial, ii, cost.depth, cost.resources):
                offsets = trial
                break
    s_m = offsets[m_name] // ii
    want = {str(ld): max(2, s_m - offsets[str(ld)] // ii + 1) for ld in loads}
    nbytes = {str(ld): _tile_nbytes(ld.result.type) for ld in loads}
    lat = {str(ld): instrs[str(ld)].latency for ld in loads}

    def exposed(depths) -> int:
        return max(lat[n] - (d - 1) * ii for n, d in depths.items())

    def shrink(depths):
        options = [n for n, d in depths.items() if d > 2]
        if not options:
            return None
        best = min(options, key=lambda n: (exposed(dict(depths, **{n: depths[n] - 1})), -nbytes[n],
                                           list(depths).index(n)))
        return dict(depths, **{best: depths[best] - 1})

    depths = dict(want)
    budget = cost.lds_budget
    while budget is not None and sum(depths[n] * nbytes[n] for n in depths) > budget:
        nxt = shrink(depths)
        if nxt is None:
            break
        depths = nxt
    plans = []
    while depths is not None:
        top = max(depths.values()) - 1
        stage_of = {n: top - depths[n] + 1 for n in depths}
        stage_of[m_name] = top
        plans.append((stage_of, dict(depths)))
        depths = shrink(depths) if cost.register_budget is not None else None
    return plans


def _tile_nbytes(t) -> int:
    return t.rows * t.cols * (2 if t.data_type == GPUType.bf16 else 4)


def _buffer_form(loop: ForOp, stage_of: Dict[str, int], depths: Dict[str, int],
                 loads: List[TMALoadOp]) -> List[Op]:
    """The reference buffer form (``:244-358``) for given stages and ring depths.

    With one depth for every ring this is the reference rewrite: prologue
    step ``p`` loads tile ``p - stage`` into its slot, the loop from
    ``num_stages - 1`` waits on the MMA's slot, refills the slots its loads
    own and runs the MMA, and drain step ``e`` waits on drain slot ``e``
    and runs the MMAs still in flight.  With depths that differ, each ring
    ``r`` of ``m_r`` slots holds tile ``t`` in slot ``t % m_r``: the loop
    waits once per ring depth, a load ``k`` stages ahead of its MMA names
    tile ``i - stage`` through an ``int_affine`` of the induction variable,
    and in the drain it loads tile ``drain + k`` (``drain_index``).
    """
    iv = loop.induction_var
    by_name: Dict[str, Op] = {str(op): op for op in loop.body}
    names = list(by_name)
    stages = max(stage_of.values()) + 1
    ring = {ld.result: Value(f"{ld.source.name.lower()}_bufs",
                             SharedBufferType(tile_type=ld.result.type, count=depths[str(ld)]))
            for ld in loads}
    mod = {ld.result: depths[str(ld)] for ld in loads}
    groups: Dict[int, List[Value]] = {}
    for ld in loads:
        groups.setdefault(mod[ld.result], []).append(ring[ld.result])

    out: List[Op] = [AllocSharedOp(result=ring[ld.result]) for ld in loads]
    # Fill: prologue step p loads logical iteration p - stage (:255-269).
    for step in range(stages - 1):
        for name in names:
            op = by_name[name]
            st = stage_of.get(name)
            if isinstance(op, TMALoadOp) and st is not None and st <= step:
                fixed = op.substitute({iv: step - st})
                out.append(TMALoadBufOp(buf=ring[op.result], slot=(step - st) % mod[op.result],
                                        source=op.source, coords=fixed.coords))

    def slot(v: Value, stage: int, value: Optional[Value] = None) -> BufSlotExpr:
        if value is not None:
            return BufSlotExpr(value=value, offset=0, modulus=mod[v])
        return BufSlotExpr(value=iv, offset=-stage, modulus=mod[v])

    mmas = [by_name[n] for n in names if isinstance(by_name[n], MMAOp)]
    s_m = stage_of[str(mmas[0])]
    body: List[Op] = [WaitBufOp(bufs=tuple(bufs), slot=BufSlotExpr(value=iv, offset=-s_m, modulus=m))
                      for m, bufs in groups.items()]
    shifted: Dict[int, Value] = {}
    for name in names:
        op = by_name[name]
        st = stage_of.get(name)
        if isinstance(op, TMALoadOp):
            coords = op.coords
            if st:
                if st not in shifted:
                    shifted[st] = Value(f"{iv.name}_s{st}", iv.type)
                    body.append(IntAffineOp(result=shifted[st], input=iv, mul=1, add=-st))
                coords = op.substitute({iv: shifted[st]}).coords
            body.append(TMALoadBufOp(buf=ring[op.result], slot=slot(op.result, st), source=op.source,
                                     coords=coords))
        elif isinstance(op, MMAOp):
            body.append(MMABufOp(result=op.result, a_buf=ring[op.a], a_slot=slot(op.a, st),
                                 b_buf=ring[op.b], b_slot=slot(op.b, st), accum=op.accum))
    body.append(next(op for op in loop.body if isinstance(op, YieldOp)))
    out.append(ForOp(induction_var=iv, start=stages - 1, stop=loop.stop, step=loop.step,
                     tile_size=loop.tile_size, iter_args=loop.iter_args, body=tuple(body),
                     results=loop.results))

    # Drain: step e waits on drain slot e and runs the MMAs still in flight
    # (:329-356); a load k stages ahead of the MMA still fetches its tile.
    for e in range(stages - 1):
        waits = [WaitBufOp(bufs=tuple(bufs), slot=BufSlotExpr(value=None, offset=e, modulus=m))
                 for m, bufs in groups.items()]
        out.extend(waits)
        for name in names:
            op = by_name[name]
            st = stage_of.get(name)
            if st is None or st < e + 1:
                continue
            if isinstance(op, TMALoadOp):
                ahead = Value(f"{iv.name}_d{e}_{s_m - st}", iv.type)
                out.append(DrainIndexOp(result=ahead, offset=s_m - st))
                out.append(TMALoadBufOp(buf=ring[op.result], slot=slot(op.result, st, ahead),
                                        source=op.source, coords=op.substitute({iv: ahead}).coords))
            elif isinstance(op, MMAOp):
                k = next(j for j, ia in enumerate(loop.iter_args) if ia.block_arg == op.accum)
                out.append(MMABufOp(result=Value(f"{op.result.name}_ep{e}", op.result.type),
                                    a_buf=ring[op.a], a_slot=BufSlotExpr(value=None, offset=e, modulus=mod[op.a]),
                                    b_buf=ring[op.b], b_slot=BufSlotExpr(value=None, offset=e, modulus=mod[op.b]),
                                    accum=loop.results[k]))
    return out


def _prefetch_loop(loop: ForOp, cost: CostModel,
                   rebuild: Optional[Callable[[List[Op]], Kernel]] = None) -> Optional[List[Op]]:
    """Buffer form for loops the reference rewrite cannot take: an MMA reads
    a loop-invariant tile (the resident Q of FlashAttention), a register
    value, or the body carries non-MMA work (the online-softmax chain).

    The loads move into a ring; the compute ops keep program order unless
    the cost model asks for a phase schedule (``CostModel.phase_schedule``),
    which places every MMA and softmax op by its unit and marks the
    placement with ``pipeline_stage`` (``_place_phases``).  With
    ``S`` ring slots chosen by the modulo schedule (the MMAs' stage behind
    their loads, at least 2, at most ``cost.max_stages``), the prologue
    loads tiles ``start .. start+S-2``; iteration ``i`` waits on slot
    ``i % S``, issues the loads of tile ``i + S - 1`` into the slot freed
    by iteration ``i - 1``, and names the tiles it reads through
    ``slot_view``.  Loads past the end of the data read zeros (TMA
    out-of-bounds semantics), so no drain steps are needed: the last
    ``S - 1`` iterations simply prefetch tiles that are never read.  With a
    register budget, a depth whose kernel the estimator puts over it gives
    way to the next shallower one (down to 2 slots).
    """
    instrs = _loop_instructions(loop, cost, transitive=True)
    manager = MSInstructionManager()
    for ins in instrs.values():
        manager.add_instruction(ins)
    prologue, _steady, _epi, _ii, stages, stage_of = manager.solve(
        max_cycles=cost.max_cycles, depth=cost.depth, resource_counts=cost.resources)
    if prologue is None:
        return None
    loads = [op for op in loop.body if isinstance(op, TMALoadOp)]
    mmas = [op for op in loop.body if isinstance(op, MMAOp)]
    if not mmas:
        raise PipelineError("loop has no MMA to pipeline")
    stages = max(cost.min_stages, stages)
    if cost.max_stages is not None:
        stages = max(2, min(stages, cost.max_stages))
    if loop.step != 1:
        raise PipelineError("the prefetch form needs a unit step")
    out: List[Op] = []
    for depth in range(stages, 1, -1):
        out = _prefetch_form(loop, cost, loads, depth)
        if _fits_registers(cost, rebuild, out):
            break
    if cost.phase_schedule is not None:
        from .register_counter import count_registers
        waves = count_registers(rebuild(out)).waves_per_simd if rebuild is not None else 2
        rewritten = out[-1]
        body = _place_phases(rewritten, list(rewritten.body), cost, waves)
        out[-1] = ForOp(induction_var=rewritten.induction_var, start=rewritten.start, stop=rewritten.stop,
                        step=rewritten.step, iter_args=rewritten.iter_args, body=tuple(body),
                        results=rewritten.results, tile_size=rewritten.tile_size)
    return out


def _prefetch_form(loop: ForOp, cost: CostModel, loads: List[TMALoadOp], stages: int) -> List[Op]:
    """``_prefetch_loop``'s rewrite for a ring of ``stages`` slots."""
    iv = loop.induction_var
    ring = {ld.result: Value(f"{ld.source.name.lower()}_bufs",
                             SharedBufferType(tile_type=ld.result.type, count=stages)) for ld in loads}
    all_rings = tuple(ring[ld.result] for ld in loads)
    out: List[Op] = [AllocSharedOp(result=ring[ld.result]) for ld in loads]
    for p in range(stages - 1):
        if isinstance(loop.start, int):
            tile, slot = loop.start + p, (loop.start + p) % stages
        else:
            # a run-time start (e.g. the first query tile of a causal key-major loop)
            tile = Value(f"{iv.name}_p{p}", iv.type)
            out.append(IntAffineOp(result=tile, input=loop.start, mul=1, add=p))
            slot = BufSlotExpr(value=loop.start, offset=p, modulus=stages)
        for ld in loads:
            out.append(TMALoadBufOp(buf=ring[ld.result], slot=slot, source=ld.source,
                                    coords=ld.substitute({iv: tile}).coords))
    nxt = Value(f"{iv.name}_pf", iv.type)
    body: List[Op] = [WaitBufOp(bufs=all_rings, slot=BufSlotExpr(value=iv, offset=0, modulus=stages)),
                      IntAffineOp(result=nxt, input=iv, mul=1, add=stages - 1)]
    # The prefetches write slot (i + S - 1) % S, which no op of iteration i
    # reads, so they may go anywhere in the body.
    prefetch = [TMALoadBufOp(buf=ring[ld.result], slot=BufSlotExpr(value=iv, offset=stages - 1, modulus=stages),
                             source=ld.source, coords=ld.substitute({iv: nxt}).coords) for ld in loads]
    if not cost.loads_after_first_mma:
        body.extend(prefetch)
        prefetch = []
    for ld in loads:
        body.append(SlotViewOp(result=ld.result, buf=ring[ld.result],
                               slot=BufSlotExpr(value=iv, offset=0, modulus=stages)))
    ring_tiles = set(ring)
    for op in loop.body:
        if isinstance(op, TMALoadOp):
            continue
        if isinstance(op, WaitOp):
            rest = tuple(v for v in op.values if v not in ring_tiles)
            if rest:
                body.append(WaitOp(values=rest))
            continue
        body.append(op)
        if isinstance(op, MMAOp) and prefetch:
            body.extend(prefetch)
            prefetch = []
    body.extend(prefetch)
    out.append(ForOp(induction_var=iv, start=loop.start, stop=loop.stop, step=loop.step,
                     iter_args=loop.iter_args, body=tuple(body), results=loop.results,
                     tile_size=loop.tile_size))
    return out


# ---------------------------------------------------------------------------
# Phase scheduling of an attention loop's compute ops
# ---------------------------------------------------------------------------
# gfx950 issue costs per wavefront, in shader cycles (in-bounds probes):
MFMA_CYCLES = 32            # one v_mfma_f32_32x32x16_bf16 (32.004 measured back to back)
VALU_CYCLES = 4             # one wave64 fp32 VALU instruction
TRANS_CYCLES = 8            # v_exp_f32 / v_log_f32: about two FMAs' cost beside an MFMA
COISSUE_PER_MFMA = 4        # independent VALU instructions an MFMA hides on its own wavefront
DEPENDENT_VALU_CYCLES = 10  # a lone wavefront's dependent VALU chain: one instruction per ~10 cycles

_VALU_OPS = (CopyOp, MulScalarOp, SubOp, MulOp, AddOp, Exp2Op, Log2Op, RowMaxOp, RowSumOp, SubRowOp,
             MulRowOp, DivRowOp, LazyMaxOp, CausalMaskOp, SubColOp)


def op_unit(op: Op) -> Optional[str]:
    """The SIMD unit a compute op of a loop body occupies: "mfma" for an MMA,
    "valu" for the element-wise, row and column ops of the softmax chain,
    None for ops that cost nothing there (zero fills, index arithmetic,
    waits, views, loads)."""
    if isinstance(op, MMAOp):
        return "mfma"
    if isinstance(op, _VALU_OPS):
        return "valu"
    return None


def _lane_elems(t) -> int:
    if isinstance(t, RegTileType):
        return max(1, t.rows * t.cols // 64)
    if isinstance(t, ColVecType):
        return max(1, t.rows // 32)
    if isinstance(t, RowVecType):
        return max(1, t.cols // 2)
    return 1


def op_cycles(op: Op) -> int:
    """Issue cycles of one wavefront's share of a compute op: MFMAs of the
    32x32x16 shape for an MMA (its per-wavefront result tile times the
    reduction depth), VALU instructions for the softmax chain (one per fp32
    element a lane holds; transcendentals count two; the bf16 pack converts
    two per instruction; a row reduction adds its cross-lane swap)."""
    if isinstance(op, MMAOp):
        t = op.result.type
        k = op.a.type.cols
        return max(1, t.rows * t.cols * k // (32 * 32 * 16)) * MFMA_CYCLES
    if isinstance(op, (RowMaxOp, RowSumOp)):
        return (_lane_elems(op.tile.type) + 1) * VALU_CYCLES
    e = _lane_elems(op.result.type)
    if isinstance(op, (Exp2Op, Log2Op)):
        return e * TRANS_CYCLES
    if isinstance(op, CopyOp) and getattr(op.result.type, "data_type", None) == GPUType.bf16:
        return max(1, e // 2) * VALU_CYCLES
    return e * VALU_CYCLES


def phase_estimates(ops: List[Op], waves_per_simd: int) -> Dict[str, int]:
    """Estimated SIMD cycles per iteration of all ``waves_per_simd``
    wavefronts for the two phase structures.  "alternate": each wavefront's
    MFMA phase runs beside the others' VALU phases, so the SIMD is bound by
    the larger of its total MFMA and VALU time (and one wavefront's own
    sequence).  "mixed": each wavefront co-issues up to COISSUE_PER_MFMA
    VALU instructions per MFMA, and the rest of its chain issues at the lone
    wavefront's dependent rate; the wavefronts then take turns."""
    mfma = sum(op_cycles(o) for o in ops if op_unit(o) == "mfma")
    valu = sum(op_cycles(o) for o in ops if op_unit(o) == "valu")
    w = max(1, waves_per_simd)
    alternate = max(w * mfma, w * valu, mfma + valu)
    hidden = COISSUE_PER_MFMA * (mfma // MFMA_CYCLES) * VALU_CYCLES
    own = mfma + max(0, valu - hidden) * DEPENDENT_VALU_CYCLES // VALU_CYCLES
    return {"alternate": alternate, "mixed": w * own}


def _phase_stages(loop: ForOp, body: List[Op], mode: str) -> Dict[int, int]:
    """Stage of each compute op of ``body`` (by ``id``) in a modulo schedule
    of phases.

    Every MMA and softmax op is an ``MSInstruction`` on its unit.  With
    "alternate" the initiation interval is two slots, an MFMA phase (slot 0)
    and a VALU phase (slot 1): ``slot_class`` pins MMAs to even and VALU ops
    to odd offsets.  With "mixed" it is one slot holding both.  An MMA's
    result is ready in the next slot (latency 1); VALU ops chain inside
    their slot (latency 0).  Data dependences have distance 0, values
    carried through the loop's iter_args distance 1.  The exact search
    (``_modsched_search``) returns the smallest interval and the earliest
    offsets; an op's stage is its offset divided by the interval, counted
    from the earliest compute op.
    """
    ops = [o for o in body if op_unit(o) is not None]
    if not ops:
        return {}
    index = {id(o): k for k, o in enumerate(ops)}
    producer = {o.result: o for o in ops if isinstance(getattr(o, "result", None), Value)}
    yld = next(o for o in body if isinstance(o, YieldOp))
    carried = {ia.block_arg: yld.values[k] for k, ia in enumerate(loop.iter_args)}
    edges = []
    for o in ops:
        for name, v in vars(o).items():
            if name == "result" or not isinstance(v, Value):
                continue
            if v in producer:
                edges.append((index[id(producer[v])], index[id(o)], 0))
            elif v in carried and carried[v] in producer:
                edges.append((index[id(producer[carried[v]])], index[id(o)], 1))
    units = [op_unit(o) for o in ops]
    if mode == "alternate":
        slot_class = [0 if u == "mfma" else 1 for u in units]
    elif mode == "mixed":
        slot_class = [0] * len(ops)
    else:
        raise ValueError(f"phase schedule {mode!r}: expected 'alternate' or 'mixed'")
    problem = _modsched_search.Problem(
        latencies=[1 if u == "mfma" else 0 for u in units], resources=units, edges=edges,
        depth=DEPTH, max_cycles=64, capacity={}, slot_class=slot_class)
    found = _modsched_search.solve(problem)
    if found is None:
        raise PipelineError("the loop's compute ops have no phase schedule")
    ii, offsets, _span = found
    first = min(offsets) // ii
    return {id(o): off // ii - first for o, off in zip(ops, offsets)}


def _place_phases(loop: ForOp, body: List[Op], cost: CostModel, waves_per_simd: int) -> List[Op]:
    """``body`` reordered by the phase schedule: stage-0 ops in program
    order, then ``pipeline_stage(s)`` and the stage-``s`` ops, then the
    yield.  Ops that are no compute op (waits, views, index arithmetic,
    loads, zero fills) stay at stage 0."""
    mode = cost.phase_schedule
    if mode == "auto":
        est = phase_estimates([o for o in body if op_unit(o)], waves_per_simd)
        mode = "mixed" if est["mixed"] < est["alternate"] else "alternate"
    stages = _phase_stages(loop, body, mode)
    last = max(stages.values(), default=0)
    if last == 0:
        return body
    yld = body[-1]
    out = [o for o in body[:-1] if stages.get(id(o), 0) == 0]
    for st in range(1, last + 1):
        out.append(PipelineStageOp(stage=st))
        out.extend(o for o in body[:-1] if stages.get(id(o), 0) == st)
    out.append(yld)
    return out


def kernel_pass(kernel: Kernel, cost_model: Optional[CostModel] = None) -> Kernel:
    """Pipeline every top-level unit-step loop of *kernel* (``:168-358``).

    Loops whose schedule has no solution are kept unchanged, as in the
    reference.  Loops of loads and MMAs get the reference's buffer form
    (with per-ring depths when the cost model asks); loops with a softmax
    chain, loop-invariant or register MMA operands (FlashAttention) get the
    prefetch form of ``_prefetch_loop`` where the reference raises
    ``KeyError`` (``:309``), with the softmax chain phase-scheduled when the
    cost model asks.  ``cost_model`` defaults to the reference's constants.
    """
    cost = cost_model or REFERENCE_COST_MODEL
    body: List[Op] = []
    for k, op in enumerate(kernel.body):
        if not isinstance(op, ForOp) or op.step != 1:
            body.append(op)
            continue

        def rebuild(ops: List[Op], k=k) -> Kernel:
            # the kernel with this loop rewritten as ``ops`` (for the register check)
            return Kernel(name=kernel.name, inputs=kernel.inputs, outputs=kernel.outputs,
                          body=tuple(body) + tuple(ops) + tuple(kernel.body[k + 1:]))

        rewritten = _pipeline_loop(op, cost, rebuild)
        body.extend([op] if rewritten is None else rewritten)
    return Kernel(name=kernel.name, inputs=kernel.inputs, outputs=kernel.outputs, body=tuple(body))


__all__ = ["MSInstructionEdge", "MSInstruction", "MSInstructionManager", "PipelineError",
           "CostModel", "REFERENCE_COST_MODEL", "GFX950_COST_MODEL", "gfx950_cost_model",
           "gfx950_attention_cost_model", "kernel_pass", "op_unit", "op_cycles", "phase_estimates"]
