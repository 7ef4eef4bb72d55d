"""WarpIR tile IR -> gfx950 (CDNA4) HIP source.

``CDNA4Lowerer().lower(kernel) -> str`` is the drop-in counterpart of the
reference's ``ThunderKittensLowerer().lower(kernel) -> str``
(``warpir/lowering/lowering.py:44,67-81``).  It keeps the reference
lowering's behavioural contract (``lowering.py:87-113,196-207,454-488,
572-606``):

* a loop's iter_arg ``init``, its ``results`` and the yielded values name
  the block argument's storage;
* ``MMAOp`` without ``transpose_b`` accumulates in place into its result
  (after copying ``accum`` there when the storages differ); with
  ``transpose_b`` it computes ``a @ b^T`` and does not read ``accum``;
* ``MMABufOp`` accumulates in place into ``accum`` and advances the drain
  counter, which every ``drain(...)`` slot reads;
* a ``tile_size`` loop runs ``ceil(stop / tile_size)`` trips;
* kernel arguments are ``inputs`` then ``outputs`` in IR order.

What differs is the machine mapping, which is CDNA4's own:

* tile loads are LDS-DMA (``global_load_lds_dwordx4``) into swizzled LDS
  tiles; out-of-bounds chunks read a zero page (TMA zero-fill);
* ``WaitOp`` / ``WaitBufOp`` become ``s_waitcnt vmcnt(N)`` + ``s_barrier``
  where ``N`` -- the loads this wave may keep in flight -- comes from a
  concrete simulation of the IR's load/wait order (``_schedule``), and a
  barrier is inserted before any load that would overwrite a tile another
  wave may still be reading (write-after-read);
* MMAs are ``v_mfma_f32_32x32x16_bf16`` (or ``16x16x32`` for 16-row
  wavefront slices) computed for the transposed product so that every
  register tile has the lane = row layout (see ``csrc/wir_cdna4.h``);
* row reductions use one ``v_permlane32_swap`` after the lane-local part;
* program ids are remapped so each XCD walks a contiguous, grouped range
  of output tiles (L2 locality).

``launch_config`` returns grid / block / LDS for concrete tensors, the
information the reference keeps in its harness strings
(``tests/test_modal_gpu.py:24-50``).
"""
from __future__ import annotations

import math
import os
import re
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple, Union

from warpir_amd.ir.ops import (
    AddOp, AllocSharedOp, BufSlotExpr, CausalMaskOp, CopyOp, DivRowOp, DrainIndexOp, Exp2Op, ForOp,
    IntAffineOp, IntDivOp, Kernel, LoadVecOp, Log2Op, MMABufOp, MMAOp, MulOp, MulRowOp, MulScalarOp, NegInftyOp,
    LazyMaxOp, Op, PipelineStageOp, ReduceSlicesOp, RowMaxOp, RowSumOp, SubColOp, SubOp, SubRowOp, TMALoadBufOp, TMALoadOp, TMAStoreOp, Value,
    WaitBufOp, WaitOp, YieldOp, ZeroOp,
)
from warpir_amd.ir.ops import SlotViewOp
from warpir_amd.ir.types import (
    ColVecType, GPUType, GlobalType, IntType, RegTileType, RowVecType, ScalarType, SharedBufferType,
    SharedTileType,
)

BUILTINS = ("blockIdx.x", "blockIdx.y", "blockIdx.z")
# Steady-state iterations the warp assigner unrolls when the lowering asks it
# for a wave-group split: one keeps the exact search to a fraction of a
# second on every kernel here, and gives the same type -> warp placement as
# longer unrolls where those finish.
ASSIGN_ITERATIONS = 1
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "csrc",
                           "wir_cdna4.h")
ROWREAD, TRREAD, BOTH = 0, 1, 2


class LoweringError(ValueError):
    """The kernel uses a shape or op combination this target cannot lower."""


@dataclass
class CDNA4Target:
    """Machine parameters and code-generation choices for gfx950.

    ``waves_per_eu`` = None takes the waves per SIMD from the
    ``register_counter`` pass (2 when a wavefront's estimated footprint fits
    256 registers per lane, else 1), at least enough for the workgroup's
    waves on four SIMDs.  ``mfma`` = None picks the
    32x32x16 MFMA when every register tile is a multiple of 32 rows and
    columns, else 16x16x32.
    """

    arch: str = "gfx950"
    lds_bytes: int = 160 * 1024
    num_xcds: int = 8
    waves_per_eu: Optional[int] = None
    mfma: Optional[int] = None
    xcd_remap: bool = True
    group_m: int = 8
    rotate_mma: bool = True
    pingpong: bool = True
    # Modulo variable expansion: unroll ring loops by their slot count so
    # every slot index is a compile-time constant.
    mve: bool = True
    # Final bf16 stores of register tiles go through LDS as whole rows.
    staged_stores: bool = True
    # Those staged stores carry the non-temporal hint (wir::store_tile_staged<true>):
    # measured +1.5% on GEMM 8192^3, +0.2-0.4% on the attention forwards.
    nontemporal_stores: bool = True
    # Wave group (0 or 1) that issues each load stream (named by its ring,
    # e.g. "k", "v") in the 8-wavefront attention ping-pong.  None: take it
    # from the warp assigner's solution for the kernel (passes.warp_assigner).
    wave_groups: Optional[Dict[str, int]] = None
    # The online-softmax step with a lazy running maximum (RowMaxOp feeding a
    # LazyMaxOp, then the exp2 / row-sum / rescale ops of that step) becomes
    # one speculative wir::lazy_softmax call: the step is computed with the
    # maximum unchanged and verified from the exponentials' lane sums; only a
    # tile that rises above the slack (and the first tile) recomputes it.
    lazy_softmax: bool = True
    # Attention ping-pong with one workgroup barrier per iteration instead of
    # one per phase: group A passes it after its V phase, group B after its
    # M phase, so the two groups' phases interleave without lock-step.
    pingpong_one_barrier: bool = True
    # With the one-barrier ping-pong on a ring of at least 5 slots: pass the
    # workgroup barrier only every second iteration (both groups load K and
    # V tiles S - 2 ahead, and each barrier still leaves the wave's newest
    # batch in flight).  1 keeps a barrier every iteration.
    pingpong_barrier_every: int = 1
    # With the one-barrier ping-pong (a barrier every iteration): group B
    # passes its barrier between the rotated PV and the QK MMA instead of
    # after the QK, so between two barriers A runs PV(i-1), QK(i), softmax(i)
    # and B runs QK(i), softmax(i), PV(i): the groups sit a third of an
    # iteration apart instead of half, and at each interval's start both
    # waves of a SIMD issue MFMAs (one's LDS operand latency under the
    # other's MFMAs).  B's V tiles are then loaded S - 2 ahead, like A's K.
    pingpong_split_barrier: bool = False
    # Attention ping-pong: B operands of the next PV MMA (V tile fragments,
    # in mma_rAB's order) each wave reads at the end of its VALU phase, when
    # its LDS reads are otherwise idle, so its MFMA phase reads that many
    # fewer (4 VGPRs each).  0 reads them all in the MFMA phase.
    pingpong_v_prefetch: int = 0
    # With the lazy softmax on scores from hoisted Q fragments: the scale c is
    # folded into those fragments (bf16 of c*q, once per program) and the
    # running max into the score MFMAs (one extra MFMA per column block
    # subtracts it), so the step needs no fma per score (wir::ScoreBias,
    # wir::lazy_softmax_fast_b / lazy_softmax_exact_b).  Off by default: the
    # second bf16 rounding of Q makes the score error grow with the logits'
    # magnitude (O error 1.3e-2 at LSE ~47, against 3.6e-3 unfolded).
    fold_softmax_scale: bool = False
    # Ask the compiler for the VGPR form of the MFMAs (LLVM's
    # -amdgpu-mfma-vgpr-form): accumulators that VALU code reads (scores)
    # stay in arch VGPRs instead of AGPRs, which removes their
    # v_accvgpr_read copies.  The flag travels in the source's first line
    # (``HIPCC_FLAGS_MARKER``), so it is part of the code-object cache key.
    mfma_vgpr_form: bool = False
    # Warp specialisation for ring-pipelined MMA loops: the workgroup gets a
    # second set of wavefronts (waves NW..2NW-1) that only issue the LDS-DMA
    # loads, while waves 0..NW-1 only read LDS and issue MFMAs.  Both sets pass
    # every barrier; gfx950 has no setmaxnreg, so both get the same register
    # allocation (two waves per SIMD: at most 256 per lane).
    warp_specialize: bool = False
    # Cache-policy bits on the tile loads' global_load_lds instructions: "" (the
    # default policy), or any of "sc0", "sc1", "nt" joined by spaces (gfx950's
    # scope and non-temporal bits).  The tiles are read once per workgroup, so
    # nothing on the path re-reads them from the CU's L1.
    dma_cache_policy: str = ""
    # The lazy softmax's speculative half sums each row's bf16 probabilities
    # on the matrix core (wir::lazy_softmax_fast_mr: four 16x16x32 MFMAs per
    # 64-key tile against a 0/1 operand) instead of 32 fp32 adds and a
    # cross-lane reduction per lane; its guard tests those sums.  32-row
    # fragments only; not with fold_softmax_scale.
    rowsum_mfma: bool = False
    # Rotated MMA pipelines: spread the step's DMAs over all its MFMAs
    # (MMAPipeAB::run<N, true>) instead of the first half, the first-loaded
    # operand's in the first half and the other's in the second.  Meant for
    # rings whose wait leaves the newest batch in flight (a deeper ring on
    # the operand loaded last), where those loads have a step more to land.
    dma_spread_whole: bool = False
    # Element-wise register-tile ops that directly precede an MMA emitted from
    # register operands (hoisted fragments, or a bf16 register A) and that the
    # MMA does not depend on run inside that MMA's MFMA stream, one group of
    # 4 registers per MFMA slot (wir::*_part in mma_*_slots), so a single
    # wavefront per SIMD issues them under its own MFMAs.
    slot_fusion: bool = False
    # Persistent programs: launch min(tiles, persistent) workgroups, each
    # walking output tiles blockIdx.x, blockIdx.x + gridDim.x, ... (the tile
    # extents come from the output tensor, the tile -> program-id map is the
    # XCD remap of the tile index, so a tile keeps its XCD when the count is a
    # multiple of 8).  The body runs once per tile, a workgroup barrier
    # between tiles.  0: one workgroup per tile.
    persistent: int = 0
    # With persistent programs and the attention ping-pong (a barrier every
    # iteration): one K/V ring stream across the tiles a program walks, so the
    # next tile's first K/V tiles load under the current tile's last steps and
    # the ping-pong never drains between tiles.  At a tile boundary, after the
    # rotated PV, each wave stores its rows of O and the LSE from registers,
    # then loads the next tile's Q and resets its running state.
    persistent_stream: bool = False


@dataclass
class LaunchConfig:
    grid: Tuple[int, int, int]
    block: Tuple[int, int, int]
    dyn_lds: int = 0


# A generated source whose first line starts with this marker is compiled with
# the hipcc flags that follow it on that line (``runtime.compile_source``).
HIPCC_FLAGS_MARKER = "// wir-hipcc-flags:"


@dataclass
class _Geometry:
    nw: int            # wavefronts per workgroup
    nw_c: int          # wavefronts along the result columns
    ms: int            # MFMA shape (32 or 16)
    waves_per_eu: int


def _cname(name: str) -> str:
    return "v_" + re.sub(r"[^0-9A-Za-z_]", "_", name)


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


class CDNA4Lowerer:
    """Lower a WarpIR ``Kernel`` to one self-contained gfx950 HIP source."""

    def __init__(self, target: Optional[CDNA4Target] = None):
        self.target = target or CDNA4Target()
        self._reset()

    # ------------------------------------------------------------------
    # public API
    # ------------------------------------------------------------------
    def lower(self, kernel: Kernel) -> str:
        """Return HIP C++ for *kernel* (``lowering.py:67-81``)."""
        self._reset()
        self.kernel = kernel
        self._drain_unreduced = any(isinstance(o, DrainIndexOp) for o in _walk(kernel.body))
        self._build_aliases(kernel.body)
        self._classify(kernel)
        self.geo = self._geometry(kernel)
        self._assign_roles(kernel.body)
        self._pending_hoist = self._hoistable()
        self._register_tiles = self._register_only_tiles()
        self._allocate_lds()
        self._staged = self._staged_stores()
        self.wait_n, self.war_barrier = _schedule(kernel, self)
        self._ws = self._warp_specialized(kernel)
        self._ws_producer_streams = self._ws_streams(kernel) if self._ws else set()
        if self._ws and self._ws_producer_streams is None:
            self._ws = False
        if self.target.lazy_softmax:
            for loop in _walk(kernel.body):
                if isinstance(loop, ForOp):
                    self._match_lazy_softmax(loop.body)
            if self.target.fold_softmax_scale:
                self._plan_score_folds(kernel)
        self._plan_pingpong_loops(kernel)
        if self.target.persistent_stream:
            self._stream = self._stream_plan(kernel)
        body: List[str] = []
        self._emit_ops(kernel.body, body, 1)
        if self._stream is not None:
            self._stream_lines = self._emit_attention_stream(*self._stream)
        return self._assemble(kernel, body)

    def _stream_plan(self, kernel: Kernel):
        """(loop, ops before it, ops after it) when the kernel takes the
        persistent stream form: persistent programs, one top-level loop in the
        one-barrier ping-pong form with a barrier every iteration (no split
        barrier, V prefetch or folded scale), whose K and V loads address
        (batch, head) = (pid_z, pid_y) at key tile = the loop index, column 0."""
        if not self.target.persistent:
            raise LoweringError("persistent_stream takes persistent programs")
        loops = [o for o in kernel.body if isinstance(o, ForOp)]
        if len(loops) != 1 or id(loops[0]) not in self._pp_forms:
            return None
        loop = loops[0]
        plan, _swap, one, every = self._pp_forms[id(loop)]
        t = self.target
        if (not one or every != 1 or t.pingpong_split_barrier or t.pingpong_v_prefetch or t.fold_softmax_scale
                or not isinstance(loop.start, int) or loop.step != 1):
            return None
        aff = self.resolve(plan["affine"].result.name)
        for ld in (plan["k_load"], plan["v_load"]):
            b, d, rt, ct = ld.coords
            if not (isinstance(b, Value) and b.name == "blockIdx.z" and isinstance(d, Value) and d.name == "blockIdx.y"
                    and isinstance(rt, Value) and self.resolve(rt.name) == aff and ct == 0):
                return None
        idx = kernel.body.index(loop)
        return loop, list(kernel.body[:idx]), list(kernel.body[idx + 1:])

    def _plan_pingpong_loops(self, kernel: Kernel) -> None:
        """Record the top-level loops that take the attention ping-pong form,
        and the prologue loads in front of each into its K and V rings: the
        ping-pong issues those tiles itself (split between its wave groups),
        so its aligned body skips them."""
        prev: List[Op] = []
        for op in kernel.body:
            if not isinstance(op, ForOp):
                prev.append(op)
                continue
            form = self._pingpong_form(op)
            if form is not None:
                self._pp_forms[id(op)] = form
                rings = {self.resolve(form[0][k].buf.name) for k in ("k_load", "v_load")}
                self._pp_prologue |= {id(o) for o in prev
                                      if isinstance(o, TMALoadBufOp) and self.resolve(o.buf.name) in rings}
            prev = []

    def launch_config(self, kernel: Kernel, tensors: Dict[str, Sequence[int]]) -> LaunchConfig:
        """Grid / block for concrete output shapes (``tensors``: name -> shape)."""
        if self.kernel is not kernel:
            self.lower(kernel)
        grid = [1, 1, 1]
        for op in _walk(kernel.body):
            if not isinstance(op, TMAStoreOp):
                continue
            shape = _as4d(tensors[op.dest.name])
            sub = op.dest.type.sub_tile_type
            units = (1, 1, sub.rows, sub.cols)
            for pos, c in enumerate(op.coords):
                if isinstance(c, Value) and c.name in BUILTINS:
                    axis = BUILTINS.index(c.name)
                    grid[axis] = max(grid[axis], _ceil_div(shape[pos], units[pos]))
        if self.target.persistent:
            total = grid[0] * grid[1] * grid[2]
            grid = [max(1, min(total, self.target.persistent)), 1, 1]
        return LaunchConfig(grid=tuple(grid), block=(self.num_threads, 1, 1), dyn_lds=0)

    def _tile_extents(self, kernel: Kernel) -> List[str]:
        """C++ expressions of the output-tile counts along blockIdx.x, .y, .z,
        from the stored globals' extents (the persistent form's grid does not
        carry them)."""
        fields = ("b", "d", "r", "c")
        ext: List[List[str]] = [[], [], []]
        for op in _walk(kernel.body):
            if not isinstance(op, TMAStoreOp):
                continue
            sub = op.dest.type.sub_tile_type
            units = (1, 1, sub.rows, sub.cols)
            for pos, c in enumerate(op.coords):
                if isinstance(c, Value) and c.name in BUILTINS:
                    e = f"globals.{_cname(op.dest.name)[2:]}.{fields[pos]}"
                    ext[BUILTINS.index(c.name)].append(e if units[pos] == 1 else
                                                       f"(({e}) + {units[pos] - 1}) / {units[pos]}")
        out = []
        for es in ext:
            expr = "1"
            for e in es:
                expr = e if expr == "1" else f"max({expr}, {e})"
            out.append(expr)
        return out

    @property
    def num_threads(self) -> int:
        return self.geo.nw * 64 * (2 if self._ws else 1)

    def _warp_specialized(self, kernel: Kernel) -> bool:
        """Whether the warp-specialised form applies: requested, four compute
        wavefronts, and every top-level loop a rotatable ring pipeline (loads
        and one buffered MMA), so that producer and consumer waves pass the
        same barriers."""
        if not self.target.warp_specialize or self.geo.nw != 4:
            return False
        def ring(loop: ForOp) -> bool:
            body = [o for o in loop.body if not isinstance(o, YieldOp)]
            return bool(body) and isinstance(body[0], WaitBufOp) and isinstance(body[-1], MMABufOp) and all(
                isinstance(o, TMALoadBufOp) for o in body[1:-1])
        loops = [op for op in kernel.body if isinstance(op, ForOp)]
        return bool(loops) and all(ring(lp) for lp in loops) and not any(
            isinstance(op, (MMAOp, CopyOp)) for op in _walk(kernel.body))

    def _ws_streams(self, kernel: Kernel):
        """Ring buffers whose loads the DMA-only waves issue; the MFMA waves
        issue the others.  The split comes from ``CDNA4Target.wave_groups``
        (stream -> group; group 1 = DMA waves) or, when that is None, from the
        warp assigner's steady-state assignment with the gfx950 costs (each
        stream's DMA issue stalls the wave that issues it): a load type placed
        on the MMA's warp stays with the MFMA waves, one placed on another
        warp goes to the DMA waves.  None if the vmcnt thresholds do not split
        between the two sets."""
        def stream(buf_name: str) -> str:
            return buf_name[:-len("_bufs")] if buf_name.endswith("_bufs") else buf_name
        bufs = sorted({self.resolve(op.buf.name) for op in _walk(kernel.body) if isinstance(op, TMALoadBufOp)})
        groups = self.target.wave_groups
        if groups is None:
            from warpir_amd.passes.warp_assigner import assign_streams, gfx950_wave_costs
            sol = assign_streams(kernel, gfx950_wave_costs(kernel, waves_per_group=self.geo.nw), num_warps=2)
            mma_warp = next((w for t, w in sol.type_warp.items() if t.startswith("mma")), 0)
            groups = {t[:-len("_load")]: int(w != mma_warp) for t, w in sol.type_warp.items() if t.endswith("_load")}
        producers = {b for b in bufs if groups.get(stream(b), 1) == 1}
        # per-wave DMA instructions of one ring step, per set
        per = {b: self.loads_per_wave(self.tile_type_of(b)) for b in bufs}
        total = sum(per.values())
        self._ws_share = (sum(per[b] for b in producers), total - sum(per[b] for b in producers), total)
        for n in self.wait_n.values():
            if n % total:
                return None
        return producers

    def _ws_wait(self, n: int) -> str:
        """wait_vm_barrier for the two wave sets: each waits on its own share of
        the n in-flight DMA instructions that one all-loading wave would have."""
        prod, cons, total = self._ws_share
        np_, nc = n // total * prod, n // total * cons
        if np_ == nc:
            return f"wir::wait_vm_barrier<{np_}>();"
        return f"if (wir_producer) wir::wait_vm_barrier<{np_}>(); else wir::wait_vm_barrier<{nc}>();"

    def _ws_issuer(self, buf_name: str) -> str:
        return "wir_producer" if self.resolve(buf_name) in self._ws_producer_streams else "!wir_producer"

    def _consumer_only(self, lines: List[str], pad: str) -> List[str]:
        """In the warp-specialised form, wrap *lines* so only MFMA waves run them."""
        if not self._ws or not lines:
            return lines
        return [f"{pad}if (!wir_producer) {{", *[("  " + ln) for ln in lines], f"{pad}}}"]

    def lds_bytes(self) -> int:
        return self.lds_total

    # ------------------------------------------------------------------
    # analysis
    # ------------------------------------------------------------------
    def _reset(self) -> None:
        self.kernel = None
        self._aliases: Dict[str, str] = {}
        self.values: Dict[str, Value] = {}
        self.roles: Dict[str, int] = {}
        self.lds_off: Dict[str, int] = {}
        self.lds_total = 0
        self.waves_per_simd: Optional[int] = None    # the amdgpu_waves_per_eu the kernel is compiled for
        self._staged: Dict[int, int] = {}
        self._stage_barrier_done = False
        self.globals: List[Value] = []
        self.drain_modulus: Optional[int] = None
        # The drain counter counts buffered MMAs without reduction when a
        # drain_index op reads it (rings of different depths); otherwise it
        # is kept reduced by the one ring size.
        self._drain_unreduced = False
        self._loop_of_yield: Dict[int, ForOp] = {}
        self._hoisted: Dict[str, Tuple[str, int]] = {}
        self._pending_hoist: Dict[str, tuple] = {}
        self._view_cache: Dict[str, SlotViewOp] = {}
        self._view_kernel = None
        self._rotated: Dict[int, str] = {}
        self._register_tiles: Dict[str, tuple] = {}
        self._aligned_checks: set = set()
        self._pp_ops: Dict[int, tuple] = {}     # id(op) -> (role, pipe name, extra)
        self._slot_const: Dict[str, int] = {}   # induction var -> its value mod the ring size
        self._slot_shift: Dict[str, int] = {}   # induction var -> offset added to its ring slots
        self._fused_loads: Dict[int, List[Op]] = {}
        self._fused_ids: set = set()
        self._var_override: Dict[str, str] = {}  # resolved value name -> C++ variable
        self._ws = False                          # warp-specialised form (producer / consumer waves)
        self._softmax_fused: Dict[int, object] = {}  # id(op) -> fused lazy-softmax plan, or "skip"
        self._slot_work: Dict[int, tuple] = {}       # id(MMA) -> (moved ops, register groups, slots form)
        self._slot_skip: set = set()                 # ids of ops emitted in an MMA's slots
        self._no_fusion = False                      # emit the fused groups' ops one by one
        self._overlapped = False                     # an attention loop took the overlapped ("mixed") form
        self._lazy_exact_only = False                # fused groups emit only the exact half
        self._score_folds: Dict[int, dict] = {}      # id(QK MMA) -> fold of its lazy-softmax group
        self._fold_live = False                      # inside a fused loop whose ScoreBias is declared
        self._pp_forms: Dict[int, tuple] = {}        # id(top-level loop) -> its attention ping-pong form
        self._pp_prologue: set = set()               # ids of prologue loads the ping-pong issues itself
        self._stream = None                          # persistent_stream: (loop, pre ops, post ops)
        self._stream_lines: List[str] = []

    def _build_aliases(self, ops) -> None:
        """iter_arg init / loop results / yielded values -> block arg (``lowering.py:87-100``)."""
        for op in ops:
            if not isinstance(op, ForOp):
                continue
            for k, ia in enumerate(op.iter_args):
                self._aliases[ia.init.name] = ia.block_arg.name
                if k < len(op.results):
                    self._aliases[op.results[k].name] = ia.block_arg.name
            for inner in op.body:
                if isinstance(inner, YieldOp):
                    for k, y in enumerate(inner.values):
                        if k < len(op.iter_args):
                            self._aliases[y.name] = op.iter_args[k].block_arg.name
            self._build_aliases(op.body)

    def resolve(self, name: str) -> str:
        seen = set()
        while name in self._aliases and name not in seen:
            seen.add(name)
            name = self._aliases[name]
        return name

    def _classify(self, kernel: Kernel) -> None:
        self.globals = list(kernel.inputs) + list(kernel.outputs)
        for v in self.globals:
            if not isinstance(v.type, (GlobalType, ScalarType)):
                raise LoweringError(f"kernel argument {v!r} must be a global or an int")
        for op in _walk(kernel.body):
            for f in vars(op).values():
                for v in _values_in(f):
                    self.values.setdefault(self.resolve(v.name), v)

    def _rtype(self, v: Value):
        return self.values[self.resolve(v.name)].type

    def _is_shared(self, v: Value) -> bool:
        return isinstance(v.type, SharedTileType)

    def _geometry(self, kernel: Kernel) -> _Geometry:
        mmas = [op for op in _walk(kernel.body) if isinstance(op, (MMAOp, MMABufOp))]
        if not mmas:
            return self._geometry_from_copies(kernel)
        nw = nw_c = None
        dims = []
        for op in mmas:
            res_t = op.result.type if isinstance(op.result.type, RegTileType) else self._rtype(op.accum)
            if not isinstance(res_t, RegTileType):
                raise LoweringError(f"MMA result {op.result!r} is not a register tile")
            r, c = res_t.rows, res_t.cols
            dims += [r, c]
            a_t, b_t, tb = _mma_operand_types(op)
            block_c = b_t.rows if tb else b_t.cols
            if block_c % c:
                raise LoweringError(f"MMA {op.result.name}: {block_c} columns do not split into {c}")
            this_c = block_c // c
            if isinstance(a_t, SharedTileType):
                if a_t.rows % r:
                    raise LoweringError(f"MMA {op.result.name}: {a_t.rows} rows do not split into {r}")
                this_nw = (a_t.rows // r) * this_c
                if nw is not None and this_nw != nw:
                    raise LoweringError("MMAs disagree on the wavefront count")
                nw = this_nw
            else:
                dims += [a_t.rows, a_t.cols]
            if nw_c is not None and this_c != nw_c:
                raise LoweringError("MMAs disagree on the wavefront column split")
            nw_c = this_c
        if nw is None:
            raise LoweringError("no MMA reads a shared tile as `a`: wavefront count unknown")
        for op in _walk(kernel.body):
            for v in _values_in(vars(op).get("result")):
                if isinstance(v.type, RegTileType):
                    dims += [v.type.rows, v.type.cols]
        ms = self.target.mfma
        if ms is None:
            ms = 32 if all(d % 32 == 0 for d in dims) else 16
        if any(d % ms for d in dims):
            raise LoweringError(f"register tiles {sorted(set(dims))} are not multiples of the MFMA shape {ms}")
        if nw * 64 > 1024:
            raise LoweringError(f"{nw} wavefronts exceed the 1024-thread workgroup limit")
        return _Geometry(nw=nw, nw_c=nw_c, ms=ms, waves_per_eu=self._waves_for(kernel, nw))

    def _waves_for(self, kernel: Kernel, nw: int) -> int:
        if self.target.waves_per_eu is not None:
            return self.target.waves_per_eu
        from warpir_amd.passes.register_counter import count_registers

        return max(count_registers(kernel).waves_per_simd, -(-nw // 4))

    def _geometry_from_copies(self, kernel: Kernel) -> _Geometry:
        """Wavefront layout of an MMA-free kernel from its shared -> register
        copies: the block tile split into the register tile's wave slices."""
        nw = nw_c = None
        dims = []
        for op in _walk(kernel.body):
            if isinstance(op, CopyOp) and isinstance(op.input.type, SharedTileType) \
                    and isinstance(op.result.type, RegTileType):
                sh, rg = op.input.type, op.result.type
                if sh.rows % rg.rows or sh.cols % rg.cols:
                    raise LoweringError(f"copy {op.result.name}: {sh.rows}x{sh.cols} does not split into "
                                        f"{rg.rows}x{rg.cols}")
                this = (sh.rows // rg.rows * (sh.cols // rg.cols), sh.cols // rg.cols)
                if nw is not None and (nw, nw_c) != this:
                    raise LoweringError("copies disagree on the wavefront layout")
                nw, nw_c = this
                dims += [rg.rows, rg.cols]
        if nw is None:
            raise LoweringError("kernel has no MMA and no shared -> register copy: wavefront count unknown")
        ms = self.target.mfma or (32 if all(d % 32 == 0 for d in dims) else 16)
        return _Geometry(nw=nw, nw_c=nw_c, ms=ms, waves_per_eu=self._waves_for(kernel, nw))

    def _assign_roles(self, ops) -> None:
        """ROWREAD for tiles read along k by rows, TRREAD for [K][N] tiles read across k,
        BOTH for tiles read both ways."""
        def use(v: Value, role: int) -> None:
            # A tile read both by rows and transposed (K in the dQ kernel, Q
            # and dO in the dK/dV kernel) takes the BOTH swizzle, conflict-free
            # for either read.
            key = self._lds_key(v)
            if key is None:
                return
            if self.roles.setdefault(key, role) != role:
                self.roles[key] = BOTH

        for op in _walk(ops):
            if isinstance(op, CopyOp) and isinstance(op.input.type, SharedTileType):
                use(op.input, ROWREAD)
            if isinstance(op, MMAOp):
                use(op.a, ROWREAD)
                use(op.b, ROWREAD if op.transpose_b else TRREAD)
            elif isinstance(op, MMABufOp):
                use(op.a_buf, ROWREAD)
                use(op.b_buf, TRREAD)

    def _lds_key(self, v: Value) -> Optional[str]:
        """Name of the LDS allocation behind a shared tile / ring / slot view."""
        name = self.resolve(v.name)
        view = self._views().get(name)
        if view is not None:
            return self.resolve(view.buf.name)
        t = self.values[name].type if name in self.values else v.type
        if isinstance(t, (SharedTileType, SharedBufferType)):
            return name
        return None

    def _views(self) -> Dict[str, SlotViewOp]:
        if self._view_kernel is not self.kernel:
            self._view_cache = {self.resolve(op.result.name): op for op in _walk(self.kernel.body)
                                if isinstance(op, SlotViewOp)}
            self._view_kernel = self.kernel
        return self._view_cache

    def _allocate_lds(self) -> None:
        off = 0
        for op in _walk(self.kernel.body):
            if isinstance(op, TMALoadOp):
                key, t, count = self.resolve(op.result.name), op.result.type, 1
                if key in self._register_tiles:
                    continue
            elif isinstance(op, AllocSharedOp):
                key, t = self.resolve(op.result.name), op.result.type.tile_type
                count = op.result.type.count
            else:
                continue
            if key in self.lds_off:
                continue
            if t.data_type != GPUType.bf16 and not _is_vec_tile(t):
                raise LoweringError(f"shared tile {key} must be bf16 (or an fp32 L x 1 vector)")
            self.roles.setdefault(key, ROWREAD)
            self.lds_off[key] = off
            off += _tile_bytes(t) * count
        self.lds_total = off
        if off > self.target.lds_bytes:
            raise LoweringError(f"LDS use {off} B exceeds the {self.target.lds_bytes} B per workgroup")

    def _staged_stores(self) -> Dict[int, int]:
        """Stores of fp32 register tiles to bf16 globals that go through LDS.

        Eligible are top-level stores after which no op touches shared
        memory: the ring buffers are dead, so each wavefront can stage its
        tile in a private LDS area (id(op) -> bytes per wavefront).  The
        first staged store is preceded by one workgroup barrier.
        """
        if not self.target.staged_stores:
            return {}
        lds_ops = (TMALoadOp, TMALoadBufOp, WaitOp, WaitBufOp, MMAOp, MMABufOp, AllocSharedOp, ForOp, SlotViewOp)
        out: Dict[int, int] = {}
        body = list(self.kernel.body)
        for i, op in enumerate(body):
            if not isinstance(op, TMAStoreOp):
                continue
            if any(isinstance(o, lds_ops) for o in body[i:]):
                continue
            st = self._rtype(op.source)
            if not (isinstance(st, RegTileType) and st.data_type == GPUType.fp32
                    and op.dest.type.data_type == GPUType.bf16):
                continue
            cpr = st.cols // 8
            per_wave = st.rows * st.cols * 2
            if st.cols % 8 or cpr & (cpr - 1) or (st.rows * cpr) % 64 or per_wave * self.geo.nw > self.target.lds_bytes:
                continue
            out[id(op)] = per_wave
        if out:
            self.lds_total = max(self.lds_total, max(out.values()) * self.geo.nw)
        return out

    # ------------------------------------------------------------------
    # emission helpers
    # ------------------------------------------------------------------
    def tile_type_of(self, key: str) -> SharedTileType:
        t = self.values[key].type
        return t.tile_type if isinstance(t, SharedBufferType) else t

    def stile(self, key: str) -> str:
        t = self.tile_type_of(key)
        return f"wir::STile<{t.rows}, {t.cols}, {self.roles.get(key, ROWREAD)}>"

    def loads_per_wave(self, tile: SharedTileType) -> int:
        if _is_vec_tile(tile):   # one global_load_lds_dword per wavefront
            if tile.rows % self.geo.nw or tile.rows // self.geo.nw > 64:
                raise LoweringError(f"vector tile {tile}: {tile.rows} elements do not split into "
                                    f"{self.geo.nw} wavefronts of at most 64")
            return 1
        chunks = tile.rows * tile.cols * 2 // 16
        if chunks % 64:
            raise LoweringError(f"tile {tile} is not a multiple of 1 KiB (64 LDS-DMA chunks)")
        instr = chunks // 64
        if instr % self.geo.nw:
            raise LoweringError(f"tile {tile}: {instr} DMA instructions do not split over {self.geo.nw} wavefronts")
        return instr // self.geo.nw

    def _int(self, x) -> str:
        if isinstance(x, int):
            return str(x)
        name = self.resolve(x.name)
        if name in BUILTINS:
            return "pid_" + name[-1]
        if any(g.name == name for g in self.globals):
            return f"globals.{_cname(name)[2:]}"
        return _cname(name)

    def _slot(self, slot) -> str:
        if isinstance(slot, int):
            return str(slot)
        if slot.value is None:
            return f"(wir_drain % {slot.modulus})" if self._drain_unreduced else "wir_drain"
        m = slot.modulus
        name = self.resolve(slot.value.name)
        off = slot.offset + self._slot_shift.get(name, 0)
        if name in self._slot_const:
            return str((self._slot_const[name] + off) % m)
        return f"((({self._int(slot.value)}) + {off % m}) % {m})"

    def _tile_ptr(self, v: Value) -> Tuple[str, str]:
        """(LDS pointer expression, LDS key) of a shared tile or slot view."""
        name = self.resolve(v.name)
        view = self._views().get(name)
        if view is not None:
            key = self.resolve(view.buf.name)
            stride = _tile_bytes(self.tile_type_of(key))
            return f"(smem + {self.lds_off[key]} + {self._slot(view.slot)} * {stride})", key
        if name not in self.lds_off:
            raise LoweringError(f"{v.name} is not a shared tile")
        return f"(smem + {self.lds_off[name]})", name

    def _buf_ptr(self, buf: Value, slot) -> Tuple[str, str]:
        key = self.resolve(buf.name)
        stride = _tile_bytes(self.tile_type_of(key))
        return f"(smem + {self.lds_off[key]} + {self._slot(slot)} * {stride})", key

    def _var(self, v: Value) -> str:
        name = self.resolve(v.name)
        return self._var_override.get(name) or _cname(name)

    def _reg_decl(self, v: Value) -> Optional[str]:
        t = v.type
        ms = self.geo.ms
        if isinstance(t, RegTileType):
            kind = "RTile" if t.data_type == GPUType.fp32 else "BTile"
            return f"wir::{kind}<{ms}, {t.rows}, {t.cols}>"
        if isinstance(t, ColVecType):
            return f"wir::RVec<{ms}, {t.rows}>"
        if isinstance(t, RowVecType):
            return f"wir::CVec<{ms}, {t.cols}>"
        return None

    # ------------------------------------------------------------------
    # op emission
    # ------------------------------------------------------------------
    def _match_lazy_softmax(self, body) -> None:
        """Find the online-softmax steps with a lazy maximum in a loop body.

        The step (``tests/attention_baseline.py:42-186`` with the running max
        replaced by ``LazyMaxOp``), matched by data flow::

            m_prev = copy(m);  cand = row_max(s, m);  m' = lazy_max(m, cand, slack)
            s_c = s * c;  m'_c = m' * c;  m_c = m_prev * c;  p = exp2(s_c - m'_c)
            corr = exp2(m_c - m'_c);  l_c = l * corr;  l' = row_sum(p, l_c)
            o' = o * corr;  pb = bf16(p)

        Every intermediate value must stay inside the group; m', l', o' and pb
        may be used after it.  The group is emitted as one ``wir::lazy_softmax``
        at the position of its first op (no op between its members may read a
        group result)."""
        ops = list(body)
        prod = {o.result.name: o for o in ops if isinstance(getattr(o, "result", None), Value)}
        uses: Dict[str, List[Op]] = {}
        for o in ops:
            for v in _op_values(o):
                if v is not getattr(o, "result", None):
                    uses.setdefault(v.name, []).append(o)

        def only(name, kind, **attrs):
            cands = [u for u in uses.get(name, []) if isinstance(u, kind)
                     and all(getattr(u, k).name == v.name if isinstance(v, Value) else getattr(u, k) == v
                             for k, v in attrs.items())]
            return cands[0] if len(cands) == 1 else None

        for lz in (o for o in ops if isinstance(o, LazyMaxOp)):
            rm = prod.get(lz.cand.name)
            if not isinstance(rm, RowMaxOp) or rm.prev.name != lz.prev.name:
                continue
            s_v, m_v = rm.tile, lz.prev
            ms_new = next((u for u in uses.get(lz.result.name, []) if isinstance(u, MulScalarOp)), None)
            if ms_new is None:
                continue
            c = ms_new.scalar
            ms_s = only(s_v.name, MulScalarOp, scalar=c)
            cp = only(m_v.name, CopyOp)
            ms_prev = cp and only(cp.result.name, MulScalarOp, scalar=c)
            sr = ms_s and only(ms_s.result.name, SubRowOp, vec=ms_new.result)
            e1 = sr and only(sr.result.name, Exp2Op)
            sb = ms_prev and only(ms_prev.result.name, SubOp, b=ms_new.result)
            e2 = sb and only(sb.result.name, Exp2Op)
            mu = e2 and only(e2.result.name, MulOp)
            rs = e1 and mu and only(e1.result.name, RowSumOp, prev=mu.result)
            mr = e2 and only(e2.result.name, MulRowOp)
            cv = e1 and only(e1.result.name, CopyOp)
            group = [cp, rm, lz, ms_s, ms_new, ms_prev, sr, e1, sb, e2, mu, rs, mr, cv]
            if any(g is None for g in group) or sb.a.name != ms_prev.result.name:
                continue
            norm = mu.a if mu.b.name == e2.result.name else mu.b
            if not (isinstance(cv.result.type, RegTileType) and cv.result.type.data_type == GPUType.bf16):
                continue
            ids = {id(g) for g in group}
            internal = [cp, rm, ms_s, ms_new, ms_prev, sr, e1, sb, e2, mu]
            if any(id(u) not in ids for g in internal for u in uses.get(g.result.name, [])):
                continue
            outputs = {g.result.name for g in (lz, rs, mr, cv)}
            inputs = {m_v.name, norm.name, mr.tile.name}
            if any(id(u) not in ids for n in inputs for u in uses.get(n, [])):
                continue
            first = min(ops.index(g) for g in group)
            last = max(ops.index(g) for g in group)
            if any(id(o) not in ids and any(v.name in outputs for v in _op_values(o)) for o in ops[first:last + 1]):
                continue
            # the fused group is emitted at its first member, so every value it
            # reads from outside (the scores, l, O) must be defined before that
            external = {s_v.name, norm.name, mr.tile.name}
            if any(isinstance(getattr(o, "result", None), Value) and o.result.name in external
                   for o in ops[first:last + 1] if id(o) not in ids):
                continue
            plan = dict(s=s_v, m_in=m_v, m_out=lz.result, l_in=norm, l_out=rs.result, o_in=mr.tile,
                        o_out=mr.result, p=cv.result, c=c, slack=lz.slack, ids=ids)
            for g in group:
                self._softmax_fused[id(g)] = "skip"
            self._softmax_fused[id(ops[first])] = plan

    def _plan_score_folds(self, kernel: Kernel) -> None:
        """Lazy-softmax groups whose scores can come out of the MFMAs already
        scaled and shifted (``CDNA4Target.fold_softmax_scale``): the group's
        score tile is S = Q K^T (or its causal mask) from a QK MMA whose Q is
        a hoisted register fragment read by that MMA alone, and the raw and
        masked scores are read by nothing outside the group.  Folding
        changes what those values hold (c*S - c*m instead of S), so every
        reader must be one of these ops."""
        if self.geo.ms != 32:
            return
        ops = list(_walk(kernel.body))
        prod = {self.resolve(o.result.name): o for o in ops if isinstance(getattr(o, "result", None), Value)}
        uses: Dict[str, List[Op]] = {}
        for o in ops:
            for v in _op_values(o):
                if v is not getattr(o, "result", None):
                    uses.setdefault(self.resolve(v.name), []).append(o)
        for plan in [p for p in self._softmax_fused.values() if isinstance(p, dict)]:
            src = prod.get(self.resolve(plan["s"].name))
            mask = None
            if isinstance(src, CausalMaskOp):
                mask, src = src, prod.get(self.resolve(src.tile.name))
            if not isinstance(src, MMAOp) or not src.transpose_b:
                continue
            q = self.resolve(src.a.name)
            if q not in self._register_tiles and q not in self._pending_hoist:
                continue
            if [id(u) for u in uses.get(q, []) if not isinstance(u, (WaitOp, WaitBufOp))] != [id(src)]:
                continue
            raw_readers = {id(mask)} if mask is not None else plan["ids"]
            if any(id(u) not in raw_readers for u in uses.get(self.resolve(src.result.name), [])):
                continue
            if mask is not None and any(id(u) not in plan["ids"]
                                        for u in uses.get(self.resolve(mask.result.name), [])):
                continue
            plan["fold"] = True
            self._score_folds[id(src)] = dict(q=q, c=plan["c"], rb=src.result.type.rows // self.geo.ms)

    def _fold_preamble(self, ops, out: List[str], depth: int) -> bool:
        """At the top of a fused lazy-softmax loop: scale the hoisted Q
        fragments of its folded QK MMA by c and declare the score bias.
        Returns whether the loop runs folded (at most one fold per loop)."""
        folds = [self._score_folds[id(o)] for o in _walk(ops) if id(o) in self._score_folds]
        if len(folds) != 1 or folds[0]["q"] not in self._hoisted:
            return False
        f = folds[0]
        pad = "  " * depth
        out.append(f"{pad}wir::scale_frags({self._hoisted[f['q']][0]}, {_flt(f['c'])});"
                   f"  // softmax scale folded into Q")
        out.append(f"{pad}wir::ScoreBias<{f['rb']}> wir_sb;   // running max folded into the score MFMAs")
        out.append(f"{pad}wir_sb.init();")
        self._fold_live = True
        return True

    def _fast_call(self, fz) -> str:
        """The speculative half of a fused group, as a C++ condition."""
        if self._fold_live and fz.get("fold"):
            guard = 2.0 ** (float(fz["slack"]) * float(fz["c"]))
            return (f"wir::lazy_softmax_fast_b({self._var(fz['s'])}, {self._var(fz['l_in'])}, "
                    f"{self._var(fz['p'])}, {_flt(guard)})")
        if self.target.rowsum_mfma and self.geo.ms != 32:
            raise LoweringError("rowsum_mfma takes the 32x32 MFMA fragment layout")
        mr = "_mr" if self.target.rowsum_mfma else ""
        return (f"wir::lazy_softmax_fast{mr}({self._var(fz['s'])}, {self._var(fz['m_in'])}, "
                f"{self._var(fz['l_in'])}, {self._var(fz['p'])}, {_flt(fz['c'])}, {_flt(fz['slack'])})")

    def _emit_lazy_softmax(self, plan, out: List[str], depth: int) -> None:
        """m, l and O are updated in place: the group's results m', l', O' name
        the C++ variables of m, l, O from here on (the matcher checked that
        nothing reads m, l, O after the group), so no register tile is copied."""
        pad = "  " * depth
        for src, dst in (("m_in", "m_out"), ("l_in", "l_out"), ("o_in", "o_out")):
            self._var_override[self.resolve(plan[dst].name)] = self._var(plan[src])
        # where the speculative half is known to fail (the first tile, whose running max is
        # -inf) or has just failed (a loop's exit to its exact path), only the exact half runs
        fn = "lazy_softmax_exact" if self._lazy_exact_only else "lazy_softmax"
        folded = self._fold_live and plan.get("fold")
        if self.target.rowsum_mfma and not folded and not self._lazy_exact_only:
            if self.geo.ms != 32:
                raise LoweringError("rowsum_mfma takes the 32x32 MFMA fragment layout")
            fn += "_mr"
        out.append(f"{pad}wir::{fn}{'_b' if folded else ''}({self._var(plan['s'])}, {self._var(plan['m_in'])}, "
                   f"{self._var(plan['l_in'])}, {self._var(plan['o_in'])}, {self._var(plan['p'])}, "
                   f"{_flt(plan['c'])}, {_flt(plan['slack'])}{', wir_sb' if folded else ''});")

    def _emit_exact(self, op: Op, out: List[str], depth: int) -> None:
        """A fused lazy-softmax group with only its exact half."""
        self._lazy_exact_only = True
        self._emit_op(op, out, depth)
        self._lazy_exact_only = False

    # element-wise register-tile ops a slot-fused MMA can carry, and the helpers they lower to
    _SLOT_OPS = (MulScalarOp, Exp2Op, SubOp, MulOp, AddOp, SubRowOp, SubColOp, CopyOp)
    _SLOT_CALL = re.compile(r"^\s*wir::(map|map2|col_apply|row_apply|to_bf16)\((.*)\);$")

    def _slot_form(self, op: Op) -> Optional[Tuple[str, int]]:
        """(helper, MFMA slot count) of an MMA that mma_*_slots can emit, or None."""
        if not isinstance(op, MMAOp) or self.geo.ms != 32:
            return None
        ms, res_t = self.geo.ms, op.result.type
        if op.transpose_b:
            hoisted = self._hoisted.get(self.resolve(op.a.name))
            if hoisted is None or (self._fold_live and id(op) in self._score_folds):
                return None
            return "mma_ABt_frags_slots", hoisted[1] * (res_t.cols // ms)
        a_t = op.a.type
        if (self._is_shared(op.a) or self._lds_key(op.a) is not None or not isinstance(a_t, RegTileType)
                or a_t.data_type != GPUType.bf16):
            return None
        groups = (a_t.cols // ms) * 4   # 4-register groups of a along k
        return "mma_rAB_slots", (groups // 2) * (res_t.cols // ms)

    def _slot_calls(self, op: Op) -> Optional[List[str]]:
        """The element-wise op as wir::*_part calls over register groups
        [WIR_G0, WIR_G1), or None when it is not one this fusion carries."""
        if not isinstance(op, self._SLOT_OPS) or not isinstance(op.result.type, RegTileType):
            return None
        if isinstance(op, CopyOp) and not (isinstance(op.input.type, RegTileType)
                                           and op.input.type.data_type == GPUType.fp32
                                           and op.result.type.data_type == GPUType.bf16):
            return None
        tmp: List[str] = []
        skipped = id(op) in self._slot_skip
        self._slot_skip.discard(id(op))
        try:
            self._emit_op(op, tmp, 0)
        finally:
            if skipped:
                self._slot_skip.add(id(op))
        calls = []
        for line in tmp:
            m = self._SLOT_CALL.match(line)
            if m is None:
                return None
            calls.append(f"wir::{m.group(1)}_part<WIR_G0, WIR_G1>({m.group(2)});")
        return calls

    def _plan_slot_fusion(self, ops: List[Op]) -> None:
        """CDNA4Target.slot_fusion: each slot-capable MMA takes into its MFMA
        slots the element-wise ops it does not depend on (transitively) from
        the contiguous run of element-wise ops and fills right before it, and
        then those right after it (up to the next other op) whose inputs all
        exist before it or come from ops it already took.  Ops that stay
        before the MMA may not read a moved op's result, and every moved op
        has the same register-tile shape (the group partition)."""
        def reads(o):
            return {self.resolve(v.name) for v in _op_values(o) if v is not getattr(o, "result", None)}

        for idx, mma in enumerate(ops):
            form = self._slot_form(mma)
            if form is None or id(mma) in self._slot_work:
                continue
            run = []
            j = idx - 1
            while j >= 0 and (isinstance(ops[j], ZeroOp) or isinstance(ops[j], self._SLOT_OPS)):
                if id(ops[j]) not in self._slot_skip:   # (ops an earlier MMA took are not in the run)
                    run.append(ops[j])
                j -= 1
            need = reads(mma)
            moved = []
            for o in run:   # nearest first
                if self.resolve(o.result.name) in need or isinstance(o, ZeroOp) or self._slot_calls(o) is None:
                    need |= reads(o)
                else:
                    moved.append(o)
            changed = True
            while changed:   # an op that stays must not read a moved result
                changed = False
                stay_reads = set().union(*(reads(o) for o in run if o not in moved)) if run else set()
                for o in list(moved):
                    if self.resolve(o.result.name) in stay_reads:
                        moved.remove(o)
                        changed = True
            moved.sort(key=ops.index)
            # ops after the MMA whose inputs exist before it (or come from ops it took)
            before = {self.resolve(o.result.name) for o in ops[:idx] if isinstance(getattr(o, "result", None), Value)
                      and o not in moved}
            later_moved = []
            k = idx + 1
            while k < len(ops) and isinstance(ops[k], self._SLOT_OPS):
                o = ops[k]
                avail = before | {self.resolve(m.result.name) for m in moved + later_moved}
                if reads(o) <= avail and self._slot_calls(o) is not None:
                    later_moved.append(o)
                k += 1
            moved += later_moved
            # a moved op writes its result while the MMA runs: never into a variable the MMA reads
            mma_vars = {self._var(v) for v in _op_values(mma) if v is not mma.result}
            moved = [o for o in moved if self._var(o.result) not in mma_vars]
            shapes = {(o.result.type.rows, o.result.type.cols) for o in moved}
            if not moved or len(shapes) != 1:
                continue
            rows, cols = shapes.pop()
            self._slot_work[id(mma)] = (moved, (rows // 32) * (cols // 32) * 4, form)
            for o in moved:
                self._slot_skip.add(id(o))

    def _emit_ops(self, ops, out: List[str], depth: int) -> None:
        ops = list(ops)
        if self.target.slot_fusion:
            self._plan_slot_fusion(ops)
        for k, op in enumerate(ops):
            if (isinstance(op, WaitBufOp) and k + 1 < len(ops) and isinstance(ops[k + 1], WaitBufOp)
                    and id(op) not in self._pp_ops and id(ops[k + 1]) not in self._pp_ops):
                # consecutive ring waits (rings of different depths) share one
                # barrier: the last one waits for the fewest loads in flight
                nxt = ops[k + 1]
                self.wait_n[id(nxt)] = min(self.wait_n.get(id(op), 0), self.wait_n.get(id(nxt), 0))
                continue
            self._emit_op(op, out, depth)

    def _emit_op(self, op: Op, out: List[str], depth: int) -> None:  # noqa: C901
        pad = "  " * depth
        ms = self.geo.ms
        w = out.append
        fused = None if self._no_fusion else self._softmax_fused.get(id(op))
        if fused is not None:
            if fused != "skip":
                self._emit_lazy_softmax(fused, out, depth)
            return
        if id(op) in self._slot_skip:
            return   # emitted in the MFMA slots of the MMA after it
        if isinstance(op, (AllocSharedOp, YieldOp, PipelineStageOp)):
            # a pipeline_stage mark is realised by the loop emitters that take
            # its placement; elsewhere the loop runs in program order
            if isinstance(op, YieldOp):
                self._emit_yield(op, out, depth)
            return
        if isinstance(op, ZeroOp) or isinstance(op, NegInftyOp):
            val = "0.f" if isinstance(op, ZeroOp) else "-__builtin_inff()"
            if isinstance(op.result.type, (RegTileType, ColVecType)):
                out.extend(self._consumer_only([f"{pad}wir::fill({self._var(op.result)}, {val});"], pad))
                return
            raise LoweringError(f"{type(op).__name__} on {op.result.type}")
        if isinstance(op, TMALoadOp) and self.resolve(op.result.name) in self._register_tiles:
            name = self.resolve(op.result.name)
            var, ks, rows, _loop = self._register_tiles[name]
            sub = op.source.type.sub_tile_type
            b, d, rt, ct = (self._int(c) for c in op.coords)
            w(f"{pad}wir::RowFrags<{ms}, {rows // ms}, {ks}> {var};")
            w(f"{pad}wir::load_row_frags_global({var}, globals.{_cname(op.source.name)[2:]}, {b}, {d}, "
              f"({rt}) * {sub.rows} + wave_row0, ({ct}) * {sub.cols});")
            self._hoisted[name] = (var, ks)
            return
        if isinstance(op, (TMALoadOp, TMALoadBufOp)):
            if id(op) in self._fused_ids:
                return
            if id(op) in self.war_barrier:
                w(f"{pad}wir::barrier();")
            if isinstance(op, TMALoadOp):
                ptr, key = self._tile_ptr(op.result)
            else:
                ptr, key = self._buf_ptr(op.buf, op.slot)
            src = op.source
            sub = src.type.sub_tile_type
            b, d, rt, ct = (self._int(c) for c in op.coords)
            call = f"{self._load_call(op, 'load<WIR_AL, WIR_INB>(', ptr, key)});"
            if self._ws:
                who = self._ws_issuer(op.buf.name) if isinstance(op, TMALoadBufOp) else "wir_producer"
                w(f"{pad}if ({who}) {call}")
            elif id(op) in self._pp_prologue:
                w(f"{pad}if constexpr (!WIR_AL) {call}   // the ping-pong loads its own prologue")
            else:
                w(f"{pad}{call}")
            return
        pp = self._pp_ops.get(id(op))
        if pp is not None and pp[0] == "skip":
            return
        if pp is not None and pp[0] in ("step", "drain"):
            self._emit_pingpong_mma(op, pp, out, depth)
            return
        if isinstance(op, (WaitOp, WaitBufOp)):
            if isinstance(op, WaitOp) and all(self.resolve(v.name) in self._register_tiles for v in op.values):
                return
            n = self.wait_n.get(id(op), 0)
            w(f"{pad}{self._ws_wait(n)}" if self._ws else f"{pad}wir::wait_vm_barrier<{n}>();")
            return
        if isinstance(op, SlotViewOp):
            return  # views are resolved to LDS pointers where they are read
        if isinstance(op, MMAOp):
            self._emit_mma(op, out, depth)
            return
        if isinstance(op, MMABufOp):
            a_ptr, a_key = self._buf_ptr(op.a_buf, op.a_slot)
            b_ptr, b_key = self._buf_ptr(op.b_buf, op.b_slot)
            t = self._rtype(op.accum)
            acc = self._var(op.accum)
            pipe = self._rotated.get(id(op))
            if pipe is not None:
                loads = self._fused_loads.get(id(op), [])
                calls, total = [], 0
                pcalls, ptotal = [], 0   # warp-specialised: the DMA waves' share
                for n_ld, ld in enumerate(loads):
                    lptr, lkey = self._buf_ptr(ld.buf, ld.slot)
                    n = self.loads_per_wave(ld.buf.type.tile_type)
                    loader = f"wir::Loader<{self.stile(lkey)}, {self.geo.nw}>"
                    g = f"globals.{_cname(ld.source.name)[2:]}"
                    sub = ld.source.type.sub_tile_type
                    bb, dd, rt, ct = (self._int(c) for c in ld.coords)
                    self._aligned_checks.add((self.stile(lkey), _cname(ld.source.name)[2:]))
                    w(f"{pad}const auto src{n_ld}_ = {loader}::prep<WIR_AL, WIR_INB>({g}, {bb}, {dd}, ({rt}) * {sub.rows}, "
                      f"({ct}) * {sub.cols});")
                    if self._ws and self.resolve(ld.buf.name) in self._ws_producer_streams:
                        pcalls.append(f"if (q >= {ptotal} && q < {ptotal + n}) {loader}::issue<WIR_AL, WIR_INB>(q - {ptotal}, "
                                      f"{lptr}, {g}, src{n_ld}_, wir_wave);")
                        ptotal += n
                        continue
                    calls.append(f"if (q >= {total} && q < {total + n}) {loader}::issue<WIR_AL, WIR_INB>(q - {total}, "
                                 f"{lptr}, {g}, src{n_ld}_, wir_wave);")
                    total += n
                if self._ws:
                    # the DMA waves issue their streams back to back; the MFMA waves
                    # run the MFMAs, spreading any streams assigned to them
                    w(f"{pad}if (wir_producer) {{")
                    w(f"{pad}  for (int q = 0; q < {ptotal}; ++q) {{")
                    for c in pcalls:
                        w(f"{pad}    {c}")
                    w(f"{pad}  }}")
                    w(f"{pad}}} else {{")
                    w(f"{pad}  {pipe}.run<{total}>({acc}, {a_ptr}, wave_row0, {b_ptr}, wave_col0, [&](int q) {{")
                    for c in calls:
                        w(f"{pad}    {c}")
                    w(f"{pad}  }});")
                    w(f"{pad}}}")
                else:
                    whole = ", true" if self.target.dma_spread_whole else ""
                    w(f"{pad}{pipe}.run<{total}{whole}>({acc}, {a_ptr}, wave_row0, {b_ptr}, wave_col0, [&](int q) {{")
                    for c in calls:
                        w(f"{pad}  {c}")
                    w(f"{pad}}});")
            else:
                out.extend(self._consumer_only(
                    [f"{pad}wir::mma_AB<{ms}, {t.rows}, {t.cols}, {self.stile(a_key)}, {self.stile(b_key)}>"
                     f"({acc}, {a_ptr}, wave_row0, {b_ptr}, wave_col0);"], pad))
            if self._var(op.result) != acc:
                w(f"{pad}{self._var(op.result)} = {acc};")
            if isinstance(op.a_slot, BufSlotExpr):
                self.drain_modulus = op.a_slot.modulus
                w(f"{pad}{self._drain_advance(op)}")
            return
        if isinstance(op, CopyOp):
            rt, it = op.result.type, op.input.type
            if isinstance(it, SharedTileType) and isinstance(rt, RegTileType):
                if rt.data_type != GPUType.fp32:
                    raise LoweringError("a shared -> register copy produces an fp32 register tile")
                ptr, key = self._tile_ptr(op.input)
                w(f"{pad}wir::load_tile<{self.stile(key)}>({self._var(op.result)}, {ptr}, wave_row0, wave_col0);")
                return
            if isinstance(rt, RegTileType) and isinstance(it, RegTileType) and rt.data_type != it.data_type:
                if it.data_type != GPUType.fp32:
                    raise LoweringError("only fp32 -> bf16 register conversion is supported")
                w(f"{pad}wir::to_bf16({self._var(op.result)}, {self._var(op.input)});")
            elif self._var(op.result) != self._var(op.input):
                w(f"{pad}{self._var(op.result)} = {self._var(op.input)};")
            return
        if isinstance(op, (MulScalarOp, Exp2Op, Log2Op)):
            fn = {MulScalarOp: f"x * {_flt(getattr(op, 'scalar', 0.0))}",
                  Exp2Op: "__builtin_amdgcn_exp2f(x)", Log2Op: "__builtin_amdgcn_logf(x)"}[type(op)]
            if isinstance(op.result.type, RegTileType):
                w(f"{pad}wir::map({self._var(op.result)}, {self._var(op.input)}, "
                  f"[](float x, int) {{ return {fn}; }});")
            else:
                vm = "cvmap" if isinstance(op.result.type, RowVecType) else "vmap"
                w(f"{pad}wir::{vm}({self._var(op.result)}, {self._var(op.input)}, [](float x) {{ return {fn}; }});")
            return
        if isinstance(op, (SubOp, MulOp, AddOp)):
            sym = {SubOp: "-", MulOp: "*", AddOp: "+"}[type(op)]
            fn = {RegTileType: "map2", RowVecType: "cvmap2"}.get(type(op.result.type), "vmap2")
            w(f"{pad}wir::{fn}({self._var(op.result)}, {self._var(op.a)}, {self._var(op.b)}, "
              f"[](float a, float b) {{ return a {sym} b; }});")
            return
        if isinstance(op, LazyMaxOp):
            fn = {RowVecType: "cvmap2"}.get(type(op.result.type), "vmap2")
            w(f"{pad}wir::{fn}({self._var(op.result)}, {self._var(op.prev)}, {self._var(op.cand)}, "
              f"[](float p, float c) {{ return c > p + {_flt(op.slack)} ? c : p; }});")
            return
        if isinstance(op, (RowMaxOp, RowSumOp)):
            red = "wir::OpMax()" if isinstance(op, RowMaxOp) else "wir::OpAdd()"
            w(f"{pad}wir::row_reduce({self._var(op.result)}, {self._var(op.tile)}, {self._var(op.prev)}, {red});")
            return
        if isinstance(op, (SubRowOp, MulRowOp, DivRowOp)):
            if isinstance(op, DivRowOp):
                w(f"{pad}{{ wir::RVec<{ms}, {op.vec.type.rows}> rcp_; "
                  f"wir::vmap(rcp_, {self._var(op.vec)}, [](float x) {{ return 1.0f / x; }});")
                w(f"{pad}  wir::row_apply({self._var(op.result)}, {self._var(op.tile)}, rcp_, "
                  f"[](float x, float s) {{ return x * s; }}); }}")
                return
            if isinstance(op, MulRowOp):
                w(f"{pad}wir::row_scale({self._var(op.result)}, {self._var(op.tile)}, {self._var(op.vec)});")
                return
            w(f"{pad}wir::row_apply({self._var(op.result)}, {self._var(op.tile)}, {self._var(op.vec)}, "
              f"[](float x, float s) {{ return x - s; }});")
            return
        if isinstance(op, SubColOp):
            w(f"{pad}wir::col_apply({self._var(op.result)}, {self._var(op.tile)}, {self._var(op.vec)}, "
              f"[](float x, float s) {{ return x - s; }});")
            return
        if isinstance(op, LoadVecOp) and isinstance(op.source.type, SharedTileType):
            ptr, _key = self._tile_ptr(op.source)
            if isinstance(op.result.type, RowVecType):
                w(f"{pad}wir::load_cvec_lds({self._var(op.result)}, {ptr}, wave_col0);")
            elif isinstance(op.result.type, ColVecType):
                w(f"{pad}wir::load_rvec_lds({self._var(op.result)}, {ptr}, wave_row0);")
            else:
                raise LoweringError(f"load_vec into {op.result.type}")
            return
        if isinstance(op, LoadVecOp):
            src = op.source
            if src.type.data_type != GPUType.fp32 or src.type.sub_tile_type.cols != 1:
                raise LoweringError(f"load_vec reads an fp32 global with L x 1 sub tiles, not {src.type}")
            n = src.type.sub_tile_type.rows
            b, d, rt, _ct = (self._int(c) for c in op.coords)
            g = f"globals.{_cname(src.name)[2:]}"
            if isinstance(op.result.type, RowVecType):
                w(f"{pad}wir::load_cvec({self._var(op.result)}, {g}, {b}, {d}, ({rt}) * {n} + wave_col0);")
            elif isinstance(op.result.type, ColVecType):
                w(f"{pad}wir::load_rvec({self._var(op.result)}, {g}, {b}, {d}, ({rt}) * {n} + wave_row0);")
            else:
                raise LoweringError(f"load_vec into {op.result.type}")
            return
        if isinstance(op, CausalMaskOp):
            t = op.tile.type
            br, bc = t.rows * (self.geo.nw // self.geo.nw_c), t.cols * self.geo.nw_c
            w(f"{pad}wir::causal_mask<{'true' if op.transposed else 'false'}>({self._var(op.result)}, "
              f"{self._var(op.tile)}, "
              f"({self._int(op.row_tile)}) * {br} + wave_row0, ({self._int(op.col_tile)}) * {bc} + wave_col0);")
            return
        if isinstance(op, IntAffineOp):
            w(f"{pad}const int {self._var(op.result)} = ({self._int(op.input)}) * {op.mul} + {op.add};")
            return
        if isinstance(op, IntDivOp):
            w(f"{pad}const int {self._var(op.result)} = ({self._int(op.input)}) / ({self._int(op.divisor)});")
            return
        if isinstance(op, DrainIndexOp):
            w(f"{pad}const int {self._var(op.result)} = wir_drain + {op.offset};")
            return
        if isinstance(op, TMAStoreOp):
            self._emit_store(op, out, depth)
            return
        if isinstance(op, ReduceSlicesOp):
            self._emit_reduce_slices(op, out, depth)
            return
        if isinstance(op, ForOp):
            self._emit_for(op, out, depth)
            return
        raise LoweringError(f"no CDNA4 lowering for {type(op).__name__}")

    def _load_call(self, op, fn: str, ptr: str, key: str) -> str:
        src = op.source
        sub = src.type.sub_tile_type
        b, d, rt, ct = (self._int(c) for c in op.coords)
        t = self.tile_type_of(key)
        if _is_vec_tile(t):
            return (f"wir::VecLoader<{t.rows}, {self.geo.nw}>::{fn}{ptr}, globals.{_cname(src.name)[2:]}, "
                    f"{b}, {d}, ({rt}) * {sub.rows}, wir_wave")
        self._aligned_checks.add((self.stile(key), _cname(src.name)[2:]))
        return (f"wir::Loader<{self.stile(key)}, {self.geo.nw}>::{fn}{ptr}, globals.{_cname(src.name)[2:]}, "
                f"{b}, {d}, ({rt}) * {sub.rows}, ({ct}) * {sub.cols}, wir_wave")

    def _emit_pingpong_mma(self, op: MMABufOp, pp, out: List[str], depth: int) -> None:
        pad = "  " * depth
        role, name, extra = pp
        a_ptr, _ = self._buf_ptr(op.a_buf, op.a_slot)
        b_ptr, _ = self._buf_ptr(op.b_buf, op.b_slot)
        acc = self._var(op.accum)
        if role == "step":
            vm, per4, loads = extra
            calls, total = [], 0
            for n_ld, ld in enumerate(loads):
                lptr, lkey = self._buf_ptr(ld.buf, ld.slot)
                n = self.loads_per_wave(ld.buf.type.tile_type) * self.geo.nw // 4
                loader = f"wir::Loader<{self.stile(lkey)}, 4>"
                g = f"globals.{_cname(ld.source.name)[2:]}"
                sub = ld.source.type.sub_tile_type
                bb, dd, rt, ct = (self._int(c) for c in ld.coords)
                self._aligned_checks.add((self.stile(lkey), _cname(ld.source.name)[2:]))
                out.append(f"{pad}const auto src{n_ld}_ = {loader}::prep<WIR_AL, WIR_INB>({g}, {bb}, {dd}, ({rt}) * {sub.rows}, "
                           f"({ct}) * {sub.cols});")
                calls.append(f"if (q >= {total} && q < {total + n}) {loader}::issue<WIR_AL, WIR_INB>(q - {total}, "
                             f"{lptr}, {g}, src{n_ld}_, wir_wave & 3);")
                total += n
            out.append(f"{pad}{name}.step<{vm}, {total}>({acc}, {a_ptr}, wave_row0, {b_ptr}, wave_col0, [&](int q) {{")
            for c in calls:
                out.append(f"{pad}  {c}")
            out.append(f"{pad}}});")
        else:
            vm, last = extra
            out.append(f"{pad}{name}.step<{vm}, 0>({acc}, {a_ptr}, wave_row0, {b_ptr}, wave_col0, [&](int) {{}});")
            if last:
                out.append(f"{pad}{name}.finish({acc});")
        if self._var(op.result) != acc:
            out.append(f"{pad}{self._var(op.result)} = {acc};")
        if isinstance(op.a_slot, BufSlotExpr):
            out.append(f"{pad}{self._drain_advance(op)}")

    def _drain_advance(self, op: MMABufOp) -> str:
        if self._drain_unreduced:
            return "wir_drain += 1;"
        return f"wir_drain = (wir_drain + 1) % {op.a_slot.modulus};"

    def _emit_yield(self, op: YieldOp, out: List[str], depth: int) -> None:
        pad = "  " * depth
        loop = self._loop_of_yield[id(op)]
        for k, v in enumerate(op.values):
            dst = self._var(loop.iter_args[k].block_arg)
            if self._var(v) != dst:
                out.append(f"{pad}{dst} = {self._var(v)};")

    def _emit_mma(self, op: MMAOp, out: List[str], depth: int) -> None:
        pad = "  " * depth
        ms = self.geo.ms
        res_t = op.result.type
        res = self._var(op.result)
        b_ptr, b_key = self._tile_ptr(op.b)
        if id(op) in self._slot_work:
            moved, ngroups, (helper, nslots) = self._slot_work[id(op)]
            calls = [c for o in moved for c in self._slot_calls(o)]
            if op.transpose_b:
                frags, ks = self._hoisted[self.resolve(op.a.name)]
                head = (f"wir::{helper}<{ms}, {res_t.rows}, {res_t.cols}, {self.stile(b_key)}, {ks}>"
                        f"({res}, {frags}, {b_ptr}, wave_col0, [&](auto wir_t) {{")
            else:
                acc = self._var(op.accum)
                if acc != res:
                    out.append(f"{pad}{res} = {acc};")
                a_t = op.a.type
                head = (f"wir::{helper}<{ms}, {a_t.rows}, {a_t.cols}, {res_t.cols}, {self.stile(b_key)}>"
                        f"({res}, {self._var(op.a)}, {b_ptr}, wave_col0, [&](auto wir_t) {{")
            out.append(f"{pad}{head}   // {len(moved)} element-wise ops in the MFMA slots")
            out.append(f"{pad}  constexpr int WIR_G0 = decltype(wir_t)::value * {ngroups} / {nslots};")
            out.append(f"{pad}  constexpr int WIR_G1 = (decltype(wir_t)::value + 1) * {ngroups} / {nslots};")
            out.extend(f"{pad}  {c}" for c in calls)
            out.append(f"{pad}}});")
            return
        if op.transpose_b:
            hoisted = self._hoisted.get(self.resolve(op.a.name))
            if hoisted is not None:
                if self._fold_live and id(op) in self._score_folds:
                    out.append(f"{pad}wir::mma_ABt_frags_bias<{ms}, {res_t.rows}, {res_t.cols}, "
                               f"{self.stile(b_key)}, {hoisted[1]}>({res}, {hoisted[0]}, wir_sb, {b_ptr}, wave_col0);")
                    return
                out.append(f"{pad}wir::mma_ABt_frags<{ms}, {res_t.rows}, {res_t.cols}, {self.stile(b_key)}, "
                           f"{hoisted[1]}>({res}, {hoisted[0]}, {b_ptr}, wave_col0);")
                return
            a_ptr, a_key = self._tile_ptr(op.a)
            out.append(f"{pad}wir::mma_ABt<{ms}, {res_t.rows}, {res_t.cols}, {self.stile(a_key)}, "
                       f"{self.stile(b_key)}>({res}, {a_ptr}, wave_row0, {b_ptr}, wave_col0);")
            return
        acc = self._var(op.accum)
        if acc != res:
            out.append(f"{pad}{res} = {acc};")
        if self._is_shared(op.a) or self._lds_key(op.a) is not None:
            a_ptr, a_key = self._tile_ptr(op.a)
            out.append(f"{pad}wir::mma_AB<{ms}, {res_t.rows}, {res_t.cols}, {self.stile(a_key)}, "
                       f"{self.stile(b_key)}>({res}, {a_ptr}, wave_row0, {b_ptr}, wave_col0);")
            return
        a_t = op.a.type
        if not (isinstance(a_t, RegTileType) and a_t.data_type == GPUType.bf16):
            raise LoweringError(f"MMA operand {op.a!r} must be a shared tile or a bf16 register tile")
        out.append(f"{pad}wir::mma_rAB<{ms}, {a_t.rows}, {a_t.cols}, {res_t.cols}, {self.stile(b_key)}>"
                   f"({res}, {self._var(op.a)}, {b_ptr}, wave_col0);")

    def _emit_store(self, op: TMAStoreOp, out: List[str], depth: int) -> None:
        pad = "  " * depth
        dest = op.dest
        if not isinstance(dest.type, GlobalType):
            raise LoweringError("tma_store destination must be a global")
        sub = dest.type.sub_tile_type
        b, d, rt, ct = (self._int(c) for c in op.coords)
        g = f"globals.{_cname(dest.name)[2:]}"
        st = self._rtype(op.source)
        if isinstance(st, RegTileType) and id(op) in self._staged:
            if not self._stage_barrier_done:
                # the loop's last prefetches (tiles past its end, or past a causal stop) may still be
                # landing in the ring: drain this wave's DMAs before any wave reuses the LDS
                out.append(f"{pad}wir::wait_vm_barrier<0>();  // ring buffers dead: LDS becomes per-wave staging")
                self._stage_barrier_done = True
            out.extend(self._consumer_only(
                [f"{pad}wir::store_tile_staged{'<true>' if self.target.nontemporal_stores else ''}"
                 f"({g}, {self._var(op.source)}, {b}, {d}, "
                 f"({rt}) * {sub.rows} + wave_row0, ({ct}) * {sub.cols} + wave_col0, "
                 f"smem + wir_wave * {self._staged[id(op)]});"], pad))
        elif isinstance(st, RegTileType):
            out.extend(self._consumer_only(
                [f"{pad}wir::store_tile({g}, {self._var(op.source)}, {b}, {d}, "
                 f"({rt}) * {sub.rows} + wave_row0, ({ct}) * {sub.cols} + wave_col0);"], pad))
        elif isinstance(st, ColVecType):
            out.append(f"{pad}if (wave_col0 == 0) wir::store_vec({g}, {self._var(op.source)}, {b}, {d}, "
                       f"({rt}) * {sub.rows} + wave_row0, ({ct}) * {sub.cols});")
        else:
            raise LoweringError("tma_store of a shared tile is not supported by the CDNA4 target")

    def _emit_reduce_slices(self, op: ReduceSlicesOp, out: List[str], depth: int) -> None:
        """Split-K fix-up after the partial store (``wir::reduce_slices``): the
        tile's counter is ``row_tile * ceil(N / TC) + col_tile``."""
        pad = "  " * depth
        part, dest, arr = op.partials, op.dest, op.arrivals
        if (part.type.data_type != GPUType.fp32 or dest.type.data_type != GPUType.bf16
                or arr.type.data_type != GPUType.u32):
            raise LoweringError("reduce_slices sums fp32 partials into a bf16 global with u32 arrivals")
        sub = dest.type.sub_tile_type
        b, _d, rt, ct = (self._int(c) for c in op.coords)
        g = lambda v: f"globals.{_cname(v.name)[2:]}"   # noqa: E731
        idx = f"({rt}) * (({g(dest)}.c + {sub.cols - 1}) / {sub.cols}) + ({ct})"
        out.append(f"{pad}wir::reduce_slices<{sub.rows}, {sub.cols}, {self.num_threads}>({g(part)}, {g(dest)}, "
                   f"{g(arr)}, {b}, ({rt}) * {sub.rows}, ({ct}) * {sub.cols}, {idx}, smem);")

    def _emit_for(self, op: ForOp, out: List[str], depth: int) -> None:
        pad = "  " * depth
        for name, (var, ks, rows, loop) in self._pending_hoist.items():
            if loop is op and name not in self._register_tiles:
                ptr, key = self._tile_ptr(self.values[name])
                out.append(f"{pad}wir::RowFrags<{self.geo.ms}, {rows // self.geo.ms}, {ks}> {var};")
                out.append(f"{pad}wir::load_row_frags<{self.stile(key)}>({var}, {ptr}, wave_row0);")
                self._hoisted[name] = (var, ks)
        for inner in op.body:
            if isinstance(inner, YieldOp):
                self._loop_of_yield[id(inner)] = op
        stop = self._int(op.stop)
        if op.tile_size:
            stop = f"(({stop}) + {op.tile_size - 1}) / {op.tile_size}"
        iv = self._var(op.induction_var)
        if self._emit_attention_overlap(op, stop, out, depth):
            return
        if self._emit_attention_pingpong(op, stop, out, depth):
            return
        if self._setup_pingpong(op, out, depth):
            self._emit_loop(op, stop, out, depth)
            return
        rotated = self._rotatable(op)
        if rotated is not None:
            mma, pipe_t = rotated
            name = f"pipe{len(self._rotated)}"
            self._rotated[id(mma)] = name
            loads = [o for o in op.body if isinstance(o, TMALoadBufOp)]
            if not any(id(o) in self.war_barrier for o in loads):
                self._fused_loads[id(mma)] = loads
                self._fused_ids |= {id(o) for o in loads}
            out.append(f"{pad}{pipe_t} {name};")
            out.extend(self._consumer_only([f"{pad}{name}.init();"], pad))
        self._emit_loop(op, stop, out, depth)
        if rotated is not None:
            out.extend(self._consumer_only(
                [f"{pad}{self._rotated[id(rotated[0])]}.finish({self._var(rotated[0].accum)});"], pad))

    def _ring_modulus(self, loop: ForOp) -> Optional[int]:
        """Slot count of the ring slots this loop indexes by its induction
        variable; for rings of different depths, their least common multiple
        (the period after which every slot index repeats)."""
        iv = self.resolve(loop.induction_var.name)
        mods = set()
        for o in loop.body:
            for f in vars(o).values():
                if isinstance(f, BufSlotExpr) and f.value is not None and self.resolve(f.value.name) == iv:
                    mods.add(f.modulus)
        if not mods:
            return None
        m = 1
        for x in mods:
            m = m * x // math.gcd(m, x)
        return m

    def _emit_loop(self, op: ForOp, stop: str, out: List[str], depth: int, mve: bool = True) -> None:
        """Emit the loop; ring loops are unrolled by their slot count S
        (modulo variable expansion) when the start is a constant and the step
        is 1: copy u of the body sees the constant slot (start + u + offset)
        % S, so LDS addresses fold into instruction offsets.  A remainder loop
        with run-time slots finishes the last (trips mod S) iterations.
        ``mve=False`` keeps one copy of the body (run-time slots)."""
        pad = "  " * depth
        iv = self._var(op.induction_var)
        ivn = self.resolve(op.induction_var.name)
        body = list(op.body)
        fused_at = next((k for k, o in enumerate(body) if isinstance(self._softmax_fused.get(id(o)), dict)), None)
        if fused_at is not None and not self._no_fusion:
            self._emit_loop_lazy(op, stop, out, depth, fused_at)
            return
        m = self._ring_modulus(op) if self.target.mve and mve else None
        # one ring size: unroll up to 4 copies; rings of different depths: up to their period 6
        m_max = 4 if m is None or len({f.modulus for o in op.body for f in vars(o).values()
                                        if isinstance(f, BufSlotExpr) and f.value is not None}) == 1 else 6
        if m is None or m < 2 or m > m_max or not isinstance(op.start, int) or op.step != 1:
            out.append(f"{pad}for (int {iv} = {self._int(op.start)}; {iv} < {stop}; {iv} += {self._int(op.step)}) {{")
            self._emit_ops(op.body, out, depth + 1)
            out.append(f"{pad}}}")
            return
        base = f"wir_base_{iv[2:]}"
        out.append(f"{pad}int {base} = {op.start};")
        # only the aligned body unrolls: the checked body's per-chunk bounds state times m copies
        # spilled (gemm_256_k64: 11 VGPRs, 43 SGPRs), and it runs every trip in the remainder loop
        out.append(f"{pad}for (; WIR_AL && {base} + {m} <= ({stop}); {base} += {m}) {{")
        for u in range(m):
            self._slot_const[ivn] = (op.start + u) % m
            out.append(f"{pad}  {{")
            out.append(f"{pad}    const int {iv} = {base} + {u};")
            self._emit_ops(op.body, out, depth + 2)
            out.append(f"{pad}  }}")
        del self._slot_const[ivn]
        out.append(f"{pad}}}")
        out.append(f"{pad}for (int {iv} = {base}; {iv} < {stop}; {iv} += 1) {{")
        self._emit_ops(op.body, out, depth + 1)
        out.append(f"{pad}}}")

    def _emit_loop_lazy(self, op: ForOp, stop: str, out: List[str], depth: int, fused_at: int) -> None:
        """A loop whose body holds a lazy softmax step (``_match_lazy_softmax``):
        the inner loop runs the step's speculative half and leaves for the exact
        path, which an outer loop runs before re-entering, so inside the inner
        loop the O accumulator is touched only by its MFMAs and keeps one
        register assignment.  The first iteration always takes the exact path
        (the running max starts at -inf), so it is peeled.

        When the ops after the step are a ``pipeline_stage(1)`` mark, the PV
        MMA (reading this iteration's ring slot) and the yield -- kernel_pass
        placed the PV one stage later -- the PV is rotated to the top of the
        next iteration, ahead of its wait: the exact path is then the softmax
        step alone, and the prefetch that overwrites that slot still comes
        after the barrier that follows the PV."""
        pad = "  " * depth
        q = pad + "  "
        iv = self._var(op.induction_var)
        ivn = self.resolve(op.induction_var.name)
        body = list(op.body)
        fz = self._softmax_fused[id(body[fused_at])]
        pre = body[:fused_at]
        post = [o for o in body[fused_at + 1:] if self._softmax_fused.get(id(o)) != "skip"]
        # kernel_pass's placement: a pipeline_stage(1) in front of the PV MMA
        rotate = (isinstance(op.start, int) and op.step == 1 and len(post) == 3
                  and isinstance(post[0], PipelineStageOp) and post[0].stage == 1 and isinstance(post[1], MMAOp)
                  and isinstance(post[2], YieldOp) and not post[1].transpose_b
                  and isinstance(pre[0], (WaitBufOp, WaitOp)))
        if rotate:
            post = post[1:]

        def fast_call(d: int) -> None:
            qq = "  " * d
            out.append(f"{qq}if (!{self._fast_call(fz)}) {{")
            out.append(f"{qq}  wir_exact = true;")
            out.append(f"{qq}  break;")
            out.append(f"{qq}}}")

        out.append(f"{pad}{{")
        was_live = self._fold_live
        self._fold_preamble(op.body, out, depth + 1)
        try:
            self._emit_loop_lazy_body(op, stop, out, depth, fused_at, fz, pre, post, rotate, fast_call)
        finally:
            self._fold_live = was_live

    def _emit_loop_lazy_body(self, op, stop, out, depth, fused_at, fz, pre, post, rotate, fast_call) -> None:
        pad = "  " * depth
        q = pad + "  "
        iv = self._var(op.induction_var)
        ivn = self.resolve(op.induction_var.name)
        body = list(op.body)

        def shifted_post(d: int) -> None:
            self._slot_shift[ivn] = self._slot_shift.get(ivn, 0) - 1
            self._emit_ops(post, out, d)
            self._slot_shift[ivn] += 1
            if self._slot_shift[ivn] == 0:
                del self._slot_shift[ivn]

        if not rotate:
            out.append(f"{q}int {iv} = {self._int(op.start)};")
            out.append(f"{q}for (;;) {{")
            out.append(f"{q}  bool wir_exact = false;")
            out.append(f"{q}  for (; {iv} < {stop}; {iv} += {self._int(op.step)}) {{")
            self._emit_ops(pre, out, depth + 3)
            fast_call(depth + 3)
            for src, dst in (("m_in", "m_out"), ("l_in", "l_out"), ("o_in", "o_out")):
                self._var_override[self.resolve(fz[dst].name)] = self._var(fz[src])
            self._emit_ops(post, out, depth + 3)
            out.append(f"{q}  }}")
            out.append(f"{q}  if (!wir_exact) break;")
            self._emit_exact(body[fused_at], out, depth + 2)
            self._emit_ops(post, out, depth + 2)
            out.append(f"{q}  {iv} += {self._int(op.step)};")
            out.append(f"{q}}}")
            out.append(f"{pad}}}")
            return
        start = op.start
        # One guard around the peeled first tile, the loop and the last PV:
        # the loop is then entered only through the first tile's block, whose
        # MFMAs already wait for the register-hoisted global fragments, so the
        # compiler sees them complete at the loop head and puts no vmcnt(0)
        # (which would also wait for this wave's ring DMAs) inside the loop.
        q2 = q + "  "
        out.append(f"{q}if (({stop}) > {start}) {{")
        out.append(f"{q2}{{")
        out.append(f"{q2}  const int {iv} = {start};")
        self._emit_ops(pre, out, depth + 3)
        self._emit_exact(body[fused_at], out, depth + 3)   # the running max starts at -inf
        out.append(f"{q2}}}")
        out.append(f"{q2}int {iv} = ({start}) + 1;")
        out.append(f"{q2}for (;;) {{")
        out.append(f"{q2}  bool wir_exact = false;")
        out.append(f"{q2}  for (; {iv} < {stop}; ++{iv}) {{")
        shifted_post(depth + 4)      # PV of the previous iteration
        self._emit_ops(pre, out, depth + 4)
        fast_call(depth + 4)
        out.append(f"{q2}  }}")
        out.append(f"{q2}  if (!wir_exact) break;")
        self._emit_exact(body[fused_at], out, depth + 3)
        out.append(f"{q2}  ++{iv};")
        out.append(f"{q2}}}")
        out.append(f"{q2}{{")
        out.append(f"{q2}  const int {iv} = ({stop});")
        shifted_post(depth + 3)      # PV of the last iteration
        out.append(f"{q2}}}")
        out.append(f"{q}}}")
        out.append(f"{pad}}}")

    def _attention_pingpong_plan(self, loop: ForOp):
        """Match the prefetch-form attention loop that the ping-pong emitter
        takes: wait on slot i, the slot views, a first MMA with B^T from
        ring K, VALU ops, a last MMA (bf16 register A, B from ring V) whose
        result is carried in place, and one prefetch load per ring into slot
        i + S - 1 with S >= 3."""
        if not self.target.pingpong or self.geo.nw != 8 or loop not in list(self.kernel.body):
            return None
        body = list(loop.body)
        if not body or not isinstance(body[0], WaitBufOp) or not isinstance(body[-1], YieldOp):
            return None
        mmas = [o for o in body if isinstance(o, MMAOp)]
        if len(mmas) != 2 or not mmas[0].transpose_b or mmas[1].transpose_b or body[-2] is not mmas[1]:
            return None
        # the placement kernel_pass marks: the PV MMA one stage behind the rest
        # (it runs at the top of the next iteration, beside S = Q K^T)
        if not (isinstance(body[-3], PipelineStageOp) and body[-3].stage == 1):
            return None
        if any(isinstance(o, PipelineStageOp) for o in body[:-3]):
            return None
        qk, pv = mmas
        views = self._views()
        vk, vv = views.get(self.resolve(qk.b.name)), views.get(self.resolve(pv.b.name))
        if vk is None or vv is None or vk.buf == vv.buf:
            return None
        loads = [o for o in body if isinstance(o, TMALoadBufOp)]
        if sorted(self.resolve(o.buf.name) for o in loads) != sorted(
                [self.resolve(vk.buf.name), self.resolve(vv.buf.name)]):
            return None
        ivn = self.resolve(loop.induction_var.name)
        mods = {o.slot.modulus for o in loads} | {vk.slot.modulus, vv.slot.modulus, body[0].slot.modulus}
        if len(mods) != 1:
            return None
        S = mods.pop()
        if S < 3 or not isinstance(loop.start, int) or loop.step != 1:
            return None
        for o in loads:
            if not (isinstance(o.slot, BufSlotExpr) and o.slot.value is not None
                    and self.resolve(o.slot.value.name) == ivn and o.slot.offset % S == S - 1):
                return None
            t = o.buf.type.tile_type
            if (t.rows * t.cols * 2 // 1024) % 4:
                return None
        for v in (vk, vv):
            if self.resolve(v.slot.value.name) != ivn or v.slot.offset % S:
                return None
        affine = [o for o in body if isinstance(o, IntAffineOp)]
        if len(affine) != 1 or affine[0].mul != 1 or affine[0].add != S - 1:
            return None
        mid = body[body.index(qk) + 1: body.index(pv) - 1]
        lds_ops = (TMALoadOp, WaitOp, WaitBufOp, MMAOp, MMABufOp, SlotViewOp, ForOp)
        if any(isinstance(o, lds_ops) for o in mid):
            return None
        yld = body[-1]
        k = list(yld.values).index(pv.result) if pv.result in yld.values else -1
        if k < 0 or self._var(loop.iter_args[k].block_arg) != self._var(pv.result):
            return None
        softmax = [o for o in mid if not isinstance(o, (TMALoadBufOp, IntAffineOp))]
        k_load = next(o for o in loads if o.buf == vk.buf)
        v_load = next(o for o in loads if o.buf == vv.buf)
        return dict(S=S, qk=qk, pv=pv, softmax=softmax, k_load=k_load, v_load=v_load, affine=affine[0],
                    yld=yld)

    def _pingpong_form(self, loop: ForOp):
        """``(plan, swap, one, every)`` when the attention ping-pong emitter
        takes *loop* (its plan, the wave group of the K stream, the
        one-barrier form, the iterations per barrier), else None."""
        one = self.target.pingpong_one_barrier
        every = self.target.pingpong_barrier_every if one else 1
        if every not in (1, 2):
            raise LoweringError(f"pingpong_barrier_every must be 1 or 2, not {every}")
        if self.target.pingpong_split_barrier and not (one and every == 1):
            raise LoweringError("pingpong_split_barrier takes the one-barrier ping-pong with a barrier "
                                "every iteration")
        plan = self._attention_pingpong_plan(loop)
        if plan is None or plan["S"] < (4 if every == 1 else 5):
            return None

        def per(ld) -> int:   # DMAs per wave of one tile, four waves issuing
            t = ld.buf.type.tile_type
            return t.rows * t.cols * 2 // 1024 // 4
        if per(plan["k_load"]) != per(plan["v_load"]):
            return None
        swap = self._pingpong_group_swap(plan)
        if swap is None:
            return None
        return plan, swap, one, every

    def _pingpong_group_swap(self, plan) -> Optional[int]:
        """Which physical wave group (0: waves 0-3, 1: waves 4-7) issues the K
        stream -- the role that runs its MFMA phase first -- as the warp
        assignment says.  The V stream must be on the other group; None
        when it is not (the ping-pong form cannot realise that assignment)."""
        def stream(ld) -> str:
            return ld.buf.name[:-len("_bufs")] if ld.buf.name.endswith("_bufs") else ld.buf.name
        ks, vs = stream(plan["k_load"]), stream(plan["v_load"])
        groups = self.target.wave_groups
        if groups is None:
            from warpir_amd.passes.warp_assigner import assign_waves
            sol = assign_waves(self.kernel, num_warps=2, iterations=ASSIGN_ITERATIONS)
            if sol is None:
                return None
            groups = {t[:-len("_load")]: w for t, w in sol.type_warp.items() if t.endswith("_load")}
        if ks not in groups or vs not in groups or groups[ks] == groups[vs]:
            return None
        return groups[ks]

    def _emit_attention_pingpong(self, loop: ForOp, stop: str, out: List[str], depth: int) -> bool:
        """Eight-wavefront attention in ping-pong form.

        Wave groups A and B (waves 0-3 and 4-7, in the order the warp
        assignment gives) share the SIMDs pairwise and run one phase apart, so
        one group's MFMA phase overlaps the other group's softmax (VALU)
        phase.  Iteration i of a group is
          M(i): O += P_{i-1} V_{i-1} (the PV MMA of the previous iteration,
                rotated), then S_i = Q K_i^T;
          V(i): the online-softmax ops of iteration i, and this group's share
                of the ring loads.
        Group A runs M(i) while group B runs V(i-1).  A barrier is
        ``vmcnt(L)`` and a workgroup barrier, L the loads one wave issues per
        tile.  With ``pingpong_one_barrier`` each wave passes one barrier per
        iteration -- group A after its V phase, group B after its M phase --
        so between two barriers A runs M(i), V(i) and B runs V(i-1), M(i),
        and neither group waits for the other inside the interval;
        otherwise every phase ends with one (lock-step).  With a ring of
        S >= 4 slots, tile t is loaded S - 2 iterations ahead into slot
        t % S: A's V(i) loads K tile i + S - 2, B's V(i) loads V tile
        i + S - 1 (B's V phase of iteration i runs during A's M(i+1)).  In
        the one-barrier form K tile t is issued in interval t - 2, complete
        at its loader's barrier closing interval t - 1 (the next batch is
        then the only one outstanding) and read in interval t; V tile t is
        issued in interval t - 2 and read in interval t + 1; the slot a load
        writes was last read two intervals (K) or one interval (V) before.
        """
        form = self._pp_forms.get(id(loop))
        if form is None:
            return False
        plan, swap, one, every = form
        pad = "  " * depth
        p1 = pad + "  "
        S, qk, pv = plan["S"], plan["qk"], plan["pv"]
        dist = S - 2
        # V load distance: B's V(i) runs in interval i + 1.  With a barrier every
        # iteration it loads V tile i + S - 1; with one every second iteration
        # tile i + S - 2, so that the slot's previous tile was read in an
        # earlier barrier interval.
        split = self.target.pingpong_split_barrier
        dv = dist + 1 if every == 1 and not split else dist
        iv = self._var(loop.induction_var)
        ivn = self.resolve(loop.induction_var.name)
        start = loop.start
        aff = self._var(plan["affine"].result)

        def dma(ld, tile: str, d: int) -> Tuple[List[str], int]:
            t = ld.buf.type.tile_type
            per = t.rows * t.cols * 2 // 1024 // 4
            key = self.resolve(ld.buf.name)
            stride = _tile_bytes(self.tile_type_of(key))
            src = ld.source
            sub = src.type.sub_tile_type
            b, dd, _rt, ct = (self._int(c) for c in ld.coords)
            self._aligned_checks.add((self.stile(key), _cname(src.name)[2:]))
            pd = "  " * d
            return [f"{pd}{{ const int {aff} = {tile};",
                    f"{pd}  wir::Loader<{self.stile(key)}, 4>::load<WIR_AL, WIR_INB>((smem + {self.lds_off[key]} + "
                    f"(({aff}) % {S}) * {stride}), globals.{_cname(src.name)[2:]}, {b}, {dd}, ({aff}) * {sub.rows}, "
                    f"({ct}) * {sub.cols}, wir_gw); }}"], per

        k_ld, v_ld = plan["k_load"], plan["v_load"]
        per = dma(k_ld, "0", 0)[1]

        npre = self.target.pingpong_v_prefetch
        pa_t, pr_t = pv.a.type, pv.result.type
        _vptr, vkey = self._tile_ptr(pv.b)
        rab = f"{self.geo.ms}, {pa_t.rows}, {pa_t.cols}, {pr_t.cols}, {self.stile(vkey)}"

        def emit_pv(dst: List[str], d: int) -> None:
            self._slot_shift[ivn] = -1
            if npre:
                pd = "  " * d
                res, acc = self._var(pv.result), self._var(pv.accum)
                if acc != res:
                    dst.append(f"{pd}{res} = {acc};")
                dst.append(f"{pd}wir::mma_rAB_pre<{rab}, {npre}>({res}, {self._var(pv.a)}, wir_vpre, "
                           f"{self._tile_ptr(pv.b)[0]}, wave_col0);")
            else:
                self._emit_op(pv, dst, d)
            del self._slot_shift[ivn]

        def v_prefetch(d: int) -> None:   # the next PV's first npre V operands (this iteration's tile)
            if npre:
                out.append(f"{'  ' * d}wir::prefetch_rAB<{rab}, {npre}>(wir_vpre, {self._tile_ptr(pv.b)[0]}, "
                           f"wave_col0);")

        # Both groups run the same loop: M(i), then V(i) with the group's ring
        # load; group B has one extra V phase (its first ring load) in front,
        # group A one extra barrier at the end, so the phases stay paired.
        q = pad + "  "
        # tensors that are not tile-aligned take the plain loop with bounds-checked loads;
        # one copy of its body keeps its registers within the ping-pong's
        out.append(f"{pad}if constexpr (!WIR_AL) {{")
        self._no_fusion = True
        self._emit_loop(loop, stop, out, depth + 1, mve=False)
        self._no_fusion = False
        if self._stream is not None and self._stream[0] is loop:
            out.append(f"{pad}}}   // (aligned tensors: the persistent stream form)")
            return True
        out.append(f"{pad}}} else {{")
        out.append(f"{q}const int wir_grp = (wir_wave >> 2) ^ {swap}, wir_gw = wir_wave & 3;"
                   f"  // group A (K loads) = physical wave group {swap}")
        if npre:
            out.append(f"{q}wir::RABPre<{npre}> wir_vpre;")
        was_live = self._fold_live
        if any(isinstance(self._softmax_fused.get(id(o)), dict) for o in plan["softmax"]):
            self._fold_preamble([qk], out, depth + 1)
        out.append(f"{q}for (int wir_t = {start}; wir_t < ({start}) + {dist}; ++wir_t) {{")
        out.append(f"{q}  if (wir_grp == 0) {{")
        out.extend(dma(k_ld, "wir_t", depth + 2)[0])
        out.append(f"{q}  }} else {{")
        out.extend(dma(v_ld, "wir_t", depth + 2)[0])
        out.append(f"{q}  }}")
        out.append(f"{q}}}")
        out.append(f"{q}wir::wait_vm_barrier<{per}>();")
        if every == 1 and not split:
            out.append(f"{q}if (wir_grp == 1) {{   // group B's first V phase: its first ring load only")
            out.extend(dma(v_ld, f"({start}) + {dist}", depth + 2)[0])
            if not one:
                out.append(f"{q}  wir::wait_vm_barrier<{per}>();")
            out.append(f"{q}}}")
        # barrier intervals of `every` iterations: a group passes its barrier in
        # iteration i only when (i - start) % every == every - 1
        odd = "" if every == 1 else f" && ((({iv}) - ({start})) & 1)"

        # Ring loads of tiles past the loop's end are skipped; a barrier whose
        # wave's latest batch was skipped drains all its loads instead (the
        # batch before is then the newest).  A's batch of V(i) is K tile
        # i + dist, B's batch of V(i) is V tile i + dist + 1.
        def pv_barrier(d: int) -> None:   # split form: B's barrier after the rotated PV(i-1)
            if split:   # B's latest batch: from its V(i-1), V tile i - 1 + dv
                out.append(f"{'  ' * d}if (wir_grp == 1) wir::wait_vm_barrier_after<{per}>(({iv}) + {dv - 1} < {stop});")

        def m_barrier(d: int) -> None:   # end of an M phase
            pd = "  " * d
            if split:
                return
            if one:   # B's latest batch: from its V(i-1), V tile i - 1 + dv
                out.append(f"{pd}if (wir_grp == 1{odd}) wir::wait_vm_barrier_after<{per}>(({iv}) + {dv - 1} < {stop});")
            else:
                out.append(f"{pd}wir::wait_vm_barrier_after<{per}>(({iv}) + {dist} - (wir_grp == 0 ? 1 : 0) < {stop});")

        def v_barrier(d: int) -> None:   # end of a V phase
            pd = "  " * d
            if one:   # A's latest batch: from this V(i)
                out.append(f"{pd}if (wir_grp == 0{odd}) wir::wait_vm_barrier_after<{per}>(({iv}) + {dist} < {stop});")
            else:
                out.append(f"{pd}wir::wait_vm_barrier_after<{per}>(({iv}) + {dist} + (wir_grp == 1 ? 1 : 0) < {stop});")
        softmax = plan["softmax"]
        fused_at = next((k for k, o in enumerate(softmax) if isinstance(self._softmax_fused.get(id(o)), dict)), None)

        def v_loads(d: int) -> None:
            qq = "  " * d
            out.append(f"{qq}if (wir_grp == 0) {{")
            out.append(f"{qq}  if (({iv}) + {dist} < {stop})")
            out.extend(dma(k_ld, f"({iv}) + {dist}", d + 2)[0])
            out.append(f"{qq}}} else {{")
            out.append(f"{qq}  if (({iv}) + {dv} < {stop})")
            out.extend(dma(v_ld, f"({iv}) + {dv}", d + 2)[0])
            out.append(f"{qq}}}")

        def v_tail(ops, d: int) -> None:
            self._emit_ops(ops, out, d)
            self._emit_op(plan["yld"], out, d)
            v_prefetch(d)
            v_barrier(d)

        def m_phase(d: int) -> None:
            emit_pv(out, d)
            pv_barrier(d)
            out.append(f"{'  ' * d}__builtin_amdgcn_sched_barrier(0);")
            self._emit_op(qk, out, d)
            m_barrier(d)

        # the first iteration (no PV yet) is peeled so the loop body's PV is
        # unconditional and O keeps one register assignment around the loop.
        # One guard holds the peeled iteration, the loop and the last M phase:
        # the loop is entered only through the peeled iteration, whose QK
        # MFMAs already wait for the register-hoisted Q, so the compiler puts
        # no vmcnt(0) for Q in the loop (it would also wait for the ring DMAs
        # this wave issued in its last V phase).
        q2 = q + "  "
        out.append(f"{q}if (({stop}) > {start}) {{")
        out.append(f"{q2}{{")
        out.append(f"{q2}  const int {iv} = {start};")
        self._emit_op(qk, out, depth + 3)
        m_barrier(depth + 3)
        v_loads(depth + 3)
        self._lazy_exact_only = True    # the first tile's running max is -inf
        v_tail(softmax, depth + 3)
        self._lazy_exact_only = False
        out.append(f"{q2}}}")
        if fused_at is None:
            out.append(f"{q2}for (int {iv} = ({start}) + 1; {iv} < {stop}; ++{iv}) {{")
            m_phase(depth + 3)
            v_loads(depth + 3)
            v_tail(softmax, depth + 3)
            out.append(f"{q2}}}")
        else:
            # A lazy softmax leaves the inner loop for its exact path (the
            # first tile was peeled above; later ones rarely rise above the
            # slack), so the inner loop touches O only through its MFMAs.
            fz = self._softmax_fused[id(softmax[fused_at])]
            pre, post = softmax[:fused_at], softmax[fused_at + 1:]
            out.append(f"{q2}int {iv} = ({start}) + 1;")
            out.append(f"{q2}for (;;) {{")
            out.append(f"{q2}  bool wir_exact = false;")
            out.append(f"{q2}  for (; {iv} < {stop}; ++{iv}) {{")
            m_phase(depth + 4)
            v_loads(depth + 4)
            self._emit_ops(pre, out, depth + 4)
            out.append(f"{q2}    if (!{self._fast_call(fz)}) {{")
            out.append(f"{q2}      wir_exact = true;")
            out.append(f"{q2}      break;")
            out.append(f"{q2}    }}")
            for src, dst in (("m_in", "m_out"), ("l_in", "l_out"), ("o_in", "o_out")):
                self._var_override[self.resolve(fz[dst].name)] = self._var(fz[src])
            v_tail(post, depth + 4)
            out.append(f"{q2}  }}")
            out.append(f"{q2}  if (!wir_exact) break;")
            self._emit_exact(softmax[fused_at], out, depth + 3)   # the step's exact half
            v_tail(post, depth + 3)
            out.append(f"{q2}  ++{iv};")
            out.append(f"{q2}}}")
        # the last M phase: PV of the last iteration
        out.append(f"{q2}{{")
        out.append(f"{q2}  const int {iv} = ({stop});")
        emit_pv(out, depth + 3)
        pv_barrier(depth + 3)
        out.append(f"{q2}}}")
        out.append(f"{q}}}")
        if not one:
            out.append(f"{q}if (wir_grp == 0) wir::wait_vm_barrier<0>();   // pairs with group B's extra V phase")
        out.append(f"{pad}}}")
        self._fold_live = was_live
        return True

    def _emit_attention_stream(self, loop: ForOp, pre_ops: List[Op], post_ops: List[Op]) -> List[str]:
        """The aligned body of the persistent stream form
        (``CDNA4Target.persistent_stream``): the one-barrier ping-pong of
        ``_emit_attention_pingpong`` over stream index ``u`` in ``[0, T)``,
        ``T`` = this program's tiles x key tiles per tile, where ``u`` is key
        tile ``u % nt`` of the program's tile ``u / nt``.  Ring slot, load
        distances and barrier conditions are the ping-pong's with the loop
        index replaced by ``u`` and the loop end by ``T`` (so the barrier
        protocol is the one its CPU model checks for a loop of ``T`` tiles);
        K and V tile ``w`` read (batch, head) of tile ``w / nt``.  After the
        rotated PV of the last key tile of a tile, each wave finishes that
        tile (O normalised in place and stored from registers, the LSE
        stored), switches the tile ids, loads the next tile's Q and resets
        its running max, sum and O; the lazy softmax of the tile's first key
        tile then takes its exact half (the max is -inf)."""
        plan, swap, _one, _every = self._pp_forms[id(loop)]
        S, qk, pv = plan["S"], plan["qk"], plan["pv"]
        dist = S - 2
        dv = dist + 1
        iv = self._var(loop.induction_var)
        ivn = self.resolve(loop.induction_var.name)
        stop = self._int(loop.stop)
        if loop.tile_size:
            stop = f"(({stop}) + {loop.tile_size - 1}) / {loop.tile_size}"
        out: List[str] = []
        w = out.append
        q = "    "

        def per(ld) -> int:
            t = ld.buf.type.tile_type
            return t.rows * t.cols * 2 // 1024 // 4
        k_ld, v_ld = plan["k_load"], plan["v_load"]
        npl = per(k_ld)

        def dma(ld, tile: str, d: int) -> List[str]:
            key = self.resolve(ld.buf.name)
            stride = _tile_bytes(self.tile_type_of(key))
            sub = ld.source.type.sub_tile_type
            self._aligned_checks.add((self.stile(key), _cname(ld.source.name)[2:]))
            pd = "  " * d
            # each wave loads stream tiles in increasing order, so a cursor (tile, key tile, batch,
            # head of the next tile it loads) replaces dividing the stream index
            return [f"{pd}{{ const int wir_w = {tile};",
                    f"{pd}  wir::Loader<{self.stile(key)}, 4>::load<WIR_AL, WIR_INB>((smem + {self.lds_off[key]} + "
                    f"((wir_w) % {S}) * {stride}), globals.{_cname(ld.source.name)[2:]}, wir_cz, wir_cy, "
                    f"(wir_ckt) * {sub.rows}, 0, wir_gw);",
                    f"{pd}  wir_adv(); }}"]

        # the tile's first and last ops: Q load and resets, and the finish (direct stores)
        pre: List[str] = []
        self._emit_ops([o for o in pre_ops if not isinstance(o, TMALoadBufOp)], pre, 0)
        decls = [ln for ln in pre if ln.lstrip().startswith("wir::RowFrags<")]
        acts = [ln for ln in pre if ln not in decls and not ln.lstrip().startswith("if constexpr (!WIR_AL)")]
        staged, over = dict(self._staged), dict(self._var_override)
        for o in post_ops:
            if isinstance(o, TMAStoreOp):
                self._staged.pop(id(o), None)
            if isinstance(o, DivRowOp):
                self._var_override[self.resolve(o.result.name)] = self._var(o.tile)   # in place
        fin: List[str] = []
        self._emit_ops(post_ops, fin, 0)
        self._staged, self._var_override = staged, over
        if any("store_tile_staged" in ln or "wait_vm_barrier" in ln for ln in fin):
            raise LoweringError("persistent_stream: the tile's finish must store from registers")

        def emit(lines: List[str], d: int) -> None:
            pd = "  " * d
            out.extend(pd + ln.strip() if ln.strip() else ln for ln in lines)

        w(f"{q}const int wir_G = gridDim.x;")
        w(f"{q}const int wir_cnt = (int)blockIdx.x < wir_nblk ? (wir_nblk - 1 - (int)blockIdx.x) / wir_G + 1 : 0;")
        w(f"{q}const int wir_nt = {stop};   // key tiles per output tile")
        w(f"{q}const int wir_T = wir_cnt * wir_nt;   // this program's stream of key tiles")
        w(f"{q}const int wir_grp = (wir_wave >> 2) ^ {swap}, wir_gw = wir_wave & 3;")
        w(f"{q}auto wir_tile = [&](int sb) {{   // tile ids of this program's sb-th tile")
        w(f"{q}  const int lid_ = wir::remap_xcd((int)blockIdx.x + sb * wir_G, wir_nblk);")
        w(f"{q}  pid_x = lid_ % nx_; pid_y = (lid_ / nx_) % ny_; pid_z = lid_ / (nx_ * ny_);")
        w(f"{q}}};")
        w(f"{q}int wir_csb = 0, wir_ckt = 0, wir_cz = 0, wir_cy = 0;   // this wave's load cursor")
        w(f"{q}auto wir_cur = [&]() {{")
        w(f"{q}  const int lid_ = wir::remap_xcd((int)blockIdx.x + wir_csb * wir_G, wir_nblk);")
        w(f"{q}  wir_cy = (lid_ / nx_) % ny_; wir_cz = lid_ / (nx_ * ny_);")
        w(f"{q}}};")
        w(f"{q}auto wir_adv = [&]() {{")
        w(f"{q}  if (++wir_ckt == wir_nt) {{ wir_ckt = 0; ++wir_csb; wir_cur(); }}")
        w(f"{q}}};")
        w(f"{q}int wir_sb = 0, wir_nb = wir_nt;   // the tile being computed; stream index of the next one")
        emit(decls, 2)
        w(f"{q}if (wir_cnt > 0) {{")
        q2 = q + "  "
        w(f"{q2}wir_tile(0);")
        w(f"{q2}wir_cur();")
        emit(acts, 3)
        w(f"{q2}for (int wir_t = 0; wir_t < {dist}; ++wir_t) {{")
        w(f"{q2}  if (wir_t < wir_T) {{")
        w(f"{q2}    if (wir_grp == 0) {{")
        out.extend(dma(k_ld, "wir_t", 6))
        w(f"{q2}    }} else {{")
        out.extend(dma(v_ld, "wir_t", 6))
        w(f"{q2}    }}")
        w(f"{q2}  }}")
        w(f"{q2}}}")
        w(f"{q2}wir::wait_vm_barrier_after<{npl}>({dist - 1} < wir_T);")
        w(f"{q2}if (wir_grp == 1 && {dist} < wir_T) {{   // group B's first V phase: its first ring load only")
        out.extend(dma(v_ld, str(dist), 4))
        w(f"{q2}}}")

        def m_barrier(d: int) -> None:   # B's latest batch: V tile u - 1 + dv
            out.append(f"{'  ' * d}if (wir_grp == 1) wir::wait_vm_barrier_after<{npl}>(({iv}) + {dv - 1} < wir_T);")

        def v_barrier(d: int) -> None:   # A's latest batch: K tile u + dist
            out.append(f"{'  ' * d}if (wir_grp == 0) wir::wait_vm_barrier_after<{npl}>(({iv}) + {dist} < wir_T);")

        def v_loads(d: int) -> None:
            qq = "  " * d
            out.append(f"{qq}if (wir_grp == 0) {{")
            out.append(f"{qq}  if (({iv}) + {dist} < wir_T)")
            out.extend(dma(k_ld, f"({iv}) + {dist}", d + 2))
            out.append(f"{qq}}} else {{")
            out.append(f"{qq}  if (({iv}) + {dv} < wir_T)")
            out.extend(dma(v_ld, f"({iv}) + {dv}", d + 2))
            out.append(f"{qq}}}")

        def emit_pv(d: int) -> None:
            self._slot_shift[ivn] = -1
            self._emit_op(pv, out, d)
            del self._slot_shift[ivn]

        def v_tail(ops, d: int) -> None:
            self._emit_ops(ops, out, d)
            self._emit_op(plan["yld"], out, d)
            v_barrier(d)

        softmax = plan["softmax"]
        fused_at = next((k for k, o in enumerate(softmax) if isinstance(self._softmax_fused.get(id(o)), dict)), None)
        if fused_at is None:
            raise LoweringError("persistent_stream takes the lazy-softmax ping-pong")
        fz = self._softmax_fused[id(softmax[fused_at])]
        pre_sm, post_sm = softmax[:fused_at], softmax[fused_at + 1:]
        # One pass of the outer loop per output tile.  The tile's first key tile is peeled: its QK
        # is the only use of the tile's freshly loaded Q fragments that the compiler must wait
        # for (the inner loop is entered only through it, so no vmcnt(0) lands in the inner loop,
        # where it would also wait for the ring DMAs in flight), and its softmax takes the exact
        # half (the running max is -inf).  The tile's last PV ends the pass, then its finish.
        q3, q4 = q2 + "  ", q2 + "    "
        w(f"{q2}int {iv} = 0;")
        w(f"{q2}for (;;) {{")
        w(f"{q3}{{")
        self._emit_op(qk, out, 7)
        m_barrier(7)
        v_loads(7)
        self._lazy_exact_only = True
        v_tail(softmax, 7)
        self._lazy_exact_only = False
        w(f"{q3}}}")
        w(f"{q3}++{iv};")
        w(f"{q3}for (;;) {{")
        w(f"{q4}bool wir_exact = false;")
        w(f"{q4}for (; {iv} < wir_nb; ++{iv}) {{")
        emit_pv(8)
        w(f"{q4}  __builtin_amdgcn_sched_barrier(0);")
        self._emit_op(qk, out, 8)
        m_barrier(8)
        v_loads(8)
        self._emit_ops(pre_sm, out, 8)
        w(f"{q4}  if (!{self._fast_call(fz)}) {{")
        w(f"{q4}    wir_exact = true;")
        w(f"{q4}    break;")
        w(f"{q4}  }}")
        for src, dst in (("m_in", "m_out"), ("l_in", "l_out"), ("o_in", "o_out")):
            self._var_override[self.resolve(fz[dst].name)] = self._var(fz[src])
        v_tail(post_sm, 8)
        w(f"{q4}}}")
        w(f"{q4}if (!wir_exact) break;")
        self._emit_exact(softmax[fused_at], out, 7)
        v_tail(post_sm, 7)
        w(f"{q4}++{iv};")
        w(f"{q3}}}")
        emit_pv(6)   # the tile's last PV ({iv} == wir_nb)
        emit(fin, 6)
        w(f"{q3}if ({iv} == wir_T) break;")
        w(f"{q3}wir_nb += wir_nt;")
        w(f"{q3}wir_tile(++wir_sb);")
        emit(acts, 6)
        w(f"{q2}}}")
        w(f"{q}}}")
        return out

    def _attention_overlap_plan(self, loop: ForOp):
        """Match the prefetch-form attention loop for the overlapped emitter:
        the placement ``kernel_pass`` marks by a ``pipeline_stage(1)`` between
        S = Q K^T and the softmax ops (tile i's softmax and PV run beside
        tile i+1's score MFMAs; the "mixed" phase schedule).

        Required: four wavefronts; body = wait on slot i, slot views, S = Q K^T
        with hoisted Q, one prefetch per ring into slot i + 1 of a 2-slot
        ring, the softmax ops, O += P V last (P a bf16 register tile, O
        carried in place).  The softmax ops split into
          E: the element-wise chain S -> P_fp32 (mul_scalar / sub_row /
             mul_row / exp2), consumed only by one row_sum and one bf16 copy;
          R: the rescale of the carried O and of row_sum's carried prev;
          M: everything else (running max, its scaled copies, the
             correction, a causal mask of S), which may read only S, the
             carried values, constants and other M results.
        Every loop-carried value must be updated in place.
        """
        if self.geo.nw != 4 or loop not in list(self.kernel.body):
            return None
        body = list(loop.body)
        marks = [o for o in body if isinstance(o, PipelineStageOp)]
        qk_at = next((k for k, o in enumerate(body) if isinstance(o, MMAOp)), None)
        if len(marks) != 1 or marks[0].stage != 1 or qk_at is None or body.index(marks[0]) < qk_at:
            return None
        if not any(isinstance(o, (Exp2Op, RowSumOp)) for o in body[body.index(marks[0]):]):
            return None
        if len(body) < 4 or not isinstance(body[0], WaitBufOp) or not isinstance(body[-1], YieldOp):
            return None
        if loop.start != 0 or loop.step != 1:
            return None
        mmas = [o for o in body if isinstance(o, MMAOp)]
        if len(mmas) != 2:
            return None
        qk, pv = mmas
        if not qk.transpose_b or pv.transpose_b or body[-2] is not pv:
            return None
        if self.resolve(qk.a.name) not in self._hoisted:
            return None
        pa = pv.a.type
        if not (isinstance(pa, RegTileType) and pa.data_type == GPUType.bf16):
            return None
        # two key column blocks: the PV MFMAs of the first block run while the
        # second block's probabilities are still being computed
        if qk.result.type.cols != 2 * self.geo.ms or pa.cols != qk.result.type.cols:
            return None
        R = self.resolve
        views = self._views()
        vk, vv = views.get(R(qk.b.name)), views.get(R(pv.b.name))
        if vk is None or vv is None or R(vk.buf.name) == R(vv.buf.name):
            return None
        ivn = R(loop.induction_var.name)
        loads = [o for o in body if isinstance(o, TMALoadBufOp)]
        if sorted(R(o.buf.name) for o in loads) != sorted([R(vk.buf.name), R(vv.buf.name)]):
            return None
        mods = {o.slot.modulus for o in loads} | {vk.slot.modulus, vv.slot.modulus, body[0].slot.modulus}
        if mods != {2}:
            return None
        affine = [o for o in body if isinstance(o, IntAffineOp)]
        if len(affine) != 1 or affine[0].mul != 1 or affine[0].add != 1 or R(affine[0].input.name) != ivn:
            return None
        for o in loads:
            if not (isinstance(o.slot, BufSlotExpr) and o.slot.value is not None and R(o.slot.value.name) == ivn
                    and o.slot.offset % 2 == 1):
                return None
            b, d, rt, ct = o.coords
            if not (isinstance(rt, Value) and R(rt.name) == R(affine[0].result.name)) or ct != 0:
                return None
            if any(isinstance(c, Value) and R(c.name) == ivn for c in (b, d)):
                return None
        for v in (vk, vv):
            if v.slot.value is None or R(v.slot.value.name) != ivn or v.slot.offset % 2:
                return None
        skip = (TMALoadBufOp, IntAffineOp, SlotViewOp, PipelineStageOp)
        mid = [o for o in body[body.index(qk) + 1: body.index(pv)] if not isinstance(o, skip)]
        if any(isinstance(o, (TMALoadOp, WaitOp, WaitBufOp, MMAOp, MMABufOp, ForOp)) for o in mid):
            return None
        producers = {}
        for o in mid:
            r = vars(o).get("result")
            if isinstance(r, Value):
                producers[R(r.name)] = o
        rowsums = [o for o in mid if isinstance(o, RowSumOp)]
        if len(rowsums) != 1:
            return None
        rs = rowsums[0]
        p_name = R(rs.tile.name)
        cvts = [o for o in mid if isinstance(o, CopyOp) and R(o.input.name) == p_name]
        if len(cvts) != 1 or R(cvts[0].result.name) != R(pv.a.name):
            return None
        cvt = cvts[0]
        chain, cur = [], rs.tile
        while True:
            prod = producers.get(R(cur.name))
            if not isinstance(prod, (MulScalarOp, SubRowOp, Exp2Op, MulRowOp)):
                break
            src = prod.input if isinstance(prod, (MulScalarOp, Exp2Op)) else prod.tile
            if not isinstance(src.type, RegTileType) or not isinstance(prod.result.type, RegTileType):
                break
            chain.insert(0, prod)
            cur = src
        if not chain:
            return None
        start = cur
        mask = producers.get(R(start.name))
        if mask is not None:
            if not isinstance(mask, CausalMaskOp) or R(mask.tile.name) != R(qk.result.name):
                return None
        elif R(start.name) != R(qk.result.name):
            return None
        acc_prod = producers.get(R(pv.accum.name))
        prev_prod = producers.get(R(rs.prev.name))
        r_ops = [o for o in (prev_prod, acc_prod) if o is not None]
        if not isinstance(acc_prod, MulRowOp):
            return None
        carried = {R(ia.block_arg.name) for ia in loop.iter_args}
        if R(acc_prod.tile.name) not in carried:
            return None
        if prev_prod is not None and not any(isinstance(x, Value) and R(x.name) in carried
                                             for x in vars(prev_prod).values()):
            return None
        e_ids = {id(o) for o in chain} | {id(rs), id(cvt)}
        r_ids = {id(o) for o in r_ops}
        m_ops = [o for o in mid if id(o) not in e_ids and id(o) not in r_ids]
        e_vals = {R(o.result.name) for o in chain} | {R(cvt.result.name)}
        r_vals = {R(o.result.name) for o in r_ops} | {R(rs.result.name)}
        s_vals = {R(qk.result.name), R(start.name)}
        rowmaxes = [o for o in m_ops if isinstance(o, RowMaxOp)]
        if len(rowmaxes) != 1 or R(rowmaxes[0].tile.name) != R(start.name):
            return None
        for o in m_ops:
            for name, x in vars(o).items():
                if name == "result" or not isinstance(x, Value):
                    continue
                n = R(x.name)
                if n in e_vals or n in r_vals:
                    return None
                if isinstance(x.type, RegTileType) and n not in s_vals:
                    return None
                if n in s_vals and not isinstance(o, (RowMaxOp, CausalMaskOp)):
                    return None
        # chain values other than P feed only the next chain op
        uses: Dict[str, int] = {}
        for o in mid + [pv, body[-1]]:
            for name, x in vars(o).items():
                for v in _values_in(x) if name != "result" else ():
                    uses[R(v.name)] = uses.get(R(v.name), 0) + 1
        for o in chain[:-1]:
            if uses.get(R(o.result.name), 0) != 1:
                return None
        if uses.get(p_name, 0) != 2:
            return None
        yld = body[-1]
        for k, v in enumerate(yld.values):
            if self._var(v) != self._var(loop.iter_args[k].block_arg):
                return None
        if self._var(pv.result) != self._var(pv.accum) and self._var(pv.result) not in {
                self._var(ia.block_arg) for ia in loop.iter_args}:
            return None
        k_load = next(o for o in loads if R(o.buf.name) == R(vk.buf.name))
        v_load = next(o for o in loads if R(o.buf.name) == R(vv.buf.name))
        return dict(qk=qk, pv=pv, chain=chain, rs=rs, cvt=cvt, start=start, mask=mask, r_ops=r_ops,
                    m_ops=m_ops, rowmax=rowmaxes[0], k_load=k_load, v_load=v_load)

    def _emit_attention_overlap(self, loop: ForOp, stop: str, out: List[str], depth: int) -> bool:
        """Software-pipelined attention loop (the "mixed" phase placement).

        Tile j's scores S_j are computed one step ahead.  Step j (j + 1 < n):
          wait + barrier (K_{j+1} and V_j landed; every wave is done with
          step j - 1), R ops of tile j (rescale O and the running sum);
          S_{j+1} = Q K_{j+1}^T, its 16 MFMAs carrying the E chain of
          S_j (exp, partial row sums, bf16 P) and the DMAs of K_{j+2} and
          V_{j+1} (into the slots that K_j and V_{j-1} have left);
          O += P_j V_j, its first MFMAs carrying the rest of E, the later
          ones the causal mask and the running max of S_{j+1} (M ops).
        The K ring runs one tile ahead of the V ring.  S alternates between
        two register tiles (the loop is unrolled by two); the last tile is
        peeled.  Tensors that are not tile-aligned take the plain loop.
        """
        plan = self._attention_overlap_plan(loop)
        if plan is None:
            return False
        self._overlapped = True
        R = self.resolve
        pad = "  " * depth
        ms = self.geo.ms
        qk, pv, rs = plan["qk"], plan["pv"], plan["rs"]
        st = qk.result.type
        rb_n = st.rows // ms
        cregs = 16 if ms == 32 else 4
        n_pairs = (st.rows * st.cols // 64) // 2
        iv = self._var(loop.induction_var)
        kl, vl = plan["k_load"], plan["v_load"]
        kkey, vkey = R(kl.buf.name), R(vl.buf.name)
        kt, vt = kl.buf.type.tile_type, vl.buf.type.tile_type
        kstile, vstile = self.stile(kkey), self.stile(vkey)
        kper, vper = self.loads_per_wave(kt), self.loads_per_wave(vt)
        kstride, vstride = _tile_bytes(kt), _tile_bytes(vt)

        def kptr(slot: int) -> str:
            return f"(smem + {self.lds_off[kkey]} + {slot} * {kstride})"

        def vptr(slot: int) -> str:
            return f"(smem + {self.lds_off[vkey]} + {slot} * {vstride})"

        def src(ld, tile_expr: str) -> Tuple[str, str]:
            g = f"globals.{_cname(ld.source.name)[2:]}"
            sub = ld.source.type.sub_tile_type
            b, d = self._int(ld.coords[0]), self._int(ld.coords[1])
            self._aligned_checks.add((self.stile(R(ld.buf.name)), _cname(ld.source.name)[2:]))
            return g, f"{b}, {d}, ({tile_expr}) * {sub.rows}, 0"

        kg, _ = src(kl, "0")
        vg, _ = src(vl, "0")
        kload = f"wir::Loader<{kstile}, 4>"
        vload = f"wir::Loader<{vstile}, 4>"
        hf_var, hf_ks = self._hoisted[R(qk.a.name)]
        s_names = {R(qk.result.name), R(plan["start"].name)}
        p_var = self._var(pv.a)
        o_var = self._var(pv.result)
        acc_var = self._var(pv.accum)
        a_t = pv.a.type
        res_t = pv.result.type

        def with_s(var: str):
            for n in s_names:
                self._var_override[n] = var

        def clear_s():
            for n in s_names:
                self._var_override.pop(n, None)

        def qk_plain(dst: List[str], d: int, svar: str, slot: int) -> None:
            dst.append(f"{'  ' * d}wir::mma_ABt_frags<{ms}, {st.rows}, {st.cols}, {kstile}, {hf_ks}>"
                       f"({svar}, {hf_var}, {kptr(slot)}, wave_col0);")

        def m_ops(dst: List[str], d: int, tile_index: str, svar: str, partial: bool) -> None:
            """The M ops for the tile in `svar` (its index `tile_index`)."""
            p_ = "  " * d
            dst.append(f"{p_}{{")
            dst.append(f"{p_}  const int {iv} = {tile_index};")
            dst.append(f"{p_}  (void){iv};")
            with_s(svar)
            for o in plan["m_ops"]:
                if partial and o is plan["mask"]:
                    continue
                if partial and o is plan["rowmax"]:
                    dst.append(f"{p_}  wir::row_finish({self._var(o.result)}, wir_mx, {self._var(o.prev)}, "
                               f"wir::OpMax());")
                    continue
                self._emit_op(o, dst, d + 1)
            clear_s()
            dst.append(f"{p_}}}")

        def r_ops(dst: List[str], d: int) -> None:
            # the rescale of the carried O is done in place (O = O * corr),
            # so no copy of the accumulator exists on either path of its skip test
            for o in plan["r_ops"]:
                if isinstance(o, MulRowOp) and R(o.result.name) == R(pv.accum.name) and \
                        self._var(o.tile) == o_var:
                    dst.append(f"{'  ' * d}wir::row_scale({o_var}, {o_var}, {self._var(o.vec)});")
                    continue
                self._emit_op(o, dst, d)
                if R(o.result.name) == R(pv.accum.name) and acc_var != o_var:
                    dst.append(f"{'  ' * d}{o_var} = {acc_var};")

        def step(dst: List[str], d: int, j: str, par: int, cur: str, nxt: str) -> None:
            p_ = "  " * d
            p2 = p_ + "  "
            dst.append(f"{p_}{{")
            dst.append(f"{p2}wir::wait_vm_barrier<0>();")
            r_ops(dst, d + 1)
            _, kc = src(kl, f"({j}) + 2")
            _, vc = src(vl, f"({j}) + 1")
            dst.append(f"{p2}const auto wir_ks = {kload}::prep<WIR_AL, WIR_INB>({kg}, {kc});")
            dst.append(f"{p2}const auto wir_vs = {vload}::prep<WIR_AL, WIR_INB>({vg}, {vc});")
            dst.append(f"{p2}for (int r_ = 0; r_ < {rb_n}; ++r_) wir_rs[r_] = 0.f;")
            dst.append(f"{p2}wir::mma_ABt_frags_slots<{ms}, {st.rows}, {st.cols}, {kstile}, {hf_ks}>"
                       f"({nxt}, {hf_var}, {kptr((par + 1) % 2)}, wave_col0, [&](auto t_) {{")
            dst.append(f"{p2}  constexpr int T = decltype(t_)::value;")
            dst.append(f"{p2}  constexpr int P0 = (T * {n_pairs} + WIR_NS - 1) / WIR_NS, "
                       f"P1 = ((T + 1) * {n_pairs} + WIR_NS - 1) / WIR_NS;")
            dst.append(f"{p2}  wir::e_pairs<P0, P1>({cur}, {p_var}, wir_rs, wir_ef);")
            dst.append(f"{p2}  if constexpr (T % 2 == 0 && T / 2 < {kper}) "
                       f"{kload}::issue<WIR_AL, WIR_INB>(T / 2, {kptr(par)}, {kg}, wir_ks, wir_wave);")
            dst.append(f"{p2}  if constexpr (T % 2 == 1 && T / 2 < {vper}) "
                       f"{vload}::issue<WIR_AL, WIR_INB>(T / 2, {vptr((par + 1) % 2)}, {vg}, wir_vs, wir_wave);")
            dst.append(f"{p2}}});")
            dst.append(f"{p2}wir::mma_rAB_slots<{ms}, {a_t.rows}, {a_t.cols}, {res_t.cols}, {vstile}>"
                       f"({o_var}, {p_var}, {vptr(par)}, wave_col0, [&](auto t_) {{")
            dst.append(f"{p2}  constexpr int T = decltype(t_)::value + WIR_NA;")
            dst.append(f"{p2}  if constexpr (T < WIR_NS) {{")
            dst.append(f"{p2}    constexpr int P0 = (T * {n_pairs} + WIR_NS - 1) / WIR_NS, "
                       f"P1 = ((T + 1) * {n_pairs} + WIR_NS - 1) / WIR_NS;")
            dst.append(f"{p2}    wir::e_pairs<P0, P1>({cur}, {p_var}, wir_rs, wir_ef);")
            dst.append(f"{p2}  }}")
            dst.append(f"{p2}  if constexpr (T == WIR_NS) {{")
            dst.append(f"{p2}    wir::row_finish({self._var(rs.result)}, wir_rs, {self._var(rs.prev)}, wir::OpAdd());")
            dst.append(f"{p2}    for (int r_ = 0; r_ < {rb_n}; ++r_) wir_mx[r_] = -__builtin_inff();")
            if plan["mask"] is not None:
                with_s(nxt)
                dst.append(f"{p2}    {{ const int {iv} = ({j}) + 1; (void){iv};")
                self._emit_op(plan["mask"], dst, d + 3)
                dst.append(f"{p2}    }}")
                clear_s()
            dst.append(f"{p2}  }}")
            n_el = 2 * n_pairs
            for c in range(n_chunks):
                e0, e1 = n_el * c // n_chunks, n_el * (c + 1) // n_chunks
                dst.append(f"{p2}  if constexpr (T == WIR_NS + {c + 1}) wir::row_partial<{e0}, {e1}>(wir_mx, {nxt}, "
                           f"wir::OpMax());")
            dst.append(f"{p2}  if constexpr (T == WIR_NS + {n_chunks + 1}) {{")
            m_ops(dst, d + 2, f"({j}) + 1", nxt, True)
            dst.append(f"{p2}  }}")
            dst.append(f"{p2}}});")
            dst.append(f"{p_}}}")

        def last(dst: List[str], d: int, j: str, par: int, cur: str) -> None:
            p_ = "  " * d
            p2 = p_ + "  "
            dst.append(f"{p_}{{")
            dst.append(f"{p2}wir::wait_vm_barrier<0>();")
            r_ops(dst, d + 1)
            dst.append(f"{p2}for (int r_ = 0; r_ < {rb_n}; ++r_) wir_rs[r_] = 0.f;")
            dst.append(f"{p2}wir::e_pairs<0, {n_pairs}>({cur}, {p_var}, wir_rs, wir_ef);")
            dst.append(f"{p2}wir::row_finish({self._var(rs.result)}, wir_rs, {self._var(rs.prev)}, wir::OpAdd());")
            dst.append(f"{p2}wir::mma_rAB<{ms}, {a_t.rows}, {a_t.cols}, {res_t.cols}, {vstile}>"
                       f"({o_var}, {p_var}, {vptr(par)}, wave_col0);")
            dst.append(f"{p_}}}")

        # PV slots after the probabilities are done: row-sum finish (+ mask),
        # the partial maxima of the next tile, then its remaining M ops
        pv_items = (a_t.cols // ms) * (cregs // 4) // 2 * (res_t.cols // ms)
        n_chunks = min(4, pv_items // 2 - 2)
        if n_chunks < 1:
            return False
        # the element-wise chain as one per-element function
        e_lines = []
        for o in plan["chain"]:
            if isinstance(o, MulScalarOp):
                e_lines.append(f"x = x * {_flt(o.scalar)};")
            elif isinstance(o, SubRowOp):
                e_lines.append(f"x = x - {self._var(o.vec)}.v[rb];")
            elif isinstance(o, MulRowOp):
                e_lines.append(f"x = x * {self._var(o.vec)}.v[rb];")
            else:
                e_lines.append("x = __builtin_amdgcn_exp2f(x);")
        p1 = pad + "  "
        out.append(f"{pad}if constexpr (!WIR_AL) {{")
        self._emit_loop(loop, stop, out, depth + 1)
        out.append(f"{pad}}} else {{")
        out.append(f"{p1}wir::RTile<{ms}, {st.rows}, {st.cols}> wir_sa, wir_sb;")
        out.append(f"{p1}float wir_rs[{rb_n}], wir_mx[{rb_n}];")
        out.append(f"{p1}constexpr int WIR_NA = {hf_ks * (st.cols // ms)};  // slots of S = Q K^T")
        out.append(f"{p1}constexpr int WIR_NS = WIR_NA + {(a_t.cols // ms) * (cregs // 4) // 2 * (res_t.cols // ms) // 2};"
                   f"  // slots carrying E")
        out.append(f"{p1}static_assert((({n_pairs} / 2 - 1) * WIR_NS) / {n_pairs} < WIR_NA, "
                   f"\"block-0 probabilities must be ready before O += P V starts\");")
        out.append(f"{p1}static_assert(WIR_NS + {n_chunks + 1} < WIR_NA + 2 * (WIR_NS - WIR_NA), "
                   f"\"running-max slots must fit\");")
        out.append(f"{p1}auto wir_ef = [&](float x, int rb) {{ (void)rb; {' '.join(e_lines)} return x; }};")
        out.append(f"{p1}const int wir_n = {stop};")
        out.append(f"{p1}if (wir_n > 0) {{")
        p2 = p1 + "  "
        _, kc1 = src(kl, "1")
        out.append(f"{p2}{kload}::load<WIR_AL, WIR_INB>({kptr(1)}, {kg}, {kc1}, wir_wave);")
        out.append(f"{p2}wir::wait_vm_barrier<{kper}>();")
        qk_plain(out, depth + 2, "wir_sa", 0)
        m_ops(out, depth + 2, "0", "wir_sa", False)
        out.append(f"{p2}int wir_j = 0;")
        out.append(f"{p2}for (; wir_j + 2 < wir_n; wir_j += 2) {{")
        step(out, depth + 3, "wir_j", 0, "wir_sa", "wir_sb")
        step(out, depth + 3, "wir_j + 1", 1, "wir_sb", "wir_sa")
        out.append(f"{p2}}}")
        out.append(f"{p2}if (wir_j + 1 < wir_n) {{")
        step(out, depth + 3, "wir_j", 0, "wir_sa", "wir_sb")
        last(out, depth + 3, "wir_j + 1", 1, "wir_sb")
        out.append(f"{p2}}} else {{")
        last(out, depth + 3, "wir_j", 0, "wir_sa")
        out.append(f"{p2}}}")
        out.append(f"{p1}}}")
        out.append(f"{pad}}}")
        return True

    def _setup_pingpong(self, loop: ForOp, out: List[str], depth: int) -> bool:
        """Eight-wavefront ring loops (steady state + drain steps) use the
        ping-pong form ``wir::PingPongAB``: two wave groups alternate between
        MFMA-only phases and LDS-read/DMA phases, one phase apart."""
        if not self.target.pingpong or self.geo.nw != 8:
            return False
        rot = self._rotatable(loop, for_pingpong=True)
        if rot is None:
            return False
        mma, _ = rot
        top = list(self.kernel.body)
        if loop not in top:
            return False
        after = top[top.index(loop) + 1:]
        drains = []
        for o in after:
            if isinstance(o, WaitBufOp) and isinstance(o.slot, BufSlotExpr) and o.slot.value is None:
                continue
            if (isinstance(o, MMABufOp) and isinstance(o.a_slot, BufSlotExpr) and o.a_slot.value is None
                    and o.a_buf == mma.a_buf and o.b_buf == mma.b_buf):
                drains.append(o)
                continue
            break
        stages = mma.a_buf.type.count
        if len(drains) != stages - 1:
            return False
        loads = [o for o in loop.body if isinstance(o, TMALoadBufOp)]
        if any(id(o) in self.war_barrier for o in loads):
            return False
        per4 = 0
        for ld in loads:
            t = ld.buf.type.tile_type
            instr = t.rows * t.cols * 2 // 16 // 64
            if instr % 4:
                return False
            per4 += instr // 4
        t = self._rtype(mma.accum)
        a_key, b_key = self.resolve(mma.a_buf.name), self.resolve(mma.b_buf.name)
        name = f"pp{len(self._pp_ops)}"
        pad = "  " * depth
        out.append(f"{pad}wir::PingPongAB<{self.geo.ms}, {t.rows}, {t.cols}, {self.stile(a_key)}, {self.stile(b_key)}> {name};")
        out.append(f"{pad}{name}.init(wir_wave);")
        self._pp_ops[id(loop.body[0])] = ("skip", name, None)
        for o in loop.body:
            if isinstance(o, TMALoadBufOp):
                self._fused_ids.add(id(o))
        self._pp_ops[id(mma)] = ("step", name, ((stages - 2) * per4, per4, loads))
        for e, d in enumerate(drains):
            self._pp_ops[id(d)] = ("drain", name, ((stages - 2 - e) * per4, e == len(drains) - 1))
        for o in after[:2 * len(drains)]:
            if isinstance(o, WaitBufOp):
                self._pp_ops[id(o)] = ("skip", name, None)
        return True

    def _rotatable(self, loop: ForOp, for_pingpong: bool = False):
        """The steady state of a ring pipeline -- ``wait_buf(slot s)``, loads,
        one ``mma_buf`` on slot ``s`` -- is emitted in rotated form
        (``wir::MMAPipeAB``): the MMA's last k-step is issued after the next
        iteration's wait, so the matrix core is busy across the barrier."""
        if not self.target.rotate_mma and not for_pingpong:
            return None
        body = [o for o in loop.body if not isinstance(o, YieldOp)]
        if not body or not isinstance(body[0], WaitBufOp):
            return None
        nwait = next(k for k, o in enumerate(body + [None]) if not isinstance(o, WaitBufOp))
        waits = body[:nwait]
        mmas = [o for o in body if isinstance(o, MMABufOp)]
        rest = [o for o in body[nwait:] if not isinstance(o, (TMALoadBufOp, MMABufOp, IntAffineOp))]
        if len(mmas) != 1 or rest or body[-1] is not mmas[0]:
            return None
        mma = mmas[0]
        # each operand's slot is the one its ring's wait names
        slot_of = {self.resolve(b.name): w.slot for w in waits for b in w.bufs}
        if (slot_of.get(self.resolve(mma.a_buf.name)) != mma.a_slot
                or slot_of.get(self.resolve(mma.b_buf.name)) != mma.b_slot):
            return None
        t = self._rtype(mma.accum)
        k = mma.a_buf.type.tile_type.cols
        if (k // (16 if self.geo.ms == 32 else 32)) % 2 and not for_pingpong:
            return None
        a_key, b_key = self.resolve(mma.a_buf.name), self.resolve(mma.b_buf.name)
        return mma, (f"wir::MMAPipeAB<{self.geo.ms}, {t.rows}, {t.cols}, {self.stile(a_key)}, "
                     f"{self.stile(b_key)}>")

    # ------------------------------------------------------------------
    # assembly
    # ------------------------------------------------------------------
    def _register_only_tiles(self) -> Dict[str, tuple]:
        """Shared tiles loaded once whose only reads are hoisted MMA fragments.

        Such a tile never needs LDS: its fragments are loaded from global
        memory straight into registers where the IR loads it, and waits on
        it need no barrier (the compiler tracks the register loads)."""
        out: Dict[str, tuple] = {}
        for name, info in self._pending_hoist.items():
            loads = [o for o in _walk(self.kernel.body)
                     if isinstance(o, TMALoadOp) and self.resolve(o.result.name) == name]
            if len(loads) != 1 or any(ld in _walk(info[3].body) for ld in loads):
                continue
            uses_ok = True
            for o in _walk(self.kernel.body):
                if isinstance(o, (TMALoadOp, WaitOp, TMALoadBufOp, WaitBufOp)):
                    continue
                for f, v in vars(o).items():
                    for x in _values_in(v):
                        if self.resolve(x.name) != name:
                            continue
                        if not (isinstance(o, MMAOp) and o.transpose_b and f == "a"):
                            uses_ok = False
            if uses_ok:
                out[name] = info
        return out

    def _hoistable(self) -> Dict[str, tuple]:
        """Shared tiles read as the row operand of a transpose_b MMA inside a
        loop that never reloads them (e.g. the resident Q tile): their MFMA
        fragments are read from LDS once, before the loop."""
        hoist: Dict[str, tuple] = {}
        for loop in _walk(self.kernel.body):
            if not isinstance(loop, ForOp):
                continue
            written = {self.resolve(o.result.name) for o in _walk(loop.body) if isinstance(o, TMALoadOp)}
            for o in _walk(loop.body):
                if isinstance(o, MMAOp) and o.transpose_b:
                    key = self._lds_key(o.a)
                    name = self.resolve(o.a.name)
                    if key is not None and key == name and name not in written and name not in hoist:
                        t = self.tile_type_of(key)
                        ks = t.cols // (16 if self.geo.ms == 32 else 32)
                        res_t = o.result.type
                        hoist[name] = (f"hf_{_cname(name)[2:]}", ks, res_t.rows, loop)
        return hoist

    def _assemble(self, kernel: Kernel, body: List[str]) -> str:
        ms = self.geo.ms
        # registers: one declaration per resolved value
        decls = []
        seen = set()
        for op in _walk(kernel.body):
            for v in _values_in(vars(op).get("result")):
                name = self.resolve(v.name)
                if name in seen:
                    continue
                seen.add(name)
                typ = self._reg_decl(self.values.get(name, v))
                if typ:
                    decls.append(f"  {typ} {_cname(name)};")
            if isinstance(op, ForOp):
                for ia in op.iter_args:
                    name = self.resolve(ia.block_arg.name)
                    if name not in seen:
                        seen.add(name)
                        typ = self._reg_decl(ia.block_arg)
                        if typ:
                            decls.append(f"  {typ} {_cname(name)};")
        fields = []
        for v in self.globals:
            if isinstance(v.type, GlobalType):
                ctype = {GPUType.bf16: "wir::bf16", GPUType.fp32: "float", GPUType.u32: "unsigned"}[v.type.data_type]
                fields.append(f"  wir::gl<{ctype}> {_cname(v.name)[2:]};")
            else:
                fields.append(f"  int {_cname(v.name)[2:]};")
        uses = {c.name for op in _walk(kernel.body) for f in vars(op).values() for c in _values_in(f)}
        dims = 3 if "blockIdx.z" in uses else 2
        # programs whose loop *stop* grows with blockIdx.x (causal query-major
        # loops) run longest first; a loop *start* that grows with it (causal
        # key-major loops) already makes the natural order longest first
        from_x = {self.resolve(op.result.name) for op in _walk(kernel.body)
                  if isinstance(op, IntAffineOp) and isinstance(op.input, Value)
                  and op.input.name == "blockIdx.x" and op.mul > 0}
        causal_x = any(isinstance(op, ForOp) and isinstance(op.stop, Value) and self.resolve(op.stop.name) in from_x
                       for op in _walk(kernel.body))
        wpe = max(self.geo.waves_per_eu, 2) if self._ws else self.geo.waves_per_eu
        if wpe > 2 and self.target.waves_per_eu is None:
            # more than two waves per SIMD only where as many workgroups fit in the LDS, and not in
            # the overlapped attention form (its second score tile is not in the register count)
            by_lds = self.target.lds_bytes // max(self.lds_total, 1024) * self.geo.nw // 4
            wpe = 2 if self._overlapped else max(2, min(wpe, by_lds))
        self.waves_per_simd = wpe
        nt = self.num_threads
        if self.target.persistent:
            if self._ws:
                raise LoweringError("persistent programs do not take the warp-specialised form")
            pid = _persistent_pid_code(self._tile_extents(kernel))
            body = ["  for (int wir_blk = blockIdx.x; wir_blk < wir_nblk; wir_blk += gridDim.x) {",
                    "  wir_drain = 0;",
                    *_persistent_tile_ids(dims, self.target, reverse_x=causal_x),
                    *body,
                    "  wir::barrier();   // the tile's LDS (ring, staging) is free before the next tile's loads",
                    "  }"]
            if self._stream is not None:
                if causal_x or dims != 3:
                    raise LoweringError("persistent_stream takes the non-causal attention forward")
                body = ["  if constexpr (WIR_AL) {", *self._stream_lines, "  } else {", *body, "  }"]
        else:
            pid = _pid_code(dims, self.target, reverse_x=causal_x)
        src = [
            *([f"{HIPCC_FLAGS_MARKER} -mllvm -amdgpu-mfma-vgpr-form=1"] if self.target.mfma_vgpr_form else []),
            "// Generated by warpir_amd.lowering.CDNA4Lowerer for gfx950 -- do not edit.",
            *([f'#define WIR_DMA_CPOL " {_dma_cpol(self.target.dma_cache_policy)}"']
              if self.target.dma_cache_policy else []),
            _header_text(),
            "",
            f"struct {kernel.name}_globals {{",
            *fields,
            "};",
            "",
            f'extern "C" __global__ void __attribute__((amdgpu_flat_work_group_size({nt}, {nt}), '
            f"amdgpu_waves_per_eu({wpe}, {wpe})))",
            f"{kernel.name}(const {kernel.name}_globals globals) {{",
            f"  __shared__ __attribute__((aligned(1024))) char smem[{max(self.lds_total, 1024)}];",
            *pid,
            *([f"  const int wir_wave_hw = wir::wave_id();",
               f"  const bool wir_producer = wir_wave_hw >= {self.geo.nw};  // DMA-only waves",
               f"  const int wir_wave = wir_wave_hw % {self.geo.nw};"] if self._ws
              else [f"  const int wir_wave = wir::wave_id();"]),
            f"  const int wave_row0 = (wir_wave / {self.geo.nw_c}) * {self._wave_rows()};",
            f"  const int wave_col0 = (wir_wave % {self.geo.nw_c}) * {self._wave_cols()};",
        ]
        checks = " && ".join(f"wir::Loader<{t}, {self.geo.nw}>::aligned(globals.{g})"
                             for t, g in sorted(self._aligned_checks)) or "true"
        inb = self._in_bounds_checks(kernel)
        if inb:
            # with these the aligned body needs no zero-page selects (WIR_INB): every tile it
            # loads lies inside its tensor; a launch that fails them takes the checked body
            checks += "".join(f" && {c}" for c in inb)
        src += [
            f"  const bool wir_aligned = {checks};",
            "  auto wir_body = [&](auto wir_tag) {",
            "  constexpr bool WIR_AL = decltype(wir_tag)::value;",
            f"  constexpr bool WIR_INB = WIR_AL && {'true' if inb else 'false'};  "
            f"// aligned tiles all inside the tensors",
            "  (void)WIR_INB;",
            "  int wir_drain = 0;",
            "  (void)wave_row0; (void)wave_col0; (void)wir_drain;",
            *decls,
        ]
        tail = ["  };",
                "  if (wir_aligned) wir_body(wir::bool_tag<true>{});",
                "  else wir_body(wir::bool_tag<false>{});",
                "}", ""]
        return "\n".join(src + body + tail)

    def _in_bounds_checks(self, kernel: Kernel) -> List[str]:
        """Run-time conditions under which every tile the aligned body loads
        lies inside its tensor, or ``[]`` when the kernel's form gives no
        such proof.  Two forms carry one:

        - the reference buffer form (MMAs on ring slots): the prologue loads
          tiles ``0 .. start-1``; iteration ``i`` loads tile ``i - k`` of a
          ring whose loads run ``k`` stages behind the first (``k = 0`` with
          one depth for every ring); a drain step loads tile ``drain + o``,
          the MMA counter plus the step's offset, which with one loop of at
          least ``start`` tiles is ``tiles - start + j + o`` in the drain's
          ``j``-th step;
        - the attention ping-pong (every top-level loop in that form): its
          prologue loads tiles ``start .. start+P-1`` of K and V (P = ring
          slots - 2, plus the one V tile of group B's first phase with a
          barrier every iteration) and its ring loads are skipped past the
          loop's end.

        Every tile coordinate is a constant, a grid index, the loop's tile
        (shifted by a constant) or a drain index.  Each coordinate's largest
        value plus one, times its tile extent, must fit the tensor's extent
        (``nx_`` / ``ny_`` / ``nz_`` for a grid index, the loop's tile count
        plus the shift for the loop's tile, and for the ping-pong also
        ``start + P``); a buffer-form loop must have at least its prologue's
        ``start`` tiles, and no coordinate may be negative.  The lazy
        attention prefetch form (slot views outside the ping-pong: it
        prefetches past the loop's end) relies on the zero page instead.
        Register-hoisted tiles are loaded with their own bounds checks and
        need no condition."""
        ops = list(_walk(kernel.body))
        if any(isinstance(o, TMALoadOp) and self.resolve(o.result.name) not in self._register_tiles for o in ops):
            return []
        loops = [op for op in kernel.body if isinstance(op, ForOp)]
        pingpong = bool(loops) and all(id(op) in self._pp_forms for op in loops)
        if not pingpong and (not any(isinstance(o, MMABufOp) for o in ops)
                             or any(isinstance(o, SlotViewOp) for o in ops)):
            return []
        conds: List[str] = []
        counts_of: Dict[str, List[str]] = {}  # integer value -> tile counts its coordinate reaches
        rows_of: Dict[int, List[str]] = {}    # id(ping-pong ring load) -> tile counts of its row coordinate
        for op in loops:
            if not isinstance(op.start, int) or not isinstance(op.stop, Value) or op.stop not in kernel.inputs:
                return []
            tiles = f"globals.{_cname(op.stop.name)[2:]}"
            if op.tile_size:
                tiles = f"(({tiles}) + {op.tile_size - 1}) / {op.tile_size}"
            if pingpong:
                plan, _swap, _one, every = self._pp_forms[id(op)]
                npro = plan["S"] - 2 + (1 if every == 1 and not self.target.pingpong_split_barrier else 0)
                for ld in (plan["k_load"], plan["v_load"]):
                    rows_of[id(ld)] = [f"({tiles})", str(op.start + npro)]
                continue
            conds.append(f"(({tiles}) >= {op.start})")
            iv = op.induction_var.name
            counts_of[iv] = [f"({tiles})"]
            for o in op.body:
                if isinstance(o, IntAffineOp) and isinstance(o.input, Value) and o.input.name == iv:
                    if o.mul != 1 or op.start + o.add < 0:
                        return []
                    counts_of[o.result.name] = [f"({tiles}) + {o.add}" if o.add else f"({tiles})"]
        if not pingpong:
            # drain indices: wir_drain counts the buffered MMAs, one per loop iteration and one
            # per drain step, so only a kernel with a single loop gives them a closed form
            loop, j = None, 0
            for op in kernel.body:
                if isinstance(op, ForOp):
                    loop, j = op, 0
                elif isinstance(op, MMABufOp):
                    j += 1
                elif isinstance(op, DrainIndexOp):
                    if loop is None or len(loops) != 1 or j + op.offset < 0:
                        return []
                    tiles = counts_of[loop.induction_var.name][0]
                    extra = j + op.offset + 1 - loop.start
                    counts_of[op.result.name] = [f"{tiles} + {extra}" if extra else tiles]
        grid = {"blockIdx.x": "nx_", "blockIdx.y": "ny_", "blockIdx.z": "nz_"}
        for op in ops:
            if not isinstance(op, TMALoadBufOp):
                continue
            if pingpong and id(op) not in rows_of:
                if id(op) in self._pp_prologue:
                    continue          # not issued by the aligned body
                return []
            g = f"globals.{_cname(op.source.name)[2:]}"
            sub = op.source.type.sub_tile_type
            for pos, (c, unit, dim) in enumerate(zip(op.coords, (1, 1, sub.rows, sub.cols), "bdrc")):
                if pingpong and pos == 2:
                    counts = rows_of[id(op)]
                elif isinstance(c, int):
                    if c < 0:
                        return []
                    counts = [str(c + 1)]
                elif isinstance(c, Value) and c.name in grid:
                    counts = [grid[c.name]]
                elif isinstance(c, Value) and c.name in counts_of:
                    counts = counts_of[c.name]
                else:
                    return []
                for count in counts:
                    cond = f"(({count}) * {unit} <= {g}.{dim})"
                    if cond not in conds:
                        conds.append(cond)
        return conds

    def _wave_tile(self) -> RegTileType:
        """The register tile shape that sets the wavefront slices: the first
        MMA's result, or in an MMA-free kernel the first shared -> register copy."""
        for op in _walk(self.kernel.body):
            if isinstance(op, (MMAOp, MMABufOp)):
                return op.result.type if isinstance(op.result.type, RegTileType) else self._rtype(op.accum)
        for op in _walk(self.kernel.body):
            if isinstance(op, CopyOp) and isinstance(op.input.type, SharedTileType):
                return op.result.type
        raise LoweringError("no MMA and no shared -> register copy")

    def _wave_rows(self) -> int:
        return self._wave_tile().rows

    def _wave_cols(self) -> int:
        return self._wave_tile().cols


# ----------------------------------------------------------------------
# schedule analysis: vmcnt per wait, write-after-read barriers
# ----------------------------------------------------------------------
def _schedule(kernel: Kernel, low: CDNA4Lowerer):
    """Simulate the kernel's load / wait / MMA order with concrete trip counts.

    Returns ``(wait_n, war)``: ``wait_n[id(wait_op)]`` is the number of this
    wave's LDS-DMA instructions that may stay in flight at the wait (the
    minimum over every simulated instance), and ``war`` the ids of load ops
    that must be preceded by a workgroup barrier because a tile they
    overwrite was read since the last barrier.
    """
    wait_n: Dict[int, int] = {}
    war: set = set()
    for trips in (0, 1, 2, 3, 5, 8):
        sim = _Sim(low, trips)
        sim.run(kernel.body)
        for k, n in sim.wait_n.items():
            wait_n[k] = min(wait_n.get(k, n), n)
        war |= sim.war
    return wait_n, war


class _Sim:
    def __init__(self, low: CDNA4Lowerer, trips: int):
        self.low = low
        self.trips = trips
        self.env: Dict[str, int] = {}
        self.drain = 0
        self.issued: List[Tuple[Tuple[str, int], int]] = []   # (key, instructions)
        self.read_since_barrier: set = set()
        self.wait_n: Dict[int, int] = {}
        self.war: set = set()
        self.landed: set = set()

    def val(self, x) -> int:
        if isinstance(x, int):
            return x
        name = self.low.resolve(x.name)
        return self.env.get(name, 0)

    def slot(self, s) -> int:
        if isinstance(s, int):
            return s
        if s.value is None:
            return self.drain % s.modulus
        return (self.val(s.value) + s.offset) % s.modulus

    def key_of_tile(self, v: Value) -> Tuple[str, int]:
        low = self.low
        name = low.resolve(v.name)
        view = low._views().get(name)
        if view is not None:
            return (low.resolve(view.buf.name), self.slot(view.slot))
        return (name, 0)

    def load(self, op, key, tile) -> None:
        if key in self.read_since_barrier:
            self.war.add(id(op))
            self.read_since_barrier.clear()
        self.landed.discard(key)
        self.issued.append((key, self.low.loads_per_wave(tile)))

    def wait(self, op, keys) -> None:
        last = -1
        for k, (key, _n) in enumerate(self.issued):
            if key in keys:
                last = k
        n_after = sum(n for _k, n in self.issued[last + 1:]) if last >= 0 else sum(n for _k, n in self.issued)
        self.wait_n[id(op)] = min(self.wait_n.get(id(op), n_after), n_after)
        for key, _n in self.issued[:last + 1]:
            self.landed.add(key)
        self.issued = self.issued[last + 1:]
        self.read_since_barrier.clear()

    def read(self, key) -> None:
        self.read_since_barrier.add(key)

    def run(self, ops) -> None:
        low = self.low
        for op in ops:
            if isinstance(op, TMALoadOp):
                if low.resolve(op.result.name) in low._register_tiles:
                    continue
                self.load(op, (low.resolve(op.result.name), 0), op.result.type)
            elif isinstance(op, TMALoadBufOp):
                key = (low.resolve(op.buf.name), self.slot(op.slot))
                self.load(op, key, op.buf.type.tile_type)
            elif isinstance(op, WaitOp):
                keys = {self.key_of_tile(v) for v in op.values if low.resolve(v.name) not in low._register_tiles}
                if keys:
                    self.wait(op, keys)
            elif isinstance(op, WaitBufOp):
                s = self.slot(op.slot)
                self.wait(op, {(low.resolve(b.name), s) for b in op.bufs})
            elif isinstance(op, MMAOp):
                for v in (op.a, op.b):
                    if low._lds_key(v) is not None and low.resolve(v.name) not in low._register_tiles:
                        self.read(self.key_of_tile(v))
            elif isinstance(op, MMABufOp):
                self.read((low.resolve(op.a_buf.name), self.slot(op.a_slot)))
                self.read((low.resolve(op.b_buf.name), self.slot(op.b_slot)))
                if isinstance(op.a_slot, BufSlotExpr):
                    self.drain += 1
            elif isinstance(op, DrainIndexOp):
                self.env[low.resolve(op.result.name)] = self.drain + op.offset
            elif isinstance(op, IntAffineOp):
                self.env[low.resolve(op.result.name)] = self.val(op.input) * op.mul + op.add
            elif isinstance(op, IntDivOp):
                self.env[low.resolve(op.result.name)] = self.val(op.input) // max(1, self.val(op.divisor))
            elif isinstance(op, ForOp):
                start = self.val(op.start)
                step = self.val(op.step) or 1
                iv = low.resolve(op.induction_var.name)
                for t in range(self.trips):
                    self.env[iv] = start + t * step
                    self.run(op.body)
                self.env[iv] = start + self.trips * step


# ----------------------------------------------------------------------
# helpers
# ----------------------------------------------------------------------
def _walk(ops):
    for op in ops:
        yield op
        if isinstance(op, ForOp):
            yield from _walk(op.body)


def _op_values(op):
    """The Values an op names in its fields (not the bodies of nested loops)."""
    import dataclasses
    for f in dataclasses.fields(op):
        if f.name in ("body", "iter_args", "results"):
            continue
        yield from _values_in(getattr(op, f.name))


def _values_in(x):
    if isinstance(x, Value):
        yield x
    elif isinstance(x, (tuple, list)):
        for y in x:
            yield from _values_in(y)
    elif isinstance(x, BufSlotExpr) and x.value is not None:
        yield x.value


def _mma_operand_types(op):
    if isinstance(op, MMAOp):
        a_t, b_t = op.a.type, op.b.type
        if isinstance(b_t, SharedBufferType):
            b_t = b_t.tile_type
        if isinstance(a_t, SharedBufferType):
            a_t = a_t.tile_type
        return a_t, b_t, op.transpose_b
    return op.a_buf.type.tile_type, op.b_buf.type.tile_type, False


def _as4d(shape) -> Tuple[int, int, int, int]:
    s = tuple(int(x) for x in shape)
    while len(s) < 4:
        s = (1,) + s
    return s


def _is_vec_tile(t) -> bool:
    """An fp32 ``L x 1`` shared tile: a vector (e.g. per-query statistics) in LDS."""
    return isinstance(t, SharedTileType) and t.data_type == GPUType.fp32 and t.cols == 1


def _tile_bytes(t) -> int:
    """LDS bytes of one shared tile (ring slot stride)."""
    if _is_vec_tile(t):
        return _align(t.rows * 4, 256)
    return _align(t.rows * t.cols * 2, 1024)


def _align(x: int, a: int) -> int:
    return _ceil_div(x, a) * a


def _flt(x: float) -> str:
    return repr(float(x)) + "f"


def _pid_code(dims: int, target: CDNA4Target, reverse_x: bool) -> List[str]:
    lines = [
        "  const int nx_ = gridDim.x, ny_ = gridDim.y, nz_ = gridDim.z;",
        "  const int hw_ = blockIdx.x + nx_ * (blockIdx.y + ny_ * blockIdx.z);",
    ]
    if target.xcd_remap:
        lines.append("  const int lid_ = wir::remap_xcd(hw_, nx_ * ny_ * nz_);")
    else:
        lines.append("  const int lid_ = hw_;")
    if dims == 2:
        lines += [
            "  int pid_x, pid_y;",
            f"  wir::grouped_tile<{target.group_m}>(lid_, nx_, ny_, pid_x, pid_y);",
            "  const int pid_z = 0;",
        ]
    else:
        lines += [
            "  int pid_x = lid_ % nx_;",
            "  const int pid_y = (lid_ / nx_) % ny_;",
            "  const int pid_z = lid_ / (nx_ * ny_);",
        ]
    if reverse_x:
        lines.append("  pid_x = nx_ - 1 - pid_x;  // longest causal rows first")
    lines.append("  (void)pid_x; (void)pid_y; (void)pid_z;")
    return lines


def _persistent_pid_code(extents: List[str]) -> List[str]:
    """Program-independent part of the persistent form: tile counts per axis
    from the output tensor, and the mutable tile ids."""
    return [
        f"  const int nx_ = {extents[0]}, ny_ = {extents[1]}, nz_ = {extents[2]};",
        "  const int wir_nblk = nx_ * ny_ * nz_;   // output tiles; this program takes every gridDim.x-th",
        "  int pid_x = 0, pid_y = 0, pid_z = 0;",
        "  (void)pid_x; (void)pid_y; (void)pid_z;",
    ]


def _persistent_tile_ids(dims: int, target: CDNA4Target, reverse_x: bool) -> List[str]:
    """Tile ids of tile wir_blk: the mapping _pid_code gives dispatch index wir_blk."""
    lines = [f"  {{ const int lid_ = {'wir::remap_xcd(wir_blk, wir_nblk)' if target.xcd_remap else 'wir_blk'};"]
    if dims == 2:
        lines.append(f"    wir::grouped_tile<{target.group_m}>(lid_, nx_, ny_, pid_x, pid_y);")
    else:
        lines.append("    pid_x = lid_ % nx_; pid_y = (lid_ / nx_) % ny_; pid_z = lid_ / (nx_ * ny_);")
    if reverse_x:
        lines.append("    pid_x = nx_ - 1 - pid_x;")
    lines.append("  }")
    return lines


_HEADER_CACHE: Dict[str, str] = {}


def _dma_cpol(policy: str) -> str:
    """The cache-policy modifiers of CDNA4Target.dma_cache_policy, checked."""
    words = policy.split()
    if not words or any(w not in ("sc0", "sc1", "nt") for w in words) or len(set(words)) != len(words):
        raise ValueError(f"dma_cache_policy: expected distinct words from sc0, sc1, nt; got {policy!r}")
    return " ".join(w for w in ("sc0", "sc1", "nt") if w in words)


def _header_text() -> str:
    if "h" not in _HEADER_CACHE:
        with open(HEADER_PATH, "r") as f:
            _HEADER_CACHE["h"] = f.read()
    return _HEADER_CACHE["h"]


__all__ = ["CDNA4Lowerer", "CDNA4Target", "LaunchConfig", "LoweringError"]
