"""SSA values and operations of the WarpIR tile IR.

The class names, field names, field order and defaults follow the
reference (``warpir/ir/ops.py:9-285``) so that IR builders written for
the reference construct the same objects here.  The ops after
``DivRowOp`` marked *additive* have no counterpart in the reference; they
carry what the MI355X configurations need (log-sum-exp output, causal
masking, data-dependent loop bounds) without changing any existing
signature.
"""
from __future__ import annotations

from dataclasses import dataclass, field, fields
from typing import Dict, Union

from .types import TypeRef


@dataclass(frozen=True)
class Value:
    """A named, typed SSA value (``ops.py:9-16``)."""

    name: str
    type: TypeRef

    def __repr__(self) -> str:
        return f"%{self.name}: {self.type}"


@dataclass(frozen=True)
class BufSlotExpr:
    """Ring-slot index ``(value + offset) % modulus`` (``ops.py:19-28``).

    ``value=None`` stands for the drain counter: a slot cursor that the
    lowering advances by one after every buffered MMA, so that the
    epilogue's drain steps consume the slots left in flight by the loop.
    """

    value: Union[Value, None]
    offset: int = 0
    modulus: int = 1


BufIdx = Union[int, BufSlotExpr]


def _subst(item, table):
    if isinstance(item, Value):
        return table.get(item, item)
    if isinstance(item, tuple):
        return tuple(_subst(x, table) for x in item)
    if isinstance(item, BufSlotExpr):
        inner = None if item.value is None else _subst(item.value, table)
        return BufSlotExpr(value=inner, offset=item.offset, modulus=item.modulus)
    return item


class Op:
    """Base class of every IR operation (``ops.py:34-50``)."""

    def __repr__(self) -> str:
        body = ", ".join(f"{k}={v}" for k, v in vars(self).items())
        return f"{type(self).__name__}({body})"

    def substitute(self, replacements: Dict[Value, Union[Value, int]]) -> "Op":
        """Return a copy with every ``Value`` operand looked up in *replacements*.

        Tuples and slot expressions are rewritten element-wise; other
        fields are kept.  Used to specialise prologue loads on a constant
        induction value (``modulo_scheduler.py:261-263``).
        """
        return type(self)(**{k: _subst(v, replacements) for k, v in vars(self).items()})


# --- tile operations (SSA form) -------------------------------------------

@dataclass(frozen=True)
class ZeroOp(Op):
    """``result`` = a tile or column vector of zeros (``ops.py:57-60``)."""

    result: Value


@dataclass(frozen=True)
class TMALoadOp(Op):
    """Asynchronous global -> shared tile load (``ops.py:63-68``).

    ``coords`` = (batch, depth, row_tile, col_tile) in units of the
    source's ``sub_tile_type``.  On CDNA4 this is a direct global->LDS
    DMA (``global_load_lds_dwordx4``) completed by a later ``WaitOp``.
    """

    result: Value
    source: Value
    coords: tuple


@dataclass(frozen=True)
class WaitOp(Op):
    """Block until the loads that produced ``values`` have landed (``ops.py:71-74``)."""

    values: tuple


@dataclass(frozen=True)
class MMAOp(Op):
    """Matrix multiply (``ops.py:77-88``).

    ``transpose_b=False``: ``result = a @ b + accum``.
    ``transpose_b=True``:  ``result = a @ b^T`` (``accum`` is not read).
    """

    result: Value
    a: Value
    b: Value
    accum: Value
    transpose_b: bool = False


@dataclass(frozen=True)
class TMAStoreOp(Op):
    """Store a tile (register or shared) to global memory (``ops.py:91-96``)."""

    source: Value
    dest: Value
    coords: tuple


# --- element-wise and row-reduction operations ----------------------------

@dataclass(frozen=True)
class NegInftyOp(Op):
    """``result`` = a tile or column vector of -inf (``ops.py:103-106``)."""

    result: Value


@dataclass(frozen=True)
class CopyOp(Op):
    """Copy, converting the element type when the types differ (``ops.py:109-113``)."""

    result: Value
    input: Value


@dataclass(frozen=True)
class MulScalarOp(Op):
    """``result = input * scalar`` for a compile-time constant (``ops.py:116-121``)."""

    result: Value
    input: Value
    scalar: float


@dataclass(frozen=True)
class SubOp(Op):
    """``result = a - b`` element-wise (``ops.py:124-129``)."""

    result: Value
    a: Value
    b: Value


@dataclass(frozen=True)
class MulOp(Op):
    """``result = a * b`` element-wise (``ops.py:132-137``)."""

    result: Value
    a: Value
    b: Value


@dataclass(frozen=True)
class Exp2Op(Op):
    """``result = 2 ** input`` element-wise (``ops.py:140-144``)."""

    result: Value
    input: Value


@dataclass(frozen=True)
class RowMaxOp(Op):
    """``result[r] = max(max_c tile[r, c], prev[r])`` (``ops.py:147-155``)."""

    result: Value
    tile: Value
    prev: Value


@dataclass(frozen=True)
class RowSumOp(Op):
    """``result[r] = sum_c tile[r, c] + prev[r]`` (``ops.py:158-166``)."""

    result: Value
    tile: Value
    prev: Value


@dataclass(frozen=True)
class SubRowOp(Op):
    """``result[r, c] = tile[r, c] - vec[r]`` (``ops.py:169-174``)."""

    result: Value
    tile: Value
    vec: Value


@dataclass(frozen=True)
class MulRowOp(Op):
    """``result[r, c] = tile[r, c] * vec[r]`` (``ops.py:177-182``)."""

    result: Value
    tile: Value
    vec: Value


@dataclass(frozen=True)
class DivRowOp(Op):
    """``result[r, c] = tile[r, c] / vec[r]`` (``ops.py:185-190``)."""

    result: Value
    tile: Value
    vec: Value


# --- additive element-wise / index operations (no reference counterpart) ---

@dataclass(frozen=True)
class AddOp(Op):
    """*Additive.* ``result = a + b`` element-wise."""

    result: Value
    a: Value
    b: Value


@dataclass(frozen=True)
class Log2Op(Op):
    """*Additive.* ``result = log2(input)`` element-wise (log-sum-exp output)."""

    result: Value
    input: Value


@dataclass(frozen=True)
class CausalMaskOp(Op):
    """*Additive.* Lower-triangular mask of a block-level score tile.

    With ``R x C`` the block-level shape of ``tile`` (all wavefront slices
    together), element ``(r, c)`` keeps its value when
    ``col_tile*C + c <= row_tile*R + r`` and becomes -inf otherwise.
    Mirrors the diagonal-tile masking of the reference's causal FA
    kernel (``kernel_examples/attention/mha_h100.cu:160-176``).  With
    ``transposed`` the tile holds transposed scores (keys along the rows,
    as in the key-major backward): ``(r, c)`` keeps its value when
    ``row_tile*R + r <= col_tile*C + c`` (``make_causal_t``,
    ``mha_h100.cu:391-403``).
    """

    result: Value
    tile: Value
    row_tile: Union[Value, int]
    col_tile: Union[Value, int]
    transposed: bool = False


@dataclass(frozen=True)
class SubColOp(Op):
    """*Additive.* ``result[r, c] = tile[r, c] - vec[c]`` (``vec`` a row_vec)."""

    result: Value
    tile: Value
    vec: Value


@dataclass(frozen=True)
class LazyMaxOp(Op):
    """*Additive.* ``result = cand if cand > prev + slack else prev`` element-wise.

    The online-softmax running max with a slack: the stabiliser only moves
    when the new maximum exceeds it by more than ``slack`` (in the units of
    ``prev``), so the rescale of the accumulators (``exp2(prev - result)``)
    is exactly 1 on most steps.  Softmax is invariant to the constant
    subtracted, so only rounding differs; the exponentials stay below
    ``2**(slack * scale)`` with ``scale`` the factor applied before ``exp2``.
    """

    result: Value
    prev: Value
    cand: Value
    slack: float


@dataclass(frozen=True)
class LoadVecOp(Op):
    """*Additive.* Synchronous load of a register vector from an fp32 global.

    The global's sub tile is ``L x 1``; ``coords = (batch, depth, tile, 0)``
    select elements ``tile*L .. tile*L + L - 1`` along its rows.  With a
    shared fp32 ``L x 1`` tile as ``source`` (loaded by ``tma_load`` like any
    tile, so it can be pipelined) and empty ``coords``, the vector is read
    from that tile.  A col_vec
    result takes them as per-row values of its tile, a row_vec result as
    per-column values.  Elements outside the tensor read 0.  (Statistics
    saved by the forward pass, e.g. the log-sum-exp, for the backward.)
    """

    result: Value
    source: Value
    coords: tuple


@dataclass(frozen=True)
class IntAffineOp(Op):
    """*Additive.* Integer ``result = input * mul + add``.

    Gives loops a data-dependent bound, e.g. the causal KV extent
    ``(q_tile + 1) * BLOCK_Q`` (``mha_h100.cu:140-145``).
    """

    result: Value
    input: Union[Value, int]
    mul: int = 1
    add: int = 0


@dataclass(frozen=True)
class IntDivOp(Op):
    """*Additive.* Integer ``result = input // divisor`` (non-negative operands).

    Maps a query head to its key/value head under grouped-query attention,
    ``kv_head = head // (query heads per kv head)`` (``mha_h100.cu:74,519``).
    """

    result: Value
    input: Union[Value, int]
    divisor: Union[Value, int]


@dataclass(frozen=True)
class DrainIndexOp(Op):
    """*Additive.* Integer ``result`` = the logical iteration of the next
    buffered MMA (the drain counter, not reduced by any ring size) plus
    ``offset``.

    Lets a drain step of a pipeline whose rings differ in depth load a
    later tile: a load scheduled ``k`` stages ahead of its MMA fetches
    tile ``drain + k`` in the drain, as it would have in the loop.
    """

    result: Value
    offset: int = 0


@dataclass(frozen=True)
class ReduceSlicesOp(Op):
    """*Additive.* Split-K fix-up of one output tile.

    ``partials`` is an fp32 ``[1, S, M, N]`` global whose depth slices are
    the K slices of a product: the program of slice ``d`` has just stored
    its tile at ``coords = (batch, d, row_tile, col_tile)``.  ``dest`` is the
    bf16 ``[1, 1, M, N]`` result and ``arrivals`` a u32 global of one
    counter per output tile (row-major over the tiles of ``dest``), zero
    before the first launch.  Once all ``S`` slices have stored the tile,
    ``dest``'s tile becomes the bf16 rounding of their fp32 sum taken in
    slice order (from 0), and its counter is zero again.  The lowering lets
    the last program to arrive do the sum; no program waits for another.
    """

    partials: Value
    dest: Value
    arrivals: Value
    coords: tuple


@dataclass(frozen=True)
class PipelineStageOp(Op):
    """*Additive.* Placement mark of a software-pipelined loop body: the ops
    after it, up to the next mark or the yield, run ``stage`` iterations
    later than the ops before the body's first mark -- each iteration
    issues them for iteration ``i - stage``, ahead of its own stage-0 work.

    It computes nothing: the loop means the same with or without it (the
    interpreter skips it).  ``kernel_pass`` writes it from the modulo
    schedule of the loop's compute ops, and the lowering follows it: with
    the PV MMA behind a ``pipeline_stage(1)``, iteration ``i`` starts with
    ``O += P_{i-1} V_{i-1}`` next to ``S_i = Q K_i^T``; with the softmax ops
    behind it, tile ``i``'s softmax runs beside ``S_{i+1}``'s MFMAs.
    """

    stage: int = 1


# --- buffer operations (post-pipeline form) --------------------------------

@dataclass(frozen=True)
class AllocSharedOp(Op):
    """Allocate a ring of shared tiles (``ops.py:197-200``)."""

    result: Value


@dataclass(frozen=True)
class TMALoadBufOp(Op):
    """Asynchronous load into ring slot ``slot`` of ``buf`` (``ops.py:203-209``)."""

    buf: Value
    slot: BufIdx
    source: Value
    coords: tuple


@dataclass(frozen=True)
class WaitBufOp(Op):
    """Block until ring slot ``slot`` of every buffer in ``bufs`` has landed (``ops.py:212-219``)."""

    bufs: tuple
    slot: BufIdx


@dataclass(frozen=True)
class MMABufOp(Op):
    """``accum += a_buf[a_slot] @ b_buf[b_slot]`` from ring slots (``ops.py:222-230``).

    The accumulation is in place into ``accum``'s storage (the reference
    lowering's ``mma_AB(accum, ...)``, ``lowering.py:472-481``); ``result``
    names the updated value.
    """

    result: Value
    a_buf: Value
    a_slot: BufIdx
    b_buf: Value
    b_slot: BufIdx
    accum: Value


@dataclass(frozen=True)
class SlotViewOp(Op):
    """*Additive.* ``result`` names the shared tile held in ring slot ``slot`` of ``buf``.

    Lets an ``MMAOp`` (with its ``transpose_b`` flag and register
    operands) read a ring slot in the buffer form of a loop whose body is
    more than loads and MMAs -- the pipelined FlashAttention loop.
    """

    result: Value
    buf: Value
    slot: BufIdx


# --- control flow -----------------------------------------------------------

@dataclass(frozen=True)
class YieldOp(Op):
    """Loop-body terminator carrying the next iteration's values (``ops.py:237-240``)."""

    values: tuple


@dataclass(frozen=True)
class IterArg:
    """A loop-carried value: ``block_arg`` starts as ``init`` (``ops.py:243-251``)."""

    block_arg: Value
    init: Value


@dataclass(frozen=True)
class ForOp(Op):
    """``scf.for``-style loop with loop-carried values (``ops.py:254-273``).

    With ``tile_size`` set the trip bound is ``ceil(stop / tile_size)``.
    ``results[i]`` is the final value of ``iter_args[i]``.
    """

    induction_var: Value
    start: Union[Value, int]
    stop: Union[Value, int]
    step: Union[Value, int]
    iter_args: tuple
    body: tuple
    results: tuple
    tile_size: Union[int, None] = None


# --- top level ---------------------------------------------------------------

@dataclass(frozen=True)
class Kernel:
    """A kernel: its launch arguments are ``inputs`` then ``outputs`` (``ops.py:280-285``)."""

    name: str
    inputs: tuple = field(default_factory=tuple)
    outputs: tuple = field(default_factory=tuple)
    body: tuple = field(default_factory=tuple)


def op_fields(op: Op) -> dict:
    """Field name -> value of an op, in declaration order."""
    return {f.name: getattr(op, f.name) for f in fields(op)}
