"""kernel_pass's phase schedule of the attention loop's compute ops (CPU).

Every MMA and softmax op of the loop body is an ``MSInstruction``: MMAs on
the MFMA unit, the softmax chain on the VALU.  The exact search places them
in phase slots -- with "alternate" phases the initiation interval is an
MFMA phase followed by a VALU phase, with "mixed" one slot holds both -- and
the pass marks the placement with ``pipeline_stage``.

Pins (beyond restating the pass):
* the solver's slot classes against a brute-force enumeration of every
  (ii, offsets) tuple on random small instances;
* the stage of every compute op of the config-4 and config-5 loops, and on
  a reduced instance (score MMA, three softmax ops, PV MMA, with the
  loop-carried edges) against a brute force over all slot assignments;
* the lowering follows the mark: without it the same loop is not rotated.
"""
import itertools
import random

import pytest

from warpir_amd import kernels
from warpir_amd.ir import ForOp, MMAOp, PipelineStageOp
from warpir_amd.lowering import CDNA4Lowerer
from warpir_amd.passes import _modsched_search as ms
from warpir_amd.passes.modulo_scheduler import (_phase_stages, gfx950_attention_cost_model, kernel_pass,
                                                op_cycles, op_unit, phase_estimates)
from warpir_amd.printing import format_kernel
from warpir_amd.workloads import build_mha_forward_kernel


def _brute(lat, edges, depth, slot_class, max_ii=6, horizon=8):
    """Smallest (ii, makespan) over every offset tuple in [0, horizon)."""
    n = len(lat)
    best = None
    for ii in range(0, max_ii + 1):
        if any(c is not None and c >= ii for c in slot_class):
            continue   # (ii = 0 only without slot classes, as in the solver)
        for offs in itertools.product(range(horizon), repeat=n):
            if any(c is not None and o % ii != c for o, c in zip(offs, slot_class)):
                continue
            if any(offs[b] + k * ii < offs[a] + lat[a] for a, b, k in edges):
                continue
            span = (depth - 1) * ii + max(o + l for o, l in zip(offs, lat))
            if best is None or (ii, span) < best:
                best = (ii, span)
        if best is not None:
            return best
    return best


@pytest.mark.parametrize("seed", range(12))
def test_slot_classes_match_brute_force(seed):
    rnd = random.Random(seed)
    n = rnd.randint(2, 4)
    lat = [rnd.randint(0, 2) for _ in range(n)]
    edges = [(a, b, 0) for a in range(n) for b in range(a + 1, n) if rnd.random() < 0.5]
    edges += [(b, a, 1) for a in range(n) for b in range(a, n) if rnd.random() < 0.2]
    slot_class = [rnd.choice([None, 0, 1]) for _ in range(n)]
    depth = 3
    p = ms.Problem(latencies=lat, resources=["u"] * n, edges=edges, depth=depth, max_cycles=30, capacity={},
                   slot_class=slot_class)
    found = ms.solve(p)
    want = _brute(lat, edges, depth, slot_class)
    if want is None:
        assert found is None or found[0] > 6
        return
    assert found is not None and (found[0], found[2]) == want
    ii, offs, _ = found
    assert all(c is None or o % ii == c for o, c in zip(offs, slot_class))


def _loop(kernel):
    return next(op for op in kernel.body if isinstance(op, ForOp))


def _stages(kernel):
    """Stage of each compute op from the marks in the pass's output loop body."""
    out, stage = {}, 0
    for op in _loop(kernel).body:
        if isinstance(op, PipelineStageOp):
            stage = op.stage
        elif op_unit(op):
            out[type(op).__name__ + ":" + op.result.name] = stage
    return out


@pytest.mark.parametrize("name", ["mha_d128", "mha_d64_causal", "mha_d128_fold", "mha_d128_s5"])
def test_alternate_phases_put_the_pv_one_stage_later(name):
    """Config 4 (eight waves, two per SIMD) and config 5 (three waves per SIMD): an MFMA phase,
    then a VALU phase.  S = Q K^T and the softmax chain of tile i share stage 0; the PV MMA
    needs P, which the VALU phase produces, so it waits for the next MFMA phase: stage 1, the
    top of iteration i + 1, next to S_{i+1}."""
    st = _stages(kernels.kernel(name))
    assert st.pop("MMAOp:o_new") == 1
    assert st.pop("MMAOp:att") == 0
    assert set(st.values()) == {0}
    body = _loop(kernels.kernel(name)).body
    assert isinstance(body[-3], PipelineStageOp) and isinstance(body[-2], MMAOp) and not body[-2].transpose_b
    assert "pipeline_stage(1)" in format_kernel(kernels.kernel(name))


def test_mixed_phases_put_the_softmax_beside_the_next_scores():
    """One co-issue phase per iteration (the FA3 / Twill placement): S_{i+1}'s MFMAs are
    issued while tile i's softmax runs, so every op that reads the scores moves to stage 1;
    the copy of the carried running max, which does not, stays at stage 0."""
    st = _stages(kernels.kernel("mha_d128_ovl"))
    assert st.pop("MMAOp:att") == 0
    assert st.pop("CopyOp:max_prev") == 0 and st.pop("MulScalarOp:max_prev_sc") == 0
    assert set(st.values()) == {1}


def test_phase_stages_match_brute_force_on_a_reduced_loop():
    """Reduced instance of the loop: S = Q K^T (MFMA), m = row_max(S, m') carried,
    X = sub_row(S, m), P = exp2(X), Pb = bf16(P), O = PV(Pb, O') carried.  Brute force over
    every slot of a three-iteration window for each op, both phase structures, taking the
    shortest span and then the earliest offsets; its stages must be the pass's."""
    import types

    from warpir_amd.ir import (ColVecType, CopyOp, Exp2Op, GPUType, IterArg, RegTileType, RowMaxOp,
                               SharedTileType, SubRowOp, Value, YieldOp)
    # (unit, producers at distance 0, producers at distance 1)
    ops = [("mfma", [], []), ("valu", [0], [1]), ("valu", [0, 1], []), ("valu", [2], []), ("valu", [3], []),
           ("mfma", [4], [5])]
    f32, b16 = RegTileType(GPUType.fp32, 32, 64), RegTileType(GPUType.bf16, 32, 64)
    cv = ColVecType(GPUType.fp32, 32, 64)
    q, kt, vt = (Value(n, SharedTileType(GPUType.bf16, 64, 64)) for n in ("q", "k", "v"))
    s_, x, p, pb = Value("s", f32), Value("x", f32), Value("p", f32), Value("pb", b16)
    m0, m1, o0, o1 = Value("m0", cv), Value("m1", cv), Value("o0", f32), Value("o1", f32)
    body = [MMAOp(result=s_, a=q, b=kt, accum=Value("z", f32), transpose_b=True), RowMaxOp(result=m1, tile=s_, prev=m0),
            SubRowOp(result=x, tile=s_, vec=m1), Exp2Op(result=p, input=x), CopyOp(result=pb, input=p),
            MMAOp(result=o1, a=pb, b=vt, accum=o0), YieldOp(values=(o1, m1))]
    loop = types.SimpleNamespace(iter_args=(IterArg(block_arg=o0, init=o0), IterArg(block_arg=m0, init=m0)))
    for mode, ii in (("alternate", 2), ("mixed", 1)):
        lat = [1 if u == "mfma" else 0 for u, _, _ in ops]
        cls = [(0 if u == "mfma" else 1) if mode == "alternate" else 0 for u, _, _ in ops]
        edges = [(a, k, 0) for k, (_, d0, _) in enumerate(ops) for a in d0]
        edges += [(a, k, 1) for k, (_, _, d1) in enumerate(ops) for a in d1]
        best = None
        for offs in itertools.product(range(3 * ii), repeat=len(ops)):
            if any(o % ii != c for o, c in zip(offs, cls)):
                continue
            if any(offs[b] + k * ii < offs[a] + lat[a] for a, b, k in edges):
                continue
            key = (max(o + l for o, l in zip(offs, lat)), offs)
            if best is None or key < best:
                best = key
        want = [o // ii - min(best[1]) // ii for o in best[1]]
        got = _phase_stages(loop, body, mode)
        assert [got[id(o)] for o in body[:6]] == want, (mode, want)
        assert want == ([0, 0, 0, 0, 0, 1] if mode == "alternate" else [0, 1, 1, 1, 1, 1])


def test_phase_estimates_prefer_alternation_on_gfx950():
    """With the measured issue costs (MFMA 32 cycles, VALU 4, exp 8, 4 VALU hidden per MFMA,
    a lone wave's dependent chain at ~10 cycles per instruction) the alternating phases are
    shorter than co-issue at every waves-per-SIMD count of the forward kernels, which matches
    the timings (the overlapped 4-wave form ran 953 against 991 TFLOP/s)."""
    for name in ("mha_d128", "mha_d64_causal"):
        ops = [o for o in _loop(kernels.kernel(name)).body if op_unit(o)]
        mfma = sum(op_cycles(o) for o in ops if op_unit(o) == "mfma")
        assert mfma == (32 if name == "mha_d128" else 16) * 32
        for w in (1, 2, 3):
            est = phase_estimates(ops, w)
            assert est["alternate"] < est["mixed"], (name, w, est)


def test_lowering_follows_the_placement_mark():
    """The same config-4 and config-5 loops without a phase schedule (no mark): the ping-pong
    form and the rotated lazy loop are not emitted; with the mark they are."""
    k_plain = kernel_pass(build_mha_forward_kernel(d=128, block_q=256, block_kv=64, wave_rows=32,
                                                   rescale_slack=kernels.LAZY_SLACK),
                          cost_model=gfx950_attention_cost_model(256, 64, 128, lds_budget=128 * 1024,
                                                                 min_stages=4))
    assert "pipeline_stage" not in format_kernel(k_plain)
    assert "const int wir_grp =" not in CDNA4Lowerer().lower(k_plain)
    assert "const int wir_grp =" in CDNA4Lowerer().lower(kernels.kernel("mha_d128"))
    c5_plain = kernel_pass(build_mha_forward_kernel(d=64, block_q=128, block_kv=64, wave_rows=32, causal=True,
                                                    name="mha_fwd_causal", rescale_slack=kernels.LAZY_SLACK),
                           cost_model=gfx950_attention_cost_model(128, 64, 64))
    rotated = CDNA4Lowerer().lower(kernels.kernel("mha_d64_causal"))
    plain = CDNA4Lowerer().lower(c5_plain)
    # the rotated loop issues the last tile's PV after the loop, at v_i = stop
    assert "const int v_i = (((v_kv_stop) + 63) / 64);" in rotated
    assert "const int v_i = (((v_kv_stop) + 63) / 64);" not in plain
