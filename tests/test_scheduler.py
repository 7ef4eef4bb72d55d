"""Modulo scheduler (CPU): the reference model's known answer and brute force.

Pins (beyond restating the model):
* the GEMM model of the reference pass has the unique optimum ii=6,
  makespan 40, stage_of {load_a: 0, load_b: 0, mma: 2}, 3 stages -- derived
  by hand from ``warpir/passes/modulo_scheduler.py:51-217``;
* the exact search agrees with an independent brute-force enumeration in C
  (``oracle/sched_bruteforce.c``, every (ii, offsets) tuple checked cycle by
  cycle) on random small instances.
"""
import os
import random
import subprocess

import pytest

from warpir_amd.passes import _modsched_search as ms
from warpir_amd.passes.modulo_scheduler import (GFX950_COST_MODEL, MSInstruction, MSInstructionEdge,
                                                MSInstructionManager, CostModel, kernel_pass)
from warpir_amd.workloads import build_gemm_kernel
from warpir_amd.ir import ForOp, MMABufOp

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BRUTE = os.path.join(ROOT, "oracle", "_bin", "sched_bruteforce")


def _gemm_manager():
    la = MSInstruction("tma", 12, "load_a", [])
    lb = MSInstruction("tma", 12, "load_b", [])
    mma = MSInstruction("tc", 4, "mma", [])
    mma.parent_edges += [MSInstructionEdge(la, mma, 0), MSInstructionEdge(lb, mma, 0),
                         MSInstructionEdge(mma, mma, 1)]
    m = MSInstructionManager()
    for x in (la, lb, mma):
        m.add_instruction(x)
    return m


def test_reference_gemm_model_known_answer():
    pro, steady, epi, ii, stages, stage_of = _gemm_manager().solve(100, 5, {"tma": 4, "tc": 1})
    assert ii == 6 and stages == 3
    assert stage_of == {"load_a": 0, "load_b": 0, "mma": 2}
    assert pro == [[(0, "load_a"), (0, "load_b")], [(1, "load_a"), (1, "load_b")]]
    assert epi == [[("mma", 1)], [("mma", 0)]] or epi == [[("mma", 2 - 1)], [("mma", 2 - 2)]]


def test_reference_gemm_model_makespan_and_uniqueness():
    if not os.path.exists(BRUTE):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    # n depth max_cycles nres / caps / (lat res)* / nedges (p c k)*
    inp = "3 5 100 2\n4 1\n12 0 12 0 4 1\n3 0 2 0 1 2 0 2 2 1\n"
    out = subprocess.run([BRUTE], input=inp, capture_output=True, text=True, check=True).stdout.split()
    assert out[0] == "40" and out[1] == "1" and out[2] == "6"
    p = ms.Problem([12, 12, 4], ["tma", "tma", "tc"], [(0, 2, 0), (1, 2, 0), (2, 2, 1)], 5, 100,
                   {"tma": 4, "tc": 1})
    ii, offsets, makespan = ms.solve(p)
    assert (ii, makespan) == (6, 40) and offsets == [0, 0, 12]


def _random_instance(rng):
    n = rng.randint(1, 4)
    lat = [rng.randint(1, 6) for _ in range(n)]
    res = [rng.randint(0, 1) for _ in range(n)]
    edges = []
    for c in range(n):
        for p in range(n):
            if p < c and rng.random() < 0.5:
                edges.append((p, c, rng.randint(0, 1)))
            elif p == c and rng.random() < 0.3:
                edges.append((p, c, 1))
    depth = rng.randint(1, 3)
    caps = [rng.randint(1, 2), rng.choice([1, 2, -1])]
    return n, lat, res, edges, depth, caps


@pytest.mark.parametrize("seed", range(40))
def test_search_matches_brute_force(seed):
    if not os.path.exists(BRUTE):
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
    rng = random.Random(seed)
    n, lat, res, edges, depth, caps = _random_instance(rng)
    max_cycles = 24
    inp = f"{n} {depth} {max_cycles} 2\n{caps[0]} {caps[1]}\n"
    inp += " ".join(f"{l} {r}" for l, r in zip(lat, res)) + "\n"
    inp += f"{len(edges)} " + " ".join(f"{p} {c} {k}" for p, c, k in edges) + "\n"
    out = subprocess.run([BRUTE], input=inp, capture_output=True, text=True, check=True).stdout.split()
    capacity = {str(r): caps[r] for r in range(2) if caps[r] >= 0}
    prob = ms.Problem(lat, [str(r) for r in res], edges, depth, max_cycles, capacity)
    got = ms.solve(prob)
    if out[0] == "none":
        assert got is None
    else:
        assert got is not None and got[2] == int(out[0])


def test_infeasible_model_keeps_loop_unchanged():
    k = build_gemm_kernel()
    tiny = CostModel(latency={t: (r, l) for t, (r, l) in GFX950_COST_MODEL.latency.items()},
                     resources={"tma": 4, "tc": 1}, max_cycles=5, depth=5)
    out = kernel_pass(k, cost_model=tiny)
    assert out.body == k.body


def test_gfx950_cost_model_gives_three_stage_ring():
    k = kernel_pass(build_gemm_kernel(256, 256, 32, 128, 128), cost_model=GFX950_COST_MODEL)
    loop = next(op for op in k.body if isinstance(op, ForOp))
    assert loop.start == 2
    drains = [op for op in k.body if isinstance(op, MMABufOp)]
    assert len(drains) == 2


# ---------------------------------------------------------------------------
# per-ring depths (short-M GEMM: B streams from HBM, A stays in L2)
# ---------------------------------------------------------------------------
def _per_ring_gemm(lds_budget=160 * 1024):
    from warpir_amd.passes.modulo_scheduler import gfx950_cost_model
    ssa = build_gemm_kernel(block_m=128, block_n=128, block_k=128, wave_m=64, wave_n=64, name="gemm_splitk",
                            split_k=True)
    return ssa, kernel_pass(ssa, cost_model=gfx950_cost_model(128, 128, 128, lds_budget=lds_budget,
                                                              hbm_sources=("B",)))


def _ring_counts(kernel):
    from warpir_amd.ir import AllocSharedOp
    return {op.result.name: op.result.type.count for op in kernel.body if isinstance(op, AllocSharedOp)}


def test_per_ring_depths_follow_each_loads_latency():
    """B (16 units, from HBM) gets three 32 KiB slots and A (8 units, L2) two, filling 160 KiB.
    Pinned by brute force over every pair of depths that fits: (A2, B3) leaves the least load
    latency uncovered, max(latency - (slots - 1) * ii) with ii = 4 (the MMA's four units)."""
    _ssa, k = _per_ring_gemm()
    assert _ring_counts(k) == {"a_bufs": 2, "b_bufs": 3}
    lat, ii, slot_bytes = {"a": 8, "b": 16}, 4, 32 * 1024
    fits = [(a, b) for a in range(2, 8) for b in range(2, 8) if (a + b) * slot_bytes <= 160 * 1024]
    exposed = {p: max(lat["a"] - (p[0] - 1) * ii, lat["b"] - (p[1] - 1) * ii) for p in fits}
    best = min(exposed.values())
    assert [p for p, e in exposed.items() if e == best] == [(2, 3)]
    # with room for everything the rings take the depths the schedule asks for:
    # A loaded as late as the MMA allows (two stages ahead), B four stages ahead
    _ssa, wide = _per_ring_gemm(lds_budget=1 << 20)
    assert _ring_counts(wide) == {"a_bufs": 3, "b_bufs": 5}


def test_per_ring_form_interprets_bitwise_like_the_ssa_form():
    """The per-ring buffer form (a stage-1 A load with its int_affine tile, waits per ring
    depth, a drain_index load in the drain) computes what the SSA loop computes, bit for bit,
    also for slices of one and two K tiles, where the drain consumes the prologue's slots."""
    import torch

    from oracle.ir_interp import run_kernel
    ssa, pip = _per_ring_gemm()
    for kc in (64, 128, 256, 384, 640, 1024):
        s, m, n = 2, 128, 256
        g = torch.Generator().manual_seed(kc)
        a = (torch.randn(m, kc * s, generator=g) * 0.1).bfloat16()
        b = (torch.randn(kc * s, n, generator=g) * 0.1).bfloat16()
        outs = []
        for kern in (ssa, pip):
            c = torch.zeros(1, s, m, n)
            run_kernel(kern, {"A": a.view(m, s, kc).permute(1, 0, 2).unsqueeze(0), "B": b.view(s, kc, n).unsqueeze(0),
                              "C_global": c}, {"N": kc})
            outs.append(c)
        assert torch.equal(outs[0], outs[1]), kc
        ref = torch.stack([a[:, j * kc:(j + 1) * kc].float() @ b[j * kc:(j + 1) * kc].float() for j in range(s)])
        assert (outs[1][0] - ref).abs().max() < 1e-5


def test_per_ring_form_structure():
    """Loop body: one wait per ring depth, A's load of tile i - 1 through int_affine, B's of tile
    i; the drain loads A's last tile through drain_index(+1)."""
    from warpir_amd.ir import DrainIndexOp, IntAffineOp, TMALoadBufOp, WaitBufOp
    from warpir_amd.printing import format_kernel
    _ssa, k = _per_ring_gemm()
    loop = next(op for op in k.body if isinstance(op, ForOp))
    assert loop.start == 2
    waits = [op for op in loop.body if isinstance(op, WaitBufOp)]
    assert [(w.bufs[0].name, w.slot.offset, w.slot.modulus) for w in waits] == [("a_bufs", -2, 2), ("b_bufs", -2, 3)]
    aff = [op for op in loop.body if isinstance(op, IntAffineOp)]
    assert len(aff) == 1 and aff[0].add == -1
    loads = {op.buf.name: op for op in loop.body if isinstance(op, TMALoadBufOp)}
    assert loads["a_bufs"].coords[3] == aff[0].result and loads["a_bufs"].slot.offset == -1
    assert loads["b_bufs"].slot.offset == 0 and loads["b_bufs"].slot.modulus == 3
    drains = [op for op in k.body if isinstance(op, DrainIndexOp)]
    assert len(drains) == 1 and drains[0].offset == 1
    assert "drain_index(+1)" in format_kernel(k)
