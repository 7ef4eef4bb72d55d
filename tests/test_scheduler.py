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
