"""Warp assignment (CPU): the reference demo's known answer and brute force.

Pins: the reference demo (``warpir/passes/warp_assigner.py:146-212``) has
optimal makespan 70 -- derived by hand: mac_k >= mac_{k-2} + 16 through
the load-ordering dependences and mac_0 >= 12, so mac_7 >= 66, plus its
4-cycle latency; load_a and load_b must sit on different warps to reach
it.  Random tiny instances are checked against an exhaustive enumerator
(``oracle/wa_bruteforce.py``).  The warp table itself is not unique, so
only the makespan is compared.
"""
import random

import pytest

from oracle.wa_bruteforce import brute_force_makespan
from warpir.passes.warp_assigner import WAInstruction, WAInstructionManager
from warpir_amd.passes.warp_assigner import assign_waves, instructions_from_pipeline


def _demo():
    ii, n = 6, 6
    mk_load = lambda name, k: WAInstruction(name, k, [], [], True, 1, 12, k * ii)  # noqa: E731
    mk_mac = lambda k, ps: WAInstruction("mac", k, ps, [], False, 1, 4, 2 * ii + k * ii)  # noqa: E731
    la, lb, macs = {}, {}, {}
    for k in range(2):
        la[k], lb[k] = mk_load("load_a", k), mk_load("load_b", k)
    for k in range(2, n + 2):
        la[k], lb[k] = mk_load("load_a", k), mk_load("load_b", k)
        ps = [la[k - 2], lb[k - 2]] + ([macs[k - 3]] if k - 3 in macs else [])
        macs[k - 2] = mk_mac(k - 2, ps)
        la[k].ordering_instructions.append(macs[k - 2])
        lb[k].ordering_instructions.append(macs[k - 2])
    for k in (n, n + 1):
        macs[k] = mk_mac(k, [la[k], lb[k], macs[k - 1]])
    return [la[k] for k in sorted(la)] + [lb[k] for k in sorted(lb)] + [macs[k] for k in sorted(macs)]


def test_reference_demo_makespan(capsys):
    m = WAInstructionManager()
    for ins in _demo():
        m.add_instruction(ins)
    sol = m.solve(500, 2, 80, ["load_a", "load_b", "mac"])
    assert sol.makespan == 70
    assert sol.type_warp["load_a"] != sol.type_warp["load_b"]
    out = capsys.readouterr().out
    assert out.startswith("warp 0:") and "warp 1:" in out and "[type: mac]" in out


def test_too_small_horizon_raises():
    m = WAInstructionManager()
    m.add_instruction(WAInstruction("x", 0, [], [], True, 1, 12, 0))
    with pytest.raises(ValueError):
        m.solve(10, 2, 80, [])


def test_infeasible_prints(capsys):
    a = WAInstruction("a", 0, [], [], False, 1, 5, 0)
    b = WAInstruction("b", 0, [a], [], False, 1, 5, 0)
    m = WAInstructionManager()
    for x in (a, b):
        m.add_instruction(x)
    assert m.solve(10, 1, 0, []) is None  # b needs start >= 5 and end <= 9 -> 5+5=10 > 9
    assert "INFEASIBLE!" in capsys.readouterr().out


def _random_instance(rng):
    n = rng.randint(2, 4)
    ins = []
    for k in range(n):
        name = rng.choice(["ld", "mm", "x"])
        parents = [p for p in ins if rng.random() < 0.4]
        order = [p for p in ins if p not in parents and rng.random() < 0.2]
        ins.append(WAInstruction(name, k, parents, order, rng.random() < 0.5, rng.randint(1, 2),
                                 rng.randint(1, 3), rng.randint(0, 3)))
    return ins


@pytest.mark.parametrize("seed", range(25))
def test_matches_brute_force(seed, capsys):
    rng = random.Random(seed)
    ins = _random_instance(rng)
    types = sorted({i.name for i in ins if i.name != "x"})
    max_cycles, warps, sync = 11, 2, rng.randint(0, 3)
    want = brute_force_makespan(ins, max_cycles, warps, sync, types)
    m = WAInstructionManager()
    for x in ins:
        m.add_instruction(x)
    got = m.solve(max_cycles, warps, sync, types)
    assert (got.makespan if got else None) == want


def test_ir_connected_assignment_of_pipelined_gemm():
    from warpir_amd.kernels import kernel
    k = kernel("gemm_256_k32")
    ins = instructions_from_pipeline(k, iterations=3)
    assert {i.name for i in ins} == {"a_load", "b_load", "mma"}
    sol = assign_waves(k, iterations=3)
    assert sol is not None and sol.makespan > 0
    # the MMA chain never pays the sync cost: every MMA sits on the MMA type's warp
    assert len({sol.warp_of[str(i)] for i in ins if i.name == "mma"}) == 1


def test_gfx950_costs_give_the_measured_faster_split():
    """With the gfx950 costs (an LDS-DMA instruction stalls its issuing wave ~20 cycles, an MFMA
    32, a tile lands ~2048 cycles after issue, a barrier between wave sets ~80; units of 32
    cycles) the steady-state periods of the warp-specialised 256x128 GEMM rank the splits as
    the timings do: both streams on the DMA waves (ws_all, 1113 TFLOP/s) ahead of A with the
    MFMA waves and B on the DMA waves (1015) -- the reference demo's constants chose the
    latter.  Periods by hand: the MMA warp issues 32 units of MFMAs, A's DMAs take 5 units of
    its issuing wave (32 KiB over 4 waves: 8 instructions), B's 3 (4 instructions); each
    3-slot ring needs (32 + issue + 64 + sync 3 off the MMA warp) / 3."""
    from warpir_amd import kernels
    from warpir_amd.passes.warp_assigner import assign_streams, gfx950_wave_costs, steady_state_period

    k = kernels.kernel("gemm_256x128_ws")
    c = gfx950_wave_costs(k)
    assert (c.load_issue, c.mma_issue, c.load_latency, c.sync) == ({"a_load": 5, "b_load": 3}, 32, 64, 3)
    period = {(a, b): steady_state_period(k, {"a_load": a, "b_load": b, "mma": 0}, c)
              for a in (0, 1) for b in (0, 1)}
    assert period[(1, 1)] == pytest.approx((32 + 5 + 64 + 3) / 3)
    assert period[(0, 1)] == 37 and period[(0, 0)] == 40 and period[(1, 0)] == 35
    assert assign_streams(k, c).type_warp == {"a_load": 1, "b_load": 1, "mma": 0}
    # the reference demo's constants over the one-iteration window keep A with the MMA
    from warpir_amd.passes.warp_assigner import assign_waves
    assert assign_waves(k, num_warps=2, iterations=1).type_warp == {"a_load": 0, "b_load": 1, "mma": 0}
