"""The attention ping-pong's barrier protocol, checked on the CPU.

The ping-pong kernel (``CDNA4Lowerer._emit_attention_pingpong``) runs two
groups of four waves: group A loads the K ring, group B the V ring, each
wave one quarter of every tile, and both groups read every tile.  Only the
workgroup barrier orders one wave's LDS-DMA against another wave's reads:
a wave's ``s_waitcnt vmcnt(N)`` before a barrier makes all but its newest
N loads land, and everything before a wave's k-th barrier happens before
everything after any wave's k-th barrier.  So

* a read of tile t needs a barrier k passed before the read such that the
  loader's wait at its k-th barrier covered the load (RAW), and
* a load into slot t % S needs every read of tile t - S to sit before a
  barrier that the loader passed before issuing the load (WAR).

``schedule`` restates the per-group event order that the emitter produces
for a loop of ``n`` tiles (prologue, peeled first iteration, loop, last PV,
final drain); ``violations`` checks RAW, WAR, equal barrier counts and that
every tile is loaded once.  Mistakes planted in the model (a 4-slot ring
with a barrier every second iteration, B's V tiles one further ahead, a
drain condition that claims a skipped batch was issued) are caught, and
the generated source is checked to carry the distances and barrier
conditions the model assumes.
"""
import pytest

from warpir_amd import kernels


def schedule(S: int, every: int, n: int, dv=None, b_cond_off=None, a_cond_off=None):
    """Per-group event lists: ("load", stream, tile), ("read", stream, tile),
    ("barrier", n_keep) with n_keep the batches the wait leaves in flight."""
    dist = S - 2
    if dv is None:
        dv = dist + 1 if every == 1 else dist
    b_cond_off = dv - 1 if b_cond_off is None else b_cond_off
    a_cond_off = dist if a_cond_off is None else a_cond_off
    ev = {"A": [], "B": []}

    def odd(i):
        return every == 1 or (i & 1) == 1

    for t in range(dist):   # the prologue loads unconditionally (tiles past the end read the zero page)
        ev["A"].append(("load", "k", t))
        ev["B"].append(("load", "v", t))
    for g in "AB":
        ev[g].append(("barrier", 1))
    if every == 1:
        ev["B"].append(("load", "v", dist))
    for i in range(n):
        for g in "AB":
            if i > 0:
                ev[g].append(("read", "v", i - 1))
            ev[g].append(("read", "k", i))
        if odd(i):
            ev["B"].append(("barrier", 1 if i + b_cond_off < n else 0))
        if i + dist < n:
            ev["A"].append(("load", "k", i + dist))
        if i + dv < n:
            ev["B"].append(("load", "v", i + dv))
        if odd(i):
            ev["A"].append(("barrier", 1 if i + a_cond_off < n else 0))
    if n > 0:
        for g in "AB":
            ev[g].append(("read", "v", n - 1))
    for g in "AB":
        ev[g].append(("barrier", 0))   # the drain before the LDS is reused for staging
    return ev


def schedule_split(S: int, n: int, dv=None, b_cond_off=None):
    """The split-barrier form (``CDNA4Target.pingpong_split_barrier``): group B
    passes its barrier after the rotated PV(i-1) instead of after QK(i), its V
    tiles are loaded S - 2 ahead like A's K tiles, there is no extra first V
    load, and B's last barrier follows the last PV."""
    dist = S - 2
    dv = dist if dv is None else dv
    b_cond_off = dv if b_cond_off is None else b_cond_off
    ev = {"A": [], "B": []}
    for t in range(dist):
        ev["A"].append(("load", "k", t))
        ev["B"].append(("load", "v", t))
    for g in "AB":
        ev[g].append(("barrier", 1))
    for i in range(n):
        for g in "AB":
            if i > 0:
                ev[g].append(("read", "v", i - 1))
        if i > 0:   # B's latest batch: V tile i - 1 + dv
            ev["B"].append(("barrier", 1 if (i - 1) + b_cond_off < n else 0))
        for g in "AB":
            ev[g].append(("read", "k", i))
        if i + dist < n:
            ev["A"].append(("load", "k", i + dist))
        if i + dv < n:
            ev["B"].append(("load", "v", i + dv))
        ev["A"].append(("barrier", 1 if i + dist < n else 0))
    if n > 0:
        for g in "AB":
            ev[g].append(("read", "v", n - 1))
        ev["B"].append(("barrier", 1 if (n - 1) + b_cond_off < n else 0))
    for g in "AB":
        ev[g].append(("barrier", 0))
    return ev


def violations(S: int, ev, n: int):
    out = []
    nb = {g: sum(1 for e in ev[g] if e[0] == "barrier") for g in ev}
    if nb["A"] != nb["B"]:
        out.append(f"barrier counts differ: {nb}")
    # per group: barriers passed before each event; landed[g][k] = loads complete at barrier k
    pos, landed = {}, {g: {} for g in ev}
    for g, es in ev.items():
        passed, issued = 0, []
        for idx, e in enumerate(es):
            if e[0] == "barrier":
                passed += 1
                keep = e[1]
                # the newest `keep` batches may stay in flight
                landed[g][passed] = set(issued[:len(issued) - keep] if keep else issued)
            else:
                pos[(g, idx)] = passed
                if e[0] == "load":
                    issued.append((e[1], e[2]))
    loads = {}
    for g, es in ev.items():
        for idx, e in enumerate(es):
            if e[0] == "load":
                if (e[1], e[2]) in loads:
                    out.append(f"tile {e[1]}{e[2]} loaded twice")
                loads[(e[1], e[2])] = (g, pos[(g, idx)])
    for stream in "kv":
        for t in range(n):
            if (stream, t) not in loads:
                out.append(f"tile {stream}{t} never loaded")
    for g, es in ev.items():
        for idx, e in enumerate(es):
            if e[0] != "read":
                continue
            key = (e[1], e[2])
            if key not in loads:
                continue
            lg = loads[key][0]
            if not any(key in landed[lg].get(k, ()) for k in range(1, pos[(g, idx)] + 1)):
                out.append(f"RAW: group {g} reads {key} before any barrier covers its load")
    for key, (lg, lpos) in loads.items():
        prev = (key[0], key[1] - S)
        for g, es in ev.items():
            for idx, e in enumerate(es):
                if e[0] == "read" and (e[1], e[2]) == prev and not pos[(g, idx)] + 1 <= lpos:
                    out.append(f"WAR: load of {key} may overwrite {prev} still read by group {g}")
    return out


@pytest.mark.parametrize("S,every", [(4, 1), (5, 1), (5, 2)])
def test_pingpong_protocol_is_race_free(S, every):
    for n in range(0, 14):
        assert violations(S, schedule(S, every, n), n) == [], (S, every, n)


def test_planted_mistakes_are_caught():
    # a 4-slot ring cannot take a barrier every second iteration
    assert any(violations(4, schedule(4, 2, n), n) for n in range(2, 10))
    # B's V tiles loaded one further ahead (the every-iteration distance) overwrite a slot still read
    assert any("WAR" in v for n in range(4, 10) for v in violations(5, schedule(5, 2, n, dv=4), n))
    # a drain condition that claims a skipped batch was issued (one tile short) keeps the batch
    # before it in flight, and the next interval reads it; the other direction only over-waits
    assert any("RAW" in v for n in range(3, 10) for v in violations(5, schedule(5, 2, n, b_cond_off=1), n))
    assert any("RAW" in v for n in range(3, 10) for v in violations(5, schedule(5, 2, n, a_cond_off=2), n))
    assert all(violations(5, schedule(5, 2, n, b_cond_off=3, a_cond_off=4), n) == [] for n in range(14))


def test_generated_source_matches_the_model():
    """The emitter's distances and barrier conditions are those the model checks: the
    every-second-iteration form (mha_d128_u2: 5-slot ring, K and V three tiles ahead, B's
    barrier covering V tile i + 2, A's K tile i + 3, both gated on odd iterations, no extra
    first V load), and the every-iteration form of the default (4 slots, K two and V three
    ahead)."""
    def loop(name):
        src = kernels.lowerer(name).lower(kernels.kernel(name))
        body = src[src.rindex('extern "C" __global__'):]
        return body[body.index("const int wir_grp ="):body.index("ring buffers dead")]

    stop = "((globals.N) + 63) / 64"
    u2 = loop("mha_d128_u2")
    assert "group B's first V phase" not in u2
    assert u2.count(f"if (wir_grp == 1 && (((v_i) - (0)) & 1)) wir::wait_vm_barrier_after<4>((v_i) + 2 < {stop});") == 2
    assert u2.count(f"if (wir_grp == 0 && (((v_i) - (0)) & 1)) wir::wait_vm_barrier_after<4>((v_i) + 3 < {stop});") == 3
    assert u2.count(f"if ((v_i) + 3 < {stop})") == 4 and f"(v_i) + 4 < {stop}" not in u2
    assert "for (int wir_t = 0; wir_t < (0) + 3; ++wir_t)" in u2 and "% 5) * 16384" in u2
    d = loop("mha_d128")
    assert "group B's first V phase" in d and "wir_t < (0) + 2;" in d
    # the model loads each tile once: the prefetch form's own prologue loads run only in the
    # plain loop's body (tensors that are not tile-aligned), never before the ping-pong
    for name in ("mha_d128", "mha_d128_u2"):
        src = kernels.lowerer(name).lower(kernels.kernel(name))
        body = src[src.rindex('extern "C" __global__'):]
        before = body[:body.index("if constexpr (!WIR_AL) {")]
        assert not [ln for ln in before.split("\n") if "::load<" in ln
                    and not ln.lstrip().startswith("if constexpr (!WIR_AL) ")], name
    assert d.count(f"if (wir_grp == 1) wir::wait_vm_barrier_after<4>((v_i) + 2 < {stop});") == 2
    assert d.count(f"if ((v_i) + 3 < {stop})") == 2 and d.count(f"if ((v_i) + 2 < {stop})") == 2


@pytest.mark.parametrize("S", [4, 5])
def test_split_barrier_protocol_is_race_free(S):
    for n in range(0, 14):
        assert violations(S, schedule_split(S, n), n) == [], (S, n)


def test_split_barrier_planted_mistakes_are_caught():
    # three slots: a V load overwrites the slot that group A's next PV still reads
    assert any(violations(3, schedule_split(3, n), n) for n in range(2, 10))
    # V one tile further ahead (the unsplit form's distance) on a 4-slot ring
    assert any("WAR" in v for n in range(3, 10) for v in violations(4, schedule_split(4, n, dv=3), n))
    # B's drain condition one tile short keeps a batch in flight that the next PV reads
    assert any("RAW" in v for n in range(2, 10) for v in violations(4, schedule_split(4, n, b_cond_off=1), n))


def test_split_barrier_source_matches_the_model():
    """mha_d128_sb: no extra first V load, K and V both two tiles ahead, B's barrier right after
    the rotated PV (in the loop, and after the last PV) covering V tile i + 1, A's after the
    softmax covering K tile i + 2, and no barrier for B after the QK MMA."""
    src = kernels.lowerer("mha_d128_sb").lower(kernels.kernel("mha_d128_sb"))
    body = src[src.rindex('extern "C" __global__'):]
    d = body[body.index("const int wir_grp ="):body.index("ring buffers dead")]
    stop = "((globals.N) + 63) / 64"
    assert "group B's first V phase" not in d and "wir_t < (0) + 2;" in d
    b_bar = f"if (wir_grp == 1) wir::wait_vm_barrier_after<4>((v_i) + 1 < {stop});"
    assert d.count(b_bar) == 2
    assert d.count(f"if (wir_grp == 0) wir::wait_vm_barrier_after<4>((v_i) + 2 < {stop});") == 3
    assert d.count(f"if ((v_i) + 2 < {stop})") == 4 and f"(v_i) + 3 < {stop}" not in d
    # each B barrier directly follows a PV MMA
    for part in d.split(b_bar)[:-1]:
        assert part.rstrip().split("\n")[-1].lstrip().startswith("wir::mma_rAB<")
