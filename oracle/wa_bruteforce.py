"""TEST INFRASTRUCTURE -- brute-force optimum of the warp-assignment model.

Enumerates every (type warps, free-instruction warps, start cycles)
combination of the model stated for CP-SAT in the reference
(``warpir/passes/warp_assigner.py:31-119``) and returns the minimum
makespan, or ``None`` when nothing is feasible.  Only for tiny instances
(a handful of instructions, short horizons); it checks the product
solver, it is never used by it.
"""
from __future__ import annotations

import itertools


def _sep(child, parent):
    gap = child.modulo_issue_cycle - parent.modulo_issue_cycle
    return max(gap, parent.total_latency) if gap > 0 else parent.total_latency


def brute_force_makespan(instrs, max_cycles, num_warps, sync_cost, types):
    n = len(instrs)
    idx = {id(x): k for k, x in enumerate(instrs)}
    ubs = [max_cycles - 1 - max(x.cuda_latency, x.total_latency) for x in instrs]
    best = None
    for tw in itertools.product(range(num_warps), repeat=len(types)):
        free = [k for k, x in enumerate(instrs) if x.name not in types]
        for fw in itertools.product(range(num_warps), repeat=len(free)):
            warp = [tw[types.index(x.name)] if x.name in types else None for x in instrs]
            for k, w in zip(free, fw):
                warp[k] = w
            for starts in itertools.product(*[range(u + 1) for u in ubs]):
                ok = True
                for k, x in enumerate(instrs):
                    for p in x.parent_instructions:
                        j = idx[id(p)]
                        extra = sync_cost if (not p.is_async and warp[j] != warp[k]) else 0
                        if starts[k] < starts[j] + _sep(x, p) + extra:
                            ok = False
                    for p in x.ordering_instructions:
                        j = idx[id(p)]
                        if starts[k] < starts[j] + _sep(x, p):
                            ok = False
                    if not ok:
                        break
                if not ok:
                    continue
                for a in range(n):
                    for b in range(a + 1, n):
                        if warp[a] != warp[b]:
                            continue
                        ea = starts[a] + instrs[a].cuda_latency
                        eb = starts[b] + instrs[b].cuda_latency
                        if starts[a] < eb and starts[b] < ea:
                            ok = False
                if not ok:
                    continue
                span = max(starts[k] + x.total_latency for k, x in enumerate(instrs))
                if span <= max_cycles - 1 and (best is None or span < best):
                    best = span
    return best
