"""Exact solver for the modulo-scheduling model of ``MSInstructionManager``.

The reference states the model for OR-Tools CP-SAT
(``warpir/passes/modulo_scheduler.py:51-101``):

* ``depth`` unrolled copies of every instruction, copy ``d`` starting at
  ``start[d][i]`` in ``[0, max_cycles - 1 - latency_i]``;
* a shared initiation interval: ``start[d+1][i] = start[d][i] + ii``;
* an edge ``p -> i`` of distance ``k``: ``start[d][i] >= end[d-k][p]``
  for every ``d >= k``;
* per listed resource, a cumulative limit: at any cycle at most
  ``resource_counts[r]`` intervals of that resource are live;
* minimise the makespan ``max end``.

Because ``start[d][i] = s_i + d * ii``, the unknowns are ``ii`` and one
offset ``s_i`` per instruction, and the makespan is
``(depth - 1) * ii + max_i (s_i + latency_i)``.  This module searches
``ii`` upward and, for each ``ii``, runs a depth-first branch-and-bound
over the offsets (topological order of the distance-0 edges, smallest
offset first), pruning on the incumbent makespan.  It returns the
optimum with the smallest ``ii`` and, among those, the
lexicographically smallest offsets in topological order -- a
deterministic choice among
CP-SAT's equally optimal answers.

Additive: ``slot_class`` restricts instruction ``i`` to offsets with
``offset % ii == slot_class[i]`` (``None`` = unrestricted), so an ``ii``
of ``P`` slots can stand for a cycle of ``P`` phases that each admit one
class of work (the attention loop's MFMA and VALU phases).  An ``ii`` at
or below the largest class is skipped.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple


class Problem:
    """Flattened solver input: index-based instructions and edges."""

    def __init__(self, latencies: Sequence[int], resources: Sequence[str],
                 edges: Sequence[Tuple[int, int, int]], depth: int, max_cycles: int,
                 capacity: Dict[str, int], slot_class: Optional[Sequence[Optional[int]]] = None):
        self.lat = list(latencies)
        self.res = list(resources)
        self.edges = list(edges)  # (parent, child, distance)
        self.depth = depth
        self.max_cycles = max_cycles
        self.cap = dict(capacity)
        self.n = len(self.lat)
        self.slot_class = list(slot_class) if slot_class is not None else [None] * self.n


def _topo_order(p: Problem) -> List[int]:
    indeg = [0] * p.n
    succ: List[List[int]] = [[] for _ in range(p.n)]
    for a, b, k in p.edges:
        if k == 0 and a != b:
            indeg[b] += 1
            succ[a].append(b)
    ready = [i for i in range(p.n) if indeg[i] == 0]
    order: List[int] = []
    while ready:
        ready.sort()
        i = ready.pop(0)
        order.append(i)
        for j in succ[i]:
            indeg[j] -= 1
            if indeg[j] == 0:
                ready.append(j)
    if len(order) != p.n:
        # A distance-0 cycle can never be satisfied (latencies are >= 0 and
        # a cycle would need start_i >= start_i + latency).  Keep the input
        # order; the search then proves infeasibility.
        return list(range(p.n))
    return order


def solve(p: Problem) -> Optional[Tuple[int, List[int], int]]:
    """Return ``(ii, offsets, makespan)`` of an optimal schedule, or ``None``."""
    if p.n == 0:
        return None
    if any(lat > p.max_cycles - 1 for lat in p.lat):
        return None  # an empty start domain, as in the CP-SAT model
    order = _topo_order(p)
    best: Optional[Tuple[int, List[int], int]] = None
    span_floor = max(p.lat)  # any schedule spans at least its longest interval
    min_ii = max([c + 1 for c in p.slot_class if c is not None], default=0)
    for ii in range(min_ii, p.max_cycles):
        base = (p.depth - 1) * ii
        if base + span_floor > p.max_cycles - 1:
            break
        if best is not None and base + span_floor >= best[2]:
            break
        limit = p.max_cycles - 1 - base  # max allowed value of max_i(s_i + lat_i)
        if best is not None:
            limit = min(limit, best[2] - 1 - base)
        found = _best_offsets(p, order, ii, limit)
        if found is not None:
            offsets, span = found
            best = (ii, offsets, base + span)
    return best


def _best_offsets(p: Problem, order: List[int], ii: int, limit: int):
    """Minimise ``max_i(s_i + lat_i)`` subject to ``<= limit`` for a fixed ``ii``."""
    n = p.n
    horizon = limit + (p.depth - 1) * ii + 1
    usage = {r: [0] * max(horizon, 1) for r in p.cap}
    s = [0] * n
    assigned = [False] * n
    best = [limit + 1, None]

    # Edge constraint in offset form: s_child + k*ii >= s_parent + lat_parent.
    into: List[List[Tuple[int, int]]] = [[] for _ in range(n)]
    outof: List[List[Tuple[int, int]]] = [[] for _ in range(n)]
    for a, b, k in p.edges:
        if k > p.depth - 1:
            continue  # no unrolled copy pair is constrained
        into[b].append((a, k))
        outof[a].append((b, k))

    def place(i: int, delta: int) -> bool:
        r = p.res[i]
        if r not in usage:
            return True
        row, cap = usage[r], p.cap[r]
        ok = True
        for d in range(p.depth):
            t0 = s[i] + d * ii
            for t in range(t0, t0 + p.lat[i]):
                row[t] += delta
                if row[t] > cap:
                    ok = False
        return ok

    def dfs(pos: int, span: int) -> None:
        if pos == n:
            if span < best[0]:
                best[0] = span
                best[1] = list(s)
            return
        i = order[pos]
        lo = 0
        for a, k in into[i]:
            if assigned[a]:
                lo = max(lo, s[a] + p.lat[a] - k * ii)
            elif a == i:
                if k * ii < p.lat[i]:
                    return  # self loop needs k*ii >= latency
        hi = min(best[0] - 1, limit) - p.lat[i]
        for b, k in outof[i]:
            if assigned[b] and b != i:
                hi = min(hi, s[b] + k * ii - p.lat[i])
        cls = p.slot_class[i]
        for v in range(lo, hi + 1):
            if max(span, v + p.lat[i]) >= best[0]:
                break  # this and every later offset cannot beat the incumbent
            if cls is not None and v % ii != cls:
                continue
            s[i] = v
            assigned[i] = True
            if place(i, +1):
                dfs(pos + 1, max(span, v + p.lat[i]))
            place(i, -1)
            assigned[i] = False

    dfs(0, 0)
    if best[1] is None:
        return None
    return best[1], best[0]
