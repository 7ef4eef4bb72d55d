/*
 * TEST INFRASTRUCTURE (oracle) -- never linked into or called by the product.
 *
 * Brute-force enumeration of the modulo-scheduling model that the reference
 * states for OR-Tools CP-SAT (warpir/passes/modulo_scheduler.py:51-101),
 * checked literally, copy by copy and cycle by cycle:
 *
 *   start[d][i] = s_i + d*ii,   0 <= start[d][i] <= max_cycles-1-lat_i   (:55-64, :89-95)
 *   edge p->i, distance k:  start[d][i] >= start[d-k][p] + lat_p for d>=k (:69-74)
 *   per constrained resource r, every cycle t: #live intervals <= cap_r  (:77-87)
 *   makespan = max_d,i start[d][i] + lat_i <= max_cycles-1, minimised   (:98-101)
 *
 * Every (ii, s_0..s_{n-1}) is enumerated.  Prints
 *   "<min_makespan> <number_of_optimal_solutions> <ii> <s_0> ... <s_{n-1}>"
 * where the listed solution is the first optimum in (ii, s_0, s_1, ...) order,
 * or "none" when the model is infeasible.
 *
 * Input (stdin, whitespace separated):
 *   n depth max_cycles nres
 *   cap_0 ... cap_{nres-1}            (-1 = unconstrained)
 *   lat_0 res_0 ... lat_{n-1} res_{n-1}
 *   nedges  (parent child distance) * nedges
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define MAXN 8
#define MAXE 64
#define MAXR 8
#define MAXT 1024

static int n, depth, max_cycles, nres, ne;
static int cap[MAXR], lat[MAXN], res[MAXN];
static int ep[MAXE], ec[MAXE], ek[MAXE];
static int s[MAXN];
static long long best = -1, count = 0;
static int best_ii, best_s[MAXN];

static void check(int ii) {
    int d, i, e, t, mk = 0;
    for (d = 0; d < depth; d++)
        for (i = 0; i < n; i++) {
            int st = s[i] + d * ii;
            if (st < 0 || st > max_cycles - 1 - lat[i]) return;
            if (st + lat[i] > mk) mk = st + lat[i];
        }
    if (mk > max_cycles - 1) return;
    for (e = 0; e < ne; e++)
        for (d = ek[e]; d < depth; d++)
            if (s[ec[e]] + d * ii < s[ep[e]] + (d - ek[e]) * ii + lat[ep[e]]) return;
    for (int r = 0; r < nres; r++) {
        static int live[MAXT];
        if (cap[r] < 0) continue;
        memset(live, 0, sizeof(int) * (size_t)(mk + 1));
        for (d = 0; d < depth; d++)
            for (i = 0; i < n; i++) {
                if (res[i] != r) continue;
                for (t = s[i] + d * ii; t < s[i] + d * ii + lat[i]; t++)
                    if (++live[t] > cap[r]) return;
            }
    }
    if (best < 0 || mk < best) {
        best = mk;
        count = 1;
        best_ii = ii;
        memcpy(best_s, s, sizeof(s));
    } else if (mk == best) {
        count++;
    }
}

static void rec(int ii, int i) {
    if (i == n) { check(ii); return; }
    int hi = max_cycles - 1 - lat[i] - (depth - 1) * ii;
    for (int v = 0; v <= hi; v++) { s[i] = v; rec(ii, i + 1); }
}

int main(void) {
    if (scanf("%d %d %d %d", &n, &depth, &max_cycles, &nres) != 4) return 2;
    if (n < 1 || n > MAXN || nres > MAXR || max_cycles > MAXT || depth < 1) return 2;
    for (int r = 0; r < nres; r++) if (scanf("%d", &cap[r]) != 1) return 2;
    for (int i = 0; i < n; i++) if (scanf("%d %d", &lat[i], &res[i]) != 2) return 2;
    if (scanf("%d", &ne) != 1 || ne > MAXE) return 2;
    for (int e = 0; e < ne; e++) if (scanf("%d %d %d", &ep[e], &ec[e], &ek[e]) != 3) return 2;
    for (int ii = 0; ii < max_cycles; ii++) rec(ii, 0);
    if (best < 0) { printf("none\n"); return 0; }
    printf("%lld %lld %d", best, count, best_ii);
    for (int i = 0; i < n; i++) printf(" %d", best_s[i]);
    printf("\n");
    return 0;
}
