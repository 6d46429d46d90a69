"""Cost router between the cluster-major exact scan (mode 10) and the cascade (mode 2).

Reference: benchmarks/phase4a_suite.py:1063-1079 (per-batch choice) and :999-1035
(calibration).  The work measure is W = B * nprobe * (N / nlist) * D; the route is mode 10
when W < W0, else mode 2.  The calibration sweeps batch sizes, times both routes with the
reference's methodology (warmup, back-to-back calls, one synchronise) and sets W0 to the
smallest work at which the cascade is at least as fast (the reference's rule);
``stable_crossover`` gives the smallest work from which the cascade wins at every larger
measured work, which ignores an isolated win at a tiny batch.

W0 is hardware-specific.  The reference's A100 value is 946,811,200 (README rounds it to
9.0e8).  On MI355X (calibrate_w0, bench.py --calibrate-w0; mode 10 timed on its faster route,
the float32 matrix cores at every calibrated batch) the stable crossovers are W = 2.56e7 at
configs[0] (B = 32), 6.4e7 at configs[1] (B = 8), 7.68e9 at configs[2] (D = 960, B = 128) and
7.68e9 at configs[3] (B = 512).  W0_MI355X is the smallest, as the reference takes the smaller
of its datasets' crossovers.

No single W0 fits all four: the crossing follows the pairs per probed cluster, not W.  From
B * nprobe = 8 nlist on, the cascade runs its batched int8 matrix-core route and wins by 4-10x;
below that it runs per (query, cluster) pair and mode 10's single float32 matrix-core pass is
faster or within 10 % (except single queries).  ``choose_mode_pairs`` routes by that (the
library's own AUTO threshold for the cascade's batched route), and ``CostRouter`` uses it unless
it is given a W0.
"""
import time
from typing import Dict, List, Optional, Sequence, Tuple

import torch

W0_REFERENCE_A100 = 946_811_200.0
# Smallest stable crossover over the calibrated configs on MI355X (configs[0]: B = 32).
W0_MI355X = 2.56e7
# Pairs per cluster from which the cascade takes its batched route (capi.hip, choose_route).
BATCHED_PAIRS_PER_CLUSTER = 8.0

MODE_CM_EXACT = 10
MODE_CASCADE = 2


def work_measure(B: int, nprobe: int, N: int, nlist: int, D: int) -> float:
    """W = B * nprobe * (N / nlist) * D (reference :1018, :1063)."""
    return float(B) * float(nprobe) * (float(N) / float(nlist)) * float(D)


def choose_mode(work: float, W0: float) -> int:
    """mode 10 (exact cluster-major scan) below W0, else mode 2 (cascade) (reference :1079)."""
    return MODE_CM_EXACT if work < W0 else MODE_CASCADE


def choose_mode_pairs(B: int, nprobe: int, nlist: int) -> int:
    """MI355X rule: mode 2 (cascade) once B * nprobe >= 8 nlist (its batched route), else
    mode 10."""
    return MODE_CASCADE if float(B) * nprobe >= BATCHED_PAIRS_PER_CLUSTER * nlist else MODE_CM_EXACT


def _time_ms(fn, warmup: int, iters: int) -> float:
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1000.0 / iters


def calibrate_w0(index, xq_pool: torch.Tensor, nprobe: int,
                 batches: Sequence[int] = (1, 4, 8, 16, 32, 64, 128, 256, 512, 1024),
                 warmup: int = 5, iters: int = 20, ub_seed: int = 0) -> Tuple[float, List[Dict]]:
    """Times mode 10 and mode 2 per batch size; W0 = min work where mode 2 is at least as fast
    (reference :999-1035).  Returns (W0, rows); W0 is +inf if mode 10 always wins."""
    rows, crossings = [], []
    N, nlist, D = index.N, index.nlist, index.D
    for b in batches:
        if b > xq_pool.shape[0] or b > index.max_batch:
            break
        q = xq_pool[:b].contiguous()
        w = work_measure(b, nprobe, N, nlist, D)
        # mode 10 on each of its routes (1: float64 per pair, 2: float32 matrix cores), the
        # faster of them standing for mode 10
        ms_routes = {}
        for rt in (1, 2):
            try:
                ms_routes[rt] = _time_ms(lambda: index.search(q, nprobe, mode=MODE_CM_EXACT, route=rt),
                                         warmup, iters)
            except RuntimeError:  # the matrix-core route does not apply (K, D or placement)
                pass
        ms_cm = min(ms_routes.values())
        ms_k2 = _time_ms(lambda: index.search(q, nprobe, mode=MODE_CASCADE, ub_seed=ub_seed), warmup, iters)
        rows.append({"batch": b, "nprobe": nprobe, "work": w, "ms_cm": ms_cm, "ms_cascade": ms_k2,
                     "ms_cm_pair": ms_routes.get(1), "ms_cm_matrix": ms_routes.get(2),
                     "qps_cm": b * 1000.0 / ms_cm, "qps_cascade": b * 1000.0 / ms_k2,
                     "cascade_faster": ms_k2 <= ms_cm})
        if ms_k2 <= ms_cm:
            crossings.append(w)
    return (min(crossings) if crossings else float("inf")), rows


def stable_crossover(rows: List[Dict]) -> float:
    """Smallest work from which the cascade is at least as fast at every larger measured work
    (+inf when mode 10 wins the largest)."""
    w0 = float("inf")
    for r in sorted(rows, key=lambda r: r["work"], reverse=True):
        if not r["cascade_faster"]:
            break
        w0 = r["work"]
    return w0


class CostRouter:
    """Routes each batch of an index to mode 10 or mode 2: ``rule="work"`` by the reference's
    work measure against W0 (W0_MI355X unless given), ``rule="pairs"`` by choose_mode_pairs;
    ``rule="auto"`` (the default) is "work" when a W0 is given, else "pairs"."""

    def __init__(self, index, W0: Optional[float] = None, rule: str = "auto"):
        if rule not in ("auto", "work", "pairs"):
            raise ValueError(f"rule must be 'auto', 'work' or 'pairs', not {rule!r}")
        self.index = index
        self.rule = ("work" if W0 is not None else "pairs") if rule == "auto" else rule
        self.W0 = W0_MI355X if W0 is None else float(W0)

    def mode_for(self, B: int, nprobe: int) -> int:
        ix = self.index
        if self.rule == "pairs":
            return choose_mode_pairs(B, nprobe, ix.nlist)
        return choose_mode(work_measure(B, nprobe, ix.N, ix.nlist, ix.D), self.W0)

    def search(self, xq: torch.Tensor, nprobe: int, **kw):
        mode = self.mode_for(int(xq.shape[0]), nprobe)
        return self.index.search(xq, nprobe, mode=mode, **kw) + (mode,)
