"""Cost router between the cluster-major exact scan (mode 10) and the cascade (mode 2).

Reference: benchmarks/phase4a_suite.py:1063-1079 (per-batch choice) and :999-1035
(calibration).  The work measure is W = B * nprobe * (N / nlist) * D; the route is mode 10
when W < W0, else mode 2.  The calibration sweeps batch sizes, times both routes with the
reference's methodology (warmup, back-to-back calls, one synchronise) and sets W0 to the
smallest work at which the cascade is at least as fast (the reference's rule);
``stable_crossover`` gives the smallest work from which the cascade wins at every larger
measured work, which ignores an isolated win at a tiny batch.

W0 is hardware-specific.  The reference's A100 value is 946,811,200 (README rounds it to
9.0e8).  On MI355X (calibrate_w0, bench.py --calibrate-w0) mode 10 is the faster route up to
B = 64 and the cascade from B = 128, where the cascade's int8 matrix-core batched route takes
over: configs[0] (N 1e5, nprobe 16) crosses at W = 1.02e8, configs[1] (N 1e6, nprobe 64) at
W = 1.02e9.  W0_MI355X is the smaller of the two, as the reference takes the smaller of its
datasets' crossovers.
"""
import time
from typing import Dict, List, Optional, Sequence, Tuple

import torch

W0_REFERENCE_A100 = 946_811_200.0
# Smallest stable crossover over the calibrated configs on MI355X (configs[0]: B = 128).
W0_MI355X = 1.024e8

MODE_CM_EXACT = 10
MODE_CASCADE = 2


def work_measure(B: int, nprobe: int, N: int, nlist: int, D: int) -> float:
    """W = B * nprobe * (N / nlist) * D (reference :1018, :1063)."""
    return float(B) * float(nprobe) * (float(N) / float(nlist)) * float(D)


def choose_mode(work: float, W0: float) -> int:
    """mode 10 (exact cluster-major scan) below W0, else mode 2 (cascade) (reference :1079)."""
    return MODE_CM_EXACT if work < W0 else MODE_CASCADE


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
    """Routes each batch of an index to mode 10 or mode 2 by the work measure."""

    def __init__(self, index, W0: Optional[float] = None):
        self.index = index
        self.W0 = W0_MI355X if W0 is None else float(W0)

    def mode_for(self, B: int, nprobe: int) -> int:
        ix = self.index
        return choose_mode(work_measure(B, nprobe, ix.N, ix.nlist, ix.D), self.W0)

    def search(self, xq: torch.Tensor, nprobe: int, **kw):
        mode = self.mode_for(int(xq.shape[0]), nprobe)
        return self.index.search(xq, nprobe, mode=mode, **kw) + (mode,)
