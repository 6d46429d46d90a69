"""Accuracy and timing helpers with the reference drivers' semantics.

eval_accuracy_v4     benchmarks/phase4a_suite.py:345-375 -- recall@10 against ground truth and
                     position-wise "strict overlap" against the exact route, where a slot also
                     matches when the distances agree within 1e-4 relative.
measure_latency_qps  benchmarks/phase4a_suite.py:377-387 -- warmup, back-to-back calls, one
                     synchronise; returns ms per call.
measure_runs         benchmarks/plan_v10/phase10_common.py:126-147 -- the same methodology in
                     rounds; returns (mean QPS, std QPS).
"""
import statistics
import time

import numpy as np


def eval_accuracy_v4(pred_ids, pred_dists, cm_ids, cm_dists, gt10, k: int = 10):
    pred_ids, pred_dists = np.asarray(pred_ids), np.asarray(pred_dists)
    cm_ids, cm_dists = np.asarray(cm_ids), np.asarray(cm_dists)
    Q = pred_ids.shape[0]
    rec, strict, full = 0, 0, 0
    for q in range(Q):
        p = pred_ids[q, :k].tolist()
        rec += len(set(p) & set(np.asarray(gt10[q])[:k].tolist()))
        row = 0
        for j in range(k):
            if p[j] == cm_ids[q, j]:
                row += 1
            else:
                dp, dc = float(pred_dists[q, j]), float(cm_dists[q, j])
                if abs(dp - dc) <= 1e-4 * max(abs(dc), 1.0) and dp >= 0:
                    row += 1
        strict += row
        full += row == k
    slots = float(Q * k)
    return rec / slots, 100.0 * strict / slots, 100.0 * full / float(Q)


def _sync():
    import torch
    if torch.cuda.is_available():
        torch.cuda.synchronize()


def measure_latency_qps(fn, warmup: int = 12, iters: int = 50) -> float:
    for _ in range(warmup):
        fn()
    _sync()
    t0 = time.perf_counter()
    for _ in range(iters):
        fn()
    _sync()
    return (time.perf_counter() - t0) * 1000.0 / float(iters)


def measure_runs(fn, warmup: int = 12, iters: int = 10, b_size: int = 1024, rounds: int = 5):
    if iters < 10:  # slow baselines: one call per round, `iters` rounds
        rounds, iters = iters, 1
    for _ in range(warmup):
        fn()
    _sync()
    qps = []
    for _ in range(rounds):
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        _sync()
        qps.append(b_size * iters / max(time.perf_counter() - t0, 1e-9))
    return statistics.mean(qps), (statistics.stdev(qps) if len(qps) > 1 else 0.0)
