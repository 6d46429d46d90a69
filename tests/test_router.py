"""Cost router closed forms (reference benchmarks/phase4a_suite.py:1018, :1063-1079)."""
import pytest

from trident_amd import router


def test_work_measure_closed_form():
    # cfg 1: B=1000, nprobe=16, N=1e5, nlist=256, D=128 -> 8.0e8
    assert router.work_measure(1000, 16, 100_000, 256, 128) == pytest.approx(8.0e8)
    # cfg 5: B=1e4, nprobe=128, N=1e8, nlist=16384, D=128 -> ~1.0e12
    assert router.work_measure(10_000, 128, 100_000_000, 16384, 128) == pytest.approx(1.0e12, rel=1e-3)


def test_choose_mode_threshold():
    W0 = router.W0_REFERENCE_A100
    assert router.choose_mode(W0 - 1, W0) == 10
    assert router.choose_mode(W0, W0) == 2
    assert router.choose_mode(8.0e8, 9.0e8) == 10   # cfg 1 with the reference's README W0


def test_router_uses_index_shape():
    class Fake:
        N, nlist, D, max_batch = 1_000_000, 1024, 128, 1024
        calls = []

        def search(self, xq, nprobe, mode, **kw):
            self.calls.append(mode)
            return (None, None, 0.0)

    class Q:
        shape = (1, 128)

    f = Fake()
    r = router.CostRouter(f, W0=1e9)
    assert r.mode_for(1, 8) == 10          # 1 * 8 * 976.6 * 128 = 1e6 < 1e9
    assert r.mode_for(10_000, 64) == 2
    assert r.search(Q(), 8)[-1] == 10 and f.calls == [10]


def test_eval_accuracy_v4_semantics():
    import numpy as np
    from trident_amd.metrics import eval_accuracy_v4, measure_latency_qps, measure_runs
    gt = np.arange(20).reshape(2, 10)
    cm_i = gt.copy()
    cm_d = np.tile(np.arange(10, dtype=np.float32), (2, 1))
    pred_i = cm_i.copy()
    pred_i[1, 9] = 99                                  # different id, same distance -> still strict
    pred_d = cm_d.copy()
    rec, strict, full = eval_accuracy_v4(pred_i, pred_d, cm_i, cm_d, gt)
    assert rec == 19 / 20 and strict == 100.0 and full == 100.0
    pred_d[1, 9] = 10.0                                 # now the distance differs too
    rec, strict, full = eval_accuracy_v4(pred_i, pred_d, cm_i, cm_d, gt)
    assert strict == 95.0 and full == 50.0
    calls = []
    assert measure_latency_qps(lambda: calls.append(1), warmup=2, iters=3) >= 0 and len(calls) == 5
    q, s = measure_runs(lambda: None, warmup=1, iters=3, b_size=10)
    assert q > 0 and s >= 0


def test_stable_crossover_ignores_an_isolated_win():
    rows = [{"work": w, "cascade_faster": f} for w, f in
            ((1e6, True), (2e6, False), (4e6, False), (8e6, True), (1.6e7, True))]
    assert router.stable_crossover(rows) == 8e6     # the reference rule would give 1e6
    assert router.stable_crossover(rows[:3]) == float("inf")
    assert router.stable_crossover([{"work": 5.0, "cascade_faster": True}]) == 5.0


def test_pairs_rule_follows_the_batched_threshold():
    """The MI355X rule: the cascade from B * nprobe = 8 nlist (its batched route) on, mode 10
    below; CostRouter takes it unless given a W0 (then the reference's work rule)."""
    assert router.choose_mode_pairs(127, 64, 1024) == 10
    assert router.choose_mode_pairs(128, 64, 1024) == 2
    assert router.choose_mode_pairs(512, 64, 4096) == 2 and router.choose_mode_pairs(511, 64, 4096) == 10

    class Fake:
        N, nlist, D, max_batch = 1_000_000, 1024, 960, 1024

    r = router.CostRouter(Fake())
    assert r.rule == "pairs" and r.mode_for(64, 64) == 10 and r.mode_for(128, 64) == 2
    w = router.CostRouter(Fake(), W0=1e9)
    assert w.rule == "work" and w.mode_for(64, 64) == 2        # W = 3.8e9 >= 1e9
    assert router.CostRouter(Fake(), rule="work").W0 == router.W0_MI355X
    with pytest.raises(ValueError):
        router.CostRouter(Fake(), rule="fastest")
