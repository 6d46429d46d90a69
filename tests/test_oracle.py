"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

Checks, each chosen so a plausible mistake fails one of them:
  * committed golden fixtures (independent numpy brute force, tests/golden/make_golden.py);
  * numpy brute force on fresh random inputs, including heavy exact ties;
  * the canonical float64 distance re-derived with exact rational arithmetic (every fma
    rounded once, in dimension order) -- pins the summation order bit for bit;
  * closed forms (1-D line, a query equal to a base row);
  * the FP32 IVF-Flat baseline: identical on integer data, only float32-rounding differences
    (audit taxonomy of benchmarks/phase3a_lossless_audit.py:76-129) on float data;
  * planted mistakes (no tie-break, a dropped dimension, a sign flip, a wrong probe order)
    are caught by the same checks.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def sorted_lists(list_ids, nlist):
    order = np.argsort(list_ids, kind="stable").astype(np.int32)
    counts = np.bincount(list_ids, minlength=nlist)
    vec_off = np.zeros(nlist + 1, np.int32)
    vec_off[1:] = np.cumsum(counts)
    return order, vec_off


def run_oracle(xb, xq, cen, lid, nprobe, K):
    order, vec_off = sorted_lists(lid, len(cen))
    cids, cd = O.coarse_probe(xq, cen, nprobe)
    d, i = O.ivf_exact(xq, cids, vec_off, xb[order], order, K)
    return cids, cd, d, i


@pytest.mark.parametrize("name", ["int_ties", "float_gmm", "short"])
def test_golden_fixture(name):
    z = np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False)
    cids, cd, d, i = run_oracle(z["xb"], z["xq"], z["centroids"], z["list_ids"], int(z["nprobe"]), int(z["K"]))
    assert np.array_equal(cids, z["probes"])
    assert np.array_equal(i, z["topk_i"])
    fin = np.isfinite(z["topk_d"])
    assert np.array_equal(np.isfinite(d), fin)
    if name == "float_gmm":
        np.testing.assert_allclose(d[fin], z["topk_d"][fin], rtol=1e-14)
        np.testing.assert_allclose(cd, z["probe_d"], rtol=1e-14)
    else:  # integer data: every summation order is exact
        assert np.array_equal(d[fin], z["topk_d"][fin])
        assert np.array_equal(cd, z["probe_d"])


@pytest.mark.parametrize("seed", range(4))
def test_brute_force_random(seed):
    rng = np.random.default_rng(seed)
    D = int(rng.integers(1, 40))
    nlist = int(rng.integers(1, 20))
    N = int(rng.integers(1, 400))
    integer = seed % 2 == 0
    draw = (lambda *s: rng.integers(0, 3, size=s)) if integer else (lambda *s: rng.standard_normal(s))
    xb = draw(N, D).astype(np.float32)
    cen = draw(nlist, D).astype(np.float32)
    lid = rng.integers(0, nlist, size=N).astype(np.int32)
    xq = draw(25, D).astype(np.float32)
    nprobe = int(rng.integers(1, nlist + 1))
    K = int(rng.integers(1, 40))
    cids, _, d, i = run_oracle(xb, xq, cen, lid, nprobe, K)
    bc, _ = O.np_coarse_probe(xq, cen, nprobe)
    assert np.array_equal(cids, bc)
    bd, bi = O.np_ivf_exact(xq, xb, lid, bc, K)
    if integer:
        assert np.array_equal(i, bi)
        assert np.array_equal(d, bd)
    else:
        assert np.array_equal(i, bi)
        np.testing.assert_allclose(d, bd, rtol=1e-12)


def fma_exact_sum(x, q):
    """Canonical distance with exact rationals: acc <- round64(t * t + acc), t = round64(x - q)."""
    acc = 0.0
    for xv, qv in zip(x.astype(np.float64).tolist(), q.astype(np.float64).tolist()):
        t = xv - qv  # float64 subtraction, rounded once (as in C)
        acc = float(Fraction(t) * Fraction(t) + Fraction(acc))  # exactly rounded fma
    return acc


def test_canonical_distance_is_sequential_fma():
    rng = np.random.default_rng(11)
    L = O.lib()
    import ctypes
    for D in (1, 7, 96, 128, 960):
        for _ in range(5):
            x = (rng.standard_normal(D) * rng.uniform(0.01, 1000)).astype(np.float32)
            q = (rng.standard_normal(D) * rng.uniform(0.01, 1000)).astype(np.float32)
            got = L.oracle_dist_f64(x.ctypes.data_as(ctypes.c_void_p), q.ctypes.data_as(ctypes.c_void_p), D)
            assert got == fma_exact_sum(x, q)


def test_closed_forms():
    # 1-D line: points 0..9 (ids = values), query 4.5 -> ties at 4/5, 3/6, ... broken by id
    xb = np.arange(10, dtype=np.float32).reshape(10, 1)
    lid = np.zeros(10, np.int32)
    cen = np.zeros((1, 1), np.float32)
    _, _, d, i = run_oracle(xb, np.array([[4.5]], np.float32), cen, lid, 1, 6)
    assert i[0].tolist() == [4, 5, 3, 6, 2, 7]
    assert d[0].tolist() == [0.25, 0.25, 2.25, 2.25, 6.25, 6.25]
    # a query equal to a base row has distance 0 and comes first
    rng = np.random.default_rng(3)
    xb = rng.standard_normal((50, 9)).astype(np.float32)
    lid = (np.arange(50) % 4).astype(np.int32)
    cen = rng.standard_normal((4, 9)).astype(np.float32)
    _, _, d, i = run_oracle(xb, xb[17:18].copy(), cen, lid, 4, 3)
    assert i[0, 0] == 17 and d[0, 0] == 0.0


def test_fp32_baseline_matches_on_integer_and_audits_on_float():
    rng = np.random.default_rng(9)
    xb = rng.integers(0, 256, size=(3000, 32)).astype(np.float32)
    lid = rng.integers(0, 16, size=3000).astype(np.int32)
    cen = rng.integers(0, 256, size=(16, 32)).astype(np.float32)
    xq = rng.integers(0, 256, size=(40, 32)).astype(np.float32)
    order, vec_off = sorted_lists(lid, 16)
    cids, _ = O.coarse_probe(xq, cen, 5)
    d64, i64 = O.ivf_exact(xq, cids, vec_off, xb[order], order, 10)
    d32, i32 = O.ivfflat_f32(xq, cids, vec_off, xb[order], order, 10)
    assert np.array_equal(i32, i64) and np.array_equal(d32, d64.astype(np.float32))
    xbf = (xb + rng.standard_normal(xb.shape)).astype(np.float32)
    xqf = (xq + rng.standard_normal(xq.shape)).astype(np.float32)
    d64, i64 = O.ivf_exact(xqf, cids, vec_off, xbf[order], order, 10)
    d32, i32 = O.ivfflat_f32(xqf, cids, vec_off, xbf[order], order, 10)
    a = O.audit(i32, i64, xbf, xqf)
    assert a["true_miss"] == 0
    np.testing.assert_allclose(d32, d64, rtol=1e-5)


def test_audit_known_answers():
    """oracle.audit on hand-built lists (reference audit_predictions,
    benchmarks/phase3a_lossless_audit.py:76-129): one exact tie, one FP32-rounding pair and one
    true miss on query 0, an identical list on query 1, and two unfilled (-1) slots on query 2."""
    xb = np.array([[1, 0], [0, 1], [2, 0], [2.000002, 0], [3, 0], [4, 0]], np.float32)
    xq = np.zeros((3, 2), np.float32)
    ref = np.array([[0, 2, 4], [0, 2, 4], [0, 2, 4]])
    pred = np.array([[1, 3, 5], [4, 0, 2], [0, -1, -1]])
    a = O.audit(pred, ref, xb, xq)
    d3 = float(xb[3, 0]) ** 2
    assert 1e-12 < (d3 - 4.0) / 4.0 <= 1e-5
    assert (a["diff_slots"], a["exact_tie"], a["f32_rounding"], a["true_miss"]) == (3, 1, 1, 3)
    assert (a["queries_strict"], a["queries_no_miss"], a["strict_id_hits"], a["total_slots"]) == (1, 1, 4, 9)
    assert a["max_rel"] == pytest.approx(7.0 / 9.0, rel=1e-12)
    assert a["strict_id_overlap_pct"] == pytest.approx(400.0 / 9.0)
    assert a["lossless_no_miss_pct"] == pytest.approx(100.0 / 3.0)
    # the same lists in the other role: the classification is symmetric in the paired ids
    b = O.audit(ref[:1], pred[:1], xb, xq[:1])
    assert (b["exact_tie"], b["f32_rounding"], b["true_miss"]) == (1, 1, 1)


# ---- planted mistakes: each mutated oracle must fail the checks above ----

def _mut_no_tiebreak(xq, xb, lid, probes, K):
    q64 = xq.astype(np.float64)
    out = np.full((len(xq), K), -1, np.int64)
    for r in range(len(xq)):
        cand = np.nonzero(np.isin(lid, probes[r]))[0][::-1]       # reversed id order
        d = ((xb[cand].astype(np.float64) - q64[r]) ** 2).sum(1)
        o = np.argsort(d, kind="stable")[:K]
        out[r, :len(o)] = cand[o]
    return out


def _mut_drop_dim(xq, xb, lid, probes, K):
    return O.np_ivf_exact(xq[:, :-1], xb[:, :-1], lid, probes, K)[1]


def _mut_sign(xq, xb, lid, probes, K):
    return O.np_ivf_exact(-xq, xb, lid, probes, K)[1]


@pytest.mark.parametrize("mutant", [_mut_no_tiebreak, _mut_drop_dim, _mut_sign])
def test_planted_mistakes_are_caught(mutant):
    z = np.load(os.path.join(GOLD, "int_ties.npz"), allow_pickle=False)
    got = mutant(z["xq"], z["xb"], z["list_ids"], z["probes"], int(z["K"]))
    assert not np.array_equal(got, z["topk_i"]), f"{mutant.__name__} was not detected"


def test_planted_probe_order_mistake_is_caught():
    z = np.load(os.path.join(GOLD, "int_ties.npz"), allow_pickle=False)
    q = z["xq"].astype(np.float64)
    cd = ((q[:, None, :] - z["centroids"].astype(np.float64)[None]) ** 2).sum(-1)
    # ties broken toward the larger cid instead of the smaller one
    wrong = np.stack([sorted(range(cd.shape[1]), key=lambda c: (cd[r, c], -c))[: int(z["nprobe"])]
                      for r in range(len(q))])
    assert not np.array_equal(wrong, z["probes"])
