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


@pytest.mark.parametrize("name", ["int_ties", "float_gmm", "short"])
def test_cluster_major_golden_fixture(name):
    """ivf_exact_cm (each list read once for all queries probing it) gives the fixture's result
    bit for bit (same canonical distances, same (d, id) order)."""
    z = np.load(os.path.join(GOLD, f"{name}.npz"), allow_pickle=False)
    order, vec_off = sorted_lists(z["list_ids"], len(z["centroids"]))
    d, i = O.ivf_exact_cm(z["xq"], z["probes"], vec_off, z["xb"][order], order, int(z["K"]))
    d0, i0 = O.ivf_exact(z["xq"], z["probes"], vec_off, z["xb"][order], order, int(z["K"]))
    assert np.array_equal(i, z["topk_i"]) and np.array_equal(i, i0)
    assert np.array_equal(d, d0, equal_nan=True)


@pytest.mark.parametrize("seed", range(6))
def test_cluster_major_matches_ivf_exact(seed):
    """Random lists with heavy exact ties and duplicated rows, empty lists, K past the probed
    rows, lists of fewer and more than the 256-row chunk and the 8-row groups, many queries per
    cluster: the cluster-major scan equals the query-major one bit for bit, and numpy brute force
    on the ids."""
    rng = np.random.default_rng(100 + seed)
    D = int(rng.integers(1, 70))
    nlist = int(rng.integers(1, 12))
    N = int(rng.integers(0, 3000))
    xb = rng.integers(0, 3, size=(N, D)).astype(np.float32) if seed % 2 == 0 else \
        rng.standard_normal((N, D)).astype(np.float32)
    if N > 10:
        xb[N // 2:N // 2 + 5] = xb[3]  # duplicated rows: ties broken by id
    lid = rng.integers(0, max(nlist - 1, 1), size=N).astype(np.int32)  # the last list may be empty
    cen = rng.standard_normal((nlist, D)).astype(np.float32)
    xq = rng.integers(0, 3, size=(60, D)).astype(np.float32) if seed % 2 == 0 else \
        rng.standard_normal((60, D)).astype(np.float32)
    nprobe = int(rng.integers(1, nlist + 1))
    K = int(rng.integers(1, 60))
    order, vec_off = sorted_lists(lid, nlist)
    cids, _ = O.coarse_probe(xq, cen, nprobe)
    d0, i0 = O.ivf_exact(xq, cids, vec_off, xb[order], order, K)
    d1, i1 = O.ivf_exact_cm(xq, cids, vec_off, xb[order], order, K, threads=3)
    assert np.array_equal(i0, i1)
    assert np.array_equal(d0, d1)
    _, bi = O.np_ivf_exact(xq, xb, lid, cids, K)
    assert np.array_equal(i1, bi)


def test_pair_dists_against_numpy():
    """pair_dists: the canonical distance of explicit (query, sorted row) pairs equals numpy's
    float64 distance on integer data (every order exact) and is within 1e-13 on floats; a mutant
    that swaps the query and row indices of the pairs fails."""
    rng = np.random.default_rng(5)
    for integer in (True, False):
        xb = (rng.integers(0, 200, size=(40, 13)) if integer else rng.standard_normal((40, 13))).astype(np.float32)
        xq = (rng.integers(0, 200, size=(7, 13)) if integer else rng.standard_normal((7, 13))).astype(np.float32)
        qids = rng.integers(0, 7, size=50).astype(np.int32)
        spos = rng.integers(0, 40, size=50).astype(np.int64)
        got = O.pair_dists(xq, xb, qids, spos)
        ref = ((xb[spos].astype(np.float64) - xq[qids].astype(np.float64)) ** 2).sum(1)
        if integer:
            assert np.array_equal(got, ref)
        else:
            np.testing.assert_allclose(got, ref, rtol=1e-13)
        for i in range(0, 50, 7):  # each value is the canonical fma chain of its pair
            assert got[i] == fma_exact_sum(xb[spos[i]], xq[qids[i]])
        swapped = ((xb[np.minimum(qids, 39)].astype(np.float64) -
                    xq[np.minimum(spos, 6)].astype(np.float64)) ** 2).sum(1)
        assert not np.allclose(got, swapped, rtol=1e-6), "a swapped-index mutant was not detected"


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


# ---------------------------------------------------------------------------------------------
# Modes 0 / 1 (oracle_ivf_sq8): pinned by an exact-rational restatement on a tiny index
# ---------------------------------------------------------------------------------------------
def _round_f32(fr: Fraction) -> float:
    """Round a rational to the nearest float32 (ties to even), once."""
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    x = abs(fr)
    e = x.numerator.bit_length() - x.denominator.bit_length()
    if Fraction(2) ** e > x:
        e -= 1
    qe = max(e - 23, -149)
    m = x / Fraction(2) ** qe
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * float(Fraction(n) * Fraction(2) ** qe)


def _fmaf(a, b, c):
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _fma64(a, b, c):
    return float(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def _tiny_sq8_index(seed=0):
    rng = np.random.default_rng(seed)
    nlist, D, D_pad, T = 3, 20, 32, 64
    sizes = [70, 5, 130]
    vec_off = np.zeros(nlist + 1, np.int32)
    vec_off[1:] = np.cumsum(sizes)
    ntile = [(n + T - 1) // T for n in sizes]
    tile_off = np.zeros(nlist + 1, np.int32)
    tile_off[1:] = np.cumsum(ntile)
    tiles = int(tile_off[-1])
    N = int(vec_off[-1])
    oids = rng.permutation(N).astype(np.int32)
    tile_oids = np.full((tiles, T), -1, np.int32)
    for c in range(nlist):
        for l in range(sizes[c]):
            tile_oids[tile_off[c] + l // T, l % T] = oids[vec_off[c] + l]
    W = np.zeros((D, nlist + D_pad), np.float32)
    W[:, :nlist] = rng.standard_normal((D, nlist)).astype(np.float32)
    W[:, nlist:nlist + D] = rng.standard_normal((D, D)).astype(np.float32) / np.sqrt(D)
    bvec = np.zeros(nlist + D_pad, np.float32)
    bvec[nlist:nlist + D] = rng.standard_normal(D).astype(np.float32) * 0.1
    vmin = (rng.standard_normal((nlist, D_pad)) - 3.0).astype(np.float32)
    delta = (rng.random((nlist, D_pad)) * 0.05 + 0.01).astype(np.float32)
    codes = rng.integers(0, 2**32, size=(tiles, D_pad // 4, T), dtype=np.uint64).astype(np.uint32)
    xb = rng.standard_normal((N, D)).astype(np.float32)
    xq = rng.standard_normal((4, D)).astype(np.float32)
    ix = dict(W_combined=W, b_combined=bvec, nlist=nlist, D_pad=D_pad, vec_off=vec_off, tile_off=tile_off,
              T=T, sq8_packed=codes, tile_oids=tile_oids, vmin=vmin, delta=delta, per_cluster=1, xb_sorted=xb)
    return ix, xq


def _exact_hats(ix, q, c):
    """Every acc_hat of cluster c for query q, exact rational fmaf / fma (one rounding each)."""
    nlist, D_pad, T = ix["nlist"], ix["D_pad"], ix["T"]
    W, bvec = ix["W_combined"], ix["b_combined"]
    xr = []
    for j in range(D_pad):
        acc = 0.0
        for d in range(q.shape[0]):
            acc = _fma64(q[d], W[d, nlist + j], acc)
        xr.append(acc + float(bvec[nlist + j]))
    base = [float(np.float32(float(ix["vmin"][c, d]) - xr[d])) for d in range(D_pad)]
    out = []
    v0, n, t0 = ix["vec_off"][c], ix["vec_off"][c + 1] - ix["vec_off"][c], ix["tile_off"][c]
    for l in range(n):
        tile, slot = t0 + l // T, l % T
        acc = 0.0
        for d in range(D_pad):
            code = (int(ix["sq8_packed"][tile, d // 4, slot]) >> (8 * (d % 4))) & 0xFF
            a = _fmaf(code, ix["delta"][c, d], base[d])
            acc = _fmaf(a, a, acc)
        out.append((acc, int(ix["tile_oids"][tile, slot]), v0 + l))
    return out


def _exact_dist(x, q):
    acc = 0.0
    for d in range(len(q)):
        t = float(x[d]) - float(q[d])
        acc = _fma64(t, t, acc)
    return acc


def test_sq8_hats_match_exact_rational_fmaf():
    """Mode 1 with K = every vector returns every acc_hat, sorted by (acc_hat, id): bit-identical
    to the exact-rational restatement (one rounding per fmaf, dims in order)."""
    ix, xq = _tiny_sq8_index()
    q = xq[:2]
    N = int(ix["vec_off"][-1])
    probes = np.array([[2, 0, 1], [1, 2, 0]], np.int32)
    d, i = O.ivf_sq8(q, probes, 0, ix, N, N, N, 0)
    for b in range(len(q)):
        ref = sorted((h, oid) for c in range(3) for (h, oid, _) in _exact_hats(ix, q[b], c))
        assert [oid for _, oid in ref] == i[b].tolist()
        assert np.array_equal(np.array([h for h, _ in ref], np.float32), d[b])
    # power of the check: an unfused a * a + acc, or the dims summed in reverse, change the
    # bits of some of these hats (so an oracle written either way fails the comparison above)
    c, nlist, D_pad, T = 2, ix["nlist"], ix["D_pad"], ix["T"]
    xr = O.rotate_query(q[0], ix["W_combined"], ix["b_combined"], nlist, D_pad)
    base = (ix["vmin"][c].astype(np.float64) - xr).astype(np.float32)
    n_unfused = n_rev = 0
    for h, _, spos in _exact_hats(ix, q[0], c)[:40]:
        l = spos - ix["vec_off"][c]
        tile, slot = ix["tile_off"][c] + l // T, l % T
        codes = [(int(ix["sq8_packed"][tile, d // 4, slot]) >> (8 * (d % 4))) & 0xFF for d in range(D_pad)]
        a = [_fmaf(codes[d], ix["delta"][c, d], base[d]) for d in range(D_pad)]
        unfused = np.float32(0)
        for d in range(D_pad):
            unfused = np.float32(unfused + np.float32(np.float32(a[d]) * np.float32(a[d])))
        rev = 0.0
        for d in reversed(range(D_pad)):
            rev = _fmaf(a[d], a[d], rev)
        n_unfused += float(unfused) != h
        n_rev += rev != h
    assert n_unfused > 0 and n_rev > 0


def _pool_ref(ix, q, probes, p_init, K, k1, k2, M):
    pool = []
    for p, c in enumerate(probes):
        kp = k1 if p < p_init else k2
        pool += sorted((h, oid, spos) for (h, oid, spos) in _exact_hats(ix, q, c))[:kp]
    pool.sort()
    if M == 0:
        top = pool[:K]
        return [h for h, _, _ in top], [oid for _, oid, _ in top]
    ranked = sorted((_exact_dist(ix["xb_sorted"][spos], q), oid) for (_, oid, spos) in pool[:M])[:K]
    return [float(np.float32(dd)) for dd, _ in ranked], [oid for _, oid in ranked]


@pytest.mark.parametrize("K,k1,k2,M,p_init", [(5, 5, 5, 0, 1), (3, 12, 4, 9, 1), (4, 40, 6, 30, 2),
                                               (10, 2, 3, 0, 0)])
def test_sq8_pool_and_rerank_match_restatement(K, k1, k2, M, p_init):
    """Per-pair truncation (k_p1 for the first p_init probes, k_p2 after), the pooled top-M and
    the exact rerank, against the exact-rational restatement."""
    ix, xq = _tiny_sq8_index(seed=1)
    probes = np.array([[2, 0, 1], [0, 1, 2], [1, 2, 0], [2, 1, 0]], np.int32)
    d, i = O.ivf_sq8(xq, probes, p_init, ix, K, k1, k2, M)
    for b in range(len(xq)):
        rd, ri = _pool_ref(ix, xq[b], probes[b], p_init, K, k1, k2, M)
        n = len(ri)
        assert i[b, :n].tolist() == ri and (i[b, n:] == -1).all()
        assert np.array_equal(d[b, :n], np.array(rd, np.float32))


def test_sq8_mode_plan_known_values():
    """The reference's split and list lengths at hand-evaluated points
    (src/trident_v4_kernels.cu:1264-1276, :1439-1443, :1071-1073)."""
    assert O.sq8_mode_plan(0, 1000, 10, 32, 100) == (2, 100, 16, 100)
    assert O.sq8_mode_plan(0, 1000, 10, 3, 100) == (1, 100, 42, 100)
    assert O.sq8_mode_plan(0, 1000, 10, 8, 20) == (1, 20, 16, 20)
    assert O.sq8_mode_plan(0, 1, 10, 8, 0) == (0, 10, 10, 0)
    assert O.sq8_mode_plan(0, 64, 10, 1, 200) == (0, 128, 200, 200)
    assert O.sq8_mode_plan(0, 64, 50, 16, 300) == (2, 128, 50, 200)
    assert O.sq8_mode_plan(0, 64, 10, 16, 300) == (2, 128, 27, 200)
    assert O.sq8_mode_plan(1, 1, 10, 8, 0) == (1, 10, 10, 0)
    assert O.sq8_mode_plan(1, 500, 10, 64, 0) == (3, 10, 10, 0)
