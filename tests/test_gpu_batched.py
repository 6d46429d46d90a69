"""GPU parity of the cluster-batched (int8 matrix-core) cascade against the float64 oracle.

Same bar as test_gpu_parity.py: ids identical on every query, float32 distances equal to the
oracle's float64 distances rounded to float32.
"""
import numpy as np
import pytest
import torch

from tests.helpers import assert_exact, build_index, oracle_search, run_search
from trident_amd import datagen, ext

pytestmark = pytest.mark.gpu


def _q(xq, dev):
    return torch.as_tensor(np.ascontiguousarray(xq, np.float32)).to(dev).contiguous()


@pytest.fixture(scope="module")
def sets(dev):
    out = {}
    xb, xq = datagen.cfg2(N=60_000, D=128, B=400, n_centers=128, seed=21)
    out["hist"] = (build_index(xb, 128, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg4(N=50_000, D=96, B=400, n_centers=256, seed=22)
    out["norm96"] = (build_index(xb, 200, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg1(N=40_000, D=128, B=300, n_centers=64, seed=23)
    out["gmm"] = (build_index(xb, 100, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg1(N=20_000, D=200, B=200, n_centers=32, seed=24)
    out["d200"] = (build_index(xb, 64, dev, max_batch=512, tile_size=256), xq.numpy())
    return out


@pytest.mark.parametrize("name", ["hist", "norm96", "gmm", "d200"])
@pytest.mark.parametrize("K", [1, 10, 64, 100, 128])
def test_batched_route_exact(sets, dev, name, K):
    b, xq = sets[name]
    for nprobe in (4, 24):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=2)
        assert_exact(d, i, rd, ri, f"batched {name} K={K} nprobe={nprobe}")


def test_batched_matches_pair_route_and_auto(sets, dev):
    b, xq = sets["hist"]
    xqd = _q(xq, dev)
    d1, i1 = run_search(b, xqd, 32, 10, mode=2, ub=1, route=1)
    d2, i2 = run_search(b, xqd, 32, 10, mode=2, ub=1, route=2)
    d0, i0 = run_search(b, xqd, 32, 10, mode=2, ub=1, route=0)
    assert np.array_equal(i1, i2) and np.array_equal(d1, d2)
    assert np.array_equal(i0, i2) and np.array_equal(d0, d2)


@pytest.mark.parametrize("name", ["hist", "norm96", "gmm"])
def test_row_norm_allowance_changes_no_result(sets, dev, name):
    """The lower-bound pass's hi-plane prefilter with the per-row code norms (vec_cn: a
    Cauchy-Schwarz allowance for the lo plane) and without them (128 sum |lo| per query): the
    prefilter only decides which tiles need the lo plane, so the results are identical, and
    exact, and so is the candidate count.  (The survivor count is not compared: the order in
    which a cluster's pairs land in its segment comes from atomics, and it decides which 32
    queries share a weight group's scale, so it varies between identical runs.)"""
    b, xq = sets[name]
    ix = b.ix
    xqd = _q(xq, dev)
    for K, nprobe in ((1, 8), (10, 24), (100, 24)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        out = []
        for keep in (True, False):
            saved = ix.vec_cn
            if not keep:
                ix.vec_cn = None
            try:
                st = torch.zeros(4, dtype=torch.int64, device=dev)
                d, i = run_search(b, xqd, nprobe, K, mode=2, ub=1, route=2, stats=st)
            finally:
                ix.vec_cn = saved
            assert_exact(d, i, rd, ri, f"batched {name} K={K} nprobe={nprobe} row norms={keep}")
            out.append((d, i, st.cpu().numpy()))
        assert np.array_equal(out[0][1], out[1][1]) and np.array_equal(out[0][0], out[1][0])
        assert out[0][2][0] == out[1][2][0] and out[0][2][1] == out[1][2][1], (out[0][2], out[1][2])


@pytest.mark.parametrize("nprobe", [1, 2, 3])
def test_batched_small_nprobe_and_single_query(sets, dev, nprobe):
    """nprobe 1 has no seeding pass (every candidate survives, candidate lists overflow and the
    merge rescans exactly); B = 1 exercises one-query chunks."""
    b, xq = sets["hist"]
    for B in (1, 33):
        _, rd, ri = oracle_search(b, xq[:B], nprobe, 10)
        d, i = run_search(b, _q(xq[:B], dev), nprobe, 10, mode=2, ub=1, route=2)
        assert_exact(d, i, rd, ri, f"batched nprobe={nprobe} B={B}")


def test_batched_overflow_fallback_on_exact_ties(dev):
    """40 copies of every row: all copies tie at the threshold, the per-query lists overflow
    nprobe * K and the merge's exhaustive rescan must still return ids by (d, id)."""
    rng = np.random.default_rng(31)
    base = rng.integers(0, 3, size=(60, 16)).astype(np.float32)
    xb = np.repeat(base, 40, axis=0)
    nlist = 6
    cen = rng.integers(0, 3, size=(nlist, 16)).astype(np.float32)
    lid = np.argmin(((xb[:, None, :] - cen[None]) ** 2).sum(-1), 1).astype(np.int32)
    xq = np.concatenate([base[:20], rng.integers(0, 3, size=(20, 16))]).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, list_ids=lid, centroids=cen, max_batch=64)
    # Repeated: every row of a tile ties with its neighbours, so a row that reads another
    # tile's sums (an accumulator read issued too early after its MFMA) changes the answer;
    # such a fault depends on timing, hence several runs.
    for rep in range(3):
        for K, nprobe in ((5, 2), (10, 4), (64, 6)):
            _, rd, ri = oracle_search(b, xq, nprobe, K)
            d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=2)
            assert_exact(d, i, rd, ri, f"ties rep={rep} K={K} nprobe={nprobe}")


def test_batched_host_mapped_base(dev):
    xb, xq = datagen.cfg2(N=30_000, D=128, B=200, n_centers=64, seed=25)
    b = build_index(xb, 64, dev, xb_placement="host", max_batch=256)
    _, rd, ri = oracle_search(b, xq.numpy(), 16, 10)
    d, i = run_search(b, _q(xq.numpy(), dev), 16, 10, mode=2, ub=1, route=2)
    assert_exact(d, i, rd, ri, "batched ooc")
    b.ix.storage._host_buf.free()


@pytest.mark.parametrize("K", [1, 10, 64])
def test_batched_large_clusters_split_into_slices(dev, K):
    """~5000 vectors per cluster: in both passes every cluster is scanned as 3 vector slices
    (units of <= 128 queries x ~2048 vectors), so survivors come from many slices."""
    xb, xq = datagen.cfg1(N=40_000, D=64, B=300, n_centers=8, seed=26)
    b = build_index(xb, 8, dev, max_batch=512)
    sizes = np.diff(b.vec_off)
    assert sizes.max() > 2048
    for nprobe in (1, 3, 8):
        _, rd, ri = oracle_search(b, xq.numpy(), nprobe, K)
        d, i = run_search(b, _q(xq.numpy(), dev), nprobe, K, mode=2, ub=1, route=2)
        assert_exact(d, i, rd, ri, f"slices K={K} nprobe={nprobe}")


@pytest.mark.parametrize("seed_rows", [0, 100, 1024, 4096])
def test_seed_rows_changes_no_result(dev, seed_rows):
    """TridentIndexView.seed_rows caps the seeding slices (0: 2048 rows; else max(512, seed_rows),
    at most 2048): ~3750 rows per cluster in residual-norm order are seeded from their first
    ~1920, 960 or 512 rows.  Only the threshold's tightness changes: every seeded threshold stays
    >= the query's exact K-th distance and the results equal the oracle's."""
    xb, xq = datagen.cfg2(N=60_000, D=128, B=300, n_centers=16, seed=31)
    b = build_index(xb, 16, dev, max_batch=512, within="residual")
    assert b.ix.storage.within == "residual" and b.ix.seed_rows > 0
    assert np.diff(b.vec_off).max() > 2048
    v = b.ix.view()
    v.seed_rows = seed_rows
    q = _q(xq.numpy(), dev)
    for nprobe, K in ((3, 10), (8, 64)):
        _, rd, ri = oracle_search(b, xq.numpy(), nprobe, K)
        d = torch.empty((q.shape[0], K), dtype=torch.float32, device=dev)
        i = torch.empty((q.shape[0], K), dtype=torch.int64, device=dev)
        tau = torch.empty(q.shape[0], dtype=torch.float32, device=dev)
        ext.search_view(v, q, nprobe, d, i, mode=2, ub_seed=1, route=2, tau_sq=tau)
        torch.cuda.synchronize()
        assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri, f"seed_rows={seed_rows} K={K}")
        t = tau.cpu().numpy().astype(np.float64)
        assert (t >= rd[:, K - 1]).all(), f"seeded threshold below the K-th distance (K={K})"


def test_batched_many_units_per_workgroup(dev):
    """~200k (query, probe) pairs in 256 clusters: thousands of work units, several per
    persistent workgroup, so every workgroup hands the next unit's index to its waves through
    LDS between units (a wave reading a stale index would scan the wrong unit)."""
    xb, xq = datagen.cfg2(N=100_000, D=128, B=4096, n_centers=256, seed=27)
    b = build_index(xb, 256, dev, max_batch=4096)
    for rep in range(2):
        _, rd, ri = oracle_search(b, xq.numpy(), 48, 10)
        d, i = run_search(b, _q(xq.numpy(), dev), 48, 10, mode=2, ub=1, route=2)
        assert_exact(d, i, rd, ri, f"many units rep={rep}")


def test_batched_rejects_k_above_128(sets, dev):
    from trident_amd._lib import TridentError
    b, xq = sets["hist"]
    with pytest.raises(TridentError, match="outside"):
        run_search(b, _q(xq, dev), 8, 129, mode=2, route=2)


def test_batched_k100_matches_pair_route(sets, dev):
    """K > 64: seeding units list their 64 smallest bounds, the threshold is the K-th over all
    of a query's units; both routes return the same lists."""
    b, xq = sets["hist"]
    xqd = _q(xq, dev)
    d1, i1 = run_search(b, xqd, 32, 100, mode=2, ub=1, route=1)
    d2, i2 = run_search(b, xqd, 32, 100, mode=2, ub=1, route=2)
    assert np.array_equal(i1, i2) and np.array_equal(d1, d2)


@pytest.fixture(scope="module")
def wide_sets(dev):
    """D_pad > 256: the scans stage 16-vector blocks and keep up to 16 steps of weights."""
    out = {}
    xb, xq = datagen.cfg3(N=24_000, D=960, B=300, n_centers=64, seed=41)
    out["d960"] = (build_index(xb, 40, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg1(N=20_000, D=288, B=300, n_centers=32, seed=42)  # last step half-full
    out["d288"] = (build_index(xb, 48, dev, max_batch=512), xq.numpy())
    return out


@pytest.mark.parametrize("name", ["d960", "d288"])
@pytest.mark.parametrize("K", [1, 10, 64, 100])
def test_batched_wide_route_exact(wide_sets, dev, name, K):
    b, xq = wide_sets[name]
    assert b.ix.D_pad > 256
    for nprobe in (3, 16):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=2)
        assert_exact(d, i, rd, ri, f"batched {name} K={K} nprobe={nprobe}")


def test_batched_wide_matches_pair_route_and_auto(wide_sets, dev):
    b, xq = wide_sets["d960"]
    xqd = _q(xq, dev)
    assert b.ix.route_for(len(xq), 16, 10) == 2  # AUTO takes the batched route at D = 960
    assert b.ix.route_for(len(xq), 16, 100) == 2  # ... for every K <= 128
    d1, i1 = run_search(b, xqd, 16, 10, mode=2, ub=1, route=1)
    d2, i2 = run_search(b, xqd, 16, 10, mode=2, ub=1, route=2)
    d0, i0 = run_search(b, xqd, 16, 10, mode=2, ub=1, route=0)
    assert np.array_equal(i1, i2) and np.array_equal(d1, d2)
    assert np.array_equal(i0, i2) and np.array_equal(d0, d2)


def test_batched_wide_host_mapped_base(dev):
    xb, xq = datagen.cfg3(N=12_000, D=960, B=120, n_centers=32, seed=43)
    b = build_index(xb, 24, dev, xb_placement="host", max_batch=128)
    _, rd, ri = oracle_search(b, xq.numpy(), 6, 10)
    d, i = run_search(b, _q(xq.numpy(), dev), 6, 10, mode=2, ub=1, route=2)
    assert_exact(d, i, rd, ri, "batched wide ooc")
    b.ix.storage._host_buf.free()


def test_batched_wide_exact_ties_and_replicas(dev):
    """D = 300 (wide layout, last 64-dim step half-full), 40 copies of every row: ties at the
    threshold everywhere.  Units of few queries make replica waves split the 64-dim steps and
    finish each block from their summed partials one block later; an early accumulator read
    or a partial summed twice changes the answer."""
    rng = np.random.default_rng(44)
    base = rng.integers(0, 3, size=(60, 300)).astype(np.float32)
    xb = np.repeat(base, 40, axis=0)
    nlist = 6
    cen = rng.integers(0, 3, size=(nlist, 300)).astype(np.float32)
    lid = np.argmin(((xb[:, None, :] - cen[None]) ** 2).sum(-1), 1).astype(np.int32)
    xq = np.concatenate([base[:20], rng.integers(0, 3, size=(20, 300))]).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, list_ids=lid, centroids=cen, max_batch=64)
    assert b.ix.D_pad == 320
    for rep in range(2):
        for K, nprobe in ((5, 2), (10, 4), (64, 6)):
            _, rd, ri = oracle_search(b, xq, nprobe, K)
            d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=2)
            assert_exact(d, i, rd, ri, f"wide ties rep={rep} K={K} nprobe={nprobe}")


def test_batched_wide_integer_range_guard(dev):
    """D = 960, identity rotation: a cluster spanning [0, 1]^960 (the all-zeros and all-ones rows
    included) and queries near 3 * ones make every weight of a pair equal and maximal, and the
    all-ones row (every code 255) is the nearest neighbour.  Without the weight scale's L1
    limit its int32 sum would be 127 * 960 * 32639 ~ 4e9 (wrapped, so the row's bounds would be
    wrong); with it the answer is exact."""
    rng = np.random.default_rng(45)
    D = 960
    c0 = rng.random((400, D), dtype=np.float32)
    c0[0], c0[1] = 0.0, 1.0
    c1 = (rng.random((400, D), dtype=np.float32) - 10.0)
    xb = np.concatenate([c0, c1])
    lid = np.repeat(np.arange(2, dtype=np.int32), 400)
    cen = np.stack([c0.mean(0), c1.mean(0)]).astype(np.float32)
    xq = (3.0 + 0.01 * rng.standard_normal((24, D))).astype(np.float32)
    b = build_index(torch.as_tensor(xb), 2, dev, list_ids=lid, centroids=cen, max_batch=32,
                    use_pca=0)
    for K, nprobe in ((10, 2), (1, 1), (64, 2)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        assert (ri[:, 0] == 1).all()  # the all-ones row
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=2)
        assert_exact(d, i, rd, ri, f"range guard K={K} nprobe={nprobe}")


@pytest.mark.parametrize("D", [64, 320])
def test_batched_short_and_empty_lists(dev, D):
    """Probed lists with fewer than K vectors in total (the missing slots must be (+inf, -1)
    as in the oracle) and probed lists that are empty (centroids nobody was assigned to), on
    the narrow and the wide layout."""
    rng = np.random.default_rng(46 + D)
    nlist = 24
    cen = (rng.standard_normal((nlist, D)) * 10.0).astype(np.float32)
    used = np.arange(0, nlist, 3)                       # lists 1, 2, 4, 5, ... stay empty
    lid = rng.choice(used, size=180).astype(np.int32)   # ~22 vectors per used list
    xb = (cen[lid] + rng.standard_normal((180, D)).astype(np.float32)).astype(np.float32)
    xq = (cen[rng.integers(0, nlist, 40)] + rng.standard_normal((40, D))).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, list_ids=lid, centroids=cen, max_batch=64)
    assert (np.diff(b.vec_off) == 0).sum() > 0
    for K, nprobe in ((64, 2), (100, 3), (10, 5), (128, 12)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=2)
        assert_exact(d, i, rd, ri, f"short/empty D={D} K={K} nprobe={nprobe}")
        assert (ri == -1).any()  # some query really has fewer than K candidates


@pytest.mark.parametrize("name", ["hist", "gmm"])
def test_cluster_bounds_table(sets, dev, name):
    """trident_cluster_bounds against a float64 restatement (A_max = 255^2 sum delta^2, r_max =
    max(2 sqrt(sum eps^2), max r_x), r_lo = min r_x, each with its 1e-12 margin), and a search
    that recomputes the table per call returns the same results as one given the table."""
    from trident_amd import ext
    b, xq = sets[name]
    ix = b.ix
    cb = ext.compute_cluster_bounds(ix.view(), dev).cpu().numpy()
    delta = ix.delta_pad.double().cpu().numpy().reshape(-1, ix.D_pad)
    eps = ix.eps_pad.double().cpu().numpy().reshape(-1, ix.D_pad)
    r = ix.vec_Ar[:, 1].double().cpu().numpy()
    vo = b.vec_off
    for c in range(ix.nlist):
        row = c if delta.shape[0] > 1 else 0
        a_max = 65025.0 * float((delta[row] ** 2).sum()) * (1 + 1e-12)
        rc = r[vo[c]:vo[c + 1]]
        r_max = max(2.0 * np.sqrt(float((eps[row] ** 2).sum())), float(rc.max()) if rc.size else 0.0)
        assert cb[c, 0] == pytest.approx(a_max, rel=1e-13), c
        assert cb[c, 1] == pytest.approx(r_max * (1 + 1e-12), rel=1e-13), c
        assert cb[c, 2] == (float(rc.min()) if rc.size else 0.0), c
    xqd = _q(xq, dev)
    d1, i1 = run_search(b, xqd, 16, 10, mode=2, ub=1, route=2)
    saved, ix.cluster_bounds = ix.cluster_bounds, None
    try:
        d2, i2 = run_search(b, xqd, 16, 10, mode=2, ub=1, route=2)
    finally:
        ix.cluster_bounds = saved
    assert np.array_equal(i1, i2) and np.array_equal(d1, d2)
