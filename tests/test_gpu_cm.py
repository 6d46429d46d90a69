"""GPU parity of mode 10's matrix-core route (float32 MFMA distances with an error band, the
listed rows refined in float64) against the float64 oracle, and its agreement with the per-pair
float64 route.  Same bar as test_gpu_parity.py: ids identical on every query, float32 distances
equal to the oracle's float64 distances rounded to float32."""
import numpy as np
import pytest
import torch

from tests.helpers import assert_exact, build_index, oracle_search, run_search
from trident_amd import datagen
from trident_amd._lib import TridentError

pytestmark = pytest.mark.gpu


def _q(xq, dev):
    return torch.as_tensor(np.ascontiguousarray(xq, np.float32)).to(dev).contiguous()


@pytest.fixture(scope="module")
def cm_sets(dev):
    out = {}
    xb, xq = datagen.cfg2(N=40_000, D=128, B=300, n_centers=64, seed=61)
    out["hist"] = (build_index(xb, 64, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg4(N=40_000, D=96, B=300, n_centers=128, seed=62)
    out["norm96"] = (build_index(xb, 128, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg1(N=30_000, D=200, B=200, n_centers=32, seed=63)
    out["d200"] = (build_index(xb, 48, dev, max_batch=512, tile_size=256), xq.numpy())
    xb, xq = datagen.cfg1(N=20_000, D=50, B=200, n_centers=32, seed=64)  # D % 4 != 0
    out["d50"] = (build_index(xb, 40, dev, max_batch=512), xq.numpy())
    return out


@pytest.mark.parametrize("name", ["hist", "norm96", "d200", "d50"])
@pytest.mark.parametrize("K", [1, 10, 16, 17, 64, 100, 128])
def test_cm_route_exact(cm_sets, dev, name, K):
    b, xq = cm_sets[name]
    for nprobe in (4, 24):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=10, route=2)
        assert_exact(d, i, rd, ri, f"cm {name} K={K} nprobe={nprobe}")


def test_cm_matches_pair_route_and_auto(cm_sets, dev):
    b, xq = cm_sets["hist"]
    xqd = _q(xq, dev)
    d1, i1 = run_search(b, xqd, 32, 10, mode=10, route=1)
    d2, i2 = run_search(b, xqd, 32, 10, mode=10, route=2)
    d0, i0 = run_search(b, xqd, 32, 10, mode=10, route=0)
    assert np.array_equal(i1, i2) and np.array_equal(d1, d2)
    assert np.array_equal(i0, i2) and np.array_equal(d0, d2)


def test_cm_exact_ties(dev):
    """40 copies of every row: the float32 band cannot separate tied rows, so every copy at the
    K-th distance must be listed and the ids resolved by (d, id) in float64."""
    rng = np.random.default_rng(65)
    base = rng.integers(0, 3, size=(60, 16)).astype(np.float32)
    xb = np.repeat(base, 40, axis=0)
    nlist = 6
    cen = rng.integers(0, 3, size=(nlist, 16)).astype(np.float32)
    lid = np.argmin(((xb[:, None, :] - cen[None]) ** 2).sum(-1), 1).astype(np.int32)
    xq = np.concatenate([base[:20], rng.integers(0, 3, size=(20, 16))]).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, list_ids=lid, centroids=cen, max_batch=64)
    for K, nprobe in ((1, 1), (5, 2), (10, 4), (16, 6), (40, 3), (100, 6)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=10, route=2)
        assert_exact(d, i, rd, ri, f"cm ties K={K} nprobe={nprobe}")


@pytest.mark.parametrize("D", [32, 64, 256])
def test_cm_short_and_empty_lists(dev, D):
    """Probed lists with fewer than K vectors in total (missing slots (+inf, -1) as in the
    oracle), empty lists, and partial 64-vector blocks."""
    rng = np.random.default_rng(66 + D)
    nlist = 24
    cen = (rng.standard_normal((nlist, D)) * 10.0).astype(np.float32)
    used = np.arange(0, nlist, 3)
    lid = rng.choice(used, size=100).astype(np.int32)  # ~12 vectors per used list
    xb = (cen[lid] + rng.standard_normal((100, D)).astype(np.float32)).astype(np.float32)
    xq = (cen[rng.integers(0, nlist, 40)] + rng.standard_normal((40, D))).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, list_ids=lid, centroids=cen, max_batch=64)
    assert (np.diff(b.vec_off) == 0).sum() > 0
    short = False
    for K, nprobe in ((16, 2), (10, 3), (16, 12), (50, 3), (128, 12)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=10, route=2)
        assert_exact(d, i, rd, ri, f"cm short/empty D={D} K={K} nprobe={nprobe}")
        short |= bool((ri == -1).any())
    assert short  # some query really has fewer than K candidates


def test_cm_large_clusters_and_many_units(dev):
    """~5000 vectors per cluster (five slices, 16 blocks each) and ~4000 queries: thousands of
    units taken from the work counter by every resident workgroup."""
    xb, xq = datagen.cfg1(N=40_000, D=64, B=2000, n_centers=8, seed=67)
    b = build_index(xb, 8, dev, max_batch=2048)
    assert np.diff(b.vec_off).max() > 2048
    for nprobe, K in ((1, 10), (3, 16), (8, 1), (2, 100), (8, 128)):
        _, rd, ri = oracle_search(b, xq.numpy(), nprobe, K)
        d, i = run_search(b, _q(xq.numpy(), dev), nprobe, K, mode=10, route=2)
        assert_exact(d, i, rd, ri, f"cm large nprobe={nprobe} K={K}")


def test_cm_route_k_above_16_matches_pair_route(cm_sets, dev):
    """K > 16: thresholds from the warm-up's listed rows (cm_seed_kernel) instead of the scan's
    16 column minima; the same results as the per-pair float64 route, on AUTO too."""
    b, xq = cm_sets["norm96"]
    xqd = _q(xq, dev)
    for K in (17, 100):
        d1, i1 = run_search(b, xqd, 24, K, mode=10, route=1)
        d2, i2 = run_search(b, xqd, 24, K, mode=10, route=2)
        d0, i0 = run_search(b, xqd, 24, K, mode=10, route=0)
        assert np.array_equal(i1, i2) and np.array_equal(d1, d2)
        assert np.array_equal(i0, i2) and np.array_equal(d0, d2)


@pytest.fixture(scope="module")
def wide_sets(dev):
    """Past 256 dims: the wide kernel (dims in 128-dim chunks), D % 4 == 0 and not."""
    out = {}
    xb, xq = datagen.cfg1(N=12_000, D=300, B=160, n_centers=16, seed=71)
    out["d300"] = (build_index(xb, 24, dev, max_batch=256, tile_size=256), xq.numpy())
    xb, xq = datagen.cfg3(N=8_000, D=960, B=96, n_centers=16, seed=72)
    out["d960"] = (build_index(xb, 16, dev, max_batch=256, tile_size=256), xq.numpy())
    xb, xq = datagen.cfg1(N=6_000, D=263, B=96, n_centers=16, seed=73)  # D % 4 == 3
    out["d263"] = (build_index(xb, 12, dev, max_batch=256, tile_size=256), xq.numpy())
    return out


@pytest.mark.parametrize("name", ["d300", "d960", "d263"])
@pytest.mark.parametrize("K", [1, 10, 16, 100])
def test_cm_wide_route_exact(wide_sets, dev, name, K):
    b, xq = wide_sets[name]
    for nprobe in (2, 8):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=10, route=2)
        assert_exact(d, i, rd, ri, f"cm wide {name} K={K} nprobe={nprobe}")


def test_cm_wide_matches_pair_route_and_auto(wide_sets, dev):
    b, xq = wide_sets["d960"]
    xqd = _q(xq, dev)
    for K in (10, 50):
        d1, i1 = run_search(b, xqd, 8, K, mode=10, route=1)
        d2, i2 = run_search(b, xqd, 8, K, mode=10, route=2)
        d0, i0 = run_search(b, xqd, 8, K, mode=10, route=0)
        assert np.array_equal(i1, i2) and np.array_equal(d1, d2)
        assert np.array_equal(i0, i2) and np.array_equal(d0, d2)


def test_cm_wide_exact_ties(dev):
    """Duplicated rows at D = 320: every copy at the K-th distance listed, ids by (d, id)."""
    rng = np.random.default_rng(74)
    base = rng.integers(0, 3, size=(40, 320)).astype(np.float32)
    xb = np.repeat(base, 20, axis=0)
    nlist = 5
    cen = rng.integers(0, 3, size=(nlist, 320)).astype(np.float32)
    lid = np.argmin(((xb[:, None, :] - cen[None]) ** 2).sum(-1), 1).astype(np.int32)
    xq = np.concatenate([base[:16], rng.integers(0, 3, size=(16, 320))]).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, list_ids=lid, centroids=cen, max_batch=64,
                    tile_size=256)
    for K, nprobe in ((1, 1), (10, 2), (30, 5)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        d, i = run_search(b, _q(xq, dev), nprobe, K, mode=10, route=2)
        assert_exact(d, i, rd, ri, f"cm wide ties K={K} nprobe={nprobe}")


def test_cm_route_requirements(cm_sets, dev):
    b, xq = cm_sets["hist"]
    xqd = _q(xq[:8], dev)
    with pytest.raises(TridentError, match="K"):
        run_search(b, xqd, 4, 129, mode=10, route=2)


def test_cm_host_base_matrix_route(dev):
    """Mode 10 on the matrix cores with the FP32 base in mapped host memory: exact on the
    explicit and the automatic route (which takes the matrix cores for a host base), and a probed
    row crosses PCIe once per unit, not once per (query, probe) pair as on the per-pair route."""
    xb, xq = datagen.cfg2(N=10_000, D=128, B=64, n_centers=16, seed=68)
    b = build_index(xb, 16, dev, xb_placement="host", max_batch=64)
    try:
        xqd = _q(xq.numpy(), dev)
        _, rd, ri = oracle_search(b, xq.numpy(), 4, 10)
        rows = {}
        for route in (2, 0, 1):
            hrows = torch.zeros(2, dtype=torch.int64, device=dev)
            d, i, _ = b.ix.search(xqd, 4, mode=10, k=10, route=route, host_rows_buf=hrows)
            torch.cuda.synchronize()
            assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri, f"cm host base route={route}")
            rows[route] = int(hrows[0])
        assert 0 < rows[2] < rows[1] and 0 < rows[0] < rows[1], rows
    finally:
        torch.cuda.synchronize()
        b.ix.storage._host_buf.free()
