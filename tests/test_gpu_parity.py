"""GPU parity: the HIP path against the float64 CPU oracle on the same seeded inputs.

Bar: ids identical on every query and float32 distances equal to the oracle's float64 distances
rounded to float32 (hence within 1e-5 relative).  Sizes keep the oracle to seconds.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_exact, build_index, oracle_search, run_search
from trident_amd import _lib, datagen, ext

pytestmark = pytest.mark.gpu


def _q(xq, dev):
    return torch.as_tensor(np.ascontiguousarray(xq, np.float32)).to(dev).contiguous()


@pytest.fixture(scope="module")
def gmm(dev):
    xb, xq = datagen.cfg1(N=30_000, D=128, B=200, n_centers=64, seed=1)
    b = build_index(xb, 96, dev, max_batch=512)
    return b, xq.numpy()


@pytest.fixture(scope="module")
def hist(dev):
    xb, xq = datagen.cfg2(N=40_000, D=128, B=200, n_centers=128, seed=2)
    b = build_index(xb, 128, dev, max_batch=512)
    return b, xq.numpy()


@pytest.fixture(scope="module")
def aniso(dev):
    xb, xq = datagen.cfg3(N=12_000, D=960, B=64, n_centers=64, seed=3)
    b = build_index(xb, 64, dev, max_batch=128)
    return b, xq.numpy()


@pytest.fixture(scope="module")
def norm96(dev):
    xb, xq = datagen.cfg4(N=40_000, D=96, B=200, n_centers=256, seed=4)
    b = build_index(xb, 256, dev, max_batch=512)
    return b, xq.numpy()


def _check_probes(b, xq, dev, nprobe):
    b.ix.search(_q(xq, dev), nprobe, mode=10, k=10)
    torch.cuda.synchronize()
    got = b.ix.probe_cids_buf[: len(xq), :nprobe].cpu().numpy()
    got_d = b.ix.probe_dqcs_buf[: len(xq), :nprobe].cpu().numpy()
    ref, ref_d = O.coarse_probe(xq, b.centroids_idx, nprobe)
    assert np.array_equal(got, ref), f"nprobe={nprobe}"
    assert np.array_equal(got_d, np.sqrt(ref_d).astype(np.float32)), f"nprobe={nprobe}"


def test_coarse_probe_matches_oracle(gmm, dev):
    for nprobe in (1, 7, 16, 96):
        _check_probes(*gmm, dev, nprobe)


def test_band_front_end_derived_centroids(gmm, dev):
    """Without the index's centroid layouts (view fields cent_*) each search derives them into
    its workspace; the probes must be the oracle's either way."""
    b, xq = gmm
    keep = b.ix.cent_band
    try:
        b.ix.cent_band = None
        for nprobe in (7, 64):
            _check_probes(b, xq, dev, nprobe)
    finally:
        b.ix.cent_band = keep


@pytest.mark.parametrize("nlist", [2048, 4096, 5000])
def test_band_front_end_wide_nlist(dev, nlist):
    """The matrix-core band front end with 32 approximations per lane in registers (nlist 2048)
    and past 2048 centroids with each wave filtering its streamed row through an LDS list."""
    xb, xq = datagen.cfg4(N=3 * nlist, D=96, B=96, n_centers=nlist, seed=43)
    b = build_index(xb, nlist, dev, max_batch=128, max_nprobe=128)
    for nprobe in (1, 64, 100, 128):
        _check_probes(b, xq.numpy(), dev, nprobe)


def test_band_front_end_far_from_origin(dev):
    """Data offset far from the origin: the matrix-core approximation loses most of its digits
    to cancellation, the band widens to many (or all) centroids, and the selection must
    still be the float64 oracle's, ties included."""
    xb, xq = datagen.cfg1(N=20_000, D=128, B=100, n_centers=128, seed=44)
    b = build_index(xb + 3.0e4, 256, dev, max_batch=128, max_nprobe=128)
    xq = (xq + 3.0e4).numpy()
    dup = np.repeat(xq[:4], 2, axis=0)  # duplicated queries: identical rows
    xq = np.concatenate([xq, dup]).astype(np.float32)
    for nprobe in (5, 64, 128):
        _check_probes(b, xq, dev, nprobe)


@pytest.mark.parametrize("low", [0x8000 + 0x40, 0xFF00])
def test_band_front_end_split_adversarial(dev, low):
    """Every stored and query value's low 16 bits set just above a bfloat16 tie (the split's
    dropped terms all of one sign) or just below the next bfloat16 value: the coarse pass's
    bfloat16 split is at its largest error, and the band must still hold every probe."""
    def hostile(t):
        u = t.contiguous().view(torch.int32)
        return ((u & ~0xFFFF) | low).view(torch.float32)

    xb, xq = datagen.cfg1(N=20_000, D=128, B=100, n_centers=128, seed=47)
    b = build_index(hostile(xb), 256, dev, max_batch=128, max_nprobe=128)
    xq = hostile(xq).numpy()
    for nprobe in (5, 64, 128):
        _check_probes(b, xq, dev, nprobe)


@pytest.mark.parametrize("nlist,offset", [(4500, 3.0e3), (4500, 3.0e4), (8195, 0.0),
                                          (8195, 3.0e3), (8195, 3.0e4)])
def test_band_front_end_stream_wide_band(dev, nlist, offset):
    """Past 2048 centroids each wave filters its row through an LDS list tightened by
    bisection; from 8192 on it filters the row's 16-centroid tile minima first and reads only
    the listed tiles (8195: rows padded to 8196 floats, a last tile of three centroids).
    Offsets from the origin widen the error band: to a few hundred centroids (the band refined
    from the list 64 at a time; more than 512 listed tiles stream the whole row) and to nearly
    all of them (the list cannot shrink, the band is taken from the row again); the probes
    must still be the oracle's."""
    xb, xq = datagen.cfg1(N=3 * nlist, D=64, B=48, n_centers=nlist, seed=45)
    b = build_index(xb + offset, nlist, dev, max_batch=64, max_nprobe=128)
    xq = (xq + offset).numpy()
    dup = np.repeat(xq[:4], 2, axis=0)
    xq = np.concatenate([xq, dup]).astype(np.float32)
    for nprobe in (5, 64, 128):
        _check_probes(b, xq, dev, nprobe)


@pytest.mark.parametrize("nlist", [1, 2, 3, 5])
def test_band_front_end_tiny_nlist(dev, nlist):
    """A handful of centroids: the approximation rows are padded to 4 floats, more than the
    nlist doubles of the coarse-distance buffer they share below 3 centroids; every query must
    still get the oracle's probes (and no row may spill into the next query's)."""
    xb, xq = datagen.cfg1(N=2_000, D=40, B=300, n_centers=8, seed=49)
    b = build_index(xb, nlist, dev, max_batch=512, max_nprobe=8)
    for nprobe in sorted({1, nlist}):
        _check_probes(b, xq.numpy(), dev, nprobe)


def test_band_front_end_stream_wide_rows(dev):
    """Rows wider than 128 dims (the float32 coarse pass) past 2048 centroids: the streaming
    selector starts from the tile minima that pass writes; the probes must be the oracle's."""
    nlist = 2500
    xb, xq = datagen.cfg1(N=3 * nlist, D=200, B=48, n_centers=nlist, seed=48)
    b = build_index(xb, nlist, dev, max_batch=64, max_nprobe=128)
    for nprobe in (5, 64, 128):
        _check_probes(b, xq.numpy(), dev, nprobe)


@pytest.mark.parametrize("D", [12, 72, 100, 112])
def test_band_front_end_query_widths(dev, D):
    """The coarse pass runs one instantiation per 32-dim step count (Dq = 16, 80, 112: one,
    three and four steps): widths the other tests do not reach, zero-padded past D."""
    xb, xq = datagen.cfg1(N=6_000, D=D, B=80, n_centers=64, seed=46 + D)
    b = build_index(xb, 96, dev, max_batch=128, max_nprobe=128)
    for nprobe in (1, 16, 96):
        _check_probes(b, xq.numpy(), dev, nprobe)


def test_coarse_probe_selectors_all_widths(dev):
    """nprobe <= 64 and <= 128 use the one-wave register selector, larger ones the block radix
    select; all must give the oracle's (d, cid) order, including at the 64 / 128 edges."""
    xb, xq = datagen.cfg4(N=20_000, D=96, B=150, n_centers=256, seed=41)
    b = build_index(xb, 256, dev, max_batch=256, max_nprobe=256)
    xq = xq.numpy()
    for nprobe in (63, 64, 65, 128, 129, 200, 256):
        b.ix.search(_q(xq, dev), nprobe, mode=10, k=10)
        torch.cuda.synchronize()
        got = b.ix.probe_cids_buf[: len(xq), :nprobe].cpu().numpy()
        ref, _ = O.coarse_probe(xq, b.centroids_idx, nprobe)
        assert np.array_equal(got, ref), f"nprobe={nprobe}"


@pytest.mark.parametrize("mode", [10, 2])
def test_gmm_k10(gmm, dev, mode):
    b, xq = gmm
    _, rd, ri = oracle_search(b, xq, 16, 10)
    d, i = run_search(b, _q(xq, dev), 16, 10, mode=mode)
    assert_exact(d, i, rd, ri, f"gmm mode={mode}")


@pytest.mark.parametrize("ub", [0, 1, 2])
def test_hist_ub_seed(hist, dev, ub):
    b, xq = hist
    _, rd, ri = oracle_search(b, xq, 24, 10)
    d, i = run_search(b, _q(xq, dev), 24, 10, mode=2, ub=ub)
    assert_exact(d, i, rd, ri, f"hist ub={ub}")


@pytest.mark.parametrize("K", [1, 10, 50, 100, 128])
def test_k_sweep_norm96(norm96, dev, K):
    b, xq = norm96
    _, rd, ri = oracle_search(b, xq, 16, K)
    for mode in (2, 10):
        d, i = run_search(b, _q(xq, dev), 16, K, mode=mode, ub=1)
        assert_exact(d, i, rd, ri, f"norm96 K={K} mode={mode}")


@pytest.mark.parametrize("K", [10, 100])
def test_d960(aniso, dev, K):
    b, xq = aniso
    _, rd, ri = oracle_search(b, xq, 12, K)
    for mode, ub in ((2, 0), (2, 1), (10, 0)):
        d, i = run_search(b, _q(xq, dev), 12, K, mode=mode, ub=ub)
        assert_exact(d, i, rd, ri, f"d960 K={K} mode={mode} ub={ub}")


@pytest.mark.parametrize("nprobe", [1, 2, 3, 17, 128])
def test_pass_split_edges(hist, dev, nprobe):
    """nprobe 1 (single pass), 2 (pass 2 empty), 3 / 17 (p_init 2 / 3), all lists."""
    b, xq = hist
    _, rd, ri = oracle_search(b, xq[:50], nprobe, 10)
    d, i = run_search(b, _q(xq[:50], dev), nprobe, 10, mode=2, ub=1)
    assert_exact(d, i, rd, ri, f"nprobe={nprobe}")


def test_single_query(hist, dev):
    b, xq = hist
    for K in (1, 10, 20):
        _, rd, ri = oracle_search(b, xq[:1], 8, K)
        d, i = run_search(b, _q(xq[:1], dev), 8, K, mode=2)
        assert_exact(d, i, rd, ri, f"B=1 K={K}")


def test_ties_duplicates_and_short_lists(dev):
    """Integer data with duplicated rows (exact distance ties broken by id), a degenerate
    dimension, empty lists and lists shorter than K (missing slots = (+inf, -1))."""
    rng = np.random.default_rng(5)
    base = rng.integers(0, 4, size=(600, 40)).astype(np.float32)
    base[:, 7] = 3.0                                   # degenerate dimension
    xb = np.concatenate([base, base[:300], base[:100]], 0)
    nlist = 24
    cen = rng.integers(0, 4, size=(nlist, 40)).astype(np.float32)
    lid = np.argmin(((xb[:, None, :] - cen[None]) ** 2).sum(-1), 1).astype(np.int32)
    lid[lid == 5] = 6                                  # list 5 empty
    cen[9] = cen[2]                                    # duplicated centroid: coarse tie
    xq = np.concatenate([rng.integers(0, 4, size=(60, 40)), base[:20]], 0).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, list_ids=lid, centroids=cen, max_batch=128)
    for K, nprobe in ((10, 4), (64, 3), (128, 24)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        for mode, ub in ((2, 0), (2, 2), (10, 0)):
            d, i = run_search(b, _q(xq, dev), nprobe, K, mode=mode, ub=ub)
            assert_exact(d, i, rd, ri, f"ties K={K} nprobe={nprobe} mode={mode} ub={ub}")


@pytest.mark.parametrize("route", [1, 2])
def test_stats_counters(hist, dev, route):
    """candidates = sum over the probed pairs of the list sizes, each pair counted once on both
    routes (the batched route's seeding pass does not count: its lower-bound pass rescans
    every probe); survivors and insertions are bounded by it."""
    b, xq = hist
    nprobe = 24
    st = torch.zeros(4, dtype=torch.int64, device=dev)
    run_search(b, _q(xq, dev), nprobe, 10, mode=2, ub=1, stats=st, route=route)
    tot, dims, surv, ins = st.tolist()
    cids, _ = O.coarse_probe(xq, b.centroids_idx, nprobe)
    sizes = np.diff(b.vec_off)
    assert tot == int(sizes[cids].sum())
    assert 0 < surv <= tot and 0 < ins <= surv
    if route == 2:
        assert dims == tot * b.ix.D_pad   # the matrix-core bound always reads every dimension
    else:
        assert tot * 32 <= dims <= tot * b.ix.D_pad


def test_sq8_bounds_bracket_exact_distance(aniso, hist, dev):
    """lb <= d64 <= ub for every (query, candidate) of the probed lists (Stage Y / X rigour)."""
    for b, xq in (aniso, hist):
        xq = xq[:8]
        cids, _ = O.coarse_probe(xq, b.centroids_idx, 4)
        qids, pc, spos = [], [], []
        for q in range(len(xq)):
            for c in cids[q]:
                for s in range(b.vec_off[c], b.vec_off[c + 1]):
                    qids.append(q), pc.append(c), spos.append(s)
        qids = np.array(qids, np.int32)
        pc = np.array(pc, np.int32)
        spos = np.array(spos, np.int64)
        d64 = O.pair_dists(xq, b.xb_sorted, qids, spos)
        ix = b.ix
        view = ext.make_index_view(
            N=ix.N, D=ix.D, D_pad=ix.D_pad, nlist=ix.nlist, tile_size=ix.tile_size,
            per_cluster_sq8=ix.per_cluster_sq8, W_combined=ix.W_combined, b_combined=ix.b_combined,
            rot_sq_min=ix.rot_sq_min, rot_sq_max=ix.rot_sq_max, sq8_packed=ix.sq8_packed,
            tile_orig_ids=ix.tile_orig_ids, tile_r_minmax=ix.tile_r_minmax,
            cluster_tile_off=ix.cluster_tile_off, cluster_vec_off=ix.storage.cluster_vec_off,
            xb_sorted=ix.storage.xb_sorted, orig_ids_sorted=ix.storage.orig_ids_sorted,
            vmin=ix.vmin_pad, delta=ix.delta_pad, eps_dim=ix.eps_pad, blk_bounds4=ix.blk_bounds4)
        L = _lib.lib()
        nbytes = L.trident_workspace_bytes(ctypes.byref(view), len(xq), 1, 1)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        tq, tc, ts = (torch.as_tensor(a).to(dev) for a in (qids, pc, spos))
        lb = torch.empty(len(qids), dtype=torch.float64, device=dev)
        ub = torch.empty_like(lb)
        xqd = _q(xq, dev)
        rc = L.trident_sq8_bounds(ctypes.byref(view), ctypes.c_void_p(xqd.data_ptr()), len(xq),
                                  ctypes.c_void_p(tq.data_ptr()), ctypes.c_void_p(tc.data_ptr()),
                                  ctypes.c_void_p(ts.data_ptr()), len(qids), ctypes.c_void_p(ws.data_ptr()),
                                  ctypes.c_size_t(nbytes), ctypes.c_void_p(lb.data_ptr()),
                                  ctypes.c_void_p(ub.data_ptr()),
                                  ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        _lib.check(rc, "trident_sq8_bounds")
        torch.cuda.synchronize()
        lb, ub = lb.cpu().numpy(), ub.cpu().numpy()
        assert (lb <= d64).all(), f"lb > d64 by {(lb - d64).max()}"
        assert (ub >= d64).all(), f"ub < d64 by {(d64 - ub).max()}"
        # the bounds must also be useful: most of the distance is captured
        assert np.median(lb / d64) > 0.5 and np.median(ub / d64) < 2.0


def test_out_of_core_host_mapped_base(dev):
    """FP32 base in hipHostMalloc-mapped host memory; Stage Z reads survivors over PCIe."""
    xb, xq = datagen.cfg2(N=30_000, D=128, B=100, n_centers=64, seed=8)
    b = build_index(xb, 64, dev, xb_placement="host", max_batch=128)
    assert b.ix.storage.xb_sorted.device.type == "cpu"
    xq = xq.numpy()
    _, rd, ri = oracle_search(b, xq, 12, 10)
    for mode, ub in ((2, 0), (2, 1), (10, 0)):
        d, i = run_search(b, _q(xq, dev), 12, 10, mode=mode, ub=ub)
        assert_exact(d, i, rd, ri, f"ooc mode={mode} ub={ub}")
    b.ix.storage._host_buf.free()


def test_group_pairs_entry_point(dev):
    """trident_group_pairs: each pass holds exactly its (cluster, query) pairs, contiguous per
    cluster at seg_off (reference counting sort, src/trident_v4_kernels.cu:168-263)."""
    rng = np.random.default_rng(12)
    B, nprobe, nlist, p_init, ld = 300, 20, 50, 3, 24
    probes = np.stack([rng.choice(nlist, nprobe, replace=False) for _ in range(B)]).astype(np.int32)
    pc = torch.zeros((B, ld), dtype=torch.int32, device=dev)
    pc[:, :nprobe] = torch.as_tensor(probes).to(dev)
    p1c = torch.full((B * p_init,), -7, dtype=torch.int32, device=dev)
    p1q = torch.full_like(p1c, -7)
    p2c = torch.full((B * (nprobe - p_init),), -7, dtype=torch.int32, device=dev)
    p2q = torch.full_like(p2c, -7)
    seg = torch.zeros(2 * (nlist + 1), dtype=torch.int32, device=dev)
    cnt = torch.zeros_like(seg)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.lib().trident_group_pairs(P(pc), ld, B, nprobe, p_init, nlist, P(p1c), P(p1q), P(p2c), P(p2q),
                                        P(seg), P(cnt), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "trident_group_pairs")
    torch.cuda.synchronize()
    seg = seg.cpu().numpy().reshape(2, nlist + 1)
    for pas, (cc, qq, lo, hi) in enumerate(((p1c, p1q, 0, p_init), (p2c, p2q, p_init, nprobe))):
        cc, qq = cc.cpu().numpy(), qq.cpu().numpy()
        want = sorted((int(probes[q, p]), q) for q in range(B) for p in range(lo, hi))
        assert sorted(zip(cc.tolist(), qq.tolist())) == want
        assert np.all(np.diff(cc) >= 0), "pairs not grouped by cluster"
        for c in range(nlist):
            assert np.all(cc[seg[pas, c]:seg[pas, c + 1]] == c)


def test_router_calibration_and_routed_search(hist, dev):
    from trident_amd import router
    b, xq = hist
    W0, rows = router.calibrate_w0(b.ix, _q(xq, dev), 16, batches=(1, 8, 64), warmup=1, iters=2)
    assert len(rows) == 3 and all(r["ms_cm"] > 0 and r["ms_cascade"] > 0 for r in rows)
    r = router.CostRouter(b.ix, W0=router.work_measure(8, 16, b.ix.N, b.ix.nlist, b.ix.D))
    _, rd, ri = oracle_search(b, xq[:64], 16, 10)
    for B, want in ((4, 10), (64, 2)):
        d, i, _, mode = r.search(_q(xq[:B], dev), 16, k=10)
        torch.cuda.synchronize()
        assert mode == want
        assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd[:B], ri[:B], f"routed B={B}")
