"""GPU parity of the code paths that only the large configurations reach, at sizes the float64
oracle checks in seconds.

* configs[4]'s shape: nlist = 16,384 with the FP32 base in mapped host memory and B * nprobe
  large enough for the batched route.  At that nlist the pair grouping's two (nlist + 1)
  counters no longer fit LDS (global-atomic count / scatter kernels), the band front end
  streams each lane's share of the approximations, and the unit tables hold 32k segments.
* a seeding pass of many 16-query units (B * p_init >> nlist, clusters over 7,168 vectors),
  which needs more work units than a 64-query-per-unit estimate provides;
* searches on two torch streams in flight at once, each with its own workspace;
* the FP32 IVF-Flat baseline against the exact result on float data, through the float64
  audit (exact ties and FP32 rounding only, no true miss).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_exact, build_index, oracle_search, run_search
from trident_amd import _lib, clustering, datagen, ext

pytestmark = pytest.mark.gpu


def _q(xq, dev):
    return torch.as_tensor(np.ascontiguousarray(xq, np.float32)).to(dev).contiguous()


def _lists(xb, nlist, dev, seed):
    """nlist distinct base rows as centroids, every row in the list of its nearest one."""
    g = torch.Generator().manual_seed(seed)
    cen = xb[torch.randperm(xb.shape[0], generator=g)[:nlist]].clone()
    lid = clustering.assign(xb.to(dev), cen.to(dev)).cpu()
    return cen.numpy(), lid.numpy().astype(np.int32)


@pytest.fixture(scope="module")
def ooc16k(dev):
    xb, xq = datagen.cfg2(N=300_000, D=128, B=1024, n_centers=1024, seed=41)
    cen, lid = _lists(xb, 16384, dev, 41)
    b = build_index(xb, 16384, dev, list_ids=lid, centroids=cen, xb_placement="host",
                    max_batch=1024, max_nprobe=128)
    yield b, xq.numpy()
    torch.cuda.synchronize()
    b.ix.storage._host_buf.free()


def test_cfg5_shape_nlist16384_host_mapped(ooc16k, dev):
    """configs[4]'s code path: nlist 16,384, nprobe 128, K 10, B 1,024, base over PCIe; the
    automatic route is the batched one, and both routes match the oracle."""
    b, xq = ooc16k
    assert b.ix.storage.xb_sorted.device.type == "cpu"
    assert 2 * (b.ix.nlist + 1) * 4 > 64 * 1024  # LDS counters do not fit: global-atomic grouping
    assert b.ix.route_for(len(xq), 128, 10, 0) == _lib.ROUTE_BATCHED
    cids, rd, ri = oracle_search(b, xq, 128, 10)
    xqd = _q(xq, dev)
    for route in (0, 1):
        d, i = run_search(b, xqd, 128, 10, mode=2, ub=1, route=route)
        assert_exact(d, i, rd, ri, f"nlist 16384 host-mapped route={route}")
        got = b.ix.probe_cids_buf[: len(xq), :128].cpu().numpy()
        assert np.array_equal(got, cids), f"probes route={route}"


def test_group_pairs_past_lds_counters(dev):
    """trident_group_pairs at nlist 12,000 (the global-atomic kernels): each pass holds exactly
    its pairs, contiguous per cluster at seg_off."""
    rng = np.random.default_rng(43)
    B, nprobe, nlist, p_init, ld = 96, 100, 12_000, 3, 100
    probes = np.stack([rng.choice(nlist, nprobe, replace=False) for _ in range(B)]).astype(np.int32)
    pc = torch.as_tensor(probes).to(dev)
    p1c = torch.full((B * p_init,), -7, dtype=torch.int32, device=dev)
    p1q = torch.full_like(p1c, -7)
    p2c = torch.full((B * (nprobe - p_init),), -7, dtype=torch.int32, device=dev)
    p2q = torch.full_like(p2c, -7)
    seg = torch.zeros(2 * (nlist + 1), dtype=torch.int32, device=dev)
    cnt = torch.zeros_like(seg)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = _lib.lib().trident_group_pairs(P(pc), ld, B, nprobe, p_init, nlist, P(p1c), P(p1q), P(p2c),
                                        P(p2q), P(seg), P(cnt),
                                        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "trident_group_pairs")
    torch.cuda.synchronize()
    seg = seg.cpu().numpy().reshape(2, nlist + 1)
    for pas, (cc, qq, lo, hi) in enumerate(((p1c, p1q, 0, p_init), (p2c, p2q, p_init, nprobe))):
        cc, qq = cc.cpu().numpy(), qq.cpu().numpy()
        want = sorted((int(probes[q, p]), q) for q in range(B) for p in range(lo, hi))
        assert sorted(zip(cc.tolist(), qq.tolist())) == want
        assert np.all(np.diff(cc) >= 0), "pairs not grouped by cluster"
        counts = np.bincount(probes[:, lo:hi].ravel(), minlength=nlist)
        assert np.array_equal(np.diff(seg[pas]), counts)


def _units(probes, sizes, p_init):
    """Work units of both batched passes (ceil(queries / 16) seeding units and ceil(queries /
    64) lower-bound units per cluster, times min(8, ceil(n / 1024)) vector slices)."""
    S = np.minimum(8, (sizes + 1023) // 1024)
    q1 = np.bincount(probes[:, :p_init].ravel(), minlength=len(sizes))
    q2 = np.bincount(probes[:, p_init:].ravel(), minlength=len(sizes))
    return int((((q1 + 15) // 16) * S).sum() + (((q2 + 63) // 64) * S).sum())


def test_batched_seeding_units_beyond_64_query_estimate(dev):
    """16 lists of 12,500 vectors (8 slices each), B = 4096, nprobe = 4 (p_init = 2): the
    seeding pass alone has ~16 * 32 * 8 = 4,096 units of <= 16 queries, more than a bound that
    assumes 64 queries per unit (2,304 for both passes).  Every unit must be scanned."""
    xb, xq = datagen.cfg2(N=200_000, D=64, B=4096, n_centers=16, seed=42)
    lid = (np.arange(200_000) % 16).astype(np.int32)          # equal lists, 12,500 rows each
    cen = np.stack([xb.numpy()[lid == c].mean(0) for c in range(16)]).astype(np.float32)
    b = build_index(xb, 16, dev, list_ids=lid, centroids=cen, max_batch=4096, max_nprobe=8)
    B, nprobe, nlist = 4096, 4, 16
    assert b.ix.route_for(B, nprobe, 10, 0) == _lib.ROUTE_BATCHED
    cids, rd, ri = oracle_search(b, xq.numpy(), nprobe, 10)
    units = _units(cids, np.diff(b.vec_off), 2)
    assert units > 8 * (B * nprobe // 64 + 2 * nlist), units
    assert units <= 8 * ((B * nprobe + 15) // 16 + 2 * nlist), units
    d, i = run_search(b, _q(xq.numpy(), dev), nprobe, 10, mode=2, ub=1, route=0)
    assert_exact(d, i, rd, ri, "seeding units past the 64-query estimate")


def test_two_streams_in_flight(dev):
    """Two searches of different shapes enqueued on two streams with no synchronisation between
    them, three times over: each stream has its own workspace, so both match the oracle."""
    xb, xq = datagen.cfg2(N=60_000, D=128, B=600, n_centers=128, seed=44)
    b = build_index(xb, 128, dev, max_batch=600)
    ix, st = b.ix, b.ix.storage
    view = ext.make_index_view(
        N=ix.N, D=ix.D, D_pad=ix.D_pad, nlist=ix.nlist, tile_size=ix.tile_size,
        per_cluster_sq8=ix.per_cluster_sq8, W_combined=ix.W_combined, b_combined=ix.b_combined,
        rot_sq_min=ix.rot_sq_min, rot_sq_max=ix.rot_sq_max, sq8_packed=ix.sq8_packed,
        tile_orig_ids=ix.tile_orig_ids, tile_r_minmax=ix.tile_r_minmax,
        cluster_tile_off=ix.cluster_tile_off, cluster_vec_off=st.cluster_vec_off,
        xb_sorted=st.xb_sorted, orig_ids_sorted=st.orig_ids_sorted, vmin=ix.vmin_pad,
        delta=ix.delta_pad, eps_dim=ix.eps_pad, blk_bounds4=ix.blk_bounds4, vec_Ar=ix.vec_Ar,
        sq8_cells=ix.sq8_cells, cent_band=ix.cent_band)
    xq = xq.numpy()
    jobs = [(xq[:400], 32, 10, 2), (xq[400:], 16, 64, 1)]   # (queries, nprobe, K, route)
    refs = [oracle_search(b, q, npb, K)[1:] for q, npb, K, _ in jobs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    xqs = [_q(q, dev) for q, *_ in jobs]
    torch.cuda.synchronize()
    for rep in range(3):
        outs = []
        for (q, npb, K, route), s, xqd in zip(jobs, streams, xqs):
            td = torch.empty((len(q), K), dtype=torch.float32, device=dev)
            ti = torch.empty((len(q), K), dtype=torch.int64, device=dev)
            s.wait_stream(torch.cuda.current_stream())
            ext.search_view(view, xqd, npb, td, ti, ub_seed=1, route=route, stream=s)
            outs.append((td, ti))
        torch.cuda.synchronize()
        for (td, ti), (rd, ri), (_, npb, K, route) in zip(outs, refs, jobs):
            assert_exact(td.cpu().numpy(), ti.cpu().numpy(), rd, ri,
                         f"stream rep={rep} nprobe={npb} K={K} route={route}")


@pytest.fixture(scope="module")
def float_sets(dev):
    out = {}
    xb, xq = datagen.cfg1(N=40_000, D=128, B=300, n_centers=64, seed=45)
    out["gmm"] = (build_index(xb, 100, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg4(N=50_000, D=96, B=300, n_centers=256, seed=46)
    out["norm96"] = (build_index(xb, 200, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg3(N=12_000, D=960, B=100, n_centers=64, seed=47)
    out["d960"] = (build_index(xb, 64, dev, max_batch=128), xq.numpy())
    return out


@pytest.mark.parametrize("name", ["gmm", "norm96", "d960"])
@pytest.mark.parametrize("K", [10, 100])
def test_fp32_ivfflat_identity_by_audit(float_sets, dev, name, K):
    """On float data the exact (float64) top-K and the reference's FP32 IVF-Flat
    (omp_cpu_ivfflat_f32) may differ only where FP32 rounding reorders near-equal distances:
    the float64 audit finds no true miss, and every differing slot is within 1e-5 relative."""
    b, xq = float_sets[name]
    nprobe = 16
    cids, rd, ri = oracle_search(b, xq, nprobe, K)
    d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=0)
    assert_exact(d, i, rd, ri, f"{name} K={K}")
    fd, fi = O.ivfflat_f32(xq, cids, b.vec_off, b.xb_sorted, b.orig_ids, K)
    a = O.audit(fi, i, b.xb, xq)
    assert a["true_miss"] == 0, a
    assert a["max_rel"] <= 1e-5, a
    # where the ids agree the FP32 distances are within 1e-5 of the exact ones
    same = fi == i
    fin = same & np.isfinite(rd)
    np.testing.assert_allclose(fd[fin].astype(np.float64), rd[fin], rtol=1e-5)


def test_configs0_at_its_stated_size(dev):
    """BASELINE.json configs[0] exactly as stated: N = 100,000, D = 128, a 256-component
    isotropic Gaussian mixture (centres U[0, 100], sigma 8), k-means nlist = 256, nprobe = 16,
    K = 10, B = 1,000 queries from the same mixture, seed 0 -- generated and clustered on the
    GPU as the bench does.  Every query is checked against the float64 oracle on both mode-2
    routes, the auto route and mode 10."""
    from trident_amd.index import SharedClusterStorage, TridentV4Index
    N, D, nlist, nprobe, K, B = 100_000, 128, 256, 16, 10, 1_000
    xb, xq = datagen.generate(1, device=dev, seed=0, N=N, D=D, B=B, n_centers=256)
    cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, nlist, seed=0, niter=20, device=dev)
    st = SharedClusterStorage(xb, lid, r, nlist, device=dev)
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=64, device=dev, max_batch=B, max_nprobe=128, k=K)
    h = ix.host_arrays()
    xq_np = xq.cpu().numpy()
    cids, _ = O.coarse_probe(xq_np, h["centroids"], nprobe)
    rd, ri = O.ivf_exact(xq_np, cids, h["vec_off"], h["xb_sorted"], h["orig_ids_sorted"], K)
    assert ix.route_for(B, nprobe, K) == _lib.ROUTE_BATCHED
    for mode, route, ub in ((2, 0, 1), (2, 1, 1), (2, 2, 0), (2, 2, 2), (10, 0, 0)):
        d, i, _ = ix.search(xq.contiguous(), nprobe, mode=mode, k=K, ub_seed=ub, route=route)
        torch.cuda.synchronize()
        probes = ix.probe_cids_buf[:B, :nprobe].cpu().numpy()
        assert np.array_equal(probes, cids), f"configs[0] probes mode={mode} route={route}"
        assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri, f"configs[0] mode={mode} route={route} ub={ub}")
