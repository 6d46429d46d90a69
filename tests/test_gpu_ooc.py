"""Out-of-core search with the second SQ level (residual codes): the bounds it takes from HBM
bracket the canonical float64 distance and are tight, and searches that use them stay exact
while refining fewer rows over PCIe than without them."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_exact, build_index, oracle_search, run_search
from trident_amd import _lib, datagen

pytestmark = pytest.mark.gpu


def _q(xq, dev):
    return torch.as_tensor(np.ascontiguousarray(xq, np.float32)).to(dev).contiguous()


@pytest.fixture(scope="module")
def host_sets(dev):
    out = {}
    xb, xq = datagen.cfg2(N=40_000, D=128, B=600, n_centers=64, seed=91)
    out["hist"] = build_index(xb, 64, dev, xb_placement="host", max_batch=1024), xq.numpy()
    xb, xq = datagen.cfg3(N=8_000, D=300, B=200, n_centers=32, seed=92)
    out["wide300"] = build_index(xb, 24, dev, xb_placement="host", max_batch=256), xq.numpy()
    xb, xq = datagen.cfg1(N=20_000, D=72, B=400, n_centers=32, seed=93)
    out["gmm72"] = build_index(xb, 40, dev, xb_placement="host", max_batch=512, per_cluster_sq8=0), xq.numpy()
    yield out
    torch.cuda.synchronize()
    for b, _ in out.values():
        b.ix.storage._host_buf.free()


@pytest.mark.parametrize("name", ["hist", "wide300", "gmm72"])
def test_fine_bounds_bracket_exact_distance(host_sets, dev, name):
    b, xq = host_sets[name]
    ix = b.ix
    assert ix.fine_codes is not None and ix.fine_qp is not None
    xq = xq[:6]
    cids, _ = O.coarse_probe(xq, b.centroids_idx, 4)
    qids, spos = [], []
    for q in range(len(xq)):
        for c in cids[q]:
            for s in range(b.vec_off[c], b.vec_off[c + 1]):
                qids.append(q), spos.append(s)
    qids = np.array(qids, np.int32)
    spos = np.array(spos, np.int64)
    d64 = O.pair_dists(xq, b.xb_sorted, qids, spos)
    view = ix.view()
    L = _lib.lib()
    nbytes = L.trident_workspace_bytes(ctypes.byref(view), len(xq), 1, 1)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    tq, ts = (torch.as_tensor(a).to(dev) for a in (qids, spos))
    lb = torch.empty(len(qids), dtype=torch.float64, device=dev)
    ub = torch.empty_like(lb)
    xqd = _q(xq, dev)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    rc = L.trident_fine_bounds(ctypes.byref(view), P(xqd), len(xq), P(tq), P(ts), len(qids), P(ws),
                              ctypes.c_size_t(nbytes), P(lb), P(ub),
                              ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "trident_fine_bounds")
    torch.cuda.synchronize()
    lb, ub = lb.cpu().numpy(), ub.cpu().numpy()
    assert (lb <= d64).all(), f"lb > d64 by {(lb - d64).max()}"
    assert (ub >= d64).all(), f"ub < d64 by {(d64 - ub).max()}"
    # a second SQ level: the bracket is a small fraction of the distance
    assert np.median((ub - lb) / d64) < 2e-2, np.median((ub - lb) / d64)


@pytest.mark.parametrize("name", ["hist", "wide300", "gmm72"])
def test_fine_mode_is_exact_and_refines_fewer_rows(host_sets, dev, name):
    b, xq = host_sets[name]
    ix = b.ix
    xqd = _q(xq, dev)
    for K, nprobe, ub in ((10, 16, 1), (1, 8, 1), (100, 6, 2), (10, 24, 0)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        kept, rows = {}, {}
        for res in (True, False):
            codes, rho = ix.fine_codes, ix.fine_qp
            if not res:
                ix.fine_codes = ix.fine_qp = None
            try:
                st = torch.zeros(4, dtype=torch.int64, device=dev)
                hr = torch.full((1,), -1, dtype=torch.int64, device=dev)
                d, i, _ = ix.search(xqd, nprobe, mode=2, k=K, ub_seed=ub, route=2, stats_buf=st,
                                    host_rows_buf=hr)
                torch.cuda.synchronize()
                assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri,
                             f"{name} res={res} K={K} nprobe={nprobe} ub={ub}")
                kept[res], rows[res] = int(st[3]), int(hr[0])
            finally:
                ix.fine_codes, ix.fine_qp = codes, rho
        # rows refined exactly and kept (d64 <= tau) were read; the residual filter reads fewer
        assert rows[True] >= kept[True] and rows[False] >= kept[False], (rows, kept)
        assert kept[True] <= kept[False] and rows[True] < rows[False], (rows, kept)


def test_uint8_copy_of_the_host_base(dev):
    """A host base of integers in [0, 255] (D a multiple of 16) gets an exact uint8 copy that
    the exact refines (seeds, Stage Z; batched route and mode 10) read instead of its float32
    rows: results equal the oracle's and the same index's without the copy, from the same host
    rows (128 instead of 512 bytes each).  Non-integer values, values past 255 and D not a
    multiple of 16 get no copy."""
    xb, xq = datagen.cfg2(N=30_000, D=128, B=500, n_centers=48, seed=95)
    b = build_index(xb, 48, dev, xb_placement="host", max_batch=512)
    st = b.ix.storage
    try:
        assert st.xb_sorted_u8 is not None
        assert torch.equal(st.xb_sorted_u8.to(torch.float32), st.xb_sorted)
        q = _q(xq.numpy(), dev)
        for K, nprobe, mode in ((10, 16, 2), (64, 8, 2), (10, 16, 10)):
            _, rd, ri = oracle_search(b, xq.numpy(), nprobe, K)
            rows = {}
            for u8 in (True, False):
                saved = st.xb_sorted_u8
                if not u8:
                    st.xb_sorted_u8 = None
                hr = torch.zeros(2, dtype=torch.int64, device=dev)
                d, i, _ = b.ix.search(q, nprobe, mode=mode, k=K, route=2, host_rows_buf=hr)
                torch.cuda.synchronize()
                st.xb_sorted_u8 = saved
                assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri, f"u8={u8} K={K} mode={mode}")
                rows[u8] = int(hr[0])
            assert rows[True] == rows[False] > 0, rows
    finally:
        st._host_buf.free()
    assert st.xb_sorted_u8 is None and st.xb_sorted is None
    for xb2 in (datagen.cfg1(N=3000, D=128, B=8, n_centers=8, seed=96)[0],   # not integers
                datagen.cfg2(N=3000, D=128, B=8, n_centers=8, seed=97)[0] * 2,  # past 255
                datagen.cfg2(N=3000, D=72, B=8, n_centers=8, seed=98)[0]):      # D % 16 != 0
        b2 = build_index(xb2, 8, dev, xb_placement="host", max_batch=8)
        assert b2.ix.storage.xb_sorted_u8 is None
        b2.ix.storage._host_buf.free()


def test_host_rows_is_zero_for_a_device_base(dev):
    xb, xq = datagen.cfg2(N=20_000, D=64, B=200, n_centers=32, seed=94)
    b = build_index(xb, 32, dev, max_batch=256)
    hr = torch.full((1,), -1, dtype=torch.int64, device=dev)
    b.ix.search(_q(xq.numpy(), dev), 8, mode=2, k=10, route=2, host_rows_buf=hr)
    torch.cuda.synchronize()
    assert int(hr[0]) == 0


def test_fine_tau_long_candidate_lists(dev):
    """Rows nearly equidistant from every query: the lower bounds let almost every probed row
    through, so the candidate lists run past 256 slots (the fine threshold's per-lane top-16
    path for K <= 16, its sorted list for K = 20) while staying within their capacity."""
    rng = np.random.default_rng(97)
    D, N, nlist = 32, 1800, 16
    u = rng.standard_normal((N, D))
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    xb = (100.0 * u * (1.0 + 1e-3 * rng.standard_normal((N, 1)))).astype(np.float32)
    xq = (0.01 * rng.standard_normal((8, D))).astype(np.float32)
    b = build_index(torch.as_tensor(xb), nlist, dev, xb_placement="host", max_batch=64)
    try:
        assert b.ix.fine_codes is not None
        for K in (1, 10, 16, 20):
            _, rd, ri = oracle_search(b, xq, nlist, K)
            st = torch.zeros(4, dtype=torch.int64, device=dev)
            d, i, _ = b.ix.search(_q(xq, dev), nlist, mode=2, k=K, ub_seed=1, stats_buf=st, route=2)
            torch.cuda.synchronize()
            assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri, f"long lists K={K}")
            assert int(st[2]) > 256 * len(xq), int(st[2])  # survivors: lists past 256 slots
    finally:
        torch.cuda.synchronize()
        b.ix.storage._host_buf.free()


@pytest.mark.parametrize("placement", ["device", "host"])
def test_stage_z_rows_not_multiple_of_four(dev, placement):
    """D = 50: rows are not 16-byte aligned, so Stage Z stages them with 4-byte loads (each lane
    dims kk + 32 m of its rows) instead of float4 runs; both routes, base in device and mapped
    host memory, against the oracle."""
    xb, xq = datagen.cfg1(N=8_000, D=50, B=96, n_centers=32, seed=71)
    b = build_index(xb, 32, dev, xb_placement=placement, max_batch=128)
    try:
        for route in (1, 2):
            for nprobe, K in ((4, 10), (12, 1)):
                _, rd, ri = oracle_search(b, xq.numpy(), nprobe, K)
                d, i = run_search(b, _q(xq.numpy(), dev), nprobe, K, mode=2, route=route)
                assert_exact(d, i, rd, ri, f"D=50 {placement} route={route} nprobe={nprobe} K={K}")
    finally:
        if placement == "host":
            torch.cuda.synchronize()
            b.ix.storage._host_buf.free()


def test_sq8_cells_only_on_the_device(dev):
    """The out-of-core configuration as the reference runs it: the base in mapped host memory,
    the fine level dropped and the reference packing released, so the device holds the SQ8
    codes once (the batched route's cells) plus ids and per-vector scalars.  Mode 2 takes the
    batched route by itself (also where AUTO would choose the per-pair route), stays exact at
    every ub_seed, reads survivors over PCIe, and refuses the per-pair route and modes 0 / 1."""
    xb, xq = datagen.cfg2(N=30_000, D=128, B=300, n_centers=48, seed=95)
    b = build_index(xb, 48, dev, xb_placement="host", max_batch=512)
    ix = b.ix
    try:
        fp0 = ix.hbm_footprint()
        ix.release_fine_level()
        ix.release_packed_codes()
        fp1 = ix.hbm_footprint()
        assert "fine_codes" in fp0 and "sq8_packed" in fp0
        assert "fine_codes" not in fp1 and "sq8_packed" not in fp1 and "xb_sorted" not in fp1
        assert fp1["sq8_cells"] == ix.sq8_cells.numel() * 4 and fp1["total"] < fp0["total"]
        xqd = _q(xq.numpy(), dev)
        for K, nprobe, ub, B in ((10, 12, 0, 300), (10, 12, 1, 300), (10, 12, 2, 300), (5, 4, 1, 3)):
            _, rd, ri = oracle_search(b, xq.numpy()[:B], nprobe, K)
            assert ix.route_for(B, nprobe, K) == _lib.ROUTE_BATCHED
            hr = torch.zeros(1, dtype=torch.int64, device=dev)
            d, i, _ = ix.search(xqd[:B], nprobe, mode=2, k=K, ub_seed=ub, host_rows_buf=hr)
            torch.cuda.synchronize()
            assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri, f"cells only K={K} ub={ub} B={B}")
            assert int(hr[0]) >= K * B  # survivors cross PCIe: no fine level
        for kw in (dict(mode=2, route=1), dict(mode=1), dict(mode=0, rerank_m=20)):
            with pytest.raises((ValueError, RuntimeError)):
                ix.search(xqd, 8, k=10, **kw)
    finally:
        torch.cuda.synchronize()
        ix.storage._host_buf.free()


@pytest.mark.parametrize("placement", ["host", "device"])
def test_overflowed_lists_are_rescanned_through_bounds(dev, placement):
    """A candidate list that overflows its capacity is rescanned through the SQ8 bounds, not
    exhaustively: the K-th smallest upper bound over the query's probed rows caps the threshold
    and only rows whose lower bound passes it are read from host memory.  Explicit lists, nlist
    8,192, base in mapped host memory: the three nearest clusters (the seeding probes) hold only
    far rows, so the seeded threshold is loose and a dense shell of rows at distance 3 in the
    other probed clusters overflows every list; the 10 true neighbours sit at distance 1.  The
    result equals the oracle's, and each query reads fewer than 2 K nprobe rows (the exhaustive
    rescan would read all 3,470 probed rows)."""
    rng = np.random.default_rng(123)
    D, nlist, nprobe, K, B = 16, 8192, 20, 10, 4

    def sphere(n, radius, jitter=0.0):
        u = rng.standard_normal((n, D))
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        return radius * u * (1.0 + jitter * rng.standard_normal((n, 1)))

    rows, lids = [], []
    for c in range(3):                        # seeding probes: far rows only
        rows.append(sphere(20, 10.0, 1e-2)); lids += [c] * 20
    for c in range(3, nprobe):                # the shell: 17 x 200 rows at distance ~3
        rows.append(sphere(200, 3.0, 1e-3)); lids += [c] * 200
    rows.append(sphere(K, 1.0, 1e-2)); lids += [3] * K   # the true neighbours
    far = nlist - nprobe                      # one distant row in every other cluster
    rows.append(sphere(far, 1000.0, 1e-2)); lids += list(range(nprobe, nlist))
    xb = torch.as_tensor(np.concatenate(rows).astype(np.float32))
    cen = np.zeros((nlist, D), np.float32)
    for c in range(nprobe):
        cen[c, c % D] = 0.05 + 0.01 * c       # probe order: clusters 0, 1, 2, then the rest
    cen[nprobe:] = sphere(far, 1000.0).astype(np.float32)
    xq = np.zeros((B, D), np.float32)
    xq[:, 0] = 0.001 * np.arange(B)
    b = build_index(xb, nlist, dev, xb_placement=placement, list_ids=np.asarray(lids, np.int32),
                    centroids=cen, max_batch=64, max_nprobe=128)
    try:
        cids, rd, ri = oracle_search(b, xq, nprobe, K)
        assert (np.sort(cids[:, :3], 1) == [0, 1, 2]).all()
        st = torch.zeros(4, dtype=torch.int64, device=dev)
        hr = torch.zeros(2, dtype=torch.int64, device=dev)
        d, i, _ = b.ix.search(_q(xq, dev), nprobe, mode=2, k=K, ub_seed=1, route=2, stats_buf=st,
                              host_rows_buf=hr)
        torch.cuda.synchronize()
        assert_exact(d.cpu().numpy(), i.cpu().numpy(), rd, ri, f"overflowed lists ({placement})")
        cap = nprobe * max(K, 64) * (2 if placement == "host" else 1)  # a fine level doubles them
        assert int(st[2]) > B * cap, (int(st[2]), B * cap)  # every list overflowed
        if placement == "host":
            stage_z = int(hr[0]) - int(hr[1])
            assert stage_z < 2 * K * nprobe * B, (int(hr[0]), int(hr[1]))
    finally:
        torch.cuda.synchronize()
        if b.ix.storage._host_buf is not None:
            b.ix.storage._host_buf.free()
