"""GPU parity of the reference's comparison modes through trident_search:

* mode 11 (Tribase): exact, so the bar of test_gpu_parity.py (ids identical to the float64
  oracle, distances equal to its float32 rounding), and the triangle skip must actually skip;
* modes 1 (K1) and 0 (K0 / CM-SQ8+RR): bit-identical ids and distances to the CPU restatement
  oracle.ivf_sq8 (acc_hat in dimension order with fmaf, per-pair list lengths and the two-pass
  split of the reference, exact float64 rerank).  Parity with the reference's own outputs is
  unpinned: its acc_hat starts from a float32 cuBLAS projection whose rounding is not published.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_exact, build_index, oracle_search, oracle_sq8, sq8_arrays
from trident_amd import datagen, ext

pytestmark = pytest.mark.gpu


def _q(xq, dev):
    return torch.as_tensor(np.ascontiguousarray(xq, np.float32)).to(dev).contiguous()


@pytest.fixture(scope="module")
def mode_sets(dev):
    out = {}
    xb, xq = datagen.cfg2(N=40_000, D=128, B=300, n_centers=128, seed=61)
    out["hist"] = build_index(xb, 128, dev, max_batch=512), xq.numpy()
    xb, xq = datagen.cfg1(N=20_000, D=96, B=200, n_centers=48, seed=62)
    out["gmm96"] = build_index(xb, 48, dev, max_batch=512, tile_size=64), xq.numpy()
    xb, xq = datagen.cfg3(N=6_000, D=300, B=64, n_centers=32, seed=63)
    out["wide300"] = build_index(xb, 24, dev, max_batch=128), xq.numpy()
    xb, xq = datagen.cfg2(N=20_000, D=64, B=128, n_centers=64, seed=64)
    out["global_host"] = build_index(xb, 40, dev, max_batch=256, per_cluster_sq8=0, xb_placement="host"), xq.numpy()
    # well-separated clusters in 32 dims: probes beyond the nearest lie far outside tau, so the
    # triangle skip must remove whole lists
    g = torch.Generator().manual_seed(65)
    cen = torch.randn(48, 32, generator=g) * 6.0
    lbl = torch.randint(0, 48, (24_000,), generator=g)
    xb = cen[lbl] + torch.randn(24_000, 32, generator=g)
    xq = cen[torch.randint(0, 48, (128,), generator=g)] + torch.randn(128, 32, generator=g)
    out["separated"] = build_index(xb, 48, dev, max_batch=256), xq.numpy()
    return out


def _search(b, xq, dev, nprobe, K, mode, rerank_m=0, stats=None):
    d, i, _ = b.ix.search(_q(xq, dev), nprobe, mode=mode, rerank_m=rerank_m, k=K, stats_buf=stats)
    torch.cuda.synchronize()
    return d.cpu().numpy().copy(), i.cpu().numpy().copy()


def _same(gd, gi, rd, ri, ctx):
    bad = np.nonzero((gi != ri).any(axis=1))[0]
    assert len(bad) == 0, f"{ctx}: {len(bad)} queries differ; q={bad[0]} gpu={gi[bad[0]].tolist()} ref={ri[bad[0]].tolist()}"
    assert np.array_equal(gd.view(np.uint32), rd.view(np.uint32)), f"{ctx}: distances differ"


@pytest.mark.parametrize("name", ["hist", "gmm96", "wide300", "global_host", "separated"])
def test_tribase_is_exact_and_skips(mode_sets, dev, name):
    """Exact on every set; on the separated set the skip must remove vectors (in 96+ dims the
    residual norms concentrate and the triangle bound rarely bites, as for the reference)."""
    b, xq = mode_sets[name]
    for K, nprobe in ((10, 8), (64, 4), (128, 3), (1, 20)):
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        stats = torch.zeros(4, dtype=torch.int64, device=dev)
        d, i = _search(b, xq, dev, nprobe, K, 11, stats=stats)
        assert_exact(d, i, rd, ri, f"mode 11 {name} K={K} nprobe={nprobe}")
        cand, dims, surv, _ = stats.cpu().tolist()
        probes = O.coarse_probe(xq, b.centroids_idx, nprobe)[0].ravel()
        assert cand == sum(int(b.vec_off[c + 1] - b.vec_off[c]) for c in probes)
        assert surv <= cand
        if name == "separated" and K <= 64 and nprobe >= 4:
            assert surv < 0.8 * cand, f"{name}: the triangle skip removed little ({surv} of {cand})"


@pytest.mark.parametrize("name", ["hist", "gmm96", "wide300", "global_host"])
def test_mode1_sq8_hat(mode_sets, dev, name):
    b, xq = mode_sets[name]
    arr = sq8_arrays(b)
    for K, nprobe in ((10, 8), (1, 1), (64, 5), (100, 17), (128, 2)):
        rd, ri = oracle_sq8(b, xq, nprobe, K, 1, arrays=arr)
        d, i = _search(b, xq, dev, nprobe, K, 1)
        _same(d, i, rd, ri, f"mode 1 {name} K={K} nprobe={nprobe}")


@pytest.mark.parametrize("name", ["hist", "gmm96", "wide300", "global_host"])
def test_mode0_rerank(mode_sets, dev, name):
    b, xq = mode_sets[name]
    arr = sq8_arrays(b)
    for K, nprobe, rr in ((10, 8, 20), (10, 32, 100), (10, 3, 50), (10, 1, 200), (50, 16, 200),
                          (128, 6, 150), (10, 12, 0), (100, 4, 0), (20, 2, 300)):
        nprobe = min(nprobe, b.ix.nlist)
        rd, ri = oracle_sq8(b, xq, nprobe, K, 0, rerank_m=rr, arrays=arr)
        d, i = _search(b, xq, dev, nprobe, K, 0, rerank_m=rr)
        _same(d, i, rd, ri, f"mode 0 {name} K={K} nprobe={nprobe} rerank_m={rr}")


def test_single_query_split(mode_sets, dev):
    """B = 1 takes the reference's single-query splits (mode 0 without rerank: one pass)."""
    b, xq = mode_sets["hist"]
    arr = sq8_arrays(b)
    for mode, rr in ((0, 0), (0, 40), (1, 0)):
        for qi in range(3):
            rd, ri = oracle_sq8(b, xq[qi:qi + 1], 9, 10, mode, rerank_m=rr, arrays=arr)
            d, i = _search(b, xq[qi:qi + 1], dev, 9, 10, mode, rerank_m=rr)
            _same(d, i, rd, ri, f"B=1 mode {mode} rerank_m={rr}")


def test_reference_call_mode11_derives_r_vec(mode_sets, dev):
    """The reference's 41-argument call for mode 11 carries no r_vec_sorted: it is derived once
    and agrees with the builder's (both round a float64 norm; the sums may differ in order)."""
    b, xq = mode_sets["gmm96"]
    ix, st = b.ix, b.ix.storage
    B, nprobe, K = len(xq), 6, 10
    ext._derived_cache.clear()
    topk_d = torch.empty((B, K), dtype=torch.float32, device=dev)
    topk_i = torch.empty((B, K), dtype=torch.int64, device=dev)
    args = (11, ix.tile_size, 0, ix.per_cluster_sq8, 0, nprobe,
            _q(xq, dev), ix.W_combined, ix.b_combined, ix.W_coarse_only, ix.b_coarse_only,
            ix.proj_buf, ix.cdists_buf, ix.probe_cids_buf, ix.probe_dqcs_buf,
            ix.p1_cids_buf, ix.p1_qids_buf, ix.p1_dqcs_buf, ix.p2_cids_buf, ix.p2_qids_buf, ix.p2_dqcs_buf,
            ix.sq8_packed, ix.tile_orig_ids, ix.tile_r_minmax, ix.cluster_tile_off, st.cluster_vec_off,
            st.xb_sorted, st.orig_ids_sorted, ix.vmin_pad, ix.delta_pad, ix.eps_pad, ix.blk_bounds4,
            topk_d, topk_i, ix.topm_buf_d, ix.topm_buf_i, ix.tau_sq_buf,
            ix.cand_buf_d, ix.cand_buf_i, ix.cand_cnt, False)
    assert len(args) == 41
    ext.launch_trident_v4_search(*args)
    torch.cuda.synchronize()
    _, rd, ri = oracle_search(b, xq, nprobe, K)
    assert_exact(topk_d.cpu().numpy(), topk_i.cpu().numpy(), rd, ri, "mode 11 reference call")
    derived = [v for k, v in ext._derived_cache.items() if k[0] == "r_vec"]
    assert len(derived) == 1
    rel = ((derived[0].double() - ix.r_vec_sorted.double()).abs() / ix.r_vec_sorted.double().clamp_min(1e-30)).max()
    assert float(rel) <= 2 ** -23
