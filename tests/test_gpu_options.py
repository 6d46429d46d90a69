"""GPU parity of the search options a reference driver can set, on both mode-2 routes:
TRIDENT_UB_SEED 0 / 1 / 2, the residual-norm tile band (use_l1), global SQ8 (per_cluster_sq8 = 0),
and the 41-argument call with reference arguments only (the batched route then derives its
per-vector scalars and code cells once per index).  Same bar as test_gpu_parity.py: ids
identical to the float64 oracle, float32 distances equal to its rounded distances."""
import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import assert_exact, build_index, oracle_search, run_search
from trident_amd import _lib, datagen, ext

pytestmark = pytest.mark.gpu


def _q(xq, dev):
    return torch.as_tensor(np.ascontiguousarray(xq, np.float32)).to(dev).contiguous()


@pytest.fixture(scope="module")
def opt_sets(dev):
    out = {}
    xb, xq = datagen.cfg2(N=50_000, D=128, B=400, n_centers=128, seed=51)
    out["hist"] = (build_index(xb, 128, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg1(N=30_000, D=96, B=300, n_centers=48, seed=52)
    out["gmm96"] = (build_index(xb, 96, dev, max_batch=512), xq.numpy())
    xb, xq = datagen.cfg3(N=8_000, D=300, B=96, n_centers=32, seed=53)
    out["wide300"] = (build_index(xb, 32, dev, max_batch=128), xq.numpy())
    return out


@pytest.mark.parametrize("route", [1, 2])
@pytest.mark.parametrize("ub", [0, 1, 2])
def test_ub_seed_schedules(opt_sets, dev, route, ub):
    """Every TRIDENT_UB_SEED schedule is exact on both routes (the batched route seeds from the
    first p_init probes for 0 and 1, from every probe for 2)."""
    for name in ("hist", "wide300"):
        b, xq = opt_sets[name]
        for K, nprobe in ((10, 12), (64, 5), (100, 3)):
            _, rd, ri = oracle_search(b, xq, nprobe, K)
            d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=ub, route=route)
            assert_exact(d, i, rd, ri, f"{name} ub={ub} route={route} K={K} nprobe={nprobe}")


@pytest.mark.parametrize("route", [1, 2])
def test_use_l1_band(opt_sets, dev, route):
    """The residual-norm tile band prunes whole tiles without changing any result."""
    for name in ("hist", "gmm96", "wide300"):
        b, xq = opt_sets[name]
        for K, nprobe in ((10, 16), (50, 6)):
            _, rd, ri = oracle_search(b, xq, nprobe, K)
            for ub in (0, 2):
                d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=ub, use_l1=1, route=route)
                assert_exact(d, i, rd, ri, f"use_l1 {name} route={route} K={K} ub={ub}")


@pytest.mark.parametrize("route", [1, 2])
def test_global_sq8(dev, route):
    """per_cluster_sq8 = 0: one vmin / delta / eps row for every cluster."""
    for gen, D, nl in ((datagen.cfg2, 128, 96), (datagen.cfg1, 200, 48)):
        xb, xq = gen(N=30_000, D=D, B=256, n_centers=64, seed=54)
        b = build_index(xb, nl, dev, per_cluster_sq8=0, max_batch=256)
        assert b.ix.vmin_pad.shape[0] == 1
        xq = xq.numpy()
        for K, nprobe in ((10, 16), (100, 8)):
            _, rd, ri = oracle_search(b, xq, nprobe, K)
            d, i = run_search(b, _q(xq, dev), nprobe, K, mode=2, ub=1, route=route)
            assert_exact(d, i, rd, ri, f"global SQ8 D={D} route={route} K={K}")


def test_reference_arguments_only_take_the_batched_route(opt_sets, dev):
    """launch_trident_v4_search with exactly the reference's 41 positional arguments (no vec_Ar,
    sq8_cells, cent_band, rot_sq_bounds): a large batch derives the batched layouts once and is
    exact; the derived per-vector scalars equal the builder's."""
    b, xq = opt_sets["hist"]
    ix, st = b.ix, b.ix.storage
    B, nprobe, K = len(xq), 32, 10
    assert B * nprobe >= 8 * ix.nlist
    ext._derived_cache.clear()
    xqd = _q(xq, dev)
    topk_d = torch.empty((B, K), dtype=torch.float32, device=dev)
    topk_i = torch.empty((B, K), dtype=torch.int64, device=dev)
    args = (2, ix.tile_size, 0, ix.per_cluster_sq8, 0, nprobe,
            xqd, ix.W_combined, ix.b_combined, ix.W_coarse_only, ix.b_coarse_only,
            ix.proj_buf, ix.cdists_buf, ix.probe_cids_buf, ix.probe_dqcs_buf,
            ix.p1_cids_buf, ix.p1_qids_buf, ix.p1_dqcs_buf, ix.p2_cids_buf, ix.p2_qids_buf, ix.p2_dqcs_buf,
            ix.sq8_packed, ix.tile_orig_ids, ix.tile_r_minmax, ix.cluster_tile_off, st.cluster_vec_off,
            st.xb_sorted, st.orig_ids_sorted, ix.vmin_pad, ix.delta_pad, ix.eps_pad, ix.blk_bounds4,
            topk_d, topk_i, ix.topm_buf_d, ix.topm_buf_i, ix.tau_sq_buf,
            ix.cand_buf_d, ix.cand_buf_i, ix.cand_cnt, False)
    assert len(args) == 41
    for _ in range(2):  # the second call reuses the derived layouts
        ext.launch_trident_v4_search(*args)
        torch.cuda.synchronize()
        assert len(ext._derived_cache) == 1
        _, rd, ri = oracle_search(b, xq, nprobe, K)
        assert_exact(topk_d.cpu().numpy(), topk_i.cpu().numpy(), rd, ri, "reference arguments only")
    vec_Ar, cells, band, vec_cn = next(iter(ext._derived_cache.values()))
    assert torch.equal(vec_Ar, ix.vec_Ar) and torch.equal(cells, ix.sq8_cells)
    assert torch.equal(vec_cn, ix.vec_cn)
    # with the derived layouts the library picks the batched route for this batch
    view = ext.make_index_view(
        N=ix.N, D=ix.D, D_pad=ix.D_pad, nlist=ix.nlist, tile_size=ix.tile_size,
        per_cluster_sq8=ix.per_cluster_sq8, W_combined=ix.W_combined, b_combined=ix.b_combined,
        rot_sq_min=ix.rot_sq_min, rot_sq_max=ix.rot_sq_max, sq8_packed=ix.sq8_packed,
        tile_orig_ids=ix.tile_orig_ids, tile_r_minmax=ix.tile_r_minmax,
        cluster_tile_off=ix.cluster_tile_off, cluster_vec_off=st.cluster_vec_off,
        xb_sorted=st.xb_sorted, orig_ids_sorted=st.orig_ids_sorted, vmin=ix.vmin_pad,
        delta=ix.delta_pad, eps_dim=ix.eps_pad, blk_bounds4=ix.blk_bounds4, vec_Ar=vec_Ar,
        sq8_cells=cells, cent_band=band)
    assert _lib.lib().trident_route_for(ctypes.byref(view), B, K, nprobe, 0) == _lib.ROUTE_BATCHED
