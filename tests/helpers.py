"""Shared test helpers: build small indexes and compare searches with the CPU oracle."""
import numpy as np
import torch

from oracle import oracle as O
from trident_amd import clustering, datagen
from trident_amd.index import SharedClusterStorage, TridentV4Index, choose_tile


class Built:
    pass


def build_index(xb, nlist, device, tile_size=None, seed=0, niter=6, per_cluster_sq8=1, var_block=0,
                max_batch=1024, max_nprobe=128, k=10, xb_placement="device", list_ids=None,
                centroids=None, use_pca=1, within="auto"):
    """Cluster (unless lists are given) and build a TridentV4Index on ``device``."""
    xb = xb.float().contiguous()
    if list_ids is None:
        cen, lid, r, mean64, R64, _ = clustering.train_clustering(xb, nlist, seed=seed, niter=niter)
    else:
        cen = np.asarray(centroids, np.float32)
        lid = np.asarray(list_ids, np.int32)
        r = clustering.residual_norms(xb, torch.as_tensor(cen), torch.as_tensor(lid, dtype=torch.int64)).numpy()
        mean64, R64 = clustering.residual_pca(xb, torch.as_tensor(cen), torch.as_tensor(lid, dtype=torch.int64))
    st = SharedClusterStorage(xb.cpu().numpy(), lid, r, nlist, device=device, xb_placement=xb_placement,
                              within=within)
    T = tile_size or choose_tile(xb.shape[1])
    ix = TridentV4Index(st, cen, mean64, R64, tile_size=T, per_cluster_sq8=per_cluster_sq8,
                        var_block=var_block, max_batch=max_batch, max_nprobe=max_nprobe, device=device, k=k,
                        use_pca=use_pca)
    b = Built()
    b.ix, b.xb, b.centroids, b.list_ids = ix, xb.cpu().numpy(), cen, np.asarray(lid)
    h = ix.host_arrays()
    b.xb_sorted, b.orig_ids, b.vec_off = h["xb_sorted"], h["orig_ids_sorted"], h["vec_off"]
    b.centroids_idx = h["centroids"]
    return b


def oracle_search(b, xq, nprobe, K):
    """float64 oracle: probes by (d, cid), exhaustive IVF top-K by (d, id)."""
    xq = np.ascontiguousarray(xq, np.float32)
    cids, _ = O.coarse_probe(xq, b.centroids_idx, nprobe)
    d, i = O.ivf_exact(xq, cids, b.vec_off, b.xb_sorted, b.orig_ids, K)
    return cids, d, i


def assert_exact(gpu_d, gpu_i, ref_d, ref_i, ctx=""):
    """IDs identical; float32 distances equal to the float64 oracle rounded to float32."""
    gpu_d = np.asarray(gpu_d)
    gpu_i = np.asarray(gpu_i)
    bad = np.nonzero((gpu_i != ref_i).any(axis=1))[0]
    assert len(bad) == 0, (f"{ctx}: {len(bad)} queries differ in ids; first q={bad[0]} "
                           f"gpu={gpu_i[bad[0]].tolist()} ref={ref_i[bad[0]].tolist()} "
                           f"gpu_d={gpu_d[bad[0]].tolist()} ref_d={ref_d[bad[0]].tolist()}")
    ref32 = ref_d.astype(np.float32)
    fin = np.isfinite(ref32)
    assert np.array_equal(np.isfinite(gpu_d), fin), f"{ctx}: missing-slot pattern differs"
    assert np.array_equal(gpu_d[fin], ref32[fin]), f"{ctx}: distances differ from float64 oracle"
    rel = np.abs(gpu_d[fin].astype(np.float64) - ref_d[fin]) / np.maximum(ref_d[fin], 1e-30)
    assert (rel <= 1e-5).all(), f"{ctx}: relative distance error {rel.max()} > 1e-5"


def run_search(b, xq_dev, nprobe, K, mode=2, ub=0, use_l1=0, stats=None, route=1):
    """route 1 = per-pair cascade (the default here, so each test pins one route), 2 = batched."""
    d, i, _ = b.ix.search(xq_dev, nprobe, mode=mode, use_l1=use_l1, k=K, ub_seed=ub, stats_buf=stats,
                          route=route)
    torch.cuda.synchronize()
    return d.cpu().numpy().copy(), i.cpu().numpy().copy()


def sq8_arrays(b):
    """numpy copies of the index tensors the SQ8 modes read (oracle.ivf_sq8's ``ix``)."""
    ix = b.ix
    return dict(W_combined=ix.W_combined.cpu().numpy(), b_combined=ix.b_combined.cpu().numpy(),
                nlist=ix.nlist, D_pad=ix.D_pad, vec_off=b.vec_off,
                tile_off=ix.cluster_tile_off.cpu().numpy(), T=ix.tile_size,
                sq8_packed=ix.sq8_packed.cpu().numpy(), tile_oids=ix.tile_orig_ids.cpu().numpy(),
                vmin=ix.vmin_pad.cpu().numpy(), delta=ix.delta_pad.cpu().numpy(),
                per_cluster=ix.per_cluster_sq8, xb_sorted=b.xb_sorted)


def oracle_sq8(b, xq, nprobe, K, mode, rerank_m=0, arrays=None):
    """Modes 0 / 1 on the CPU oracle with the reference's split and list lengths."""
    xq = np.ascontiguousarray(xq, np.float32)
    cids, _ = O.coarse_probe(xq, b.centroids_idx, nprobe)
    p_init, k1, k2, M = O.sq8_mode_plan(mode, len(xq), K, nprobe, rerank_m)
    d, i = O.ivf_sq8(xq, cids, p_init, arrays or sq8_arrays(b), K, k1, k2, M)
    return d, i
