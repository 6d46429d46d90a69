"""trident_search_noalloc (the entry point with a fixed, library-owned scratch array) against
trident_search with a caller-owned workspace, through the C ABI: identical ids and distances on
two calls in a row (the second with a smaller batch, so the scratch holds the first call's
leftovers), on both mode-2 routes and the exact route, and an oversized batch is refused."""
import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import build_index, oracle_search
from trident_amd import _lib, datagen, ext
from trident_amd._lib import TridentSearchOutputs, TridentSearchParams

pytestmark = pytest.mark.gpu


def _view(ix):
    st = ix.storage
    return ext.make_index_view(
        N=ix.N, D=ix.D, D_pad=ix.D_pad, nlist=ix.nlist, tile_size=ix.tile_size,
        per_cluster_sq8=ix.per_cluster_sq8, W_combined=ix.W_combined, b_combined=ix.b_combined,
        rot_sq_min=ix.rot_sq_min, rot_sq_max=ix.rot_sq_max, sq8_packed=ix.sq8_packed,
        tile_orig_ids=ix.tile_orig_ids, tile_r_minmax=ix.tile_r_minmax,
        cluster_tile_off=ix.cluster_tile_off, cluster_vec_off=st.cluster_vec_off,
        xb_sorted=st.xb_sorted, orig_ids_sorted=st.orig_ids_sorted, vmin=ix.vmin_pad,
        delta=ix.delta_pad, eps_dim=ix.eps_pad, blk_bounds4=ix.blk_bounds4, vec_Ar=ix.vec_Ar,
        sq8_cells=ix.sq8_cells, cent_band=ix.cent_band)


def _call(view, xq, mode, nprobe, K, route, noalloc):
    L = _lib.lib()
    dev = xq.device
    B = int(xq.shape[0])
    td = torch.full((B, K), -1.0, dtype=torch.float32, device=dev)
    ti = torch.full((B, K), -7, dtype=torch.int64, device=dev)
    sp = TridentSearchParams(mode, B, K, nprobe, 1, 0, -1, route)
    out = TridentSearchOutputs()
    out.topk_d, out.topk_i = td.data_ptr(), ti.data_ptr()
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if noalloc:
        rc = L.trident_search_noalloc(ctypes.byref(view), ctypes.byref(sp), ctypes.c_void_p(xq.data_ptr()),
                                      ctypes.byref(out), stream)
        _lib.check(rc, "trident_search_noalloc")
    else:
        nbytes = L.trident_workspace_bytes(ctypes.byref(view), B, nprobe, K)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = L.trident_search(ctypes.byref(view), ctypes.byref(sp), ctypes.c_void_p(xq.data_ptr()),
                              ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(nbytes), ctypes.byref(out),
                              stream)
        _lib.check(rc, "trident_search")
    torch.cuda.synchronize()
    return td.cpu().numpy(), ti.cpu().numpy()


def test_noalloc_matches_workspace_entry_point(dev):
    xb, xq = datagen.cfg2(N=40_000, D=128, B=400, n_centers=128, seed=61)
    b = build_index(xb, 128, dev, max_batch=400)
    view = _view(b.ix)
    xqd = torch.as_tensor(xq.numpy()).to(dev).contiguous()
    for mode, route, nprobe, K in ((2, 0, 16, 10), (2, 1, 16, 10), (2, 2, 24, 64), (10, 0, 8, 10)):
        for B in (400, 150):  # the second call is smaller: the scratch holds the first's data
            q = xqd[:B].contiguous()
            d0, i0 = _call(view, q, mode, nprobe, K, route, noalloc=False)
            d1, i1 = _call(view, q, mode, nprobe, K, route, noalloc=True)
            ctx = f"mode={mode} route={route} nprobe={nprobe} K={K} B={B}"
            assert np.array_equal(i1, i0), ctx
            assert np.array_equal(d1, d0), ctx
            _, rd, ri = oracle_search(b, xq.numpy()[:B], nprobe, K)
            assert np.array_equal(i1, ri), ctx


def test_noalloc_refuses_batches_beyond_its_scratch(dev):
    xb, xq = datagen.cfg2(N=20_000, D=128, B=64, n_centers=64, seed=62)
    b = build_index(xb, 64, dev, max_batch=64)
    view = _view(b.ix)
    L = _lib.lib()
    B, nprobe, K = 20_000, 64, 10
    assert L.trident_workspace_bytes(ctypes.byref(view), B, nprobe, K) > _lib.NOALLOC_SCRATCH_BYTES
    sp = TridentSearchParams(2, B, K, nprobe, 1, 0, -1, 0)
    out = TridentSearchOutputs()
    td = torch.empty((1, K), dtype=torch.float32, device=dev)
    ti = torch.empty((1, K), dtype=torch.int64, device=dev)
    out.topk_d, out.topk_i = td.data_ptr(), ti.data_ptr()
    rc = L.trident_search_noalloc(ctypes.byref(view), ctypes.byref(sp), ctypes.c_void_p(td.data_ptr()),
                                  ctypes.byref(out), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 3 and b"scratch" in L.trident_last_error()
