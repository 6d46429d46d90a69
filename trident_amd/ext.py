"""Drop-in search entry point with the reference's Python signature.

``launch_trident_v4_search`` keeps the 41 positional arguments and 3 keywords of the
reference PyBind11 export (src/trident_v4_kernels.cu:1606-1627, C++ body :1172-1604) and
returns the kernel milliseconds when ``record_events`` is true, else 0.0.  It forwards to
the C ABI ``trident_search`` of libtrident_hip.so on torch's current HIP stream.

Differences from the reference, all stricter supersets:
* shapes, dtypes and devices are validated and errors raise ``TridentError``;
* K is read from ``topk_d.size(1)`` and honoured for every K <= 128 (the reference folds
  the cascade and merge back to K = 10, src/trident_v4_kernels.cu:575-576, :984);
* ``TRIDENT_UB_SEED`` is read here (once per call) and passed explicitly; the keyword
  ``ub_seed`` overrides it;
* the per-query candidate buffers are sized nprobe * K inside the library workspace, so
  nothing is dropped (the reference silently drops past ``cand_buf_d.size(1)``, :955-958).
  The reference workspace tensors (proj_buf, cdists_buf, p1_*/p2_*, topm_*, cand_*) are
  accepted for signature compatibility; probe_cids_buf / probe_dqcs_buf receive the probes
  and tau_sq the pass-1 threshold, as in the reference;
* modes 0 (CM-SQ8+RR), 1 (K1) and 11 (Tribase), the reference's comparison routes, run
  the reference algorithms: modes 0 / 1 rank by the SQ8 reconstruction distance acc_hat in
  the rotated space (float64 rotation rounded once, see ``trident_search``), mode 0 then
  reranks the top M = min(max(rerank_m, K), 200) exactly; mode 11 is exact.  use_l1 is
  applied by mode 2 only (for modes 0 / 1 the reference's tile skip compares acc_hat with
  original-space norms and bounds nothing).  When ``r_vec_sorted`` is not given, mode 11
  derives it (float64 |x - c| rounded to float32) once per index;
* ``warp_refine`` only selected a refinement schedule and does not change results, so it
  is accepted and ignored.
"""
import ctypes
import os
import threading
from typing import Optional

import torch

from . import _lib
from ._lib import TridentIndexView, TridentSearchOutputs, TridentSearchParams, check

_ws_lock = threading.Lock()
_ws_cache = {}
_rot_cache = {}
_derived_lock = threading.Lock()
_derived_cache = {}  # index identity -> (vec_Ar, sq8_cells, cent_band, vec_cn), at most two indexes


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise _lib.TridentError(msg)


def _check_tensor(name, t, dtype, device, dims=None, allow_host=False):
    _need(isinstance(t, torch.Tensor), f"{name} must be a torch.Tensor")
    _need(t.dtype == dtype, f"{name} must be {dtype}, got {t.dtype}")
    _need(t.is_contiguous(), f"{name} must be contiguous")
    if dims is not None:
        _need(t.dim() == dims, f"{name} must be {dims}-D, got shape {tuple(t.shape)}")
    if allow_host and t.device.type == "cpu":
        try:
            device_pointer(t)
        except _lib.TridentError as e:
            raise _lib.TridentError(f"{name} on the host must be device-mapped pinned memory "
                                    f"(hipHostMalloc): {e}") from None
    else:
        _need(t.device == device, f"{name} must be on {device}, got {t.device}")


def device_pointer(t: torch.Tensor) -> int:
    """Device address of a tensor; pinned host tensors map through hipHostGetDevicePointer."""
    if t.device.type != "cpu":
        return t.data_ptr()
    out = ctypes.c_void_p()
    check(_lib.lib().trident_host_device_pointer(ctypes.c_void_p(t.data_ptr()), ctypes.byref(out)),
          "trident_host_device_pointer")
    return out.value


def rotation_sq_bounds(W_combined: torch.Tensor, nlist: int, D: int):
    """(min, max) squared singular values of the rotation block R = W_combined[:, nlist:nlist+D],
    widened by 1e-12 relative; cached per tensor version."""
    key = (W_combined.data_ptr(), tuple(W_combined.shape), W_combined._version, nlist, D)
    hit = _rot_cache.get(key)
    if hit is None:
        R = W_combined[:, nlist:nlist + D].detach().to("cpu", torch.float64)
        s = torch.linalg.svdvals(R)
        hit = (float(s.min()) ** 2 * (1.0 - 1e-12), float(s.max()) ** 2 * (1.0 + 1e-12))
        _rot_cache.clear()
        _rot_cache[key] = hit
    return hit


class _Workspace:
    """One grow-only scratch buffer for the searches enqueued on one (device, stream).

    The buffer is allocated while its stream is current, so the caching allocator orders its
    reuse after the work queued on that stream when it is replaced by a larger one; ``lock`` is
    held from taking the buffer until the search is enqueued, so two host threads that share a
    stream cannot interleave their launches over the same scratch memory."""

    __slots__ = ("buf", "lock")

    def __init__(self):
        self.buf = None
        self.lock = threading.Lock()


def _ws_key(device, stream):
    d = torch.device(device)
    if d.type == "cuda" and d.index is None:
        d = torch.device("cuda", torch.cuda.current_device())
    return (d, int(stream.cuda_stream))


def _workspace_slot(device: torch.device, stream) -> _Workspace:
    key = _ws_key(device, stream)
    with _ws_lock:
        slot = _ws_cache.get(key)
        if slot is None:
            slot = _ws_cache[key] = _Workspace()
        return slot


def workspace(device: torch.device, nbytes: int, stream=None) -> torch.Tensor:
    """Grow-only scratch buffer of at least ``nbytes`` for searches on ``stream`` (default:
    the device's current stream); the library itself never allocates.  The caller must hold
    the slot's lock while the buffer is in use from the host (``search_view`` does)."""
    st = stream if stream is not None else torch.cuda.current_stream(device)
    slot = _workspace_slot(device, st)
    return _grow(slot, device, nbytes, st)


def _grow(slot: _Workspace, device, nbytes: int, st) -> torch.Tensor:
    if slot.buf is None or slot.buf.numel() < nbytes:
        slot.buf = None
        with torch.cuda.stream(st):
            slot.buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
    return slot.buf


def release_workspace(device: torch.device, stream) -> None:
    """Drop the workspace of one (device, stream); the next search on it allocates again."""
    key = _ws_key(device, stream)
    with _ws_lock:
        slot = _ws_cache.pop(key, None)
    if slot is not None:
        with slot.lock:
            slot.buf = None


def release_workspaces() -> None:
    with _ws_lock:
        for slot in _ws_cache.values():
            with slot.lock:
                slot.buf = None
        _ws_cache.clear()


def make_index_view(*, N, D, D_pad, nlist, tile_size, per_cluster_sq8, W_combined, b_combined,
                    rot_sq_min, rot_sq_max, sq8_packed, tile_orig_ids, tile_r_minmax,
                    cluster_tile_off, cluster_vec_off, xb_sorted, orig_ids_sorted, vmin, delta,
                    eps_dim, blk_bounds4, vec_Ar=None, sq8_cells=None,
                    cent_band=None, r_vec_sorted=None, fine_codes=None, fine_qp=None,
                    cluster_bounds=None, vec_cn=None, seed_rows=0, xb_sorted_u8=None) -> TridentIndexView:
    v = TridentIndexView()
    v.N, v.D, v.D_pad, v.nlist = int(N), int(D), int(D_pad), int(nlist)
    v.tile_size = int(tile_size)
    v.total_tiles = int(tile_orig_ids.shape[0]) if tile_orig_ids is not None else 0
    v.num_blocks = int(blk_bounds4.numel() - 1) if blk_bounds4 is not None else 0
    v.per_cluster_sq8 = int(per_cluster_sq8)
    v.W_combined = _ptr(W_combined)
    v.b_combined = _ptr(b_combined)
    v.rot_sq_min, v.rot_sq_max = float(rot_sq_min), float(rot_sq_max)
    v.sq8_packed = _ptr(sq8_packed)
    v.tile_orig_ids = _ptr(tile_orig_ids)
    v.tile_r_minmax = _ptr(tile_r_minmax) if tile_r_minmax is not None and tile_r_minmax.numel() > 0 else None
    v.cluster_tile_off = _ptr(cluster_tile_off)
    v.cluster_vec_off = _ptr(cluster_vec_off)
    v.xb_sorted = device_pointer(xb_sorted) if xb_sorted is not None else None
    v.orig_ids_sorted = _ptr(orig_ids_sorted) if orig_ids_sorted is not None and orig_ids_sorted.device.type != "cpu" else None
    v.vmin, v.delta, v.eps_dim = _ptr(vmin), _ptr(delta), _ptr(eps_dim)
    v.blk_bounds4 = _ptr(blk_bounds4)
    v.vec_Ar = _ptr(vec_Ar)
    v.sq8_cells = _ptr(sq8_cells)
    v.r_vec_sorted = _ptr(r_vec_sorted)
    v.fine_codes = _ptr(fine_codes)
    v.fine_qp = _ptr(fine_qp)
    v.cluster_bounds = _ptr(cluster_bounds)
    v.vec_cn = _ptr(vec_cn)
    v.seed_rows = int(seed_rows)
    v.xb_sorted_u8 = device_pointer(xb_sorted_u8) if xb_sorted_u8 is not None else None
    if cent_band is not None:
        rows, tiles, norms, nmax = cent_band
        v.cent_rows, v.cent_tiles, v.cent_norms = _ptr(rows), _ptr(tiles), _ptr(norms)
        v.cent_norm_max = float(nmax)
    return v


def compute_cluster_bounds(view: TridentIndexView, device) -> torch.Tensor:
    """The index-constant per-cluster table of the batched route ([nlist, 4] float64), filled by
    trident_cluster_bounds on the current stream; pass it back as ``cluster_bounds``."""
    out = torch.empty((int(view.nlist), 4), dtype=torch.float64, device=device)
    st = torch.cuda.current_stream(device).cuda_stream
    _lib.check(_lib.lib().trident_cluster_bounds(ctypes.byref(view), out.data_ptr(), st),
               "trident_cluster_bounds")
    return out


def band_dq(D: int) -> int:
    """Row length of the matrix-core coarse layouts: D rounded up to 16."""
    return (int(D) + 15) & ~15


def centroid_band_layouts(W_combined: torch.Tensor, nlist: int):
    """(rows [nlist, Dq], tiles, norms [nlist], max norm) of the centroids c_d = -W[d, c] / 2,
    the optional TridentIndexView fields cent_*: built once per index instead of per search."""
    D = int(W_combined.shape[0])
    Dq = band_dq(D)
    dev = W_combined.device
    cen = (-0.5 * W_combined[:, :nlist]).t().contiguous()          # exact: power-of-two scale
    rows = torch.zeros((nlist, Dq), device=dev, dtype=torch.float32)
    rows[:, :D] = cen
    nl16 = (nlist + 15) // 16 * 16
    pad = torch.zeros((nl16, Dq), device=dev, dtype=torch.float32)
    pad[:nlist] = rows
    S = Dq // 4
    # [t, m, g, j, e] -> [t, j, g, m, e]: float4 (t S/4 + j) 64 + (m + 16 g) = dims g S + 4 j + e
    tiles = pad.view(nl16 // 16, 16, 4, S // 4, 4).permute(0, 3, 2, 1, 4).contiguous().view(-1)
    n64 = (rows.double() ** 2).sum(1)
    return rows, tiles, n64.to(torch.float32), float(n64.max()) if nlist else 0.0


def _identity(*ts):
    return tuple((int(t.data_ptr()), tuple(t.shape), int(t._version)) for t in ts)


def derived_layouts(W_combined, b_combined, sq8_packed, cluster_vec_off, cluster_tile_off, xb_sorted,
                    vmin, delta, per_cluster_sq8: int, nlist: int, tile_size: int):
    """(vec_Ar, sq8_cells, cent_band, vec_cn) for an index passed in the reference layout alone,
    derived once per index (tensor identities and versions) and cached: the per-vector scalars
    measured on the data (index.derive_vec_Ar), the code cells regrouped from sq8_packed
    (index.cells_from_packed), the centroid layouts of the matrix-core coarse pass and the
    per-row code norms (index.derive_vec_cn)."""
    from . import index as _index
    key = _identity(W_combined, b_combined, sq8_packed, cluster_vec_off, cluster_tile_off, xb_sorted,
                    vmin, delta) + (int(per_cluster_sq8), int(nlist), int(tile_size))
    with _derived_lock:
        hit = _derived_cache.get(key)
        if hit is not None:
            return hit
        D_pad = int(W_combined.shape[1]) - int(nlist)
        vec_Ar = _index.derive_vec_Ar(sq8_packed, cluster_vec_off, cluster_tile_off, xb_sorted,
                                      W_combined, b_combined, vmin, delta, per_cluster_sq8, nlist,
                                      tile_size)
        cells = _index.cells_from_packed(sq8_packed, D_pad, int(tile_size))
        band = centroid_band_layouts(W_combined, nlist)
        vec_cn = _index.derive_vec_cn(cells, cluster_vec_off, cluster_tile_off, D_pad, int(tile_size))
        if len(_derived_cache) >= 2:
            _derived_cache.pop(next(iter(_derived_cache)))
        _derived_cache[key] = (vec_Ar, cells, band, vec_cn)
        return vec_Ar, cells, band, vec_cn


def derived_r_vec(W_combined, cluster_vec_off, xb_sorted, nlist: int, chunk_rows: int = 1 << 20):
    """Mode 11's per-vector |x - c| [N] float32 (float64 norm, rounded to nearest) for an index
    passed in the reference layout without r_vec_sorted; centroids c_d = -W_combined[d, c] / 2.
    Cached like derived_layouts."""
    key = ("r_vec",) + _identity(W_combined, cluster_vec_off, xb_sorted) + (int(nlist),)
    with _derived_lock:
        hit = _derived_cache.get(key)
        if hit is not None:
            return hit
        dev = W_combined.device
        cen = (-0.5 * W_combined[:, :nlist]).t().to(torch.float64)
        vec_off = cluster_vec_off.to(dev, torch.int64)
        lid = torch.repeat_interleave(torch.arange(nlist, device=dev), vec_off[1:] - vec_off[:-1])
        N = int(xb_sorted.shape[0])
        out = torch.empty(N, device=dev, dtype=torch.float32)
        for s in range(0, N, chunk_rows):
            e = min(N, s + chunk_rows)
            x = xb_sorted[s:e].to(dev, torch.float64)
            out[s:e] = torch.sqrt(((x - cen[lid[s:e]]) ** 2).sum(1)).to(torch.float32)
        if len(_derived_cache) >= 2:
            _derived_cache.pop(next(iter(_derived_cache)))
        _derived_cache[key] = out
        return out


def env_ub_seed() -> int:
    return int(os.environ.get("TRIDENT_UB_SEED", "0") or 0)


def search_view(view: TridentIndexView, xq: torch.Tensor, nprobe: int, topk_d: torch.Tensor,
                topk_i: torch.Tensor, *, mode: int = 2, ub_seed: int = 0, use_l1: int = 0,
                p_init: int = -1, route: int = 0, rerank_m: int = 0,
                probe_cids: Optional[torch.Tensor] = None,
                probe_dqcs: Optional[torch.Tensor] = None, tau_sq: Optional[torch.Tensor] = None,
                stats: Optional[torch.Tensor] = None, record_events: bool = False,
                stream: Optional[torch.cuda.Stream] = None, stage_events=None,
                host_rows: Optional[torch.Tensor] = None) -> float:
    """Runs trident_search on an index view; all tensors already validated by the caller."""
    B, K = int(xq.shape[0]), int(topk_d.shape[1])
    L = _lib.lib()
    # mode 0's merged lists hold M = min(max(rerank_m, K), 200) entries
    k_ws = max(K, min(int(rerank_m), 200)) if int(mode) == _lib.MODE_SQ8_RERANK else K
    nbytes = L.trident_workspace_bytes(ctypes.byref(view), max(B, 1), int(nprobe), k_ws)
    st = stream if stream is not None else torch.cuda.current_stream(xq.device)
    slot = _workspace_slot(xq.device, st)
    sp = TridentSearchParams(int(mode), B, K, int(nprobe), int(ub_seed), int(use_l1), int(p_init), int(route),
                             int(rerank_m))
    out = TridentSearchOutputs()
    out.topk_d, out.topk_i = topk_d.data_ptr(), topk_i.data_ptr()
    out.probe_cids = _ptr(probe_cids)
    out.probe_dqcs = _ptr(probe_dqcs)
    ld = 0
    if probe_cids is not None:
        ld = int(probe_cids.shape[1])
    elif probe_dqcs is not None:
        ld = int(probe_dqcs.shape[1])
    out.probe_ld = ld
    out.tau_sq = _ptr(tau_sq)
    out.stats = _ptr(stats)
    out.host_rows = _ptr(host_rows)
    # a 2-entry host_rows buffer also receives the seeding pass's share in its second entry
    out.host_rows_seed = host_rows.data_ptr() + 8 if host_rows is not None and host_rows.numel() >= 2 else None
    if stage_events is not None:
        out.events = stage_events.handles
        out.n_events = _lib.EV_COUNT
    ev0 = ev1 = None
    if record_events:
        ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ev0.record(st)
    with slot.lock:
        ws = _grow(slot, xq.device, nbytes, st)
        rc = L.trident_search(ctypes.byref(view), ctypes.byref(sp), ctypes.c_void_p(xq.data_ptr()),
                              ctypes.c_void_p(ws.data_ptr()), ctypes.c_size_t(ws.numel()),
                              ctypes.byref(out), ctypes.c_void_p(st.cuda_stream))
    check(rc, "trident_search")
    if record_events:
        ev1.record(st)
        ev1.synchronize()
        return float(ev0.elapsed_time(ev1))
    return 0.0


def launch_trident_v4_search(
    mode, tile_size, use_l1, per_cluster_sq8, rerank_m, nprobe,
    xq_orig, W_combined, b_combined, W_coarse_only, b_coarse_only,
    proj_buf, cdists_buf, probe_cids_buf, probe_dqcs_buf,
    p1_cids_buf, p1_qids_buf, p1_dqcs_buf, p2_cids_buf, p2_qids_buf, p2_dqcs_buf,
    sq8_packed, tile_orig_ids, tile_r_minmax, cluster_tile_off, cluster_vec_off,
    xb_sorted, orig_ids_sorted, vmin, delta, eps_dim, blk_bounds4,
    topk_d, topk_i, topm_buf_d, topm_buf_i, tau_sq,
    cand_buf_d, cand_buf_i, cand_cnt, record_events,
    warp_refine=1, stats_buf=None, r_vec_sorted=None,
    *, ub_seed: Optional[int] = None, rot_sq_bounds=None, p_init: int = -1, stage_events=None,
    vec_Ar: Optional[torch.Tensor] = None, route: int = 0,
    sq8_cells: Optional[torch.Tensor] = None,
    cent_band=None,
    fine_codes: Optional[torch.Tensor] = None, fine_qp: Optional[torch.Tensor] = None,
    host_rows: Optional[torch.Tensor] = None,
    cluster_bounds: Optional[torch.Tensor] = None,
    vec_cn: Optional[torch.Tensor] = None,
    seed_rows: int = 0,
    xb_sorted_u8: Optional[torch.Tensor] = None,
):
    """Batched lossless IVF search; signature of the reference extension (see module doc)."""
    mode, nprobe = int(mode), int(nprobe)
    _need(int(seed_rows) >= 0, "seed_rows must be >= 0")
    _need(mode in (0, 1, 2, 10, 11), f"unknown mode {mode} (0, 1, 2, 10 or 11)")
    _need(int(rerank_m) >= 0, "rerank_m must be >= 0")
    sq8 = mode in (0, 1, 2)  # modes reading the SQ8 codes
    dev = xq_orig.device
    _need(dev.type == "cuda", "xq_orig must be a device tensor")
    _check_tensor("xq_orig", xq_orig, torch.float32, dev, 2)
    B, D = int(xq_orig.shape[0]), int(xq_orig.shape[1])
    _check_tensor("W_coarse_only", W_coarse_only, torch.float32, dev, 2)
    nlist = int(W_coarse_only.shape[1])
    _check_tensor("W_combined", W_combined, torch.float32, dev, 2)
    _need(W_combined.shape[0] == D, "W_combined rows must equal D")
    D_pad = int(W_combined.shape[1]) - nlist
    _need(D_pad >= D and D_pad % 32 == 0, f"W_combined implies D_pad={D_pad}; expected a multiple of 32 >= D")
    _check_tensor("b_combined", b_combined, torch.float32, dev)
    _need(b_combined.numel() == nlist + D_pad, "b_combined must have nlist + D_pad entries")
    _check_tensor("topk_d", topk_d, torch.float32, dev, 2)
    _check_tensor("topk_i", topk_i, torch.int64, dev, 2)
    _need(topk_d.shape[0] == B and tuple(topk_i.shape) == tuple(topk_d.shape),
          "topk_d / topk_i must be [B, K]")
    K = int(topk_d.shape[1])
    _check_tensor("cluster_vec_off", cluster_vec_off, torch.int32, dev, 1)
    _check_tensor("cluster_tile_off", cluster_tile_off, torch.int32, dev, 1)
    _need(cluster_vec_off.numel() == nlist + 1 and cluster_tile_off.numel() == nlist + 1,
          "cluster offsets must have nlist + 1 entries")
    _check_tensor("xb_sorted", xb_sorted, torch.float32, dev, 2, allow_host=True)
    _need(xb_sorted.shape[1] == D, "xb_sorted must be [N, D]")
    N = int(xb_sorted.shape[0])
    _check_tensor("tile_orig_ids", tile_orig_ids, torch.int32, dev, 2)
    _need(int(tile_orig_ids.shape[1]) == int(tile_size),
          f"tile_size={tile_size} does not match the packed tiles ({tile_orig_ids.shape[1]})")
    tiles = int(tile_orig_ids.shape[0])
    _check_tensor("orig_ids_sorted", orig_ids_sorted, torch.int32, dev, 1)
    _need(orig_ids_sorted.numel() == N, f"orig_ids_sorted must hold N={N} int32 ids")
    if tile_r_minmax is not None and tile_r_minmax.numel() > 0:
        _check_tensor("tile_r_minmax", tile_r_minmax, torch.float32, dev)
        _need(tile_r_minmax.numel() == 2 * tiles, f"tile_r_minmax must be [tiles={tiles}, 2] float32")
    else:
        tile_r_minmax = None
    _need(not (int(use_l1) and mode == 2 and tile_r_minmax is None), "use_l1 needs tile_r_minmax")
    # mode 2 on an index that keeps only the batched route's cells (TridentV4Index.
    # release_packed_codes): an empty sq8_packed, and the batched route
    packed = sq8 and not (mode == 2 and sq8_packed is not None and sq8_packed.numel() == 0 and
                          sq8_cells is not None and vec_Ar is not None)
    if sq8 and not packed:
        _need(int(route) != 1, "the per-pair route reads sq8_packed, which this index released")
    if packed:
        _check_tensor("sq8_packed", sq8_packed, torch.int32, dev)
        _need(sq8_packed.numel() == tiles * (D_pad // 4) * int(tile_size),
              "sq8_packed must hold [tiles, D_pad/4, tile_size] words")
    if sq8:
        rows = nlist if int(per_cluster_sq8) else 1
        for name, t in (("vmin", vmin), ("delta", delta), ("eps_dim", eps_dim)):
            _check_tensor(name, t, torch.float32, dev)
            _need(t.numel() == rows * D_pad, f"{name} must be [{rows}, D_pad]")
        _check_tensor("blk_bounds4", blk_bounds4, torch.int32, dev, 1)
    if fine_codes is not None or fine_qp is not None:
        _need(fine_codes is not None and fine_qp is not None, "fine_codes and fine_qp go together")
        _check_tensor("fine_codes", fine_codes, torch.int16, dev, 2)
        _need(tuple(fine_codes.shape) == (N, D_pad), "fine_codes must be [N, D_pad] int16 (uint16 bits)")
        _check_tensor("fine_qp", fine_qp, torch.float32, dev, 2)
        _need(tuple(fine_qp.shape) == (N, 4), "fine_qp must be [N, 4] float32")
    if cluster_bounds is not None:
        _need(vec_Ar is not None, "cluster_bounds is derived from vec_Ar: pass both")
        _check_tensor("cluster_bounds", cluster_bounds, torch.float64, dev, 2)
        _need(tuple(cluster_bounds.shape) == (nlist, 4), "cluster_bounds must be [nlist, 4] float64")
    if vec_Ar is not None:
        _check_tensor("vec_Ar", vec_Ar, torch.float32, dev, 2)
        _need(tuple(vec_Ar.shape) == (N, 2), "vec_Ar must be [N, 2] float32")
    if vec_cn is not None:
        _check_tensor("vec_cn", vec_cn, torch.float32, dev, 1)
        _need(vec_cn.numel() == N, f"vec_cn must hold N={N} floats")
    if xb_sorted_u8 is not None:
        _check_tensor("xb_sorted_u8", xb_sorted_u8, torch.uint8, dev, 2, allow_host=True)
        _need(tuple(xb_sorted_u8.shape) == (N, D) and D % 16 == 0,
              "xb_sorted_u8 must be [N, D] uint8 with D a multiple of 16")
    if sq8_cells is not None:
        _check_tensor("sq8_cells", sq8_cells, torch.int32, dev)
        _need(sq8_cells.numel() == tiles * (D_pad // 16) * int(tile_size) * 4,
              "sq8_cells must hold [tiles, tile_size/V, D_pad/16, V, 4] words")
    if cent_band is not None:
        Dq = band_dq(D)
        rows_t, tiles_t, norms_t, _ = cent_band
        for name, t, numel in (("cent_band rows", rows_t, nlist * Dq),
                               ("cent_band tiles", tiles_t, (nlist + 15) // 16 * 16 * Dq),
                               ("cent_band norms", norms_t, nlist)):
            _check_tensor(name, t, torch.float32, dev)
            _need(t.numel() == numel, f"{name} must hold {numel} floats")
    if stats_buf is not None:
        _check_tensor("stats_buf", stats_buf, torch.int64, dev)
        _need(stats_buf.numel() >= 4, "stats_buf needs 4 entries")
    if host_rows is not None:
        _check_tensor("host_rows", host_rows, torch.int64, dev)
        _need(host_rows.numel() >= 1, "host_rows needs 1 entry")
    if probe_cids_buf is not None:
        _check_tensor("probe_cids_buf", probe_cids_buf, torch.int32, dev, 2)
        _need(probe_cids_buf.shape[0] >= B and probe_cids_buf.shape[1] >= nprobe, "probe_cids_buf too small")
    if probe_dqcs_buf is not None:
        _check_tensor("probe_dqcs_buf", probe_dqcs_buf, torch.float32, dev, 2)
        _need(probe_dqcs_buf.shape[0] >= B and probe_dqcs_buf.shape[1] >= nprobe, "probe_dqcs_buf too small")
        if probe_cids_buf is not None:
            _need(probe_dqcs_buf.shape[1] == probe_cids_buf.shape[1], "probe buffers need one row stride")
    if tau_sq is not None:
        _check_tensor("tau_sq", tau_sq, torch.float32, dev)
        _need(tau_sq.numel() >= B, "tau_sq needs B entries")

    if mode == 11:
        if r_vec_sorted is not None:
            _check_tensor("r_vec_sorted", r_vec_sorted, torch.float32, dev)
            _need(r_vec_sorted.numel() == N, f"r_vec_sorted must hold N={N} floats")
        else:
            r_vec_sorted = derived_r_vec(W_combined, cluster_vec_off, xb_sorted, nlist)
    else:
        r_vec_sorted = None
    if rot_sq_bounds is None:
        rot_sq_bounds = rotation_sq_bounds(W_combined, nlist, D)
    if mode == 2 and (vec_Ar is None or sq8_cells is None) and int(route) != 1 and \
            (int(route) == 2 or B * nprobe >= 8 * nlist) and D_pad <= 1024 and K <= 128:
        # a reference caller passes neither: derive them (once per index) so that the batched
        # route can run, as it would for an index built by TridentV4Index
        vec_Ar, sq8_cells, band, vec_cn = derived_layouts(W_combined, b_combined, sq8_packed,
                                                          cluster_vec_off, cluster_tile_off, xb_sorted,
                                                          vmin, delta, per_cluster_sq8, nlist, tile_size)
        if cent_band is None:
            cent_band = band
    view = make_index_view(
        N=N, D=D, D_pad=D_pad, nlist=nlist, tile_size=tile_size, per_cluster_sq8=per_cluster_sq8,
        W_combined=W_combined, b_combined=b_combined, rot_sq_min=rot_sq_bounds[0],
        rot_sq_max=rot_sq_bounds[1], sq8_packed=sq8_packed if packed else None,
        tile_orig_ids=tile_orig_ids, tile_r_minmax=tile_r_minmax,
        cluster_tile_off=cluster_tile_off, cluster_vec_off=cluster_vec_off, xb_sorted=xb_sorted,
        orig_ids_sorted=orig_ids_sorted, vmin=vmin if sq8 else None,
        delta=delta if sq8 else None, eps_dim=eps_dim if sq8 else None,
        blk_bounds4=blk_bounds4, vec_Ar=vec_Ar if mode == 2 else None,
        sq8_cells=sq8_cells if mode == 2 else None, cent_band=cent_band, r_vec_sorted=r_vec_sorted,
        fine_codes=fine_codes if mode == 2 else None, fine_qp=fine_qp if mode == 2 else None,
        cluster_bounds=cluster_bounds if mode == 2 else None, vec_cn=vec_cn if mode == 2 else None,
        seed_rows=seed_rows, xb_sorted_u8=xb_sorted_u8 if mode in (2, 10) else None)
    ub = env_ub_seed() if ub_seed is None else int(ub_seed)
    return search_view(view, xq_orig, nprobe, topk_d, topk_i, mode=mode, ub_seed=ub,
                       use_l1=int(use_l1), p_init=p_init, route=route,
                       rerank_m=int(rerank_m) if mode == 0 else 0, probe_cids=probe_cids_buf,
                       probe_dqcs=probe_dqcs_buf, tau_sq=tau_sq, stats=stats_buf, host_rows=host_rows,
                       record_events=bool(record_events), stage_events=stage_events)
