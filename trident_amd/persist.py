"""On-disk index: one directory of ``meta.npz`` plus raw ``.bin`` arrays, loaded by memory map.

The reference's 100M engine keeps its built index as ``meta.npz`` (centroids, mean64, R64,
sort_perm, vec_off, tile_off, vmin, delta) next to ``sq8_packed.bin``, ``tile_orig_ids.bin``
and the base as raw memmaps (benchmarks/phase8_ooc_100m_4080.py:228-248), written by its GPU
build (scripts/phase7_step2_gpu_build_verify.py:68-272).  This format keeps that split -- the
small arrays and scalars in ``meta.npz``, every array proportional to N in a ``.bin`` file read
with ``numpy.memmap`` and streamed to the device in chunks -- and stores everything a
``TridentV4Index`` holds, so loading rebuilds nothing:

  meta.npz            format, version, sizes and options, rot_sq_min / rot_sq_max, centroids,
                      mean64, R64 (the clustering's float64 rotation, kept for reference),
                      W_combined, b_combined, vec_off, tile_off, vmin, delta, eps, blk_bounds4,
                      tile_r_minmax, and the .bin manifest (name, dtype, shape)
  sort_perm.bin       int32 [N]            original id of each sorted row (orig_ids_sorted)
  sq8_packed.bin      int32 [tiles, D_pad/4, T]   the reference's code packing
  tile_orig_ids.bin   int32 [tiles, T]
  vec_Ar.bin          float32 [N, 2]       per-vector scalars of the batched route
  r_vec_sorted.bin    float32 [N]          |x - c| (mode 11)
  fine_codes.bin      int16 [N, D_pad]     fine level: 16-bit row codes (when the index has it)
  fine_qp.bin         float32 [N, 4]       their offset, step and error bound
  xb_sorted.bin       float32 [N, D]       the cluster-sorted base (optional)

The code cells of the batched route, their per-row norms and the centroid layouts of the
coarse pass are regrouped / recomputed from sq8_packed / W_combined on load (cheap, on the
device).

Consistency.  A save first removes any ``meta.npz`` already in the directory, writes every
``.bin`` under a temporary name and renames it into place (``os.replace``), and writes
``meta.npz`` last, so an interrupted save leaves a directory without a ``meta.npz``, which the
loader refuses.  Every ``.bin`` ends with the save's 16-byte random token (after the array's
bytes), and ``meta.npz`` records it: a ``.bin`` left over from another save (a re-save over an
index of the same shapes, interrupted after some files were replaced) carries another token and
is refused.  The loader also checks the format, the version, every file's size and shape
against the manifest and the index sizes (N, D, D_pad, nlist, tiles, T), and the list offsets
(0 = vec_off[0] <= ... <= vec_off[nlist] = N, the same for the tile offsets), before anything is
copied to the device.  Callers may store their own scalars (``user`` = {name: int/float/str})
and read them back with ``read_user_meta``.
"""
import os
import time
from typing import Optional

import numpy as np
import torch

from . import ext as _ext
from .index import SharedClusterStorage, TridentV4Index, cells_from_packed, derive_vec_cn

FORMAT = "trident-amd-ivf-sq8"
VERSION = 2
_TOKEN_BYTES = 16

_CHUNK_ROWS = 1 << 20
_SCALARS = ("N", "D", "D_pad", "nlist", "tile_size", "per_cluster_sq8", "use_pca", "var_block",
            "total_tiles")


def _write_bin(path: str, t: torch.Tensor, token: bytes, chunk_rows: int = _CHUNK_ROWS):
    """Streams a tensor (device, host or pinned) to ``path`` row chunk by row chunk, then the
    save's token."""
    tmp = f"{path}.tmp-{os.getpid()}"
    with open(tmp, "wb") as f:
        n = int(t.shape[0]) if t.dim() else 1
        for s in range(0, max(n, 1), chunk_rows):
            part = t[s:s + chunk_rows] if t.dim() else t
            f.write(part.detach().to("cpu").contiguous().numpy().tobytes())
        f.write(token)
    os.replace(tmp, path)


def save_index(ix: TridentV4Index, path: str, include_base: bool = True, mean64=None, R64=None,
               user: Optional[dict] = None) -> dict:
    """Writes ``ix`` (and, with ``include_base``, its sorted base) under directory ``path``.
    ``user``: the caller's own scalars, stored in meta.npz (``read_user_meta``).  Returns the
    manifest."""
    os.makedirs(path, exist_ok=True)
    meta_f = os.path.join(path, "meta.npz")
    if os.path.exists(meta_f):  # until the new meta lands, the directory is no index
        os.remove(meta_f)
    token = os.urandom(_TOKEN_BYTES)
    st = ix.storage
    bins = {
        "sort_perm": st.orig_ids_sorted,
        "sq8_packed": ix.packed_codes(),  # rebuilt from the cells if the index released it
        "tile_orig_ids": ix.tile_orig_ids,
        "vec_Ar": ix.vec_Ar,
        "r_vec_sorted": ix.r_vec_sorted,
    }
    if getattr(ix, "fine_codes", None) is not None:
        bins["fine_codes"] = ix.fine_codes
        bins["fine_qp"] = ix.fine_qp
    if include_base:
        _need(st.xb_sorted is not None, "the storage's base has been freed")
        bins["xb_sorted"] = st.xb_sorted
    manifest = {}
    for name, t in bins.items():
        _write_bin(os.path.join(path, name + ".bin"), t, token)
        manifest[name] = (str(t.dtype).replace("torch.", ""), tuple(int(s) for s in t.shape))
    meta = {k: np.int64(getattr(ix, k)) for k in _SCALARS}
    meta.update(
        format=np.array(FORMAT), version=np.int64(VERSION),
        within=np.array(getattr(st, "within", "id")),
        token=np.frombuffer(token, np.uint8).copy(),
        rot_sq_min=np.float64(ix.rot_sq_min), rot_sq_max=np.float64(ix.rot_sq_max),
        centroids=ix.centroids.cpu().numpy(),
        W_combined=ix.W_combined.cpu().numpy(), b_combined=ix.b_combined.cpu().numpy(),
        vec_off=st.cluster_vec_off.cpu().numpy(), tile_off=ix.cluster_tile_off.cpu().numpy(),
        vmin=ix.vmin_pad.cpu().numpy(), delta=ix.delta_pad.cpu().numpy(), eps=ix.eps_pad.cpu().numpy(),
        blk_bounds4=ix.blk_bounds4.cpu().numpy(), tile_r_minmax=ix.tile_r_minmax.cpu().numpy(),
        bin_names=np.array(list(manifest)),
        bin_dtypes=np.array([manifest[n][0] for n in manifest]),
        bin_shapes=np.array([",".join(map(str, manifest[n][1])) for n in manifest]),
    )
    if mean64 is not None:
        meta["mean64"] = np.asarray(mean64, np.float64)
    if R64 is not None:
        meta["R64"] = np.asarray(R64, np.float64)
    for k2, v in (user or {}).items():
        _need(isinstance(v, (int, float, str, np.integer, np.floating)), f"user[{k2!r}] must be a scalar")
        meta["user_" + str(k2)] = np.array(v)
    tmp = os.path.join(path, f"meta.tmp-{os.getpid()}.npz")
    np.savez(tmp, **meta)
    os.replace(tmp, meta_f)
    return manifest


def read_user_meta(path: str) -> dict:
    """The ``user`` scalars a save stored (empty when the directory holds no index)."""
    meta_f = os.path.join(path, "meta.npz")
    if not os.path.exists(meta_f):
        return {}
    with np.load(meta_f, allow_pickle=False) as z:
        return {k2[5:]: z[k2].item() for k2 in z.files if k2.startswith("user_")}


def _need(cond: bool, msg: str):
    if not cond:
        raise ValueError(msg)


_NP = {"int32": np.int32, "float32": np.float32, "int16": np.int16}
_TORCH = {"int32": torch.int32, "float32": torch.float32, "int16": torch.int16}


def _expected_shapes(sc: dict) -> dict:
    N, D, DP, T, tiles = sc["N"], sc["D"], sc["D_pad"], sc["tile_size"], sc["total_tiles"]
    return {"sort_perm": ((N,), "int32"), "sq8_packed": ((tiles, DP // 4, T), "int32"),
            "tile_orig_ids": ((tiles, T), "int32"), "vec_Ar": ((N, 2), "float32"),
            "r_vec_sorted": ((N,), "float32"), "fine_codes": ((N, DP), "int16"),
            "fine_qp": ((N, 4), "float32"), "xb_sorted": ((N, D), "float32")}


def _open_bins(path: str, meta, sc: dict) -> dict:
    out = {}
    token = bytes(np.asarray(meta["token"], np.uint8))
    want_shapes = _expected_shapes(sc)
    for name, dt, shp in zip(meta["bin_names"], meta["bin_dtypes"], meta["bin_shapes"]):
        name, dt = str(name), str(dt)
        shape = tuple(int(s) for s in str(shp).split(",") if s)
        _need(name in want_shapes, f"{path}: unknown array {name!r} in the manifest")
        _need((shape, dt) == want_shapes[name],
              f"{path}: {name} is {dt} {shape} in the manifest, the index sizes say "
              f"{want_shapes[name][1]} {want_shapes[name][0]}")
        f = os.path.join(path, name + ".bin")
        _need(os.path.exists(f), f"{f} is missing")
        want = int(np.prod(shape)) * np.dtype(_NP[dt]).itemsize
        got = os.path.getsize(f)
        _need(got == want + _TOKEN_BYTES, f"{f}: {got} bytes, the manifest says {want + _TOKEN_BYTES}")
        with open(f, "rb") as fh:
            fh.seek(want)
            _need(fh.read(_TOKEN_BYTES) == token, f"{f} belongs to another save (token mismatch)")
        out[name] = np.memmap(f, dtype=_NP[dt], mode="r", shape=shape) if want else np.zeros(shape, _NP[dt])
    for name in ("sort_perm", "sq8_packed", "tile_orig_ids", "vec_Ar", "r_vec_sorted"):
        _need(name in out, f"{path}: {name}.bin is not in the manifest")
    _need(("fine_codes" in out) == ("fine_qp" in out), f"{path}: the fine level is incomplete")
    return out


def _check_offsets(path: str, off: np.ndarray, n_lists: int, total: int, what: str):
    off = np.asarray(off)
    _need(off.ndim == 1 and off.shape[0] == n_lists + 1, f"{path}: {what} must have nlist + 1 entries")
    _need(int(off[0]) == 0 and int(off[-1]) == total, f"{path}: {what} must run from 0 to {total}")
    _need(bool(np.all(np.diff(off.astype(np.int64)) >= 0)), f"{path}: {what} is not monotone")


def _check_meta(path: str, meta, sc: dict):
    N, D, DP, nlist, T, tiles = (sc["N"], sc["D"], sc["D_pad"], sc["nlist"], sc["tile_size"],
                                 sc["total_tiles"])
    _need(N >= 0 and D >= 1 and nlist >= 1 and T >= 64 and T % 64 == 0 and DP >= D and DP % 32 == 0,
          f"{path}: inconsistent sizes {sc}")
    _check_offsets(path, meta["vec_off"], nlist, N, "vec_off")
    _check_offsets(path, meta["tile_off"], nlist, tiles, "tile_off")
    _need(tuple(meta["centroids"].shape) == (nlist, D), f"{path}: centroids must be [{nlist}, {D}]")
    _need(tuple(meta["W_combined"].shape) == (D, nlist + DP), f"{path}: W_combined must be [{D}, {nlist + DP}]")
    _need(meta["b_combined"].size == nlist + DP, f"{path}: b_combined must hold {nlist + DP} values")
    rows = nlist if sc["per_cluster_sq8"] else 1
    for name in ("vmin", "delta", "eps"):
        _need(meta[name].shape[-1] == DP and meta[name].size in (DP, rows * DP),
              f"{path}: {name} must be [{rows}, {DP}]")
    _need(meta["tile_r_minmax"].size == 2 * tiles, f"{path}: tile_r_minmax must be [{tiles}, 2]")


def _to_device(a: np.ndarray, dev, chunk_rows: int = _CHUNK_ROWS) -> torch.Tensor:
    t = torch.empty(a.shape, dtype=_TORCH[str(a.dtype)], device=dev)
    n = a.shape[0] if a.ndim else 1
    for s in range(0, n, chunk_rows):
        t[s:s + chunk_rows] = torch.from_numpy(np.array(a[s:s + chunk_rows]))
    return t


def load_index(path: str, device="cuda:0", xb_placement: str = "device", xb_raw=None,
               max_batch: int = 1024, max_nprobe: int = 512, k: int = 10) -> TridentV4Index:
    """Loads an index written by ``save_index``.  The base comes from ``xb_sorted.bin`` when the
    directory has one, else from ``xb_raw`` (the original-order base, sorted here by sort_perm).
    ``xb_placement`` = "device" (HBM) or "host" (device-mapped pinned host memory)."""
    t0 = time.perf_counter()
    meta_f = os.path.join(path, "meta.npz")
    _need(os.path.exists(meta_f), f"{meta_f} is missing (not a saved index, or an interrupted save)")
    with np.load(meta_f, allow_pickle=False) as z:
        meta = {k2: z[k2] for k2 in z.files}
    _need(str(meta["format"]) == FORMAT, f"{path}: format {meta['format']!s}, expected {FORMAT}")
    _need(int(meta["version"]) == VERSION, f"{path}: version {int(meta['version'])}, expected {VERSION}")
    sc = {k2: int(meta[k2]) for k2 in _SCALARS}
    _check_meta(path, meta, sc)
    bins = _open_bins(path, meta, sc)
    N, D, nlist = sc["N"], sc["D"], sc["nlist"]
    dev = torch.device(device)
    sort_perm = np.asarray(bins["sort_perm"])
    if "xb_sorted" in bins:
        xb_sorted = bins["xb_sorted"]
    else:
        _need(xb_raw is not None, f"{path} holds no base: pass xb_raw (the base in original order)")
        _need(tuple(xb_raw.shape) == (N, D), f"xb_raw must be [{N}, {D}]")
        xb_sorted = None
    st = SharedClusterStorage.from_sorted(xb_sorted, sort_perm, meta["vec_off"], device=dev,
                                          xb_placement=xb_placement, xb_raw=xb_raw)
    # the row order within clusters (indexes saved before it was recorded are in id order)
    st.within = str(meta["within"]) if "within" in meta else "id"
    ix = TridentV4Index.__new__(TridentV4Index)
    ix.storage, ix.dev = st, dev
    for k2, v in sc.items():
        setattr(ix, k2, v)
    ix.W_tile = ix.tile_size // 32
    ix.D4 = ix.D_pad // 4
    ix.k = int(k)
    ix.rot_sq_min, ix.rot_sq_max = float(meta["rot_sq_min"]), float(meta["rot_sq_max"])
    f32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.float32).to(dev)
    i32 = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32).to(dev)
    ix.centroids = f32(meta["centroids"])
    ix.W_combined, ix.b_combined = f32(meta["W_combined"]), f32(meta["b_combined"])
    ix.W_coarse_only = ix.W_combined[:, :nlist].contiguous()
    ix.b_coarse_only = ix.b_combined[:, :nlist].contiguous()
    ix.cent_band = _ext.centroid_band_layouts(ix.W_combined, nlist)
    ix.vmin_pad, ix.delta_pad, ix.eps_pad = f32(meta["vmin"]), f32(meta["delta"]), f32(meta["eps"])
    ix.blk_bounds4 = i32(meta["blk_bounds4"])
    ix.tile_r_minmax = f32(meta["tile_r_minmax"])
    ix.cluster_tile_off = i32(meta["tile_off"])
    ix.sq8_packed = _to_device(bins["sq8_packed"], dev)
    ix.sq8_cells = cells_from_packed(ix.sq8_packed, ix.D_pad, ix.tile_size)
    ix.vec_cn = derive_vec_cn(ix.sq8_cells, st.cluster_vec_off, ix.cluster_tile_off, ix.D_pad, ix.tile_size)
    ix.tile_orig_ids = _to_device(bins["tile_orig_ids"], dev)
    ix.vec_Ar = _to_device(bins["vec_Ar"], dev)
    ix.r_vec_sorted = _to_device(bins["r_vec_sorted"], dev)
    ix.fine_codes = _to_device(bins["fine_codes"], dev) if "fine_codes" in bins else None
    ix.fine_qp = _to_device(bins["fine_qp"], dev) if "fine_qp" in bins else None
    ix.max_batch, ix.max_nprobe = int(max_batch), int(max_nprobe)
    ix._fill_cluster_bounds()
    ix._alloc_buffers()
    if dev.type == "cuda":
        torch.cuda.synchronize(dev)
    ix.build_time_s = 0.0
    ix.load_time_s = time.perf_counter() - t0
    return ix
