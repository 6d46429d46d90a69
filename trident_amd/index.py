"""Index layout producer and search wrapper with the reference's Python API.

``SharedClusterStorage`` and ``TridentV4Index`` mirror benchmarks/phase4a_suite.py:75-342
(``choose_tile`` :61-62): same constructor arguments, same device tensors, same
``search(...) -> (topk_d, topk_i, kern_ms)``.  The build runs as torch ops on the index
device (the GPU at scale, in the manner of scripts/phase7_step2_gpu_build_verify.py:68-208)
instead of per-cluster Python loops.

What differs, and why:
* Rotation map.  The query rotation the kernels apply is x -> x R + b with R and b exactly the
  float32 values stored in W_combined / b_combined, evaluated in float64.  The base is rotated
  with the same map (float64 GEMM), so base and query agree up to float64 rounding; the
  orthogonality defect of the float32 R is measured once (``rot_sq_min``, ``rot_sq_max``,
  squared extreme singular values) and enters the bounds as a factor.
* eps is rigorous: eps[c, d] >= max over the cluster of |x_rot(exact) - (vmin + code delta)|,
  computed in float64 and rounded up, plus the float64 rotation error bound.  The production
  reference uses 0.5001 * delta (phase4a_suite.py:179), which does not bound the float32
  rounding of the rotated coordinates; the strict variant it cites
  (benchmarks/phase3a_benchmark.py:302) plays the same role as this one.
* Codes follow the reference's closed form: code = clip(round_half_even((x32 - vmin) / delta),
  0, 255) with delta = max((vmax - vmin) / 255, 1e-12) in float32 (phase4a_suite.py:163-176).
* K is explicit (``k=``); output buffers are [max_batch, k].
"""
import math
import time
from typing import Optional

import numpy as np
import torch

import ctypes

from . import _lib
from . import ext as _ext

_U53 = 2.0 ** -53


def cell_block(D_pad: int) -> int:
    """Slots per contiguous block of sq8_cells: the batched route's scan block (64 vectors up to
    256 dims, 16 beyond)."""
    return 64 if D_pad <= 256 else 16


def choose_tile(dim: int) -> int:
    """Tile rule of benchmarks/phase4a_suite.py:61-62."""
    return 256 if dim >= 256 else 64


def _as_tensor(x, device, dtype):
    if isinstance(x, torch.Tensor):
        return x.to(device=device, dtype=dtype)
    return torch.as_tensor(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


# Slice length of the seeding pass's units on the narrow layout (kSplitVecNarrow in
# csrc/kernels.hpp): the seeding pass scans the first slice of each seeding cluster.
SEED_SLICE_ROWS = 2048
# Rows per seeding slice for rows ordered by residual norm (TridentIndexView.seed_rows): on
# histogram-like data with ~6,100 rows per cluster (configs[4]'s shape) the first 1024 rows of a
# cluster seed a threshold 1.044x the K-th distance within the whole cluster (seed_order_scores)
# against 1.032x for 2048 rows, and the seeding pass reads half the codes.
SEED_ROWS_RESIDUAL = 1024


def seed_order_scores(xb, lid: torch.Tensor, r: torch.Tensor, nlist: int, sv: int = SEED_SLICE_ROWS,
                      K: int = 10, samples: int = 512, seed: int = 0) -> dict:
    """How well a cluster's first slice seeds the threshold under each within-cluster order:
    for up to ``samples`` database rows taken as queries (a fixed random sample), the K-th
    smallest distance among the first slice of the row's own cluster (the row itself left out)
    over the K-th smallest among the whole cluster, averaged: {"id": ..., "residual": ...} (1 is
    perfect; larger is a looser seeded threshold).  Slices as the search cuts them: S =
    min(8, ceil(n / sv)) slices of ceil(n / S) rows rounded up to 64."""
    dev = lid.device
    N = int(lid.numel())
    order_id = torch.argsort(lid, stable=True)
    by_r = torch.argsort(r, stable=True)
    order_r = by_r[torch.argsort(lid[by_r], stable=True)]
    del by_r
    off = torch.zeros(nlist + 1, dtype=torch.int64, device=dev)
    off[1:] = torch.cumsum(torch.bincount(lid, minlength=nlist), 0)
    off = off.cpu().tolist()
    g = torch.Generator(device="cpu").manual_seed(seed)
    picks = torch.randint(0, N, (min(samples, N),), generator=g).tolist()
    lid_c = lid.cpu() if N <= (1 << 24) else None

    def rows(idx):
        return xb[idx.to(xb.device)].to(dev, torch.float32)

    tot = {"id": 0.0, "residual": 0.0}
    used = 0
    for i in picks:
        c = int(lid_c[i]) if lid_c is not None else int(lid[i])
        a, b = off[c], off[c + 1]
        n = b - a
        if n <= K + 1:
            continue
        S = max(1, min(8, -(-n // sv)))
        L = min(n, (-(-n // S) + 63) // 64 * 64)
        x = rows(torch.tensor([i], device=dev))
        used += 1
        for name, order in (("id", order_id), ("residual", order_r)):
            idx = order[a:b]
            d = ((rows(idx) - x) ** 2).sum(1, dtype=torch.float64)
            d[idx == i] = math.inf
            tt = float(torch.kthvalue(d, K).values)
            ts = float(torch.kthvalue(d[:L], K).values) if L > K else math.inf
            tot[name] += (ts / tt) if tt > 0 else (1.0 if ts == 0 else 2.0)
    return {k: v / max(used, 1) for k, v in tot.items()}


def round_up_f32(x64: torch.Tensor) -> torch.Tensor:
    """Smallest float32 >= each float64 value."""
    x32 = x64.to(torch.float32)
    low = x32.to(torch.float64) < x64
    if bool(low.any()):
        x32 = torch.where(low, torch.nextafter(x32, torch.full_like(x32, math.inf)), x32)
    return x32


def cells_from_packed(sq8_packed: torch.Tensor, D_pad: int, T: int) -> torch.Tensor:
    """The batched route's code cells from the reference tile packing: cell (t, b, g, v) = dims
    16 g .. 16 g + 15 of slot b V + v of tile t (words 4 g .. 4 g + 3 of sq8_packed[t, :, slot]),
    every byte c stored as c ^ 0x80, V = cell_block(D_pad) slots per contiguous block."""
    dev = sq8_packed.device
    tiles = int(sq8_packed.numel()) // ((D_pad // 4) * T)
    packed = sq8_packed.view(tiles, D_pad // 4, T)
    G16, V = D_pad // 16, cell_block(D_pad)
    cells = torch.empty((tiles, T // V, G16, V, 4), device=dev, dtype=torch.int32)
    flip = torch.tensor(-0x7f7f7f80, dtype=torch.int32, device=dev)  # 0x80808080
    tstep = max(1, (1 << 24) // max(T * (D_pad // 4), 1))
    for ts in range(0, tiles, tstep):
        te = min(tiles, ts + tstep)
        cells[ts:te] = packed[ts:te].view(te - ts, G16, 4, T // V, V).permute(0, 3, 1, 4, 2) ^ flip
    return cells


def packed_from_cells(sq8_cells: torch.Tensor, D_pad: int, T: int) -> torch.Tensor:
    """The reference tile packing [tiles, D_pad/4, T] from the batched route's cells (the
    inverse of ``cells_from_packed``)."""
    dev = sq8_cells.device
    G16, V = D_pad // 16, cell_block(D_pad)
    tiles = int(sq8_cells.numel()) // (G16 * T * 4)
    cells = sq8_cells.view(tiles, T // V, G16, V, 4)
    packed = torch.empty((tiles, D_pad // 4, T), device=dev, dtype=torch.int32)
    flip = torch.tensor(-0x7f7f7f80, dtype=torch.int32, device=dev)  # 0x80808080
    tstep = max(1, (1 << 24) // max(T * (D_pad // 4), 1))
    for ts in range(0, tiles, tstep):
        te = min(tiles, ts + tstep)
        packed[ts:te] = (cells[ts:te].permute(0, 2, 4, 1, 3) ^ flip).reshape(te - ts, D_pad // 4, T)
    return packed


def derive_vec_cn(sq8_cells: torch.Tensor, cluster_vec_off, cluster_tile_off, D_pad: int, T: int,
                  chunk_tiles: int = 1 << 14) -> torch.Tensor:
    """Per-row code norms [N] float32 in sorted order: sqrt(sum_d (code_d - 128)^2) over the
    D_pad dims, rounded up (the sum is an exact integer, the float64 root is raised by 2^-50
    before the upward rounding), from the cells (whose bytes are code - 128 as int8).  The
    lower-bound pass bounds the lo weight plane's share of a row's sum by this norm times the
    plane's norm (Cauchy-Schwarz)."""
    dev = sq8_cells.device
    G16, V = D_pad // 16, cell_block(D_pad)
    tiles = int(sq8_cells.numel()) // (G16 * T * 4)
    cells = sq8_cells.view(tiles, T // V, G16, V, 4)
    per_slot = torch.empty((tiles, T), device=dev, dtype=torch.float32)
    for ts in range(0, tiles, chunk_tiles):
        te = min(tiles, ts + chunk_tiles)
        c8 = cells[ts:te].contiguous().view(torch.int8).view(te - ts, T // V, G16, V, 16).to(torch.int32)
        ssq = (c8 * c8).sum(dim=(2, 4)).reshape(te - ts, T)   # exact: <= 2^14 D_pad
        per_slot[ts:te] = round_up_f32(torch.sqrt(ssq.double()) * (1.0 + 2.0 ** -50))
    vec_off = cluster_vec_off.to(dev, torch.int64)
    tile_off = cluster_tile_off.to(dev, torch.int64)
    N = int(vec_off[-1])
    counts = vec_off[1:] - vec_off[:-1]
    lid = torch.repeat_interleave(torch.arange(counts.numel(), device=dev), counts)
    local = torch.arange(N, device=dev) - vec_off[lid]
    tile = tile_off[lid] + torch.div(local, T, rounding_mode="floor")
    return per_slot[tile, local % T].contiguous()


def derive_vec_Ar(sq8_packed, cluster_vec_off, cluster_tile_off, xb_sorted, W_combined, b_combined,
                  vmin, delta, per_cluster_sq8: int, nlist: int, T: int, chunk_rows: int = 1 << 20):
    """The batched route's per-vector scalars [N, 2] of any index in the reference layout, from
    its own tensors: A = sum_d (code_d delta_d)^2 (rounded down after a 1e-13 margin) and
    r >= |x R + b - x_hat| with R, b the float32 rotation stored in W_combined / b_combined (the
    map the query path applies), x_hat = vmin + code delta from sq8_packed, plus the float64
    rotation error bound (rounded up).  r is measured on the data, so it holds whatever rotation
    or eps produced the codes (the reference quantises a float64 rotation with eps = 0.5001
    delta)."""
    dev = sq8_packed.device
    N, D = int(xb_sorted.shape[0]), int(xb_sorted.shape[1])
    D_pad = int(W_combined.shape[1]) - nlist
    R = W_combined[:, nlist:nlist + D].to(dev, torch.float64)
    b = b_combined.reshape(-1)[nlist:nlist + D].to(dev, torch.float64)
    colabs = R.abs().sum(0)
    rot_err_coef = (D + 2) * 2.0 * _U53
    vec_off = cluster_vec_off.to(dev, torch.int64)
    tile_off = cluster_tile_off.to(dev, torch.int64)
    counts = vec_off[1:] - vec_off[:-1]
    lid = torch.repeat_interleave(torch.arange(nlist, device=dev), counts)
    local = torch.arange(N, device=dev) - vec_off[lid]
    tile = tile_off[lid] + torch.div(local, T, rounding_mode="floor")
    slot = local % T
    packed = sq8_packed.view(-1, D_pad // 4, T)
    rows = nlist if per_cluster_sq8 else 1
    vm_all = vmin.reshape(rows, D_pad).to(dev, torch.float64)
    dl_all = delta.reshape(rows, D_pad).to(dev, torch.float64)
    out = torch.empty((N, 2), device=dev, dtype=torch.float32)
    for s in range(0, N, chunk_rows):
        e = min(N, s + chunk_rows)
        codes = packed[tile[s:e], :, slot[s:e]].contiguous().view(torch.uint8)   # [n, D_pad]
        ci = lid[s:e] if per_cluster_sq8 else torch.zeros(e - s, dtype=torch.int64, device=dev)
        cdl = codes.double() * dl_all[ci]
        xhat = vm_all[ci] + cdl
        x = xb_sorted[s:e].to(dev, torch.float64)
        xr = torch.zeros((e - s, D_pad), device=dev, dtype=torch.float64)
        xr[:, :D] = x @ R + b
        rerr = rot_err_coef * (x.abs().amax(1, keepdim=True) * colabs + b.abs())
        a64 = (cdl * cdl).sum(1) * (1.0 - 1e-13)
        r = torch.sqrt(((xr - xhat) ** 2).sum(1)) + torch.sqrt((rerr ** 2).sum(1))
        out[s:e, 0] = -round_up_f32(-a64)
        out[s:e, 1] = round_up_f32(r * (1.0 + 1e-12) + 1e-300)
    return out


class PinnedHostBuffer:
    """Device-mapped pinned host memory from ``hipHostMalloc`` (C ABI), viewed as a CPU tensor.

    Replaces the torch ``pin_memory=True`` buffer of the out-of-core engine
    (benchmarks/phase8_ooc_100m_4080.py:501-507): torch's caching host allocator rounds large
    requests up, hipHostMalloc gives exactly the bytes asked for.
    """

    def __init__(self, shape, dtype=torch.float32, owner=None):
        self._owner = owner  # object whose xb_sorted / xb_sorted_u8 is this buffer's tensor
        self.children = []   # buffers freed with this one
        nbytes = int(np.prod(shape)) * torch.empty(0, dtype=dtype).element_size()
        ptr = ctypes.c_void_p()
        _lib.check(_lib.lib().trident_host_alloc_mapped(ctypes.c_size_t(max(nbytes, 1)), ctypes.byref(ptr)),
                   "trident_host_alloc_mapped")
        self._ptr = ptr.value
        self.nbytes = nbytes
        np_dtype = {torch.float32: np.float32, torch.int32: np.int32, torch.uint8: np.uint8}[dtype]
        buf = (ctypes.c_char * max(nbytes, 1)).from_address(self._ptr)
        arr = np.frombuffer(buf, dtype=np_dtype, count=int(np.prod(shape))).reshape(shape)
        self.tensor = torch.from_numpy(arr)

    def free(self):
        """Releases the host memory.  The owning storage's ``xb_sorted`` (a view of it) is
        cleared first, so nothing keeps a tensor over freed memory; every search using that
        storage must have completed (synchronise its stream before freeing)."""
        for c in self.children:
            c.free()
        self.children = []
        if self._ptr:
            for attr in ("xb_sorted", "xb_sorted_u8"):
                if self._owner is not None and getattr(self._owner, attr, None) is self.tensor:
                    setattr(self._owner, attr, None)
            self.tensor = None
            _lib.lib().trident_host_free(ctypes.c_void_p(self._ptr))
            self._ptr = None


class SharedClusterStorage:
    """Cluster-sorted base (reference benchmarks/phase4a_suite.py:75-92).

    ``xb_placement="device"`` keeps the FP32 base in HBM; ``"host"`` puts it in device-mapped
    pinned host memory (the out-of-core mode) while ids and offsets stay on the device.  With
    ``host_u8`` (the default) a host base whose every value is an integer in [0, 255] (u8
    descriptors such as SIFT / BIGANN stored as float32) and D a multiple of 16 also gets an
    exact uint8 copy in host memory, ``xb_sorted_u8`` (N * D more bytes, freed with the base):
    the exact refines read their rows from it, a quarter of the PCIe bytes for the same
    distances.

    Within a cluster, rows follow one of two orders; search results do not depend on it, but
    the seeding pass scans the first slice of each seeding cluster, so the order decides how
    tight the seeded threshold is:
      ``within="id"``: by original id (the reference's order), so a slice is an unbiased sample
        of its cluster;
      ``within="residual"``: by residual norm |x - c| ascending (ties by original id), so the
        first slice holds the rows nearest the centroid, whose expected distance to a query of
        the cluster is the smallest (|q - c|^2 + |x - c|^2 on average).  On blob-like clusters
        (configs[4]'s histogram data) the seeded threshold drops from 1.10x to 1.03x the true
        K-th neighbour distance; on elongated ones queries far from the core get no
        near seeds (up to 190x);
      ``within="auto"`` (the default): ``seed_order_scores`` on a sample of the data picks
        "residual" when its score is at least 1 % better, else "id".  ``self.within`` records
        the order taken.
    """

    def __init__(self, xb_raw, list_ids, r_vec, nlist: int, device="cuda:0", xb_placement: str = "device",
                 within: str = "auto", host_u8: bool = True):
        self.dev = torch.device(device)
        lid = _as_tensor(list_ids, self.dev, torch.int64)
        self.N = int(lid.numel())
        self.nlist = int(nlist)
        if within not in ("auto", "residual", "id"):
            raise ValueError(f"within={within!r}: 'auto', 'residual' or 'id'")
        xb = xb_raw if isinstance(xb_raw, torch.Tensor) else torch.as_tensor(np.ascontiguousarray(xb_raw))
        rv = None if r_vec is None else _as_tensor(r_vec, self.dev, torch.float32)
        self.seed_scores = None
        if rv is None:
            within = "id"
        elif within == "auto":
            sc = self.seed_scores = seed_order_scores(xb, lid, rv, self.nlist)
            within = "residual" if sc["residual"] < 0.99 * sc["id"] else "id"
        self.within = within
        if within == "residual":
            by_r = torch.argsort(rv, stable=True)
            sort_perm = by_r[torch.argsort(lid[by_r], stable=True)]
            del by_r
        else:
            sort_perm = torch.argsort(lid, stable=True)
        self.D = int(xb.shape[1])
        self.placement = xb_placement
        self._host_buf = None
        if xb_placement == "host":
            self._host_buf = PinnedHostBuffer((self.N, self.D), torch.float32, owner=self)
            self.xb_sorted = self._host_buf.tensor
            u8 = self._u8_start(host_u8)
            step = 1 << 22
            perm_cpu = sort_perm.cpu()
            for s in range(0, self.N, step):
                idx = perm_cpu[s:s + step]
                rows = xb[idx.to(xb.device)]
                u8 = self._u8_put(u8, s, rows)
                self.xb_sorted[s:s + step] = rows.to("cpu", torch.float32)
            self._u8_finish(u8)
        else:
            self.xb_sorted_u8 = None
            self.xb_sorted = xb.to(self.dev, torch.float32)[sort_perm].contiguous()
        self.orig_ids_sorted = sort_perm.to(torch.int32).contiguous()
        counts = torch.bincount(lid, minlength=nlist).to(torch.int32)
        vec_off = torch.zeros(nlist + 1, dtype=torch.int32, device=self.dev)
        vec_off[1:] = torch.cumsum(counts, 0).to(torch.int32)
        self.cluster_vec_off = vec_off
        self.counts = counts.cpu().numpy()
        self.sort_perm = self.orig_ids_sorted.cpu().numpy()
        self.list_ids_sorted = lid[sort_perm].to(torch.int32).contiguous()
        self.r_vec_sorted = None if r_vec is None else _as_tensor(r_vec, self.dev, torch.float32)[sort_perm].contiguous()

    def _u8_start(self, host_u8: bool):
        """The buffer of the base's uint8 copy (xb_sorted_u8), or None: kept for a base in host
        memory with D a multiple of 16 while every value is an integer in [0, 255]."""
        self.xb_sorted_u8 = None
        if not host_u8 or self.placement != "host" or self.D % 16 != 0 or self.N == 0:
            return None
        return PinnedHostBuffer((self.N, self.D), torch.uint8, owner=self)

    @staticmethod
    def _u8_put(buf, s: int, rows: torch.Tensor):
        """Writes sorted rows [s, s + len(rows)) into the uint8 copy; at the first value that
        uint8 does not hold exactly the copy is freed (returns None)."""
        if buf is None:
            return None
        r = rows.to(torch.float32)
        if not bool(((r >= 0) & (r <= 255) & (r == torch.round(r))).all()):
            buf.free()
            return None
        buf.tensor[s:s + r.shape[0]] = r.to(torch.uint8).cpu()
        return buf

    def _u8_finish(self, buf):
        if buf is not None:
            self._host_buf.children.append(buf)  # freed with the FP32 base
            self.xb_sorted_u8 = buf.tensor

    @classmethod
    def from_sorted(cls, xb_sorted, sort_perm, vec_off, device="cuda:0", xb_placement: str = "device",
                    xb_raw=None, chunk_rows: int = 1 << 22, host_u8: bool = True):
        """Storage of an already sorted layout (a saved index): rows come from ``xb_sorted``
        ([N, D], e.g. a memmap) or, when it is None, from ``xb_raw[sort_perm]``; nothing is
        re-sorted.  ``sort_perm`` [N] holds the original id of each sorted row.  ``within`` is
        "id" (set it to "residual" for a layout ordered by residual norm within clusters)."""
        self = cls.__new__(cls)
        self.dev = torch.device(device)
        self.within, self.seed_scores = "id", None
        perm = np.ascontiguousarray(sort_perm, np.int64)
        voff = np.ascontiguousarray(vec_off, np.int64)
        self.N, self.nlist = int(perm.shape[0]), int(voff.shape[0]) - 1
        src = xb_sorted if xb_sorted is not None else xb_raw
        self.D = int(src.shape[1])
        self.placement = xb_placement
        self._host_buf = None
        if xb_placement == "host":
            self._host_buf = PinnedHostBuffer((self.N, self.D), torch.float32, owner=self)
            self.xb_sorted = self._host_buf.tensor
        else:
            self.xb_sorted = torch.empty((self.N, self.D), device=self.dev, dtype=torch.float32)
        u8 = self._u8_start(host_u8)
        for s in range(0, self.N, chunk_rows):
            e = min(self.N, s + chunk_rows)
            if xb_sorted is not None:
                rows = torch.from_numpy(np.array(xb_sorted[s:e], dtype=np.float32))
            else:
                xr = xb_raw if isinstance(xb_raw, torch.Tensor) else torch.as_tensor(np.asarray(xb_raw))
                rows = xr[torch.as_tensor(perm[s:e]).to(xr.device)].to(torch.float32)
            u8 = self._u8_put(u8, s, rows)
            self.xb_sorted[s:e] = rows.to(self.xb_sorted.device)
        self._u8_finish(u8)
        self.orig_ids_sorted = torch.as_tensor(perm.astype(np.int32)).to(self.dev)
        self.cluster_vec_off = torch.as_tensor(voff.astype(np.int32)).to(self.dev)
        counts = (voff[1:] - voff[:-1]).astype(np.int32)
        self.counts = counts
        self.sort_perm = perm.astype(np.int32)
        self.list_ids_sorted = torch.repeat_interleave(
            torch.arange(self.nlist, dtype=torch.int32), torch.as_tensor(counts.astype(np.int64))).to(self.dev)
        self.r_vec_sorted = None
        return self

    def xb_sorted_host(self) -> np.ndarray:
        return self.xb_sorted.cpu().numpy() if self.xb_sorted.device.type != "cpu" else self.xb_sorted.numpy()


class TridentV4Index:
    """PCA-rotated, per-cluster SQ8 index in the wave64 tile layout plus search buffers.

    Layout (all on the index device; see the module docstring for the arithmetic):
      sq8_packed   int32 [tiles, D_pad/4, T]: word [t, d4, s] packs dims 4*d4..4*d4+3 of slot
                   s of tile t, byte 0 = dim 4*d4 (reference packing :221-228); for T = 64 a
                   wave's 64 lanes read one contiguous 256-byte row per d4.
      sq8_cells    int32 [tiles, T/V, D_pad/16, V, 4], V = cell_block(D_pad) (64, or 16 past
                   256 dims): the same codes as 16-byte cells (16 dims of one slot), bytes XOR
                   0x80, every V-slot block contiguous -- the batched route's matrix-core operand
                   layout (one scan block is one contiguous run).
      vec_cn       f32 [N] sorted order: |code - 128|_2 per row, rounded up (the lower-bound
                   pass's Cauchy-Schwarz allowance for its lo weight plane)
      tile_orig_ids int32 [tiles, T] (-1 padded), tile_r_minmax f32 [tiles, 2]
      cluster_tile_off int32 [nlist + 1]; vmin / delta / eps_pad f32 [nlist or 1, D_pad]
      blk_bounds4  int32 [nb + 1] (32-dim blocks, or the variable scheme of :233-247)
      W_combined [D, nlist + D_pad] = [-2 C^T | R | 0], b_combined = [|c|^2 | b | 0]
      cent_band    the centroids for the matrix-core coarse pass (rows, tile layout, norms,
                   max norm; ext.centroid_band_layouts)
    """

    def __init__(self, storage: SharedClusterStorage, centroids, mean64, R64, tile_size: int = 256,
                 per_cluster_sq8: int = 1, use_pca: int = 1, var_block: int = 0, max_batch: int = 1024,
                 max_nprobe: int = 512, device="cuda:0", k: int = 10, chunk_rows: int = 1 << 20,
                 fine_level: Optional[bool] = None):
        """``fine_level`` (default: when the base is in host memory) also builds the fine level
        (``fine_codes``, ``fine_qp``: 16-bit codes of every rotated row on its own grid) that the
        out-of-core search bounds its rows with."""
        t_start = time.perf_counter()
        if fine_level is None:
            fine_level = getattr(storage, "placement", "device") == "host"
        self.storage = storage
        self.dev = torch.device(device)
        self.N, self.D, self.nlist = storage.N, storage.D, storage.nlist
        self.tile_size = int(tile_size)
        assert self.tile_size % 64 == 0, "tile_size must be a multiple of 64"
        self.per_cluster_sq8 = int(per_cluster_sq8)
        self.use_pca = int(use_pca)
        self.var_block = int(var_block)
        self.W_tile = self.tile_size // 32
        self.D_pad = ((self.D + 31) // 32) * 32
        self.D4 = self.D_pad // 4
        self.k = int(k)
        dev, N, D, D_pad, nlist, T = self.dev, self.N, self.D, self.D_pad, self.nlist, self.tile_size

        # ---- rotation map x -> x R + b, R and b exactly the stored float32 values ----
        if use_pca:
            R32 = _as_tensor(R64, "cpu", torch.float64).to(torch.float32)
            mean = _as_tensor(mean64, "cpu", torch.float64)
        else:
            R32 = torch.eye(D, dtype=torch.float32)
            mean = torch.zeros(D, dtype=torch.float64)
        b32 = (-(mean @ R32.to(torch.float64))).to(torch.float32)
        s = torch.linalg.svdvals(R32.to(torch.float64))
        self.rot_sq_min = float(s.min()) ** 2 * (1.0 - 1e-12)
        self.rot_sq_max = float(s.max()) ** 2 * (1.0 + 1e-12)
        R64d = R32.to(dev, torch.float64)
        b64d = b32.to(dev, torch.float64)
        colabs = R64d.abs().sum(0)                      # sum_j |R_jd|
        rot_err_coef = (D + 2) * 2.0 * _U53             # generous float64 dot-product bound

        # ---- coarse / fused projection matrices ----
        cen = _as_tensor(centroids, dev, torch.float32).contiguous()
        self.centroids = cen
        c_norm_sq = (cen.double() ** 2).sum(1).to(torch.float32)
        self.W_coarse_only = (-2.0 * cen.t()).contiguous()
        self.b_coarse_only = c_norm_sq.unsqueeze(0).contiguous()
        total_cols = nlist + D_pad
        self.W_combined = torch.zeros((D, total_cols), device=dev, dtype=torch.float32)
        self.b_combined = torch.zeros((1, total_cols), device=dev, dtype=torch.float32)
        self.W_combined[:, :nlist] = self.W_coarse_only
        self.W_combined[:, nlist:nlist + D] = R32.to(dev)
        self.b_combined[0, :nlist] = c_norm_sq
        self.b_combined[0, nlist:nlist + D] = b32.to(dev)
        self.cent_band = _ext.centroid_band_layouts(self.W_combined, nlist)

        # ---- rotate, quantise, bound (chunked over sorted rows) ----
        vec_off = storage.cluster_vec_off.to(torch.int64)
        counts = (vec_off[1:] - vec_off[:-1])
        lid_sorted = storage.list_ids_sorted.to(dev, torch.int64)
        xb_src = storage.xb_sorted
        rows_dev = lambda s, e: xb_src[s:e].to(dev, torch.float32)

        def rotate(s, e):
            x = rows_dev(s, e)
            xr64 = torch.zeros((e - s, D_pad), device=dev, dtype=torch.float64)
            xr64[:, :D] = x.double() @ R64d + b64d
            err = torch.zeros_like(xr64)
            err[:, :D] = rot_err_coef * (x.double().abs().amax(1, keepdim=True) * colabs + b64d.abs())
            return xr64, err

        rows = nlist if self.per_cluster_sq8 else 1
        vmin = torch.full((rows, D_pad), math.inf, device=dev, dtype=torch.float32)
        vmax = torch.full((rows, D_pad), -math.inf, device=dev, dtype=torch.float32)
        for s in range(0, N, chunk_rows):
            e = min(N, s + chunk_rows)
            xr32 = rotate(s, e)[0].to(torch.float32)
            if self.per_cluster_sq8:
                idx = lid_sorted[s:e].unsqueeze(1).expand(-1, D_pad)
                vmin.scatter_reduce_(0, idx, xr32, reduce="amin", include_self=True)
                vmax.scatter_reduce_(0, idx, xr32, reduce="amax", include_self=True)
            else:
                vmin = torch.minimum(vmin, xr32.amin(0, keepdim=True))
                vmax = torch.maximum(vmax, xr32.amax(0, keepdim=True))
        empty = torch.isinf(vmin).all(1, keepdim=True)
        vmin = torch.where(empty, torch.zeros_like(vmin), vmin)
        vmax = torch.where(empty, torch.zeros_like(vmax), vmax)
        delta = torch.clamp((vmax - vmin) / 255.0, min=1e-12)
        delta = torch.where(empty, torch.ones_like(delta), delta)
        codes = torch.empty((N, D_pad), device=dev, dtype=torch.uint8)
        err_max = torch.zeros((rows, D_pad), device=dev, dtype=torch.float64)
        # Per-vector scalars of the batched (matrix-core) bound, sorted order, float32 pairs:
        #   vec_Ar[v, 0] <= A_v * (1 - 1e-13),  A_v = sum_d (code_d * delta_d)^2 (exact products;
        #                   the float64 sum is within D * 2^-53 relative, far inside the margin)
        #   vec_Ar[v, 1] >= r_v >= |x_rot(exact) - x_hat|_2   (quantisation + rotation error)
        # The kernel uses vec_Ar[v, 0] * (1 + 2^-22) >= A_v as the upper value of A_v.
        self.vec_Ar = torch.empty((N, 2), device=dev, dtype=torch.float32)
        # residual norms |x - c(x)| in float64, for the tile band of use_l1 (tile_r_minmax)
        res_norm = torch.empty(N, device=dev, dtype=torch.float64)
        # Fine level: per row, offset = the smallest rotated coordinate (rounded down to float32),
        # step = its range / 65535 (rounded up), code = rint((x_rot - offset) / step) in 16 bits
        # (stored as int16 bit patterns), x_fine = offset + code * step (the product is exact in
        # float64, the sum rounded once, as the kernels compute it) and rho >= |x_rot(exact) -
        # x_fine| (the float64 rotation's error included), rounded up.
        self.fine_codes = torch.empty((N, D_pad), device=dev, dtype=torch.int16) if fine_level else None
        self.fine_qp = torch.zeros((N, 4), device=dev, dtype=torch.float32) if fine_level else None
        for s in range(0, N, chunk_rows):
            e = min(N, s + chunk_rows)
            res_norm[s:e] = torch.sqrt(((rows_dev(s, e).double() - cen[lid_sorted[s:e]].double()) ** 2).sum(1))
            xr64, rerr = rotate(s, e)
            xr32 = xr64.to(torch.float32)
            ci = lid_sorted[s:e] if self.per_cluster_sq8 else torch.zeros(e - s, dtype=torch.int64, device=dev)
            vm, dl = vmin[ci], delta[ci]
            cd = torch.clamp(torch.round((xr32 - vm) / dl), 0.0, 255.0)
            codes[s:e] = cd.to(torch.uint8)
            cdl = cd.double() * dl.double()
            xhat = vm.double() + cdl
            err = (xr64 - xhat).abs() + rerr
            idx = ci.unsqueeze(1).expand(-1, D_pad)
            err_max.scatter_reduce_(0, idx, err, reduce="amax", include_self=True)
            a64 = (cdl * cdl).sum(1) * (1.0 - 1e-13)
            self.vec_Ar[s:e, 0] = -round_up_f32(-a64)
            r_q = torch.sqrt(((xr64 - xhat) ** 2).sum(1)) + torch.sqrt((rerr ** 2).sum(1))
            self.vec_Ar[s:e, 1] = round_up_f32(r_q * (1.0 + 1e-12) + 1e-300)
            if fine_level:
                lo = -round_up_f32(-xr64.amin(1))                            # offset <= min
                span = (xr64.amax(1) - lo.double()) / 65535.0
                st = round_up_f32(torch.clamp(span * (1.0 + 2.0 ** -40), min=2.0 ** -100))
                c = torch.clamp(torch.round((xr64 - lo.double().unsqueeze(1)) / st.double().unsqueeze(1)), 0.0, 65535.0)
                self.fine_codes[s:e] = (c - 65536.0 * (c >= 32768.0)).to(torch.int16)
                xf = lo.double().unsqueeze(1) + c * st.double().unsqueeze(1)
                rho = torch.sqrt(((xr64 - xf) ** 2).sum(1)) + torch.sqrt((rerr ** 2).sum(1))
                self.fine_qp[s:e, 0] = lo
                self.fine_qp[s:e, 1] = st
                self.fine_qp[s:e, 2] = round_up_f32(rho * (1.0 + 1e-12) + 1e-300)
        self.vmin_pad = vmin.contiguous()
        self.delta_pad = delta.contiguous()
        self.eps_pad = round_up_f32(err_max * (1.0 + 2.0 ** -20) + 1e-300).contiguous()

        # ---- tiles (vectorised packing) ----
        tile_counts = (counts + T - 1) // T
        self.total_tiles = int(tile_counts.sum().item())
        tile_off = torch.zeros(nlist + 1, dtype=torch.int64, device=dev)
        tile_off[1:] = torch.cumsum(tile_counts, 0)
        self.cluster_tile_off = tile_off.to(torch.int32).contiguous()
        tiles = self.total_tiles
        tile_cid = torch.repeat_interleave(torch.arange(nlist, device=dev), tile_counts)
        tile_local = torch.arange(tiles, device=dev) - tile_off[tile_cid]
        slot = torch.arange(T, device=dev).unsqueeze(0)
        vidx = vec_off[tile_cid].unsqueeze(1) + tile_local.unsqueeze(1) * T + slot
        valid = vidx < vec_off[tile_cid + 1].unsqueeze(1)
        safe = torch.clamp(vidx, 0, max(N - 1, 0))
        oids = storage.orig_ids_sorted.to(dev)
        self.tile_orig_ids = torch.where(valid, oids[safe], torch.full_like(safe, -1).to(torch.int32)).to(torch.int32).contiguous()
        codes32 = codes.view(torch.int32)                    # [N, D4], byte 0 = lowest dim
        self.sq8_packed = torch.zeros((tiles, self.D4, T), device=dev, dtype=torch.int32)
        tstep = max(1, (1 << 24) // max(T * self.D4, 1))
        for ts in range(0, tiles, tstep):
            te = min(tiles, ts + tstep)
            g = codes32[safe[ts:te]]                         # [nt, T, D4]
            g = torch.where(valid[ts:te].unsqueeze(-1), g, torch.zeros_like(g))
            self.sq8_packed[ts:te] = g.permute(0, 2, 1)
        # Batched-route copy: 16-byte cells, every scan block of V slots one contiguous run
        self.sq8_cells = cells_from_packed(self.sq8_packed, D_pad, T)
        self.vec_cn = derive_vec_cn(self.sq8_cells, storage.cluster_vec_off, self.cluster_tile_off, D_pad, T)
        # The tile band (reference :198-230 takes it from the clustering's float32 r_vec): the
        # smallest and largest |x - c| of each tile, measured here in float64 and rounded
        # outward to float32 (an empty tile gets [+inf, -inf]: never reached).
        self.tile_r_minmax = torch.empty((tiles, 2), device=dev, dtype=torch.float32)
        for ts in range(0, tiles, tstep):
            te = min(tiles, ts + tstep)
            r = res_norm[safe[ts:te]]
            v = valid[ts:te]
            rmin = torch.where(v, r, torch.full_like(r, math.inf)).amin(1) * (1.0 - 1e-12)
            rmax = torch.where(v, r, torch.full_like(r, -math.inf)).amax(1) * (1.0 + 1e-12)
            self.tile_r_minmax[ts:te, 0] = -round_up_f32(-rmin)
            self.tile_r_minmax[ts:te, 1] = round_up_f32(rmax)
        # mode 11's per-vector |x - c| (reference r_vec_sorted): the float64 norm rounded to nearest
        self.r_vec_sorted = res_norm.to(torch.float32)
        del codes, codes32, res_norm

        # ---- dimension blocks (reference :231-255) ----
        if var_block:
            if D_pad <= 128:
                blk_dims = [16, 16, 32, 32, 32]
            elif D_pad <= 256:
                blk_dims = [16, 16, 32, 32, 64, 64, 32]
            else:
                blk_dims = [16, 16, 32, 32, 64, 64, 64, 128, 128, 256, 256]
            bounds, cur = [0], 0
            for bd in blk_dims:
                cur += bd
                if cur <= D_pad:
                    bounds.append(cur // 4)
            if bounds[-1] < self.D4:
                bounds.append(self.D4)
        else:
            bounds = [0] + [d // 4 for d in range(32, D_pad + 1, 32)]
            if bounds[-1] < self.D4:
                bounds.append(self.D4)
        self.blk_bounds4 = torch.tensor(bounds, device=dev, dtype=torch.int32)

        # ---- search buffers (reference :257-278, K explicit) ----
        self.max_batch, self.max_nprobe = int(max_batch), int(max_nprobe)
        self._fill_cluster_bounds()
        self._alloc_buffers()
        self.build_time_s = time.perf_counter() - t_start

    def _alloc_buffers(self):
        dev, mb, mnp = self.dev, self.max_batch, self.max_nprobe
        total_cols = self.nlist + self.D_pad
        self.proj_buf = torch.zeros((1, total_cols), device=dev, dtype=torch.float32)
        self.cdists_buf = torch.zeros((1, self.nlist), device=dev, dtype=torch.float32)
        self.probe_cids_buf = torch.zeros((mb, mnp), device=dev, dtype=torch.int32)
        self.probe_dqcs_buf = torch.zeros((mb, mnp), device=dev, dtype=torch.float32)
        z32 = torch.zeros(1, device=dev, dtype=torch.int32)
        zf = torch.zeros(1, device=dev, dtype=torch.float32)
        self.p1_cids_buf = self.p2_cids_buf = self.p1_qids_buf = self.p2_qids_buf = z32
        self.p1_dqcs_buf = self.p2_dqcs_buf = zf
        self.topk_d_buf = torch.zeros((mb, self.k), device=dev, dtype=torch.float32)
        self.topk_i_buf = torch.zeros((mb, self.k), device=dev, dtype=torch.int64)
        self.topm_buf_d = torch.zeros((1, 1), device=dev, dtype=torch.float32)
        self.topm_buf_i = torch.zeros((1, 1), device=dev, dtype=torch.int64)
        self.tau_sq_buf = torch.zeros(mb, device=dev, dtype=torch.float32)
        self.cand_buf_d = torch.zeros((1, 1), device=dev, dtype=torch.float32)
        self.cand_buf_i = torch.zeros((1, 1), device=dev, dtype=torch.int64)
        self.cand_cnt = torch.zeros(mb, device=dev, dtype=torch.int32)

    def set_k(self, k: int):
        if int(k) != self.k:
            self.k = int(k)
            self.topk_d_buf = torch.zeros((self.max_batch, self.k), device=self.dev, dtype=torch.float32)
            self.topk_i_buf = torch.zeros((self.max_batch, self.k), device=self.dev, dtype=torch.int64)

    def sq8_bytes(self) -> int:
        """Bytes of SQ8 codes held in HBM: the reference packing plus, when built, the batched
        route's cells (the same codes regrouped)."""
        n = int(self.sq8_packed.numel()) * 4
        if getattr(self, "sq8_cells", None) is not None:
            n += int(self.sq8_cells.numel()) * 4
        return n

    @property
    def has_packed_codes(self) -> bool:
        return int(self.sq8_packed.numel()) > 0

    def release_packed_codes(self):
        """Frees the reference-packed codes (``sq8_packed``) on the device, keeping the batched
        route's cells (the same codes): mode 2 then runs the batched route only (the per-pair
        route and modes 0 / 1 read the packing and are refused).  ``packed_codes()`` rebuilds
        the packing from the cells when it is needed again (``save_index`` does)."""
        if self.sq8_cells is None:
            raise ValueError("the index has no sq8_cells: the packed codes are its only copy")
        self.sq8_packed = torch.empty(0, dtype=torch.int32, device=self.dev)

    def packed_codes(self) -> torch.Tensor:
        """``sq8_packed`` [tiles, D_pad/4, T] (int32): the device tensor, or, once released, the
        packing rebuilt from the cells (a new device tensor)."""
        if self.has_packed_codes:
            return self.sq8_packed
        return packed_from_cells(self.sq8_cells, self.D_pad, self.tile_size)

    def release_fine_level(self):
        """Drops the fine level (``fine_codes``, ``fine_qp``): an out-of-core search then bounds
        its seeds and survivors with the SQ8 codes alone and reads them from host memory."""
        self.fine_codes = self.fine_qp = None

    def hbm_footprint(self) -> dict:
        """Bytes of every index tensor resident in device memory (the library's workspace and
        the search buffers excluded), by name, plus their total under "total"."""
        st = self.storage
        named = {
            "sq8_packed": self.sq8_packed, "sq8_cells": getattr(self, "sq8_cells", None),
            "tile_orig_ids": self.tile_orig_ids, "tile_r_minmax": self.tile_r_minmax,
            "vec_Ar": getattr(self, "vec_Ar", None), "vec_cn": getattr(self, "vec_cn", None),
            "r_vec_sorted": getattr(self, "r_vec_sorted", None),
            "fine_codes": getattr(self, "fine_codes", None), "fine_qp": getattr(self, "fine_qp", None),
            "cluster_bounds": getattr(self, "cluster_bounds", None),
            "vmin_delta_eps": None, "centroids_and_projection": None,
            "xb_sorted": st.xb_sorted, "orig_ids_sorted": st.orig_ids_sorted,
            "list_ids_sorted": getattr(st, "list_ids_sorted", None),
            "offsets": None,
        }
        out = {}
        for k2, t in named.items():
            if isinstance(t, torch.Tensor) and t.device.type == "cuda":
                out[k2] = int(t.numel() * t.element_size())
        small = lambda ts: sum(int(t.numel() * t.element_size()) for t in ts
                               if isinstance(t, torch.Tensor) and t.device.type == "cuda")
        out["vmin_delta_eps"] = small((self.vmin_pad, self.delta_pad, self.eps_pad))
        out["centroids_and_projection"] = small(
            (self.centroids, self.W_combined, self.b_combined, self.W_coarse_only, self.b_coarse_only)
            + tuple(t for t in (self.cent_band or ()) if isinstance(t, torch.Tensor)))
        out["offsets"] = small((self.cluster_tile_off, st.cluster_vec_off, self.blk_bounds4))
        out = {k2: v for k2, v in out.items() if v}
        out["total"] = sum(out.values())
        return out

    def search(self, xq_gpu: torch.Tensor, nprobe: int, mode: int = 2, use_l1: int = 0, rerank_m: int = 0,
               tile_override: int = 0, warp_refine: int = 1, stats_buf: Optional[torch.Tensor] = None,
               record_kernel_ms: bool = False, k: Optional[int] = None, ub_seed: Optional[int] = None,
               stage_events=None, route: int = 0, p_init: int = -1,
               host_rows_buf: Optional[torch.Tensor] = None):
        """Reference TridentV4Index.search (phase4a_suite.py:280-342) plus ``k=``, ``ub_seed=``,
        ``route=`` (0 auto, 1 per-pair cascade, 2 cluster-batched matrix-core cascade) and
        ``p_init=`` (probes of the first pass per query; -1 = the reference's rule) and
        ``host_rows_buf=`` (int64 [1]: receives the base rows read from host memory)."""
        if k is not None:
            self.set_k(k)
        B = int(xq_gpu.shape[0])
        if B > self.max_batch:
            raise ValueError(f"batch {B} exceeds max_batch={self.max_batch}")
        if nprobe > self.max_nprobe:
            raise ValueError(f"nprobe {nprobe} exceeds max_nprobe={self.max_nprobe}")
        tsize = tile_override if tile_override > 0 else self.tile_size
        topk_d = self.topk_d_buf[:B]
        topk_i = self.topk_i_buf[:B]
        st = self.storage
        kern_ms = _ext.launch_trident_v4_search(
            int(mode), int(tsize), int(use_l1), int(self.per_cluster_sq8), int(rerank_m), int(nprobe),
            xq_gpu, self.W_combined, self.b_combined, self.W_coarse_only, self.b_coarse_only,
            self.proj_buf, self.cdists_buf, self.probe_cids_buf, self.probe_dqcs_buf,
            self.p1_cids_buf, self.p1_qids_buf, self.p1_dqcs_buf,
            self.p2_cids_buf, self.p2_qids_buf, self.p2_dqcs_buf,
            self.sq8_packed, self.tile_orig_ids, self.tile_r_minmax, self.cluster_tile_off,
            st.cluster_vec_off, st.xb_sorted, st.orig_ids_sorted,
            self.vmin_pad, self.delta_pad, self.eps_pad, self.blk_bounds4,
            topk_d, topk_i, self.topm_buf_d, self.topm_buf_i, self.tau_sq_buf,
            self.cand_buf_d, self.cand_buf_i, self.cand_cnt,
            bool(record_kernel_ms), int(warp_refine), stats_buf,
            ub_seed=ub_seed, rot_sq_bounds=(self.rot_sq_min, self.rot_sq_max), stage_events=stage_events,
            p_init=p_init,
            vec_Ar=self.vec_Ar, route=route, sq8_cells=self.sq8_cells, cent_band=self.cent_band,
            r_vec_sorted=self.r_vec_sorted, fine_codes=self.fine_codes, fine_qp=self.fine_qp,
            host_rows=host_rows_buf, cluster_bounds=self.cluster_bounds, vec_cn=getattr(self, "vec_cn", None),
            seed_rows=self.seed_rows, xb_sorted_u8=getattr(st, "xb_sorted_u8", None))
        return topk_d, topk_i, kern_ms

    def view(self):
        """The C-ABI view (TridentIndexView) of this index; it holds raw pointers, so the index
        must outlive it."""
        st = self.storage
        return _ext.make_index_view(
            N=st.N, D=self.D, D_pad=self.D_pad, nlist=self.nlist, tile_size=self.tile_size,
            per_cluster_sq8=self.per_cluster_sq8, W_combined=self.W_combined, b_combined=self.b_combined,
            rot_sq_min=self.rot_sq_min, rot_sq_max=self.rot_sq_max,
            sq8_packed=self.sq8_packed if self.has_packed_codes else None,
            tile_orig_ids=self.tile_orig_ids, tile_r_minmax=self.tile_r_minmax,
            cluster_tile_off=self.cluster_tile_off, cluster_vec_off=st.cluster_vec_off,
            xb_sorted=st.xb_sorted, orig_ids_sorted=st.orig_ids_sorted, vmin=self.vmin_pad,
            delta=self.delta_pad, eps_dim=self.eps_pad, blk_bounds4=self.blk_bounds4, vec_Ar=self.vec_Ar,
            sq8_cells=self.sq8_cells, cent_band=self.cent_band, r_vec_sorted=self.r_vec_sorted,
            fine_codes=self.fine_codes, fine_qp=self.fine_qp,
            cluster_bounds=getattr(self, "cluster_bounds", None), vec_cn=getattr(self, "vec_cn", None),
            seed_rows=self.seed_rows, xb_sorted_u8=getattr(st, "xb_sorted_u8", None))

    @property
    def seed_rows(self) -> int:
        """Rows per seeding slice the batched route scans (TridentIndexView.seed_rows): with rows
        ordered by residual norm within each cluster a cluster's first rows are its best seeds,
        so SEED_ROWS_RESIDUAL of them seed almost as tight a threshold as SEED_SLICE_ROWS; 0
        (the library's 2048-row slices) for the id order."""
        return SEED_ROWS_RESIDUAL if getattr(self.storage, "within", "id") == "residual" else 0

    def _fill_cluster_bounds(self):
        """The batched route's per-cluster constants (A_max, r_max, r_lo), once per index."""
        self.cluster_bounds = None
        if self.dev.type == "cuda":
            self.cluster_bounds = _ext.compute_cluster_bounds(self.view(), self.dev)

    def route_for(self, B: int, nprobe: int, k: Optional[int] = None, route: int = 0, mode: int = 2) -> int:
        """The route (_lib.ROUTE_PAIR / ROUTE_BATCHED) a search of B queries takes (mode 2, or
        mode 10 whose batched route is the float32 matrix-core scan)."""
        view = self.view()
        r = _lib.lib().trident_route_for_mode(ctypes.byref(view), int(mode), int(B), int(k or self.k),
                                              int(nprobe), int(route))
        if r < 0:
            _lib.check(-r, "trident_route_for")
        return int(r)

    # ---- views used by tests / oracle (host copies) ----
    def host_arrays(self):
        st = self.storage
        return dict(
            xb_sorted=st.xb_sorted_host(),
            orig_ids_sorted=st.orig_ids_sorted.cpu().numpy(),
            vec_off=st.cluster_vec_off.cpu().numpy(),
            centroids=self.centroids.cpu().numpy(),
        )
