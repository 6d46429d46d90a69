"""Pipelined search of a query stream held in host memory.

The reference searches one device-resident batch per call and leaves upload and readback to
its callers (benchmarks/phase4a_suite.py:280-342).  ``SearchPipeline`` serves a query set of
any size from host memory: it splits it into batches and keeps ``depth`` batches in flight,
each on its own HIP stream with its own pinned staging buffers, device buffers and library
workspace.  On one stream a batch runs upload -> search -> readback in order; across streams
the batches overlap, so one batch's copies and its PCIe-bound stages (the exact refinement of
an out-of-core base) run beside another batch's HBM-bound scans.  All streams have the default
priority.  Results are identical to searching each batch alone: every batch's kernels read
only its own buffers and the shared read-only index.

Ordering with the caller's work: every slot stream waits for the caller's current stream when
``run`` starts, so an index whose build kernels (cluster bounds, derived layouts) are still
queued there is complete before any batch reads it.  ``close`` (or leaving a ``with`` block)
drains the slots and frees their workspaces.
"""
import numpy as np
import torch

from . import _lib
from . import ext as _ext


class _Slot:
    def __init__(self, dev, batch, D, k):
        self.stream = torch.cuda.Stream(device=dev)
        self.host_q = torch.empty((batch, D), dtype=torch.float32, pin_memory=True)
        self.host_d = torch.empty((batch, k), dtype=torch.float32, pin_memory=True)
        self.host_i = torch.empty((batch, k), dtype=torch.int64, pin_memory=True)
        # allocated on the slot's own stream, the only stream that writes them
        with torch.cuda.stream(self.stream):
            self.dev_q = torch.empty((batch, D), dtype=torch.float32, device=dev)
            self.dev_d = torch.empty((batch, k), dtype=torch.float32, device=dev)
            self.dev_i = torch.empty((batch, k), dtype=torch.int64, device=dev)
        self.done = torch.cuda.Event()
        self.pending = None  # (start, end) of the batch whose results are in flight


class SearchPipeline:
    """``run(xq)`` searches every row of a host query matrix in batches of ``batch`` rows with
    ``depth`` batches in flight; returns (distances [Q, k] float32, ids [Q, k] int64) as numpy
    arrays.  Search options as ``TridentV4Index.search``."""

    def __init__(self, ix, nprobe: int, k: int, batch: int, depth: int = 2, mode: int = 2,
                 ub_seed=None, use_l1: int = 0, route: int = 0, rerank_m: int = 0):
        if depth < 1 or batch < 1:
            raise ValueError("depth and batch must be >= 1")
        if ix.dev.type != "cuda":
            raise ValueError("the pipeline needs a device index")
        self.ix, self.nprobe, self.k, self.batch, self.depth = ix, int(nprobe), int(k), int(batch), int(depth)
        self.mode, self.use_l1, self.route, self.rerank_m = int(mode), int(use_l1), int(route), int(rerank_m)
        self.ub_seed = _ext.env_ub_seed() if ub_seed is None else int(ub_seed)
        if self.nprobe < 1 or self.nprobe > ix.nlist:
            raise ValueError(f"nprobe {nprobe} outside [1, nlist={ix.nlist}]")
        self._view = ix.view()
        self._slots = [_Slot(ix.dev, self.batch, ix.D, self.k) for _ in range(self.depth)]

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
        return False

    def close(self) -> None:
        """Wait for the slots' streams and free their library workspaces (each slot stream
        holds one, sized for a full batch)."""
        for slot in self._slots:
            slot.stream.synchronize()
            _ext.release_workspace(self.ix.dev, slot.stream)
            slot.pending = None

    def _drain(self, slot, out_d, out_i):
        if slot.pending is None:
            return
        slot.done.synchronize()
        s, e = slot.pending
        out_d[s:e] = slot.host_d[:e - s].numpy()
        out_i[s:e] = slot.host_i[:e - s].numpy()
        slot.pending = None

    def run(self, xq):
        xq = np.ascontiguousarray(xq.numpy() if isinstance(xq, torch.Tensor) else xq, np.float32)
        if xq.ndim != 2 or xq.shape[1] != self.ix.D:
            raise ValueError(f"queries must be [Q, {self.ix.D}] float32")
        Q = xq.shape[0]
        out_d = np.empty((Q, self.k), np.float32)
        out_i = np.empty((Q, self.k), np.int64)
        caller = torch.cuda.current_stream(self.ix.dev)
        for slot in self._slots:  # the index and anything the caller queued come first
            slot.stream.wait_stream(caller)
        for b, s in enumerate(range(0, Q, self.batch)):
            e = min(Q, s + self.batch)
            n = e - s
            slot = self._slots[b % self.depth]
            self._drain(slot, out_d, out_i)  # this slot's previous batch is read back first
            slot.host_q[:n].numpy()[:] = xq[s:e]
            st = slot.stream
            with torch.cuda.stream(st):
                slot.dev_q[:n].copy_(slot.host_q[:n], non_blocking=True)
                _ext.search_view(self._view, slot.dev_q[:n], self.nprobe, slot.dev_d[:n], slot.dev_i[:n],
                                 mode=self.mode, ub_seed=self.ub_seed, use_l1=self.use_l1, route=self.route,
                                 rerank_m=self.rerank_m, stream=st)
                slot.host_d[:n].copy_(slot.dev_d[:n], non_blocking=True)
                slot.host_i[:n].copy_(slot.dev_i[:n], non_blocking=True)
                slot.done.record(st)
            slot.pending = (s, e)
        for slot in self._slots:
            self._drain(slot, out_d, out_i)
        return out_d, out_i
