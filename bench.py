#!/usr/bin/env python3
"""QPS at 100% exact top-10 on one MI355X, with the dominant kernel's roofline and the CPU
baseline.

Workload (default): BASELINE.json configs[4], the largest single-GPU configuration -- N = 1e8
histogram-like descriptors, D = 128 (integer values 0-255 stored as float32), nlist = 16,384,
nprobe = 128, K = 10, B = 10,000 queries; the FP32 base (51.2 GB) in hipHostMalloc-mapped pinned
host memory, read over PCIe for exact distances only; in HBM the SQ8 codes (as the batched
route's cells and the reference packing), ids, per-vector scalars and the 16-bit fine level.
Data and index are generated and built on the GPU first (untimed).  ``--cfg 1..4`` selects an
in-HBM configuration instead.

One step = one full batched search of B queries (front end + seeding pass + lower-bound pass +
exact refine + merge) with the queries already resident in HBM.  W warmup steps, then exactly K
timed steps in R rounds (K / R steps each, bracketed by torch.cuda.synchronize()); ``value`` is
B * K / (total timed seconds), ``rounds`` gives the per-round mean and standard deviation.
Afterwards (untimed):
  * exactness: ids and distances of every query of the batch against the float64 CPU oracle
    (the cluster-major form of the exhaustive scan over the same probes);
  * roofline of the dominant kernel (batched route: the lower-bound pass on the int8 matrix
    cores, 4 * D_pad int8 ops per probed (query, vector) pair -- multiply + add over two
    weight planes -- against the 5.0 POP/s dense int8 peak; per-pair route: SQ8 code bytes at
    full depth against 8 TB/s), its duration from HIP events on the library's stream, and its
    HBM bytes per launch from the committed rocprofv3 PMC summary of the same workload;
  * the HBM footprint of every index tensor, and the host bytes of the base;
  * out of core: base rows read from host memory in this run (the library's own counter; 4 D
    bytes each), split into the seeding pass and Stage Z;
  * cpu_baseline: the reference's CPU IVF-Flat (omp_cpu_ivfflat_f32, restated in oracle/,
    FP32, OpenMP) on the same probes over a bounded query sample, the box's thread share,
    threads pinned (OMP_PROC_BIND=spread, OMP_PLACES=cores), warmup 1 + 3 rounds; on float
    data its ids are audited against the exact ones (exact tie / FP32 rounding / true miss).
With ``--pipeline-batches`` > 0 (default 12): ``pipelined_from_host`` (queries uploaded from host
memory, searched and read back with 1 / 2 / 3 batches in flight; PCIe-inclusive) and
``two_streams_resident`` (queries resident in HBM, batches alternating between two streams so
that one search's PCIe-bound refinement overlaps the next one's scans); both are reported beside
``value``, which stays the one-stream step.
With configs[4] (the default) the line also carries, under ``extra``:
  * ``cfg5_sq8_only``: the same index with the fine level dropped and the reference packing
    released, i.e. the configuration as BASELINE.json states it (SQ8 codes, ids and per-vector
    scalars in HBM, FP32 survivors over PCIe), at TRIDENT_UB_SEED 0, 1 and 2;
  * ``configs``: every config x K x nprobe BASELINE.json lists (configs[0]; configs[1] at
    nprobe 32/64/128; configs[2] at K 10/100; configs[3] at K 1/10/50/100), each timed and
    checked against the oracle on every query.
"""
import os

# The CPUs this process may use, read before an OpenMP runtime binds its initial thread to one
# place (after that, sched_getaffinity of the main thread names that place only).
AFFINITY_CPUS = len(os.sched_getaffinity(0))
# OpenMP reads its placement once, when the runtime loads (torch or the oracle library).
os.environ.setdefault("OMP_PROC_BIND", "spread")
os.environ.setdefault("OMP_PLACES", "cores")

import argparse  # noqa: E402
import json  # noqa: E402
import platform  # noqa: E402
import statistics  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "QPS at 100% exact top-10, 1×MI355X; achieved HBM GB/s vs peak"  # BASELINE.json metric, verbatim
HBM_PEAK_GBPS = 8000.0
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix throughput
FP32_PEAK_TFLOPS = 157.3  # MI355X dense float32 matrix throughput
PROFILES = os.path.join(ROOT, "profiles")
T_START = time.perf_counter()


def log(*a):
    print(f"[bench {time.perf_counter() - T_START:6.1f}s]", *a, file=sys.stderr, flush=True)


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_threads() -> int:
    """The OpenMP threads the CPU baseline uses: OMP_NUM_THREADS when the host sets it (the GPU
    boxes set it to their CPU share for one GPU), else every CPU this process may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return AFFINITY_CPUS


# BASELINE.json configs; `cpu` is the default CPU-baseline sample (-1 = all B), `sweep` the
# (nprobe, K) variants BASELINE.json lists for it.
CONFIGS = {
    1: dict(N=100_000, D=128, nlist=256, nprobe=16, K=10, B=1_000, T=64, n_centers=256, host=False,
            cpu=-1, sweep=[(16, 10)], desc="configs[0]: 256-component isotropic Gaussian mixture"),
    2: dict(N=1_000_000, D=128, nlist=1024, nprobe=64, K=10, B=10_000, T=64, n_centers=1024, host=False,
            cpu=-1, sweep=[(32, 10), (64, 10), (128, 10)],
            desc="configs[1]: histogram-like u8-valued descriptors"),
    3: dict(N=1_000_000, D=960, nlist=1024, nprobe=64, K=10, B=1_000, T=256, n_centers=1024, host=False,
            cpu=-1, sweep=[(64, 10), (64, 100)], desc="configs[2]: anisotropic power-law Gaussian, D=960"),
    4: dict(N=10_000_000, D=96, nlist=4096, nprobe=64, K=10, B=10_000, T=64, n_centers=4096, host=False,
            cpu=2000, sweep=[(64, 1), (64, 10), (64, 50), (64, 100)],
            desc="configs[3]: L2-normalised 4096-centre mixture, D=96"),
    5: dict(N=100_000_000, D=128, nlist=16384, nprobe=128, K=10, B=10_000, T=64, n_centers=1024, host=True,
            cpu=1000, sweep=[(128, 10)], desc="configs[4]: histogram-like u8-valued descriptors, out of core"),
}
FLOAT_CONFIGS = (1, 3, 4)


def load_profile(name, **match):
    """A committed rocprofv3 summary (profiles/<name>.json) if it was measured on this
    workload (every key of `match` equal), else None."""
    path = os.path.join(PROFILES, name + ".json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        p = json.load(f)
    return p if all(p.get(k) == v for k, v in match.items()) else None


class Workload:
    """Synthetic data + index of one configuration, built on the GPU."""

    def __init__(self, cfg_id, cfg, xb_host, dev, index_cache=""):
        import torch
        from trident_amd import clustering, datagen, persist
        from trident_amd.index import SharedClusterStorage, TridentV4Index
        self.cfg_id, self.cfg, self.xb_host = cfg_id, cfg, xb_host
        N, D, nlist, K, B = cfg["N"], cfg["D"], cfg["nlist"], cfg["K"], cfg["B"]
        max_k = max([K] + [k for _, k in cfg["sweep"]])
        max_np = max([128, cfg["nprobe"]] + [n for n, _ in cfg["sweep"]])
        t0 = time.perf_counter()
        xb, xq = datagen.generate(cfg_id, device=dev, seed=0, N=N, D=D, B=B, n_centers=cfg["n_centers"])
        torch.cuda.synchronize()
        log(f"generated cfg{cfg_id} N={N} D={D} B={B} in {time.perf_counter() - t0:.1f}s")
        t1 = time.perf_counter()
        placement = "host" if xb_host else "device"
        # the workload a saved index was built for: its generator, seed and sizes
        ident = {"cfg": int(cfg_id), "seed": 0, "N": int(N), "D": int(D), "nlist": int(nlist),
                 "n_centers": int(cfg["n_centers"]), "T": int(cfg["T"])}
        cached = index_cache and os.path.exists(os.path.join(index_cache, "meta.npz"))
        if cached:
            saved = persist.read_user_meta(index_cache)
            if saved != ident:
                raise SystemExit(f"{index_cache} holds an index of another workload ({saved}, "
                                 f"this run needs {ident}): remove it or pass another directory")
            # the saved index holds no base: the regenerated one is sorted by its sort_perm
            self.ix = persist.load_index(index_cache, device=dev, xb_placement=placement, xb_raw=xb,
                                         max_batch=B, max_nprobe=max_np, k=max_k)
            self.st = self.ix.storage
        else:
            cen, lid, r, mean64, R64, t_train = clustering.train_clustering(
                xb, nlist, seed=0, niter=20, max_train=min(N, max(64 * nlist, 256 * 1024)), device=dev)
            self.st = SharedClusterStorage(xb, lid, r, nlist, device=dev, xb_placement=placement)
            self.ix = TridentV4Index(self.st, cen, mean64, R64, tile_size=cfg["T"], device=dev, max_batch=B,
                                     max_nprobe=max_np, k=max_k)
        del xb
        torch.cuda.synchronize()
        self.build_s = time.perf_counter() - t1
        if cached:
            log(f"index loaded from {index_cache} in {self.build_s:.1f}s")
        else:
            log(f"k-means {t_train:.1f}s, index build {self.ix.build_time_s:.1f}s, total {self.build_s:.1f}s; "
                f"rows within a cluster by {getattr(self.st, 'within', 'id')} "
                f"(seeding scores {getattr(self.st, 'seed_scores', None)})")
            if index_cache:
                t2 = time.perf_counter()
                persist.save_index(self.ix, index_cache, include_base=False, mean64=mean64, R64=R64,
                                   user=ident)
                log(f"index saved to {index_cache} in {time.perf_counter() - t2:.1f}s")
        log("HBM footprint (MB): " + ", ".join(f"{k} {v / 1e6:.1f}" for k, v in self.ix.hbm_footprint().items()))
        self.xq = xq.contiguous()
        self.xq_np = xq.cpu().numpy()
        self._refs = {}

    def reference(self, nprobe, K):
        """float64 oracle over every query of the batch: (probes, d [B, K], ids [B, K]).  One
        cluster-major scan per nprobe at the largest K asked for; smaller K take its prefix (the
        top-K by (d, id) is the first K entries of any longer such list)."""
        from oracle import oracle as O
        kmax = max([K] + [k for n, k in self.cfg["sweep"] if n == nprobe])
        hit = self._refs.get(nprobe)
        if hit is None or hit[0] < K:
            h = self.host_arrays()
            tc = time.perf_counter()
            cids, _ = O.coarse_probe(self.xq_np, h["centroids"], nprobe)
            d, i = O.ivf_exact_cm(self.xq_np, cids, h["vec_off"], h["xb_sorted"], h["orig_ids_sorted"], kmax)
            log(f"oracle nprobe={nprobe} K={kmax}: {len(self.xq_np)} queries in {time.perf_counter() - tc:.1f}s")
            hit = self._refs[nprobe] = (kmax, cids, d, i)
        return hit[1], hit[2][:, :K], hit[3][:, :K]

    def host_arrays(self):
        if not hasattr(self, "_host"):
            self._host = self.ix.host_arrays()
        return self._host

    def free(self):
        import torch
        torch.cuda.synchronize()
        if self.st._host_buf is not None:
            self.st._host_buf.free()
        self.ix = self.st = None
        self._refs, self._host = {}, None
        torch.cuda.empty_cache()


def time_steps(run, steps, warmup, rounds):
    """W warmup steps, then `steps` timed steps in `rounds` rounds; returns (ms per step over the
    whole timed region, per-round ms per step, stage events of every timed step)."""
    import torch
    from trident_amd import _lib
    for _ in range(warmup):
        run(None)
    rounds = max(1, min(rounds, steps))
    per = [steps // rounds + (1 if r < steps % rounds else 0) for r in range(rounds)]
    evs = [_lib.StageEvents() for _ in range(steps)]
    torch.cuda.synchronize()
    t_all, round_ms, k = 0.0, [], 0
    for n in per:
        torch.cuda.synchronize()
        ts = time.perf_counter()
        for _ in range(n):
            run(evs[k])
            k += 1
        torch.cuda.synchronize()
        dt = time.perf_counter() - ts
        t_all += dt
        round_ms.append(dt * 1000.0 / n)
    return t_all * 1000.0 / steps, round_ms, evs


def stage_breakdown(evs):
    from trident_amd import _lib as E
    pairs = {"front_end_ms": (E.EV_START, E.EV_PROBED), "group_pairs_ms": (E.EV_PROBED, E.EV_GROUPED),
             "pass1_scan_ms": (E.EV_GROUPED, E.EV_P1_SCAN), "pass1_merge_ms": (E.EV_P1_SCAN, E.EV_P1_MERGE),
             "pass2_scan_ms": (E.EV_P1_MERGE, E.EV_P2_SCAN), "pass2_merge_ms": (E.EV_P2_SCAN, E.EV_END),
             "gpu_total_ms": (E.EV_START, E.EV_END)}
    out = {k: statistics.mean(e.elapsed_ms(a, b) for e in evs) for k, (a, b) in pairs.items()}
    for e in evs:
        e.destroy()
    return out


class _RowsById:
    """xb_sorted indexed by original id (for the audit), without a reordered copy."""

    def __init__(self, xb_sorted, orig_ids):
        import numpy as np
        self.xb = xb_sorted
        self.pos = np.empty(len(orig_ids), np.int64)
        self.pos[orig_ids] = np.arange(len(orig_ids))

    def __getitem__(self, i):
        return self.xb[self.pos[i]]


def search_once(w, nprobe, K, mode, ub, route):
    """One untimed search with telemetry: (d, i, probes, stats, host rows [total, seeding])."""
    import torch
    dev = w.xq.device
    stats = torch.zeros(4, dtype=torch.int64, device=dev)
    hrows = torch.zeros(2, dtype=torch.int64, device=dev)
    d_out, i_out, _ = w.ix.search(w.xq, nprobe, mode=mode, ub_seed=ub, stats_buf=stats, route=route,
                                  host_rows_buf=hrows, k=K)
    torch.cuda.synchronize()
    B = w.xq.shape[0]
    return (d_out.cpu().numpy().copy(), i_out.cpu().numpy().copy(),
            w.ix.probe_cids_buf[:B, :nprobe].cpu().numpy().copy(),
            [int(v) for v in stats.tolist()], [int(v) for v in hrows.tolist()])


def exactness(w, nprobe, K, gpu_d, gpu_i, probes):
    import numpy as np
    ref_cids, ref_d, ref_i = w.reference(nprobe, K)
    B = len(gpu_i)
    return {"queries_checked": B, "of_batch": B,
            "probes_identical": int((ref_cids == probes).all(axis=1).sum()),
            "ids_identical": int((ref_i == gpu_i).all(axis=1).sum()),
            "distances_identical": int((ref_d.astype(np.float32) == gpu_d).all(axis=1).sum())}


def roofline(w, stage, probes, mode, route_used):
    """The dominant kernel's roofline from this run's stage events (the lower-bound pass)."""
    import numpy as np
    from trident_amd import _lib
    ix = w.ix
    sizes = np.diff(w.st.cluster_vec_off.cpu().numpy().astype(np.int64))
    rows_all = int(sizes[probes].sum())
    t_scan = stage["pass2_scan_ms"] * 1e-3
    if route_used == _lib.ROUTE_BATCHED and mode == 10:
        flops = 2.0 * rows_all * ix.D_pad  # float32 matrix cores: 2 D_pad flops per (query, row)
        achieved = flops / t_scan / 1e12
        kname = "cm_scan_kernel<D4>" if ix.D_pad <= 256 else "cm_scan_wide_kernel"
        roof = {"bound": "mfma", "kernel": f"{kname} (mode 10, float32 matrix cores)",
                "achieved": round(achieved, 2), "peak": FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / FP32_PEAK_TFLOPS, 4), "flops_alg_per_launch": flops}
    elif route_used == _lib.ROUTE_BATCHED:
        ops_alg = 4 * rows_all * ix.D_pad
        achieved = ops_alg / t_scan / 1e12
        kname = "lb_scan_kernel<KS>" if ix.D_pad <= 256 else "lb_scan_wide_kernel<KS>"
        roof = {"bound": "mfma", "kernel": f"{kname} (lower-bound pass, int8 matrix cores)",
                "achieved": round(achieved, 2), "peak": INT8_PEAK_TOPS, "unit": "TOP/s",
                "frac": round(achieved / INT8_PEAK_TOPS, 4), "ops_alg_per_launch": ops_alg}
    else:
        byts = rows_all * ix.D_pad
        achieved = byts / t_scan / 1e9
        roof = {"bound": "hbm", "kernel": "pair_scan_kernel (pass 2)" if mode == 2 else "pair_scan_kernel (CM)",
                "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBPS, 4), "bytes_alg_per_launch": byts}
    roof["launch_ms"] = round(stage["pass2_scan_ms"], 4)
    return roof, rows_all, int(sizes[np.unique(probes)].sum())


def cpu_baseline(w, nprobe, K, probes, gpu_d, gpu_i, nc):
    import numpy as np
    from oracle import oracle as O
    from trident_amd import metrics
    h = w.host_arrays()
    threads = cpu_threads()
    B = len(gpu_i)
    nc = B if nc < 0 else min(nc, B)
    fn = lambda: O.ivfflat_f32(w.xq_np[:nc], probes[:nc], h["vec_off"], h["xb_sorted"], h["orig_ids_sorted"],
                               K, threads=threads)
    fn()
    rounds = []
    for _ in range(3):
        tb = time.perf_counter()
        fd, fi = fn()
        rounds.append(nc / (time.perf_counter() - tb))
    f32_same = int((fi == gpu_i[:nc]).all(axis=1).sum())
    cpu = {"value": round(statistics.mean(rounds), 1), "unit": "queries/s", "cores": threads, "kind": "port",
           "sample": f"first {nc} of {B} queries, nprobe={nprobe}, same probes as the GPU; warmup 1 + 3 "
                     f"rounds (std {statistics.pstdev(rounds):.1f} QPS); {threads} OpenMP threads "
                     f"(OMP_PROC_BIND={os.environ.get('OMP_PROC_BIND')}, OMP_PLACES={os.environ.get('OMP_PLACES')}) "
                     f"of {os.cpu_count()} online CPUs, {AFFINITY_CPUS} in this process's "
                     f"affinity at start; CPU: {cpu_model()}; FP32 ids identical to the GPU's exact ids on "
                     f"{f32_same}/{nc} queries",
           "online_cpus": os.cpu_count(), "cpu_model": cpu_model()}
    if w.cfg_id in FLOAT_CONFIGS:
        a = O.audit(fi, gpu_i[:nc], _RowsById(h["xb_sorted"], h["orig_ids_sorted"]), w.xq_np[:nc])
        rec, strict, full = metrics.eval_accuracy_v4(fi, fd, gpu_i[:nc], gpu_d[:nc], gpu_i[:nc], k=K)
        cpu["fp32_audit_vs_exact"] = {
            "diff_slots": a["diff_slots"], "exact_tie": a["exact_tie"], "f32_rounding_le_1e-5": a["f32_rounding"],
            "true_miss": a["true_miss"], "max_rel": a["max_rel"],
            "strict_overlap_pct": round(strict, 4), "queries_all_slots_pct": round(full, 2)}
    log(f"cpu baseline: {cpu['value']:,.1f} QPS on {threads} threads over {nc} queries")
    return cpu


def measure_variant(w, nprobe, K, mode, ub, route, steps, warmup, rounds, label=""):
    """Times one (nprobe, K, mode, ub) on a built workload and checks every query."""
    from trident_amd import _lib
    ix = w.ix
    B = w.cfg["B"]

    def run(events):
        return ix.search(w.xq, nprobe, mode=mode, ub_seed=ub, stage_events=events, route=route, k=K)

    ms, round_ms, evs = time_steps(run, steps, warmup, rounds)
    stage = stage_breakdown(evs)
    gd, gi, probes, stats, hrows = search_once(w, nprobe, K, mode, ub, route)
    ex = exactness(w, nprobe, K, gd, gi, probes)
    route_used = ix.route_for(B, nprobe, K, route, mode=mode)
    roof, rows_all, rows_unique = roofline(w, stage, probes, mode, route_used)
    round_qps = [B / (m / 1000.0) for m in round_ms]
    out = {"qps": round(B / (ms / 1000.0), 1), "ms_per_step": round(ms, 4), "steps": steps,
           "rounds_qps_mean": round(statistics.mean(round_qps), 1),
           "rounds_qps_std": round(statistics.pstdev(round_qps), 1),
           "route": (("cm_matrix" if mode == 10 else "batched") if route_used == _lib.ROUTE_BATCHED
                     else "pair"),
           "exact": ex, "roofline": roof, "stages_ms": {k: round(v, 4) for k, v in stage.items()},
           "pruning": {"candidates": stats[0], "survivors": stats[2], "refined_kept": stats[3]}}
    if w.xb_host:
        D = w.cfg["D"]
        # the exact refines read the base's uint8 copy when it has one (the rescan of an
        # overflowed candidate list reads float32 rows)
        u8 = getattr(w.st, "xb_sorted_u8", None) is not None
        rb = D if u8 else 4 * D
        out["pcie"] = {"host_rows_read": hrows[0], "seeding_pass_rows": hrows[1],
                       "stage_z_rows": hrows[0] - hrows[1], "row_bytes": rb,
                       "row_format": "uint8 copy of the float32 base" if u8 else "float32",
                       "bytes_per_query": round(hrows[0] * rb / B, 1),
                       "seeding_bytes_per_query": round(hrows[1] * rb / B, 1),
                       "stage_z_bytes_per_query": round((hrows[0] - hrows[1]) * rb / B, 1)}
    log(f"{label} nprobe={nprobe} K={K} mode={mode} ub={ub}: {ms:.3f} ms/step, {B / ms * 1e3:,.0f} QPS; "
        f"exact ids {ex['ids_identical']}/{B}, distances {ex['distances_identical']}/{B}; "
        f"{roof['kernel'].split(' ')[0]} {roof['frac']:.3f} of peak in {roof['launch_ms']} ms")
    return out, (gd, gi, probes, stats, hrows, stage, ms, round_ms, roof, rows_all, rows_unique, route_used)


def two_streams_resident(w, nprobe, K, mode, ub, route, nb, gpu_d, gpu_i):
    """Queries resident in HBM, `nb` searches of the same batch alternating between two streams
    (own outputs and library workspace each), so one search's PCIe-bound refinement runs beside
    the next one's scans; the bench's `value` stays the one-stream step.  Not PCIe-inclusive."""
    import numpy as np
    import torch
    from trident_amd import ext
    ix, dev = w.ix, w.ix.dev
    B = int(w.xq.shape[0])
    view = ix.view()
    streams = [torch.cuda.Stream(device=dev) for _ in range(2)]
    outs = [(torch.empty((B, K), dtype=torch.float32, device=dev),
             torch.empty((B, K), dtype=torch.int64, device=dev)) for _ in range(2)]

    def run(n):
        for k in range(n):
            s = streams[k % 2]
            with torch.cuda.stream(s):
                ext.search_view(view, w.xq, nprobe, outs[k % 2][0], outs[k % 2][1], mode=mode, ub_seed=ub,
                                route=route, stream=s)

    for s in streams:
        s.wait_stream(torch.cuda.current_stream(dev))
    run(4)  # warm-up: both streams' workspaces
    torch.cuda.synchronize(dev)
    tb = time.perf_counter()
    run(nb)
    torch.cuda.synchronize(dev)
    sec = time.perf_counter() - tb
    same = all(bool(np.array_equal(o[1].cpu().numpy(), gpu_i) and np.array_equal(o[0].cpu().numpy(), gpu_d))
               for o in outs)
    for s in streams:
        ext.release_workspace(dev, s)
    res = {"batches": nb, "batch": B, "qps": round(nb * B / sec, 1), "ms_per_batch": round(sec * 1e3 / nb, 3),
           "results_identical": same}
    log(f"two streams, queries resident: {res['qps']:,.0f} QPS ({res['ms_per_batch']:.3f} ms per batch of "
        f"{B}), results identical {same}")
    return res


def measure_primary(cfg_id, cfg, args, dev):
    """The headline line's fields: the config at its stated nprobe / K, timed, checked on every
    query, with roofline, footprint, PCIe split and the CPU baseline."""
    import numpy as np
    from trident_amd import _lib

    w = Workload(cfg_id, cfg, cfg["host"], dev, index_cache=args.index_cache)
    ix = w.ix
    N, D, K, B, nprobe = cfg["N"], cfg["D"], cfg["K"], cfg["B"], cfg["nprobe"]
    mode, ub = args.mode, args.ub
    v, raw = measure_variant(w, nprobe, K, mode, ub, args.route, args.steps, args.warmup, args.rounds,
                             label=f"cfg{cfg_id}")
    gpu_d, gpu_i, probes, stats, hrows, stage, ms, round_ms, roof, rows_all, rows_unique, route_used = raw
    prof = load_profile(f"lb_scan_cfg{cfg_id}_traffic", N=N, nprobe=nprobe, K=K, B=B) if mode == 2 else None
    roof["traffic"] = prof["hbm_bytes_per_launch"] if prof else None
    if prof:
        roof["traffic_source"] = (f"profiles/lb_scan_cfg{cfg_id}_traffic.json: rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                  "of this kernel on this workload, a separate profiled run")
    p_init = _lib.lib().trident_p_init_rule(mode, B, K, nprobe, 0) if mode == 2 else 0
    tot, dims, surv, ins = stats
    out = {"qps": B / (ms / 1000.0), "ms_per_step": ms, "round_qps": [B / (m / 1000.0) for m in round_ms],
           "stage": stage, "roof": roof, "exact": v["exact"], "route": route_used, "p_init": p_init,
           "rows_all": rows_all, "rows_unique": rows_unique,
           "pruning": {"candidates": tot, "dims_scanned_frac": round(dims / max(tot * ix.D_pad, 1), 4),
                       "survivors_frac": round(surv / max(tot, 1), 6), "refined_kept": ins},
           "nprobe": nprobe, "K": K, "B": B, "N": N, "D": D, "nlist": cfg["nlist"],
           "row_order": getattr(w.st, "within", "id"),
           "hbm_footprint": ix.hbm_footprint(),
           "host_bytes": (int(w.st.xb_sorted.numel() * 4) + (0 if getattr(w.st, "xb_sorted_u8", None) is None
                                                             else int(w.st.xb_sorted_u8.numel())))
                         if w.xb_host else 0}
    if w.xb_host:
        out["out_of_core"] = dict(v["pcie"], fine_level=ix.fine_codes is not None,
                                  pass_b_survivors=surv, stage_z_ms=round(stage["pass2_merge_ms"], 4))
        pp = load_profile(f"refine_cfg{cfg_id}_pcie", N=N, nprobe=nprobe, K=K, B=B)
        if pp:
            out["out_of_core"]["pcie_counter_profile"] = {
                "source": f"profiles/refine_cfg{cfg_id}_pcie.json (rocprofv3, a separate profiled run)",
                "bytes_per_search": pp["pcie_bytes_per_search"],
                "bytes_per_query": round(pp["pcie_bytes_per_search"] / B, 1), "counter": pp["counter"]}

    if not args.no_cpu_baseline:
        out["cpu"] = cpu_baseline(w, nprobe, K, probes, gpu_d, gpu_i, cfg["cpu"] if args.cpu_queries == -1
                                  else args.cpu_queries)
    else:
        out["cpu"] = None

    if args.pipeline_batches > 0:
        # End to end from host memory (PCIe-inclusive): queries uploaded, searched and read back
        # in batches of B, `depth` batches in flight on separate streams (trident_amd.pipeline).
        from trident_amd.pipeline import SearchPipeline
        nb = args.pipeline_batches
        xq_all = np.concatenate([w.xq_np] * nb)
        pipe_out = {}
        for depth in (1, 2, 3):
            with SearchPipeline(ix, nprobe, K, batch=B, depth=depth, mode=mode, ub_seed=ub,
                                route=args.route) as pipe:
                pipe.run(xq_all[:B * depth])  # warm-up: every slot's workspace and buffers
                tb = time.perf_counter()
                pd_, pi_ = pipe.run(xq_all)
                sec = time.perf_counter() - tb
            same = bool(np.array_equal(pi_[:B], gpu_i) and np.array_equal(pd_[-B:], gpu_d))
            pipe_out[f"depth{depth}"] = {"qps": round(len(xq_all) / sec, 1), "ms_per_batch": round(sec * 1e3 / nb, 3),
                                         "results_identical": same}
            log(f"pipelined from host, depth {depth}: {len(xq_all) / sec:,.0f} QPS "
                f"({sec * 1e3 / nb:.3f} ms per batch of {B}), results identical {same}")
        out["pipelined_from_host"] = dict(batches=nb, batch=B, **pipe_out)
        out["two_streams_resident"] = two_streams_resident(w, nprobe, K, mode, ub, args.route, nb, gpu_d, gpu_i)

    if w.xb_host and mode == 2 and not args.no_float32_rows and getattr(w.st, "xb_sorted_u8", None) is not None:
        # the same search with every exact refine reading the float32 rows (uint8 copy unset)
        u8_saved = w.st.xb_sorted_u8
        w.st.xb_sorted_u8 = None
        try:
            sv, _ = measure_variant(w, nprobe, K, mode, ub, args.route, args.extra_steps, 3, 2,
                                    label=f"cfg{cfg_id} float32 refine rows")
        finally:
            w.st.xb_sorted_u8 = u8_saved
        out["float32_refine_rows"] = sv

    if args.sweep:
        sweep = {}
        for npb, md, u in ((nprobe // 2, 2, ub), (nprobe * 2, 2, ub), (nprobe, 10, 0)):
            if npb > ix.max_nprobe or npb < 1:
                continue
            sv, _ = measure_variant(w, npb, K, md, u, args.route, 5, 2, 1, label="sweep")
            sweep[f"nprobe{npb}_mode{md}_ub{u}"] = sv
        out["sweep"] = sweep
    if args.calibrate_w0:
        from trident_amd import router
        W0, rows = router.calibrate_w0(ix, w.xq, nprobe,
                                       batches=(1, 2, 4, 8, 16, 32, 64, 128, 256, 512, 1024, 2048,
                                                4096, 8192, B),
                                       warmup=3, iters=10, ub_seed=ub)
        for r_ in rows:
            mx = r_["ms_cm_matrix"]
            log(f"W0 sweep B={r_['batch']:5d} W={r_['work']:.3e} cm={r_['ms_cm']:.3f}ms "
                f"(pair {r_['ms_cm_pair']:.3f}, matrix {'-' if mx is None else f'{mx:.3f}'}) "
                f"cascade={r_['ms_cascade']:.3f}ms -> {'cascade' if r_['cascade_faster'] else 'cm'}")
        out["w0_calibration"] = {"W0": W0, "W0_stable": router.stable_crossover(rows), "rows": rows}

    if w.xb_host and mode == 2 and not args.no_sq8_only:
        # The configuration as BASELINE.json states it: SQ8 codes (once), ids and per-vector
        # scalars in HBM, FP32 survivors over PCIe -- the fine level dropped, the reference
        # packing released (the batched route reads the cells).
        ix.release_fine_level()
        ix.release_packed_codes()
        import torch
        torch.cuda.empty_cache()
        sq = {"hbm_footprint": ix.hbm_footprint()}
        for u in (0, 1, 2):
            sv, _ = measure_variant(w, nprobe, K, mode, u, args.route, args.extra_steps, 3, 2,
                                    label=f"cfg{cfg_id} sq8-only")
            sq[f"ub{u}"] = sv
        out["sq8_only"] = sq
    w.free()
    return out


def measure_sweeps(args, dev, cfg_ids):
    """Every (nprobe, K) BASELINE.json lists for the in-HBM configs: one build each."""
    res = {}
    for cid in cfg_ids:
        cfg = dict(CONFIGS[cid])
        w = Workload(cid, cfg, False, dev)
        for npb, K in cfg["sweep"]:
            v, raw = measure_variant(w, npb, K, 2, args.ub, args.route, args.extra_steps, 5, 2,
                                     label=f"cfg{cid}")
            v["workload"] = (f"BASELINE {cfg['desc']}, N={cfg['N']}, D={cfg['D']}, nlist={cfg['nlist']}, "
                             f"nprobe={npb}, K={K}, B={cfg['B']}")
            if (npb, K) == (cfg["nprobe"], cfg["K"]) and not args.no_cpu_baseline:
                gd, gi, probes = raw[0], raw[1], raw[2]
                v["cpu_baseline"] = cpu_baseline(w, npb, K, probes, gd, gi, cfg["cpu"])
            res[f"configs[{cid - 1}]_nprobe{npb}_K{K}"] = v
        # mode 10 (exact cluster-major scan; the reference's router sends configs[0] there) at the
        # config's stated nprobe and K, on the library's AUTO route (float32 matrix cores here)
        npb, K = cfg["nprobe"], cfg["K"]
        v, _ = measure_variant(w, npb, K, 10, 0, 0, args.extra_steps, 5, 2, label=f"cfg{cid} mode 10")
        v["workload"] = (f"BASELINE {cfg['desc']}, N={cfg['N']}, D={cfg['D']}, nlist={cfg['nlist']}, "
                         f"nprobe={npb}, K={K}, B={cfg['B']}, mode 10")
        res[f"configs[{cid - 1}]_nprobe{npb}_K{K}_mode10"] = v
        w.free()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=12)
    ap.add_argument("--rounds", type=int, default=5, help="timed steps are split into this many rounds")
    ap.add_argument("--cfg", type=int, default=5, choices=sorted(CONFIGS))
    ap.add_argument("--nprobe", type=int, default=0, help="0 = the config's value")
    ap.add_argument("--K", type=int, default=0, help="0 = the config's value")
    ap.add_argument("--ub", type=int, default=1, help="TRIDENT_UB_SEED for the timed runs")
    ap.add_argument("--mode", type=int, default=2, help="2 cascade, 10 CM exact")
    ap.add_argument("--route", type=int, default=0, help="mode-2 route: 0 auto, 1 per-pair, 2 batched")
    ap.add_argument("--N", type=int, default=0)
    ap.add_argument("--B", type=int, default=0)
    ap.add_argument("--cpu-queries", type=int, default=-1, help="CPU-baseline sample (-1 = config default)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--xb-host", action="store_true", help="FP32 base in mapped pinned host memory (out of core)")
    ap.add_argument("--xb-device", action="store_true", help="FP32 base in HBM (cfg 5 defaults to host)")
    ap.add_argument("--no-extra", action="store_true", help="skip the config sweeps after cfg 5")
    ap.add_argument("--no-sq8-only", action="store_true", help="skip the SQ8-only out-of-core lines")
    ap.add_argument("--no-float32-rows", action="store_true",
                    help="skip the out-of-core line whose refines read float32 rows instead of the uint8 copy")
    ap.add_argument("--extra-cfgs", default="1,2,3,4", help="configs swept after cfg 5")
    ap.add_argument("--pipeline-batches", type=int, default=12,
                    help="batches of B host queries for the pipelined end-to-end line (0 = skip)")
    ap.add_argument("--index-cache", default="", help="directory of a saved index (trident_amd.persist): "
                    "loaded when present and built for this workload, else written after the build")
    ap.add_argument("--extra-steps", type=int, default=10)
    ap.add_argument("--sweep", action="store_true", help="also time other nprobe values and the CM route")
    ap.add_argument("--calibrate-w0", action="store_true", help="router crossover sweep over batch sizes")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (--gpus {args.gpus} requested): this build's path runs on a "
              "single MI355X; sharding across GPUs is a design, not part of this build.", file=sys.stderr)
        sys.exit(2)
    cfg = dict(CONFIGS[args.cfg])
    for k in ("N", "B", "K", "nprobe"):
        if getattr(args, k):
            cfg[k] = getattr(args, k)
    if args.K or args.nprobe:
        cfg["sweep"] = [(cfg["nprobe"], cfg["K"])]
    if args.xb_host:
        cfg["host"] = True
    if args.xb_device:
        cfg["host"] = False

    import torch
    dev = torch.device("cuda:0")
    r = measure_primary(args.cfg, cfg, args, dev)
    from trident_amd import _lib
    roof = r["roof"]
    t_l = roof["launch_ms"] * 1e-3
    # SURVEY's algorithmic bytes (every probed (query, list) pair's codes at full depth) and the
    # compulsory bytes (each probed list's codes once) of the dominant kernel's launch
    D_pad = (cfg["D"] + 31) // 32 * 32
    byt_alg, byt_cmp = r["rows_all"] * D_pad, r["rows_unique"] * D_pad
    hv = {"bytes_alg_per_launch": byt_alg, "alg_GBps": round(byt_alg / t_l / 1e9, 1),
          "alg_over_peak": round(byt_alg / t_l / 1e9 / HBM_PEAK_GBPS, 3),
          "bytes_compulsory_per_launch": byt_cmp, "compulsory_GBps": round(byt_cmp / t_l / 1e9, 1),
          "compulsory_frac_of_peak": round(byt_cmp / t_l / 1e9 / HBM_PEAK_GBPS, 3),
          "note": "bytes_alg counts each probed list once per query (SURVEY 8(d)); it exceeds the HBM peak "
                  "because a staged slice serves every query of its unit from LDS.  bytes_compulsory reads "
                  "each probed list once."}
    if roof.get("traffic"):
        hv.update({"physical_bytes_per_launch": roof["traffic"],
                   "physical_GBps": round(roof["traffic"] / t_l / 1e9, 1),
                   "physical_frac_of_peak": round(roof["traffic"] / t_l / 1e9 / HBM_PEAK_GBPS, 3)})
    line = {
        "metric": METRIC, "value": round(r["qps"], 1), "unit": "queries/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(r["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8 codes x int8 weights (i32 MFMA) / f32 bounds / f64 exact distances", "data": "synthetic",
        "config": {"workload": f"BASELINE {cfg['desc']}, N={r['N']}, D={r['D']}, nlist={r['nlist']}, "
                               f"nprobe={r['nprobe']}, K={r['K']}, B={r['B']}",
                   "route": ("batched" if r["route"] == _lib.ROUTE_BATCHED else "pair") if args.mode == 2 else "cm_exact",
                   "ub_seed": args.ub, "p_init": r["p_init"], "tile_size": cfg["T"], "row_order": r["row_order"],
                   "parallelism": "single GPU",
                   "xb_placement": "host (mapped, out of core)" if cfg["host"] else "device",
                   "host_rows": (r["out_of_core"]["row_format"] if "out_of_core" in r else None)},
        "roofline": roof,
        "cpu_baseline": r["cpu"],
        "rounds": {"n": len(r["round_qps"]), "qps_mean": round(statistics.mean(r["round_qps"]), 1),
                   "qps_std": round(statistics.pstdev(r["round_qps"]), 1)},
        "exact": r["exact"],
        "stages_ms": {k: round(v, 4) for k, v in r["stage"].items()},
        "pruning": r["pruning"],
        "hbm_view": hv,
        "hbm_footprint_bytes": r["hbm_footprint"],
        "host_bytes": r["host_bytes"],
    }
    for k in ("out_of_core", "sweep", "w0_calibration", "pipelined_from_host", "two_streams_resident"):
        if k in r:
            line[k] = r[k]
    extra = {}
    if "sq8_only" in r:
        extra[f"cfg{args.cfg}_sq8_only"] = r["sq8_only"]
    if "float32_refine_rows" in r:
        extra[f"cfg{args.cfg}_float32_refine_rows"] = r["float32_refine_rows"]
    if args.cfg == 5 and not args.no_extra:
        cids = [int(c) for c in args.extra_cfgs.split(",") if c.strip()]
        extra["configs"] = measure_sweeps(args, dev, cids)
    if extra:
        line["extra"] = extra
    log(f"done in {time.perf_counter() - T_START:.0f}s")
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
