"""trident_amd -- MI355X-native lossless IVF query path (TRIDENT's search, rebuilt for gfx950).

Public surface, mirroring the reference's Python API (benchmarks/phase4a_suite.py):
  choose_tile, SharedClusterStorage, TridentV4Index       (index layout + search wrapper)
  get_cuda_ext()  -> module exposing launch_trident_v4_search (reference PyBind11 export)
  train_clustering (load_or_train_clustering), metrics.eval_accuracy_v4, metrics.measure_latency_qps,
  metrics.measure_runs
  router.CostRouter / router.calibrate_w0                  (cost router)
The compute path is libtrident_hip.so (hand-written HIP for gfx950) behind the C ABI in
include/trident_hip.h; importing the package does not load it, calling a search does.
"""
from .index import SharedClusterStorage, TridentV4Index, choose_tile  # noqa: F401
from .clustering import train_clustering  # noqa: F401


def get_cuda_ext():
    """Returns the extension module (reference get_cuda_ext, phase4a_suite.py:65-72)."""
    from . import ext
    from . import _lib
    _lib.lib()
    return ext
