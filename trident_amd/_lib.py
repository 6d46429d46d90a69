"""ctypes binding of libtrident_hip.so (declarations: include/trident_hip.h).

The library is built in-tree by ``trident_amd._build`` (``__graft_entry__.build()``).  If
it is missing this module raises immediately: there is no fallback implementation.
"""
import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libtrident_hip.so")

TRIDENT_OK = 0
ABI_VERSION = 6  # TRIDENT_ABI_VERSION
MODE_SQ8_RERANK = 0
MODE_SQ8 = 1
MODE_CASCADE = 2
MODE_CM_EXACT = 10
MODE_TRIBASE = 11

_P = ctypes.c_void_p
_i32 = ctypes.c_int32
_f64 = ctypes.c_double

NOALLOC_SCRATCH_BYTES = 64 << 20  # TRIDENT_NOALLOC_SCRATCH_BYTES


class TridentIndexView(ctypes.Structure):
    _fields_ = [
        ("N", _i32), ("D", _i32), ("D_pad", _i32), ("nlist", _i32),
        ("tile_size", _i32), ("total_tiles", _i32), ("num_blocks", _i32), ("per_cluster_sq8", _i32),
        ("W_combined", _P), ("b_combined", _P),
        ("rot_sq_min", _f64), ("rot_sq_max", _f64),
        ("sq8_packed", _P), ("tile_orig_ids", _P), ("tile_r_minmax", _P),
        ("cluster_tile_off", _P), ("cluster_vec_off", _P),
        ("xb_sorted", _P), ("orig_ids_sorted", _P),
        ("vmin", _P), ("delta", _P), ("eps_dim", _P), ("blk_bounds4", _P), ("vec_Ar", _P),
        ("sq8_cells", _P),
        ("cent_rows", _P), ("cent_tiles", _P), ("cent_norms", _P), ("cent_norm_max", _f64),
        ("r_vec_sorted", _P), ("fine_codes", _P), ("fine_qp", _P), ("cluster_bounds", _P),
        ("vec_cn", _P), ("seed_rows", _i32), ("xb_sorted_u8", _P),
    ]


class TridentSearchParams(ctypes.Structure):
    _fields_ = [("mode", _i32), ("B", _i32), ("K", _i32), ("nprobe", _i32),
                ("ub_seed", _i32), ("use_l1", _i32), ("p_init", _i32), ("route", _i32),
                ("rerank_m", _i32)]


ROUTE_AUTO, ROUTE_PAIR, ROUTE_BATCHED = 0, 1, 2


class TridentSearchOutputs(ctypes.Structure):
    _fields_ = [("topk_d", _P), ("topk_i", _P), ("probe_cids", _P), ("probe_dqcs", _P),
                ("probe_ld", _i32), ("n_events", _i32), ("tau_sq", _P), ("stats", _P),
                ("events", ctypes.POINTER(_P)), ("host_rows", _P), ("host_rows_seed", _P)]


# Stage boundaries recorded into TridentSearchOutputs.events (enum TridentStageEvent).
EV_START, EV_PROBED, EV_GROUPED, EV_P1_SCAN, EV_P1_MERGE, EV_P2_SCAN, EV_END, EV_COUNT = range(8)


EXPORTS = {
    "trident_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(TridentIndexView), _i32, _i32, _i32]),
    "trident_search": (ctypes.c_int, [ctypes.POINTER(TridentIndexView), ctypes.POINTER(TridentSearchParams),
                                      _P, _P, ctypes.c_size_t, ctypes.POINTER(TridentSearchOutputs), _P]),
    "trident_search_noalloc": (ctypes.c_int, [ctypes.POINTER(TridentIndexView), ctypes.POINTER(TridentSearchParams),
                                              _P, ctypes.POINTER(TridentSearchOutputs), _P]),
    "trident_coarse_probe": (ctypes.c_int, [ctypes.POINTER(TridentIndexView), _P, _i32, _i32, _P,
                                            ctypes.c_size_t, _P, _P, _i32, _P]),
    "trident_group_pairs": (ctypes.c_int, [_P, _i32, _i32, _i32, _i32, _i32, _P, _P, _P, _P, _P, _P, _P]),
    "trident_p_init_rule": (_i32, [_i32, _i32, _i32, _i32, _i32]),
    "trident_route_for": (_i32, [ctypes.POINTER(TridentIndexView), _i32, _i32, _i32, _i32]),
    "trident_route_for_mode": (_i32, [ctypes.POINTER(TridentIndexView), _i32, _i32, _i32, _i32, _i32]),
    "trident_sq8_bounds": (ctypes.c_int, [ctypes.POINTER(TridentIndexView), _P, _i32, _P, _P, _P, _i32,
                                          _P, ctypes.c_size_t, _P, _P, _P]),
    "trident_cluster_bounds": (ctypes.c_int, [ctypes.POINTER(TridentIndexView), _P, _P]),
    "trident_fine_bounds": (ctypes.c_int, [ctypes.POINTER(TridentIndexView), _P, _i32, _P, _P, _i32,
                                          _P, ctypes.c_size_t, _P, _P, _P]),
    "trident_host_alloc_mapped": (ctypes.c_int, [ctypes.c_size_t, ctypes.POINTER(_P)]),
    "trident_host_free": (ctypes.c_int, [_P]),
    "trident_host_device_pointer": (ctypes.c_int, [_P, ctypes.POINTER(_P)]),
    "trident_event_create": (ctypes.c_int, [ctypes.POINTER(_P)]),
    "trident_event_destroy": (ctypes.c_int, [_P]),
    "trident_event_elapsed_ms": (ctypes.c_int, [_P, _P, ctypes.POINTER(ctypes.c_float)]),
    "trident_last_error": (ctypes.c_char_p, []),
    "trident_abi_version": (ctypes.c_int, []),
}

_LIB = None


def lib():
    """Load libtrident_hip.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                "(the lossless IVF path has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in EXPORTS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.trident_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI version {L.trident_abi_version()}, these bindings "
                               f"expect {ABI_VERSION}: rebuild it")
        _LIB = L
    return _LIB


class TridentError(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    if rc != TRIDENT_OK:
        msg = lib().trident_last_error().decode(errors="replace")
        raise TridentError(f"{what} failed (code {rc}): {msg}")


class StageEvents:
    """One hipEvent_t per stage boundary, for timing the library's kernels on their stream."""

    def __init__(self):
        self.handles = (_P * EV_COUNT)()
        for i in range(EV_COUNT):
            h = _P()
            check(lib().trident_event_create(ctypes.byref(h)), "trident_event_create")
            self.handles[i] = h.value

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = ctypes.c_float()
        check(lib().trident_event_elapsed_ms(self.handles[a], self.handles[b], ctypes.byref(ms)),
              "trident_event_elapsed_ms")
        return float(ms.value)

    def destroy(self):
        for i in range(EV_COUNT):
            if self.handles[i]:
                lib().trident_event_destroy(self.handles[i])
                self.handles[i] = None
