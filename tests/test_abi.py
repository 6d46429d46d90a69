"""The C ABI boundary on the CPU (no kernel launches): the library loads, exports every symbol
include/trident_hip.h declares, its structs match the ctypes mirror byte for byte, and the
host-side rules and argument checks behave."""
import ctypes
import os
import re
import subprocess

import pytest
import torch

from trident_amd import _lib, ext
from trident_amd._lib import TridentIndexView, TridentSearchOutputs, TridentSearchParams

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "trident_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(trident_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(L, n), f"{n} declared in trident_hip.h but not exported"
        assert n in _lib.EXPORTS, f"{n} has no ctypes prototype"
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (trident_[a-z0-9_]+)", out))
    assert exported == set(names), f"undeclared exports: {exported - set(names)}"
    assert L.trident_abi_version() == _lib.ABI_VERSION == 6


def test_struct_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "trident_hip.h"\n'
        "#define F(S, f) printf(#S \" \" #f \" %zu\\n\", offsetof(S, f));\n"
        "int main(void){\n"
        + "".join(f"F(TridentIndexView,{f})" for f, _ in TridentIndexView._fields_)
        + "".join(f"F(TridentSearchParams,{f})" for f, _ in TridentSearchParams._fields_)
        + "".join(f"F(TridentSearchOutputs,{f})" for f, _ in TridentSearchOutputs._fields_)
        + 'printf("size TridentIndexView %zu\\nsize TridentSearchParams %zu\\nsize TridentSearchOutputs %zu\\n",'
          " sizeof(TridentIndexView), sizeof(TridentSearchParams), sizeof(TridentSearchOutputs));return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.dirname(HEADER), str(src), "-o", str(exe)], check=True)
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines()
    structs = {"TridentIndexView": TridentIndexView, "TridentSearchParams": TridentSearchParams,
               "TridentSearchOutputs": TridentSearchOutputs}
    for line in lines:
        a, b, c = line.split()
        if a == "size":
            assert ctypes.sizeof(structs[b]) == int(c), line
        else:
            assert getattr(structs[a], b).offset == int(c), line


def test_p_init_rule():
    f = _lib.lib().trident_p_init_rule
    # reference src/trident_v4_kernels.cu:1264-1276: modes 1 / 2 / 11 share one rule, mode 0 has
    # its own (by rerank_m), mode 10 is single-pass
    for mode in (1, 2, 11):
        assert f(mode, 1000, 10, 1, 0) == 0
        assert f(mode, 1, 10, 64, 0) == 1
        assert f(mode, 1, 11, 64, 0) == 3
        assert f(mode, 1000, 10, 16, 0) == 2
        assert f(mode, 1000, 10, 2, 0) == 2
        assert f(mode, 1000, 10, 17, 0) == 3
    assert f(10, 1000, 10, 64, 0) == 0
    assert f(0, 1000, 10, 1, 100) == 0
    assert f(0, 1, 10, 32, 0) == 0
    assert f(0, 1, 10, 32, 50) == 2
    assert f(0, 1000, 10, 32, 20) == 1
    assert f(0, 1000, 11, 4, 0) == 2
    assert f(0, 1000, 11, 3, 0) == 1


def _fake_view():
    """A view whose pointers are never dereferenced (argument checks only)."""
    v = TridentIndexView()
    v.N, v.D, v.D_pad, v.nlist, v.tile_size, v.num_blocks = 1000, 128, 128, 16, 64, 4
    v.rot_sq_min = v.rot_sq_max = 1.0
    for f in ("W_combined", "b_combined", "cluster_vec_off", "cluster_tile_off", "xb_sorted",
              "tile_orig_ids", "sq8_packed", "vmin", "delta", "eps_dim", "blk_bounds4"):
        setattr(v, f, 256)
    return v


def test_mode_arguments_are_checked_before_any_launch():
    L = _lib.lib()
    out = TridentSearchOutputs()
    out.topk_d = out.topk_i = 256
    v = _fake_view()
    sp = TridentSearchParams(7, 4, 10, 8, 0, 0, -1, 0, 0)
    assert L.trident_search(ctypes.byref(v), ctypes.byref(sp), None, None, 0, ctypes.byref(out), None) == 2
    assert b"mode 7" in L.trident_last_error()
    sp = TridentSearchParams(11, 4, 10, 8, 0, 0, -1, 0, 0)
    assert L.trident_search(ctypes.byref(v), ctypes.byref(sp), None, None, 0, ctypes.byref(out), None) == 1
    assert b"r_vec_sorted" in L.trident_last_error()
    sp = TridentSearchParams(0, 4, 10, 8, 0, 0, -1, 0, -5)
    assert L.trident_search(ctypes.byref(v), ctypes.byref(sp), None, None, 0, ctypes.byref(out), None) == 1
    assert b"rerank_m" in L.trident_last_error()
    # mode 0's merged lists need room for M = min(max(rerank_m, K), 200) entries
    assert L.trident_workspace_bytes(ctypes.byref(v), 64, 8, 200) > L.trident_workspace_bytes(
        ctypes.byref(v), 64, 8, 10)


def test_host_validation_errors_without_gpu():
    L = _lib.lib()
    sp = TridentSearchParams(2, 4, 10, 8, 0, 0, -1, 0, 0)
    out = TridentSearchOutputs()
    rc = L.trident_search(None, ctypes.byref(sp), None, None, 0, ctypes.byref(out), None)
    assert rc == 1 and b"NULL" in L.trident_last_error()
    v = TridentIndexView()
    v.N, v.D, v.D_pad, v.nlist, v.tile_size, v.num_blocks = 100, 128, 100, 8, 64, 4
    rc = L.trident_search(ctypes.byref(v), ctypes.byref(sp), None, None, 0, ctypes.byref(out), None)
    assert rc == 1 and b"D_pad" in L.trident_last_error()
    assert L.trident_workspace_bytes(None, 1, 1, 1) == 0


def test_noalloc_refuses_oversized_batches_without_touching_the_device():
    """trident_search_noalloc checks the batch against its fixed scratch before any HIP call
    (the view's pointers are never dereferenced here)."""
    L = _lib.lib()
    v = TridentIndexView()
    v.N, v.D, v.D_pad, v.nlist, v.tile_size, v.num_blocks = 1_000_000, 128, 128, 1024, 64, 4
    v.rot_sq_min = v.rot_sq_max = 1.0
    for f in ("W_combined", "b_combined", "cluster_vec_off", "cluster_tile_off", "xb_sorted",
              "tile_orig_ids"):
        setattr(v, f, 256)
    out = TridentSearchOutputs()
    sp = TridentSearchParams(2, 10_000, 10, 64, 1, 0, -1, 0, 0)
    need = L.trident_workspace_bytes(ctypes.byref(v), 10_000, 64, 10)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    rc = L.trident_search_noalloc(ctypes.byref(v), ctypes.byref(sp), None, ctypes.byref(out), None)
    assert rc == 3 and str(need).encode() in L.trident_last_error()


def test_workspace_size_scales_with_batch():
    v = TridentIndexView()
    v.N, v.D, v.D_pad, v.nlist = 1000, 128, 128, 64
    a = _lib.lib().trident_workspace_bytes(ctypes.byref(v), 100, 16, 10)
    b = _lib.lib().trident_workspace_bytes(ctypes.byref(v), 200, 16, 10)
    c = _lib.lib().trident_workspace_bytes(ctypes.byref(v), 100, 16, 100)
    assert 0 < a < b and a < c
    # dominated by float64 coarse distances + candidate lists: B*(nlist*8 + nprobe*K*12) + ...
    assert b - a >= 100 * (64 * 8 + 16 * 10 * 12)


def test_python_boundary_rejects_bad_inputs():
    cpu = torch.zeros(4, 8)
    with pytest.raises(_lib.TridentError, match="unknown mode 3"):
        ext.launch_trident_v4_search(3, 64, 0, 1, 0, 4, *([None] * 35))
    with pytest.raises(_lib.TridentError, match="device tensor"):
        ext.launch_trident_v4_search(2, 64, 0, 1, 0, 4, cpu, *([None] * 34))
    with pytest.raises(_lib.TridentError, match="rerank_m"):
        ext.launch_trident_v4_search(0, 64, 0, 1, -1, 4, cpu, *([None] * 34))


def test_ub_seed_env(monkeypatch):
    monkeypatch.setenv("TRIDENT_UB_SEED", "2")
    assert ext.env_ub_seed() == 2
    monkeypatch.delenv("TRIDENT_UB_SEED")
    assert ext.env_ub_seed() == 0
