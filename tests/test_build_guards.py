"""Build guards, checked on the built library's own device code (CPU only).

* No packed FP32 instructions: the build passes ``-Xclang -target-feature -Xclang
  -packed-fp32-ops`` (trident_amd/_build.py); every gfx950 code object in libtrident_hip.so is
  disassembled and searched for v_pk_add_f32 / v_pk_mul_f32 / v_pk_fma_f32, and a float2
  kernel that the compiler turns into packed instructions without the flag is compiled both
  ways, so the check shows that the flag is what keeps them out.
* Register budget of the hot kernels: their VGPR and scratch use from the code objects'
  metadata (what the compiler's resource report prints) -- no VGPR spills and no scratch.
"""
import os
import re
import subprocess

import pytest

from trident_amd import _build

LLVM = "/opt/rocm/llvm/bin"
TOOLS = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump", "llvm-readelf")]
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
PACKED_F32 = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")

pytestmark = pytest.mark.skipif(not all(os.path.exists(t) for t in TOOLS) or not os.path.exists(_build.LIB),
                                reason="needs the ROCm LLVM tools and a built libtrident_hip.so")


@pytest.fixture(scope="module")
def code_objects(tmp_path_factory):
    """The gfx950 code objects of the built library (one per source file)."""
    d = tmp_path_factory.mktemp("co")
    fat = d / "fatbin.bin"
    subprocess.run([TOOLS[0], f"--dump-section=.hip_fatbin={fat}", _build.LIB, str(d / "stripped.so")],
                   check=True)
    blob = fat.read_bytes()
    starts = [m.start() for m in re.finditer(rb"__CLANG_OFFLOAD_BUNDLE__", blob)] + [len(blob)]
    out = []
    for n, (a, b) in enumerate(zip(starts, starts[1:])):
        part, co = d / f"b{n}.bin", d / f"b{n}.co"
        part.write_bytes(blob[a:b])
        subprocess.run([TOOLS[1], "--unbundle", "--type=o", f"--input={part}", f"--targets={TARGET}",
                        f"--output={co}"], check=True)
        out.append(co)
    assert len(out) == len(_build.SOURCES), (len(out), _build.SOURCES)
    return out


def test_no_packed_fp32_in_the_library(code_objects):
    n_insn = 0
    for co in code_objects:
        asm = subprocess.run([TOOLS[2], "-d", str(co)], check=True, capture_output=True, text=True).stdout
        n_insn += asm.count("\n\t") + asm.count("\n ")
        hits = PACKED_F32.findall(asm)
        assert not hits, f"{co.name}: {len(hits)} packed FP32 instructions"
    assert n_insn > 10_000  # the disassembly really holds the kernels


def test_the_flag_is_what_keeps_them_out(tmp_path):
    src = tmp_path / "pk.hip"
    src.write_text(
        "#include <hip/hip_runtime.h>\n"
        "__global__ void k(float2* a, const float2* b, const float2* c, int n) {\n"
        "  int i = blockIdx.x * blockDim.x + threadIdx.x;\n"
        "  if (i < n) { float2 x = a[i], y = b[i], z = c[i];\n"
        "    x.x = x.x * y.x + z.x; x.y = x.y * y.y + z.y; x.x += y.x; x.y += y.y; a[i] = x; }\n"
        "}\n")
    base = [_build.HIPCC, f"--offload-arch={_build.ARCH}", "-O3", "-ffp-contract=fast", "--cuda-device-only", "-S"]
    flag = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    subprocess.run(base + [str(src), "-o", str(tmp_path / "a.s")], check=True, capture_output=True)
    subprocess.run(base + flag + [str(src), "-o", str(tmp_path / "b.s")], check=True, capture_output=True)
    assert PACKED_F32.search((tmp_path / "a.s").read_text()), "the probe no longer produces packed FP32"
    assert not PACKED_F32.search((tmp_path / "b.s").read_text())
    assert all(f in _build.CFLAGS for f in flag)


def kernel_resources(code_objects):
    """{mangled kernel name: {vgpr_count, vgpr_spill_count, sgpr_spill_count,
    private_segment_fixed_size}} from the code objects' metadata notes."""
    res = {}
    for co in code_objects:
        notes = subprocess.run([TOOLS[3], "--notes", str(co)], check=True, capture_output=True, text=True).stdout
        for block in notes.split("  - .agpr_count")[1:]:
            name = re.search(r"\.name:\s+(\S+)", block)
            if not name:
                continue
            vals = {k: int(v) for k, v in re.findall(
                r"\.(vgpr_count|vgpr_spill_count|sgpr_spill_count|private_segment_fixed_size):\s+(\d+)", block)}
            res[name.group(1)] = vals
    return res


# The hot kernels of the batched route: each must keep its working set in registers (a scratch
# reload inside their loops serialises the loads in flight).
HOT = ("lb_scan_kernelILi1E", "lb_scan_kernelILi2E", "ub_scan_kernelILi2ELi4E", "coarse_gemm_bf16_kernelILi4E",
       "select_band_kernel", "refine_survivors_kernelILb1ELi256E", "cm_scan_kernelILi32E")


def test_hot_kernels_do_not_spill(code_objects):
    res = kernel_resources(code_objects)
    assert len(res) > 50
    for key in HOT:
        found = [n for n in res if key in n]
        assert found, key
        for n in found:
            r = res[n]
            assert r["vgpr_spill_count"] == 0 and r["private_segment_fixed_size"] == 0, (n, r)
