"""Resource fit of every kernel in the built liblfamd.so, read on the CPU from its own
gfx950 code object (the AMDGPU metadata notes of the library this repository builds).

A workgroup of W waves puts ceil(W / 4) of them on each SIMD at once; a SIMD holds 512
VGPRs per lane (arch VGPRs, then AGPRs at a 4-aligned offset), allocated in granules of 8.
Inline asm that names registers above what a kernel's launch bound allows only draws a
compiler warning (the build makes it an error) and yields a kernel whose workgroup cannot
be dispatched: the queue aborts with HSA_STATUS_ERROR_INVALID_ISA. The launch code checks
the same rule at run time (check_fit in lf_runtime.hip); this test checks the artefact."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "laplacianformer_amd", "liblfamd.so")
LLVM = "/opt/rocm/llvm/bin"


def _tools():
    tools = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")]
    if not all(os.path.exists(t) for t in tools):
        pytest.skip("ROCm LLVM tools not present")
    return tools


def _parse_notes(co):
    notes = subprocess.run([_tools()[2], "--notes", co], check=True, capture_output=True, text=True).stdout
    body = notes.split("amdhsa.kernels:", 1)[1]
    kernels = []
    for entry in re.split(r"\n  - ", "\n" + body)[1:]:
        kv = {}
        for line in ("    " + entry).splitlines():
            m = re.match(r"^    \.([a-z_]+):\s+(\S+)\s*$", line)
            if m:
                kv[m.group(1)] = m.group(2)
        if "name" in kv:
            kernels.append(kv)
    return kernels


MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _gfx950_kernels(host_binary, tmp_path):
    """Kernels of every gfx950 code object in the binary's .hip_fatbin section (one
    offload bundle per translation unit, concatenated)."""
    objcopy, bundler, _ = _tools()
    fat = tmp_path / "x.fatbin"
    subprocess.run([objcopy, f"--dump-section=.hip_fatbin={fat}", host_binary, str(tmp_path / "stripped")],
                   check=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    kernels = []
    for i, a in enumerate(starts):
        b = starts[i + 1] if i + 1 < len(starts) else len(data)
        part, co = tmp_path / f"b{i}.bundle", tmp_path / f"b{i}.co"
        part.write_bytes(data[a:b])
        subprocess.run([bundler, "--type=o", f"--input={part}", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--output={co}", "--unbundle"], check=True)
        kernels += _parse_notes(str(co))
    return kernels


def _kernels(tmp_path):
    if not os.path.exists(LIB):
        pytest.skip("the library is not built")
    return _gfx950_kernels(LIB, tmp_path)


def fits(k):
    """True when one workgroup of the kernel's launch bound fits a CU."""
    vgpr, agpr = int(k["vgpr_count"]), int(k.get("agpr_count", 0))
    total = (vgpr + 3) // 4 * 4 + agpr if agpr else vgpr
    waves = -(-int(k["max_flat_workgroup_size"]) // 64)
    per_simd = -(-waves // 4)
    alloc = -(-total // 8) * 8
    return alloc * per_simd <= 512 and int(k["group_segment_fixed_size"]) <= 160 * 1024


def test_every_kernel_fits_its_launch_bound(tmp_path):
    kernels = _kernels(tmp_path)
    assert len(kernels) > 100
    bad = [(k["name"], k["vgpr_count"], k.get("agpr_count"), k["max_flat_workgroup_size"])
           for k in kernels if not fits(k)]
    assert not bad, bad


def test_asm_bound_kernels_shape(tmp_path):
    """The hand-scheduled L1 kernels: the register budget their generated loops assume
    (128 VGPRs at 16 waves, 168 at 12, 256 at 8) and no spills."""
    kernels = {k["name"]: k for k in _kernels(tmp_path)}
    seen = 0
    for name, k in kernels.items():
        m = re.search(r"laplace_(fwd2|fwd3|bwd2)(_seg)?_kernel", name)
        if not m:
            continue
        seen += 1
        waves = int(k["max_flat_workgroup_size"]) // 64
        budget = {16: 128, 12: 168, 8: 256}[waves]
        assert int(k["vgpr_count"]) <= budget, (name, k["vgpr_count"], waves)
        assert int(k.get("vgpr_spill_count", 0)) == 0 and int(k.get("private_segment_fixed_size", 0)) == 0, name
    assert seen >= 20


PROBE = r"""
#include <hip/hip_runtime.h>
__global__ void __launch_bounds__(1024) high_asm(float* o) {
  float x = o[threadIdx.x];
  asm volatile("v_mov_b32 v200, 0" ::: "v200");
  o[threadIdx.x] = x;
}
__global__ void __launch_bounds__(1024) plain(float* o) { o[threadIdx.x] += 1.0f; }
"""


def test_fit_rule_on_the_probe_shape(tmp_path):
    """The shape that aborted a probe's queue (compiled here, never run): inline asm naming
    v200 in a 1024-thread kernel. Without -Werror=inline-asm hipcc only warns and emits a
    201-VGPR kernel, which the rule rejects (4 waves per SIMD x 208 > 512); with the flag
    the product build uses, the same source does not compile."""
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not present")
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    base = [hipcc, "--offload-arch=gfx950", "-O3", "-c", str(src)]
    r = subprocess.run(base + ["-o", str(tmp_path / "probe.o")], capture_output=True, text=True)
    assert r.returncode == 0 and "reserved registers" in r.stderr
    ks = {k["name"]: k for k in _gfx950_kernels(str(tmp_path / "probe.o"), tmp_path)}
    high = next(k for n, k in ks.items() if "high_asm" in n)
    plain = next(k for n, k in ks.items() if "plain" in n)
    assert int(high["vgpr_count"]) == 201 and not fits(high)
    assert fits(plain)
    r = subprocess.run(base + ["-Werror=inline-asm", "-o", str(tmp_path / "probe2.o")], capture_output=True,
                       text=True)
    assert r.returncode != 0 and "reserved registers" in r.stderr
