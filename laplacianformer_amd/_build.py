"""In-tree build of the two native libraries.

* ``liblfamd.so`` - the gfx950 HIP kernels behind the C ABI of
  ``include/laplacianformer_amd.h`` (hipcc, no PyTorch dependency).
* ``Laplace_subtraction_cuda.so`` - the drop-in PyTorch extension with the
  reference module name and exports (reference ``setup.py:8-33``,
  ``src/wrapper.cpp:73-99``), compiled with g++ against the PyTorch-ROCm headers
  and linked to ``liblfamd.so``. Sources are already HIP, so no hipify step runs.

Both land next to this file so that they travel with the repository tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "liblfamd.so")
EXT_NAME = "Laplace_subtraction_cuda"
EXT_PATH = os.path.join(PKG_DIR, EXT_NAME + ".so")

HIP_SOURCES = ["laplace_kernels.hip", "laplace_bwd2.hip", "laplace_fwd2.hip", "newton_kernels.hip", "mix_kernels.hip",
               "layer_kernels.hip", "lf_runtime.hip", "laplace_noalloc.hip"]
TORCH_SOURCES = ["wrapper.cpp", "LaplaceSubtraction_hip.cpp", "NewtonInverse_hip.cpp", "LaplacianAttention_hip.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Packed fp32 VALU ops are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Inline asm naming a register above what a kernel's launch bounds allow
    # only draws a warning, and gives a kernel whose workgroup cannot be
    # dispatched: make it a build error.
    "-Werror=inline-asm",
    "-Wno-unused-command-line-argument",
]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}):\n{' '.join(cmd)}\n{r.stdout}")
    return r.stdout


def _torch_paths():
    import torch
    from torch.utils import cpp_extension as ce

    inc = ce.include_paths(device_type="cuda")
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, libdir, abi


def generate(verbose=False):
    """Writes csrc/l1_asm_gen.h from csrc/gen_l1_asm.py (unchanged files are left alone)."""
    _run([sys.executable, os.path.join(CSRC, "gen_l1_asm.py"), os.path.join(CSRC, "l1_asm_gen.h")], verbose)


def build_hip(verbose=False, jobs=4):
    os.makedirs(BUILD_DIR, exist_ok=True)
    generate(verbose)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        objs.append(obj)
        cmds.append([HIPCC, *HIP_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs,
          "-Wl,-soname,liblfamd.so"], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def build_torch_ext(verbose=False, jobs=4):
    inc, libdir, abi = _torch_paths()
    os.makedirs(BUILD_DIR, exist_ok=True)
    py_inc = sysconfig.get_paths()["include"]
    cflags = [
        "-O2", "-std=c++17", "-fPIC", "-DWITH_HIP", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-unused-function", "-Wno-deprecated-declarations",
        *[f"-I{p}" for p in inc], f"-I{py_inc}", f"-I{os.path.join(CSRC, 'torch', 'include')}",
    ]
    objs = []
    cmds = []
    for src in TORCH_SOURCES:
        obj = os.path.join(BUILD_DIR, "torch_" + src + ".o")
        objs.append(obj)
        cmds.append(["g++", *cflags, "-c", os.path.join(CSRC, "torch", src), "-o", obj])
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = EXT_PATH + ".tmp"
    _run(["g++", "-shared", "-fPIC", "-o", tmp, *objs,
          f"-L{PKG_DIR}", "-llfamd", f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
          "-ltorch_hip", "-ltorch_python", "-lamdhip64",
          # $ORIGIN: next to liblfamd.so inside the package; $ORIGIN/laplacianformer_amd:
          # the same file installed as the top-level module next to the package (setup.py).
          "-Wl,-rpath,$ORIGIN", "-Wl,-rpath,$ORIGIN/laplacianformer_amd", f"-Wl,-rpath,{libdir}"], verbose)
    os.replace(tmp, EXT_PATH)
    return EXT_PATH


def build(verbose=False):
    """Compile both libraries (always recompiles)."""
    build_hip(verbose)
    build_torch_ext(verbose)
    return LIB_PATH, EXT_PATH


def _newest(paths):
    return max((os.path.getmtime(p) for p in paths if os.path.exists(p)), default=0.0)


def build_if_stale(verbose=False):
    """Compile what is missing or older than its sources (setup.py's build step)."""
    hip_inputs = [os.path.join(CSRC, f) for f in os.listdir(CSRC)
                  if f.endswith((".hip", ".h", ".py")) and f != "l1_asm_gen.h"]
    hip_inputs.append(os.path.join(REPO_DIR, "include", "laplacianformer_amd.h"))
    hip_inputs.append(os.path.abspath(__file__))
    if not os.path.exists(LIB_PATH) or os.path.getmtime(LIB_PATH) < _newest(hip_inputs):
        build_hip(verbose)
    tdir = os.path.join(CSRC, "torch")
    torch_inputs = [os.path.join(tdir, f) for f in os.listdir(tdir) if f.endswith(".cpp")]
    torch_inputs += [os.path.join(tdir, "include", f) for f in os.listdir(os.path.join(tdir, "include"))]
    torch_inputs += [LIB_PATH, os.path.abspath(__file__)]
    if not os.path.exists(EXT_PATH) or os.path.getmtime(EXT_PATH) < _newest(torch_inputs):
        build_torch_ext(verbose)
    return LIB_PATH, EXT_PATH


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", LIB_PATH, EXT_PATH)
