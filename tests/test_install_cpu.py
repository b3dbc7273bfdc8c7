"""The drop-in installs like the reference's extension: ``pip install .`` puts a
top-level ``Laplace_subtraction_cuda`` module (reference setup.py:7-40) next to the
``laplacianformer_amd`` package, importable from a fresh interpreter that does not
see this repository, with the reference's ten exports (src/wrapper.cpp:73-99)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

REFERENCE_EXPORTS = [
    "get_compiler_version", "get_cuda_version", "has_cuda",
    "LaplaceSubtraction_forward", "LaplaceSubtraction_backward_query", "LaplaceSubtraction_backward_key",
    "LaplaceSubtraction_reduce_forward", "NewtonInverse_forward", "NewtonInverse_backward",
    "NewtonInverse_is_supported",
]


def test_pip_install_dropin(tmp_path):
    target = tmp_path / "site"
    env = dict(os.environ, PIP_DISABLE_PIP_VERSION_CHECK="1", PIP_NO_INPUT="1")
    r = subprocess.run([sys.executable, "-m", "pip", "install", "--no-deps", "--no-build-isolation", "--no-index",
                        "--target", str(target), ROOT],
                       capture_output=True, text=True, timeout=1200, env=env)
    assert r.returncode == 0, (r.stdout[-4000:], r.stderr[-4000:])
    assert (target / "Laplace_subtraction_cuda.so").exists()
    assert (target / "laplacianformer_amd" / "liblfamd.so").exists()
    code = (
        "import sys, Laplace_subtraction_cuda as m\n"
        f"names = {REFERENCE_EXPORTS!r}\n"
        "missing = [n for n in names if not callable(getattr(m, n, None))]\n"
        "assert not missing, missing\n"
        "assert isinstance(m.NewtonInverse_is_supported(64), bool)\n"
        "print(m.__file__)\n"
        "import laplacianformer_amd\n"
        "print(laplacianformer_amd.__file__)\n"
    )
    env2 = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    env2["PYTHONPATH"] = str(target)
    r = subprocess.run([sys.executable, "-c", code], cwd=str(tmp_path), capture_output=True, text=True,
                       timeout=600, env=env2)
    assert r.returncode == 0, (r.stdout[-4000:], r.stderr[-4000:])
    lines = r.stdout.strip().splitlines()
    assert lines[0].startswith(str(target)), lines
    assert lines[1].startswith(str(target)), lines
