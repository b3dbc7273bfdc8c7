"""The concatenated row plan of the column-split backward (the attention layer's
one launch over K_mm, K_qm and K_km rows): ``tests/b2_plan_check.cpp`` builds the
plan header with the host compiler and checks every planned shape's wave tables
(each row taken once, waves within one source and their register budget, LDS rows
disjoint). CPU only."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_concatenated_row_plan(tmp_path):
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        pytest.skip("no host C++ compiler")
    exe = tmp_path / "b2_plan_check"
    subprocess.run([cxx, "-O2", "-std=c++17", "-Wall", "-Werror", os.path.join(HERE, "b2_plan_check.cpp"), "-o",
                    str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    ok, planned, shapes = out.stdout.split()
    assert ok == "ok" and int(planned) > 1000 and int(shapes) > int(planned), out.stdout
