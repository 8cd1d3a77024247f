"""CPU check of the grouped GEMM kernels' persistent-grid tile schedule
(csrc/gemm_sched.hpp, shared by the kernels and their launchers): every tile is
run exactly once, the launchers' grid keeps each workgroup within the LDS row
table of the gathered kernels (which compute nothing past it), and the panel
order of a group's tiles is a bijection. The C++
check is built with g++ from tests/gemm_schedule_check.cpp."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_gemm_schedule_covers_every_tile_and_fits_the_row_table(tmp_path):
    exe = tmp_path / "gemm_schedule_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror",
                    os.path.join(HERE, "gemm_schedule_check.cpp"), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.strip() == "OK", res.stdout + res.stderr
