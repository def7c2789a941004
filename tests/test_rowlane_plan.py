"""CPU test of the row-per-lane matvec's launch planning (arm_ai_amd/csrc/rl_plan.h).

The header is plain C++ that k_rowlane.hip plans every launch with; here it is
compiled with g++ and swept over every weight kind, 1-64 groups and rows up to
300000: each planned grid must pass the check that every launch passes
(`rl::grid_ok`), cover every row, and the check must refuse grids with a
workgroup past the chunks -- among them the 512-workgroup persistent grid on a
286-chunk shape that faulted during development (a chunk past the rows made
an out-of-range weight descriptor)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ is not installed")
def test_rowlane_launch_plans_pass_the_grid_check(tmp_path):
    exe = str(tmp_path / "rl_plan_check")
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-o", exe,
                    os.path.join(HERE, "c", "rl_plan_check.cc")], check=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failures" in r.stdout
