"""grid_round (floating-point formulation, used by the kernels) against
grid_round_int (integer operations on the bit pattern) on the host: every
f32 of the binades that round to something on grid j, plus special values,
for grids at both ends of the range and in between."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("grids", [["-126", "-125", "-100"], ["0", "100", "127"]])
def test_grid_round_fp_equals_int(tmp_path, grids):
    exe = tmp_path / "grc"
    subprocess.run(["g++", "-O2", "-std=c++17", os.path.join(HERE, "grid_round_check.cpp"), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)] + grids, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.startswith("ok ")
