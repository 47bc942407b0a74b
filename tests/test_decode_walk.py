"""The persistent decode kernel's loader walk against the compute waves' row order (no GPU).

tests/walk_check.cpp includes the kernel's own walk (cudallm_amd/csrc/decode_walk.h) and checks, for every weight
type and segment, that the 1 KiB lines the loader streams are the lines of the rows the compute side multiplies.
The kernel requires grid % 8 == 0 (the qkv rows of a wave's consecutive units are then a fixed stride apart); the
walk must match for every such grid the kernel accepts, and a grid outside that rule must show why it is refused.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
GRIDS_OK = [64, 72, 128, 200, 256, 304, 1024, 4096]


@pytest.fixture(scope="module")
def walk_check(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("walk") / "walk_check"
    cmd = [gxx, "-O1", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           f"-I{ROOT / 'cudallm_amd' / 'csrc'}", str(ROOT / "tests" / "walk_check.cpp"), "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def test_walk_matches_compute_rows_for_accepted_grids(walk_check):
    r = subprocess.run([str(walk_check), *map(str, GRIDS_OK)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.split() == [w for g in GRIDS_OK for w in ("ok", str(g))]


def test_walk_breaks_for_a_grid_the_kernel_refuses(walk_check):
    # 66 workgroups: NW = 264 is not a multiple of 32, so a wave's next qkv unit is not 2 NW rows further on.
    r = subprocess.run([str(walk_check), "66"], capture_output=True, text=True)
    assert r.returncode == 1
    assert "segment 0" in r.stdout
