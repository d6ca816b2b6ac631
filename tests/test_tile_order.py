"""CPU test of the attention launches' workgroup -> (tile, head) mapping
(``map_tile`` / ``tile_order`` in csrc/attn_tiles.h): tests/native/
tile_order_check.cpp is built with hipcc for the host only and checks, over
head counts, tile counts and occupancy targets, that the mapping is a
bijection, keeps each head on XCD bh % 8, and puts the held-back cheap ranks
after every heavy one.  No GPU is used.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "pku-aiprogramming_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

pytestmark = pytest.mark.skipif(not (os.path.exists(HIPCC) or shutil.which("hipcc")), reason="hipcc not available")


def test_tile_order_is_a_bijection_with_xcd_affinity(tmp_path):
    exe = str(tmp_path / "tile_order_check")
    src = os.path.join(ROOT, "tests", "native", "tile_order_check.cpp")
    build = subprocess.run([HIPCC, "--cuda-host-only", "-x", "hip", "-std=c++17", "-O1", "-I", CSRC,
                            "-I", os.path.join(ROOT, "include"), src, "-o", exe],
                           stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert build.returncode == 0, build.stdout
    run = subprocess.run([exe], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=120)
    assert run.returncode == 0, run.stdout[-4000:]
    assert "tile order checks passed" in run.stdout
