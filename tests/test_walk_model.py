"""CPU: the persistent GEMMs' tile walk covers every output tile exactly once.

Builds tests/walk_model.cpp, which compiles the kernels' own TileWalk (afd_common.h) as host
code, and runs it: every row-tile count 1..300 with 1-16 column tiles and grids of 3-256
workgroups (split over the 8 XCDs or not), with the 2-row blocks of the MXFP4 GEMMs, the
4-row blocks of the bf16-activation GEMMs and the 8-row blocks of the FP8 GEMMs, statically and
with the dynamic claims interleaved in a seeded random order."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def test_every_tile_taken_once(tmp_path):
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc is not available to build the host model")
    exe = tmp_path / "walk_model"
    subprocess.run([HIPCC, "-O2", "-std=c++17", "-x", "hip", "--cuda-host-only",
                    os.path.join(HERE, "walk_model.cpp"), "-o", str(exe)], check=True,
                   stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    res = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=300)
    assert res.returncode == 0, res.stdout
    assert res.stdout.startswith("ok: 72000 walks"), res.stdout
