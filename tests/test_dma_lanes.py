"""Host check of the lane offsets the grouped global -> LDS copies use
(dma_blocks4 / dma_blocks4_nt, tpr_kernel_util.h): blocks 1-3 of a group are
addressed through the instruction offset 1024 j, so each lane's register
holds v_j - 1024 j as an unsigned 32-bit offset, and must not wrap. A wrapped
offset made one development variant read about 4 GB out of bounds.

tests/dma_lanes_check.cpp is compiled with g++ against the header the kernels
take their offset functions from (bridge_amd/csrc/tpr_lanes.h) and run for
the row strides of every committed test and benchmark plan: for each lane,
wave and block it checks no wrap, the row and chunk bounds, the swizzle and
that every 16-byte chunk of a tile or dS block is fetched exactly once. CPU
only."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# (Hq, Hkv) of the plans the tests and bench.py build on the MFMA paths
HEADS = [(32, 8), (16, 8), (32, 4), (28, 4), (8, 2), (4, 4), (6, 2), (16, 2), (4, 1), (8, 1), (4, 2),
         (2, 2), (12, 4), (1, 1), (64, 8), (64, 64)]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not found")
    out = str(tmp_path_factory.mktemp("lanes") / "dma_lanes_check")
    subprocess.run([gxx, "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "bridge_amd", "csrc"),
                    os.path.join(ROOT, "tests", "dma_lanes_check.cpp"), "-o", out], check=True)
    return out


def test_grouped_copy_offsets_do_not_wrap_and_stay_in_bounds(checker):
    strides = sorted({256 * h for hq, hkv in HEADS for h in (hq, hkv)})
    run = subprocess.run([checker, *map(str, strides)], stdout=subprocess.PIPE, text=True)
    print(run.stdout)
    assert run.returncode == 0 and run.stdout.strip().endswith("ok")
    assert int(run.stdout.split("checks ")[1].split()[0]) == len(strides) * 4 * 64 * 4 + 2 * 64 * 4


def test_checker_catches_the_partial_tile_wrap(checker):
    """The development fault: a partial tile (rows clamped to its last row)
    given to the immediate-offset grouped copy. With one row, block 1's
    register would be 0 * stride + chunk - 1024 < 0, i.e. wrapped; the checker
    reports it (the kernels copy partial tiles with dma_blocks4_m0, which
    steps M0 and passes the offsets unchanged)."""
    run = subprocess.run([checker, "--clamped", "1", "2048"], stdout=subprocess.PIPE, text=True)
    assert run.returncode == 1 and "clamped tile wraps" in run.stdout
    # a full-length "partial" tile is the full tile: no wrap
    run = subprocess.run([checker, "--clamped", "64", "2048"], stdout=subprocess.PIPE, text=True)
    assert run.returncode == 0
