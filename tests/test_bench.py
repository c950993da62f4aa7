"""CPU checks of bench.py's accounting: the workloads are the benchmark
configurations with the visible-pair and FLOP counts the reference's
benchmark table states (14 * Hq * D * sum of visible pairs for fwd + bwd),
the multi-GPU request is refused, and roofline.traffic comes from the
committed HBM-traffic profile of its own workload only."""

from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def _flops(name):
    _, meta, hq, _, d, _ = bench.workload(name)
    pairs = meta.visible_pairs()
    return pairs, 14 * hq * d * pairs


@pytest.mark.parametrize("name, pairs, tflop", [
    ("plumbing-fp32", 786_944, 0.00282),     # prefix 512 + 2 x 512, MHA 4, d64
    ("qwen3-4b", 100_671_488, 5.773),        # prefix 4096 + 4 x 4096, GQA 32/8, d128
    ("long-session", 553_656_320, 31.75),    # prefix 32768 + 8 x 2048
    ("turn-tree", 58_728_448, 3.368),        # leaf level of root 2048 -> 4 x 1024 -> 16 x 1024
])
def test_workload_pairs_and_flops_match_the_benchmark_table(name, pairs, tflop):
    got_pairs, flops = _flops(name)
    assert got_pairs == pairs
    assert flops / 1e12 == pytest.approx(tflop, rel=1e-3)


def test_headline_flops_exactly():
    pairs, flops = _flops("qwen3-4b")
    # S_i P + S_i (S_i + 1) / 2 per sibling, four siblings
    assert pairs == 4 * (4096 * 4096 + 4096 * 4097 // 2)
    assert flops == 5_772_905_807_872


def test_ragged_workload_is_the_seeded_draw():
    import torch
    _, meta, hq, hkv, d, dtype = bench.workload("ragged")
    g = torch.Generator(device="cpu").manual_seed(0)
    lens = torch.randint(256, 8193, (16,), generator=g).tolist()
    assert meta.suffix_lengths() == tuple(lens) and meta.total_prefix == 8192
    assert (hq, hkv, d, dtype) == (32, 8, 128, torch.bfloat16)
    assert meta.visible_pairs() == sum(s * 8192 + s * (s + 1) // 2 for s in lens)


def test_turn_tree_shape():
    _, meta, *_ = bench.workload("turn-tree")
    assert meta.num_leaves == 16 and meta.suffix_lengths() == (1024,) * 16
    # every leaf sees the root (2048) and its branch (1024) in full
    assert all(meta.prefix_length(i) == 3072 for i in range(16))


def test_traffic_comes_from_the_own_workloads_profile():
    with open(os.path.join(ROOT, "profiles", "hbm_traffic.json")) as f:
        data = json.load(f)
    assert data["workload"] == "qwen3-4b"
    e = data["per_launch"]["tpr::mfma_dkdv"]
    assert bench.traffic_bytes("qwen3-4b", "tpr::mfma_dkdv") == e["read_bytes"] + e["write_bytes"]
    assert bench.traffic_bytes("long-session", "tpr::mfma_dkdv") is None
    assert bench.traffic_bytes("qwen3-4b", "tpr::no_such_kernel") is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""
