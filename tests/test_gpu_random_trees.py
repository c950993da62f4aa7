"""GPU parity on seeded random prefix trees (through the C ABI) against the fp64 oracle.

Each case draws a random segment tree (segments attach to a random earlier
segment; lengths 0..150, so empty nodes and leaves occur), lowers it with
``TPRPrefixMeta.from_segment_tree`` (the reference's SegmentPlan order,
segment_plan.py:266-275), then relabels the prefix nodes with a random
permutation. The relabelling moves the nodes around in prefix_k/v, so a
leaf's ancestors form anywhere from one key run to one run per node, while
the attention each leaf computes is unchanged."""

from __future__ import annotations

import math
import random

import pytest
import torch

from _helpers import (
    BF16_FWD_COS,
    BF16_FWD_MAX_ABS,
    BF16_GRAD_COS,
    BF16_PREFIX_GRAD_REL_L2,
    FP32_TOL,
    cosine,
    make_inputs,
    max_abs,
    oracle,
    rel_l2,
)

pytestmark = pytest.mark.gpu


def random_meta(seed: int, deep: bool = False):
    """deep: 24-40 segments, each attached to the previous one with probability
    0.75 (long chains with side branches, so leaves reach 9+ ancestors)."""
    from bridge_amd import TPRPrefixMeta
    rng = random.Random(seed)
    nseg = rng.randint(24, 40) if deep else rng.randint(5, 16)
    parents = {0: None}
    lengths = {0: rng.choice([0, 64, rng.randint(1, 150)])}
    for s in range(1, nseg):
        parents[s] = s - 1 if deep and rng.random() < 0.75 else rng.randrange(s)
        lengths[s] = rng.choice([0, 64, 128, rng.randint(1, 150), rng.randint(1, 150)])
    meta, _, _ = TPRPrefixMeta.from_segment_tree(parents, lengths)
    m = meta.num_nodes
    perm = list(range(m))
    rng.shuffle(perm)                       # old node id -> new node id
    node_len = [meta.node_offsets[n + 1] - meta.node_offsets[n] for n in range(m)]
    new_len = [0] * m
    for old, new in enumerate(perm):
        new_len[new] = node_len[old]
    offsets = [0]
    for n in range(m):
        offsets.append(offsets[-1] + new_len[n])
    ancestors = tuple(tuple(perm[n] for n in path) for path in meta.leaf_ancestors)
    return TPRPrefixMeta(meta.cu_seqlens_q, tuple(offsets), ancestors)


def _run(meta, q, k, v, pk, pv, dout, scale, recompute_dq=False):
    from bridge_amd import TPRPrefixAttention
    tensors = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    out, lse = TPRPrefixAttention.apply(*tensors, meta, scale, None, recompute_dq)
    out.backward(dout)
    torch.cuda.synchronize()
    return out.detach(), lse.detach(), [t.grad for t in tensors]


def _describe(meta, plan):
    runs = int(plan.host[29])
    return (f"leaves={meta.num_leaves} nodes={meta.num_nodes} depth={meta.max_depth} tq={meta.total_q} "
            f"tp={meta.total_prefix} max_key_runs={runs} path={plan.path}")


HEADS = [(8, 2), (4, 4), (6, 2), (4, 1)]


@pytest.mark.parametrize("recompute_dq", [False, True], ids=["ds_store", "recompute"])
@pytest.mark.parametrize("seed", range(10))
def test_random_tree_mfma_bf16(seed, recompute_dq, cuda_device):
    """Both dQ plans: from the dS store, and recomputing S and dP; seeds 8
    and 9 are deep trees whose leaves have more key runs than the kernels
    hold in registers (the run-list instances)."""
    meta = random_meta(seed, deep=seed >= 8)
    hq, hkv = HEADS[seed % len(HEADS)]
    d = 128
    scale = 1.0 / math.sqrt(d)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device, recompute_dq=recompute_dq)
    print(f"[random mfma seed={seed} recompute_dq={recompute_dq}] hq={hq} hkv={hkv} {_describe(meta, plan)}",
          flush=True)
    assert plan.path == "mfma" and plan.dq_from_ds == (not recompute_dq)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=100 + seed, device=cuda_device)
    out, lse, grads = _run(meta, q, k, v, pk, pv, dout, scale, recompute_dq)
    ro, rl, rg = oracle(meta, q, k, v, pk, pv, dout, scale)
    print(f"  out max_abs={max_abs(out, ro):.3e} cos={cosine(out, ro):.6f} lse max_abs={max_abs(lse, rl):.3e}",
          flush=True)
    assert max_abs(out, ro) <= BF16_FWD_MAX_ABS and cosine(out, ro) >= BF16_FWD_COS
    assert max_abs(lse, rl) <= 1e-3
    for label, g, r in zip(("dq", "dk", "dv", "dpk", "dpv"), grads, rg):
        print(f"  {label}: cos={cosine(g, r):.6f} rel_l2={rel_l2(g, r):.3e}", flush=True)
        assert cosine(g, r) >= BF16_GRAD_COS
    for g, r in zip(grads[3:], rg[3:]):
        assert rel_l2(g, r) <= BF16_PREFIX_GRAD_REL_L2


@pytest.mark.parametrize("seed", range(4))
def test_random_tree_simt_fp32(seed, cuda_device):
    meta = random_meta(1000 + seed)
    hq, hkv = HEADS[seed % len(HEADS)]
    d = 64
    scale = 1.0 / math.sqrt(d)
    plan = meta.plan(hq, hkv, d, torch.float32, cuda_device)
    print(f"[random simt seed={seed}] hq={hq} hkv={hkv} {_describe(meta, plan)}", flush=True)
    assert plan.path == "simt"
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.float32, seed=200 + seed, device=cuda_device)
    out, lse, grads = _run(meta, q, k, v, pk, pv, dout, scale)
    ro, rl, rg = oracle(meta, q, k, v, pk, pv, dout, scale)
    assert max_abs(out, ro) <= FP32_TOL and max_abs(lse, rl) <= FP32_TOL
    for g, r in zip(grads, rg):
        assert max_abs(g, r) <= FP32_TOL
