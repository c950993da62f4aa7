"""GPU parity of the head_dim-64 / 256 bf16 MFMA kernels (tpr_mfma16.hip, through
the C ABI) against the fp64 oracle.

The cases mirror the head_dim-128 MFMA suite (tests/test_gpu_parity.py) and
the cases the SIMT kernels ran at these sizes before: shared prefixes at GQA
ratios 1, 2, 3, 4 and 8 (1, 2 and 4 query heads per forward workgroup), no
prefix, tile-aligned and ragged lengths, a depth-3 tree, an unused node, empty
leaves, a 12-level chain as one key run and as 12 separate runs (the run-list
variant), split prefix tiles (fp32 partials + ordered reduction), seeded
random trees (also the relabelled and deep ones of the head_dim-128 suite,
at head_dim 256 with both dQ plans), and determinism."""

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
    cosine,
    make_inputs,
    max_abs,
    oracle,
    rel_l2,
)

pytestmark = pytest.mark.gpu

_DEEP_LENS = (29, 66, 2, 40, 17, 90, 5, 33, 64, 1, 70, 13)


def _offsets(lens):
    out = [0]
    for n in lens:
        out.append(out[-1] + n)
    return tuple(out)


def _cases():
    from bridge_amd import TPRPrefixMeta as M
    return {
        # name: (meta, hq, hkv)
        "gqa4": (M.shared_prefix(200, [100, 37]), 8, 2),
        "mha": (M.shared_prefix(96, [80]), 4, 4),
        "gqa2": (M.shared_prefix(64, [90]), 4, 2),
        "gqa3": (M.shared_prefix(70, [45, 20]), 6, 2),
        "gqa8": (M.shared_prefix(130, [70, 64]), 8, 1),
        "no_prefix": (M.shared_prefix(0, [70, 33]), 4, 1),
        "tile_aligned": (M.shared_prefix(128, [64, 64, 128]), 8, 2),
        "depth3_tree": (M(cu_seqlens_q=(0, 33, 98, 138, 155), node_offsets=(0, 130, 200, 270),
                          leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2))), 8, 2),
        "unused_node": (M(cu_seqlens_q=(0, 40), node_offsets=(0, 10, 30), leaf_ancestors=((0,),)), 4, 1),
        "empty_leaf": (M.shared_prefix(50, [0, 60, 0]), 4, 1),
        "deep_chain_one_run": (M(cu_seqlens_q=(0, 50, 179, 243), node_offsets=_offsets(_DEEP_LENS),
                                 leaf_ancestors=(tuple(range(12)), tuple(range(9)), tuple(range(3)))), 8, 2),
        "deep_run_list": (M(cu_seqlens_q=(0, 50, 179, 243), node_offsets=_offsets(_DEEP_LENS[::-1]),
                            leaf_ancestors=(tuple(range(11, -1, -1)), tuple(range(11, 2, -1)),
                                            tuple(range(11, 8, -1)))), 8, 2),
        # 64-key tiles: 6 (three pairs at head_dim 256), 3 (a pair and a lone
        # middle tile), 2 with a 1-key mirror, and 5 tiles
        "paired_suffix_tiles": (M.shared_prefix(100, [333, 150, 65, 260]), 8, 2),
    }


def _run(meta, q, k, v, pk, pv, dout, scale, recompute_dq=False):
    from bridge_amd import TPRPrefixAttention
    tensors = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    out, lse = TPRPrefixAttention.apply(*tensors, meta, scale, None, recompute_dq)
    out.backward(dout)
    torch.cuda.synchronize()
    return out.detach(), lse.detach(), [t.grad for t in tensors]


def _check(tag, meta, hq, hkv, d, seed, device, recompute_dq=False):
    scale = 1.0 / math.sqrt(d)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, device, recompute_dq=recompute_dq)
    print(f"[mfma16 {tag}] d={d} hq={hq} hkv={hkv} tq={meta.total_q} tp={meta.total_prefix} "
          f"path={plan.path} mfma={plan.mfma_shape} slots={int(plan.host[25])} recompute_dq={recompute_dq}",
          flush=True)
    assert plan.path == "mfma" and plan.mfma_shape == "16x16x32"
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=seed, device=device)
    out, lse, grads = _run(meta, q, k, v, pk, pv, dout, scale, recompute_dq)
    ro, rl, rg = oracle(meta, q, k, v, pk, pv, dout, scale)
    print(f"  out max_abs={max_abs(out, ro):.3e} cos={cosine(out, ro):.6f} lse max_abs={max_abs(lse, rl):.3e}",
          flush=True)
    for label, g, r in zip(("dq", "dk", "dv", "dpk", "dpv"), grads, rg):
        print(f"  {label}: cos={cosine(g, r):.6f} rel_l2={rel_l2(g, r):.3e}", flush=True)
    assert max_abs(out, ro) <= BF16_FWD_MAX_ABS and cosine(out, ro) >= BF16_FWD_COS
    assert max_abs(lse, rl) <= 1e-3
    for g, r in zip(grads, rg):
        assert cosine(g, r) >= BF16_GRAD_COS
    for g, r in zip(grads[3:], rg[3:]):
        assert rel_l2(g, r) <= BF16_PREFIX_GRAD_REL_L2
    # every 64-key dK/dV tile of every leaf on its own (at head_dim 256 a
    # leaf's tiles are paired with their mirrors): a tile written by the wrong
    # item, or not at all, has a relative error near 1
    for s, (a, b) in enumerate(zip(meta.cu_seqlens_q[:-1], meta.cu_seqlens_q[1:])):
        for k0 in range(a, b, 64):
            for g, r in zip(grads[1:3], rg[1:3]):
                assert rel_l2(g[k0:min(b, k0 + 64)], r[k0:min(b, k0 + 64)]) <= 0.1, (s, k0 - a)
    return grads


@pytest.mark.parametrize("d", [64, 256])
@pytest.mark.parametrize("name", list(_cases()))
def test_mfma16_matches_oracle(name, d, cuda_device):
    meta, hq, hkv = _cases()[name]
    grads = _check(name, meta, hq, hkv, d, seed=5, device=cuda_device)
    if name == "unused_node":
        assert torch.count_nonzero(grads[3][10:]) == 0 and torch.count_nonzero(grads[4][10:]) == 0


@pytest.mark.parametrize("name", list(_cases()))
def test_mfma16_head_dim_256_recomputing_dq_matches_oracle(name, cuda_device):
    """The same cases at head_dim 256 with the recomputing dQ plan (m16_dq
    instead of the dS store and m16_dqs; head_dim 64 always recomputes)."""
    meta, hq, hkv = _cases()[name]
    _check(name, meta, hq, hkv, 256, seed=5, device=cuda_device, recompute_dq=True)


@pytest.mark.parametrize("d", [64, 256])
def test_mfma16_split_prefix_tiles(d, cuda_device):
    """80 query blocks under one prefix: its tiles' query range is split into
    fp32 partials and summed by the reduction in leaf order."""
    from bridge_amd import TPRPrefixMeta
    meta = TPRPrefixMeta.shared_prefix(100, [1300, 1300, 70, 2400])
    plan = meta.plan(4, 1, d, torch.bfloat16, cuda_device)
    assert int(plan.host[25]) > 0  # partial slots
    _check("split", meta, 4, 1, d, seed=9, device=cuda_device)


def _random_meta(seed):
    from bridge_amd import TPRPrefixMeta
    rng = random.Random(seed)
    nseg = rng.randint(5, 14)
    parents = {0: None}
    lengths = {0: rng.choice([0, 64, rng.randint(1, 150)])}
    for s in range(1, nseg):
        parents[s] = rng.randrange(s)
        lengths[s] = rng.choice([0, 64, 128, rng.randint(1, 150), rng.randint(1, 150)])
    meta, _, _ = TPRPrefixMeta.from_segment_tree(parents, lengths)
    return meta


@pytest.mark.parametrize("seed", range(4))
def test_mfma16_random_trees(seed, cuda_device):
    d = (64, 256)[seed % 2]
    hq, hkv = [(8, 2), (4, 4), (6, 2), (4, 1)][seed]
    _check(f"random{seed}", _random_meta(300 + seed), hq, hkv, d, seed=400 + seed, device=cuda_device)


@pytest.mark.parametrize("plan", ["d64", "d256_ds_store", "d256_recompute"])
@pytest.mark.parametrize("seed", range(4))
def test_mfma16_relabelled_random_trees(seed, plan, cuda_device):
    """The head_dim-128 suite's random trees on the 16-wide kernels: node ids
    relabelled (a leaf's ancestors form one to many key runs in prefix_k/v),
    seeds 2 and 3 deep chains whose 11 and 9 runs take the run-list kernels;
    head_dim 64, and 256 with both dQ plans."""
    from test_gpu_random_trees import random_meta
    meta = random_meta(500 + seed, deep=seed >= 2)
    d = 64 if plan == "d64" else 256
    hq, hkv = [(8, 2), (4, 1), (6, 2), (4, 4)][seed]
    runs = int(meta.plan(hq, hkv, d, torch.bfloat16, torch.device("cpu")).host[29])
    assert (runs > 8) == (seed >= 2)
    _check(f"relabelled{seed}", meta, hq, hkv, d, seed=600 + seed, device=cuda_device,
           recompute_dq=plan == "d256_recompute")


@pytest.mark.parametrize("d", [64, 256])
def test_mfma16_is_deterministic(d, cuda_device):
    from bridge_amd import TPRPrefixMeta
    meta = TPRPrefixMeta.shared_prefix(150, [90, 61, 128])
    q, k, v, pk, pv, dout = make_inputs(meta, 8, 2, d, torch.bfloat16, seed=77, device=cuda_device)
    first = _run(meta, q, k, v, pk, pv, dout, 1.0 / math.sqrt(d))
    second = _run(meta, q, k, v, pk, pv, dout, 1.0 / math.sqrt(d))
    assert torch.equal(first[0], second[0]) and torch.equal(first[1], second[1])
    for a, b in zip(first[2], second[2]):
        assert torch.equal(a, b)
