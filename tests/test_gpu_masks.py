"""GPU: physical key masks -- the reference's custom-mask mode
(rectangular_attention.py:112-122, sparse mode 0: the mask is the only
visibility rule) -- on the masked SIMT kernels, through the C ABI, against the
fp64 oracle (oracle/tpr_oracle.py tree_forward / tree_backward with ``mask``).

Masks are random (about 40% of each row's keys hidden, so rows also see later
keys of their own suffix) with a few rows that see no key at all, which must
come out as output 0, lse -inf and zero gradient. The trees are fixed cases
and the relabelled (and deep) random trees of the head_dim-128 suite."""

from __future__ import annotations

import math

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
    random_key_mask,
    rel_l2,
    tree_of,
)

pytestmark = pytest.mark.gpu


def _cases():
    from bridge_amd import TPRPrefixMeta as M
    return {
        # name: (meta, hq, hkv, rows that see no key)
        "single_leaf_gqa2": (M.shared_prefix(70, [90]), 4, 2, (0, 89)),
        "siblings_empty_leaf": (M.shared_prefix(100, [64, 37, 0, 80]), 8, 2, (63, 100)),
        "depth3_tree": (M(cu_seqlens_q=(0, 33, 98, 138, 155), node_offsets=(0, 130, 200, 270),
                          leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2))), 8, 2, (40,)),
        "no_prefix": (M.shared_prefix(0, [70, 33]), 4, 1, ()),
    }


KINDS = [(torch.float32, 64), (torch.float32, 96), (torch.bfloat16, 64), (torch.bfloat16, 128),
         (torch.bfloat16, 256)]


@pytest.mark.parametrize("dtype, d", KINDS, ids=[f"{str(t).split('.')[1]}_d{d}" for t, d in KINDS])
@pytest.mark.parametrize("name", ["single_leaf_gqa2", "siblings_empty_leaf", "depth3_tree", "no_prefix"])
def test_masked_kernels_match_oracle(name, dtype, d, cuda_device):
    meta, hq, hkv, empty = _cases()[name]
    _check_masked(name, meta, hq, hkv, empty, dtype, d, d + len(name), cuda_device)


@pytest.mark.parametrize("dtype, d", [(torch.float32, 64), (torch.bfloat16, 128)], ids=["float32_d64", "bfloat16_d128"])
@pytest.mark.parametrize("seed", range(3))
def test_masked_kernels_on_relabelled_random_trees(seed, dtype, d, cuda_device):
    """The head_dim-128 suite's random trees (node ids relabelled, seed 2 a
    deep chain with side branches) under random masks, the first and last
    query rows seeing no key."""
    from test_gpu_random_trees import random_meta
    meta = random_meta(800 + seed, deep=seed == 2)
    assert meta.total_q > 1
    _check_masked(f"random{seed}", meta, (4, 8, 6)[seed], 2, (0, meta.total_q - 1), dtype, d, 900 + seed,
                  cuda_device)


def _check_masked(name, meta, hq, hkv, empty, dtype, d, mask_seed, cuda_device):
    from bridge_amd import tpr_prefix_attention
    scale = 1.0 / math.sqrt(d)
    mask = random_key_mask(tree_of(meta), torch.Generator().manual_seed(mask_seed), empty_rows=empty)
    plan = meta.plan(hq, hkv, d, dtype, cuda_device, masked=True)
    assert plan.path == "simt" and plan.masked
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, dtype, seed=17, device=cuda_device)
    print(f"[masked {name} {dtype} d{d}] mask {tuple(mask.shape)}, {len(empty)} empty rows", flush=True)
    tensors = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    out, lse = tpr_prefix_attention(*tensors, meta, scale, attention_mask=mask.to(cuda_device))
    out.backward(dout)
    torch.cuda.synchronize()
    grads = [t.grad for t in tensors]
    ro, rl, rg = oracle(meta, q, k, v, pk, pv, dout, scale, mask=mask)
    # rows that see no key: output 0, lse -inf, no query gradient
    for r in empty:
        assert torch.count_nonzero(out[r]) == 0 and torch.count_nonzero(grads[0][r]) == 0
        assert bool(torch.isneginf(lse[:, r]).all())
    seen = torch.ones(meta.total_q, dtype=torch.bool)
    seen[list(empty)] = False
    lse_c, rl_c = lse.cpu()[:, seen], rl[:, seen]
    if dtype == torch.float32:
        assert max_abs(out, ro) <= FP32_TOL and max_abs(lse_c, rl_c) <= FP32_TOL
        for g, r in zip(grads, rg):
            assert max_abs(g, r) <= FP32_TOL
        return
    assert max_abs(out, ro) <= BF16_FWD_MAX_ABS and cosine(out, ro) >= BF16_FWD_COS
    assert max_abs(lse_c, rl_c) <= 1e-3
    for g, r in zip(grads, rg):
        assert cosine(g, r) >= BF16_GRAD_COS
    for g, r in zip(grads[3:], rg[3:]):
        if r.numel():
            assert rel_l2(g, r) <= BF16_PREFIX_GRAD_REL_L2


def test_causal_mask_on_the_masked_kernels_equals_the_causal_kernels(cuda_device):
    """fp32: the causal mask passed as a physical mask (masked kernels, every
    suffix key streamed) gives the unmasked SIMT kernels' results."""
    from bridge_amd import TPRPrefixMeta, tpr_prefix_attention
    meta = TPRPrefixMeta.shared_prefix(50, [70, 33])
    tree = tree_of(meta)
    mask = torch.ones(meta.total_q, meta.max_keys(), dtype=torch.bool)
    for s in range(meta.num_leaves):
        a, b = tree.leaf_range(s)
        for i in range(b - a):
            mask[a + i, :50 + i + 1] = False
    q, k, v, pk, pv, dout = make_inputs(meta, 4, 2, 64, torch.float32, seed=5, device=cuda_device)
    results = []
    for m in (None, mask.to(cuda_device)):
        tensors = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
        out, lse = tpr_prefix_attention(*tensors, meta, 0.125, attention_mask=m)
        out.backward(dout)
        torch.cuda.synchronize()
        results.append([out.detach(), lse] + [t.grad for t in tensors])
    for x, y in zip(*results):
        assert max_abs(x, y) <= 1e-6


def test_mask_contract_errors(cuda_device):
    from bridge_amd import TPRPrefixMeta, tpr_prefix_attention
    meta = TPRPrefixMeta.shared_prefix(8, [4, 6])
    q, k, v, pk, pv, _ = make_inputs(meta, 4, 2, 64, torch.bfloat16, seed=1, device=cuda_device)
    good = torch.zeros(10, 14, dtype=torch.bool, device=cuda_device)
    tpr_prefix_attention(q, k, v, pk, pv, meta, attention_mask=good)
    with pytest.raises(TypeError, match="torch.Tensor or None"):
        tpr_prefix_attention(q, k, v, pk, pv, meta, attention_mask=[[False]])
    with pytest.raises(ValueError, match="torch.bool"):
        tpr_prefix_attention(q, k, v, pk, pv, meta, attention_mask=good.to(torch.uint8))
    with pytest.raises(ValueError, match="must be on"):
        tpr_prefix_attention(q, k, v, pk, pv, meta, attention_mask=good.cpu())
    with pytest.raises(ValueError, match="L >= 14"):
        tpr_prefix_attention(q, k, v, pk, pv, meta, attention_mask=good[:, :13])
    with pytest.raises(ValueError, match="shape"):
        tpr_prefix_attention(q, k, v, pk, pv, meta, attention_mask=good[:9])
