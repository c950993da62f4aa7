"""GPU: a forest of rollout tries lowered to ONE launch (every segment of every
tree, all levels) matches the oracle's per-segment visits of the same trees
(the reference executor's order, kv_stack.py:139-154) in fp32.

The prefix K/V are ``k.index_select(0, prefix_index)`` inside autograd, so the
gradient that reaches k/v already includes every descendant's contribution."""

from __future__ import annotations

import math

import pytest
import torch

from _helpers import BF16_FWD_COS, BF16_FWD_MAX_ABS, BF16_GRAD_COS, cosine, max_abs

pytestmark = pytest.mark.gpu


def _rollouts(seed):
    """3 uid groups of 4-6 rollouts: shared prompts, partly shared responses."""
    g = torch.Generator().manual_seed(seed)
    keys, rows = [], []
    for u in range(3):
        prompt = torch.randint(0, 50000, (int(torch.randint(150, 600, (1,), generator=g)),), generator=g)
        firsts = []
        for i in range(int(torch.randint(4, 7, (1,), generator=g))):
            if firsts and torch.rand(1, generator=g).item() < 0.5:
                base = firsts[int(torch.randint(0, len(firsts), (1,), generator=g))]
                cut = int(torch.randint(1, base.numel() + 1, (1,), generator=g))
                tail = torch.randint(0, 50000, (int(torch.randint(1, 300, (1,), generator=g)),), generator=g)
                row = torch.cat([prompt, base[:cut], tail])
            else:
                resp = torch.randint(0, 50000, (int(torch.randint(50, 400, (1,), generator=g)),), generator=g)
                firsts.append(resp)
                row = torch.cat([prompt, resp])
            keys.append(f"uid{u}_s_{i}")
            rows.append(row)
    return keys, {"input_ids": rows}


def test_lowered_forest_matches_the_per_segment_visits(cuda_device):
    from bridge_amd import TPRPrefixAttention
    from bridge_amd.topology import build_trajectory_trees, lower_forest
    from oracle.trie_oracle import segment_visits
    keys, batch = _rollouts(3)
    trees = build_trajectory_trees(keys, batch)
    launch = lower_forest(trees)
    meta = launch.meta
    hq, hkv, d = 8, 2, 128
    scale = 1.0 / math.sqrt(d)
    tq = meta.total_q
    depth = max(len(a) for a in meta.leaf_ancestors)
    print(f"[forest] trees={len(trees)} segments={meta.num_leaves} prefix_nodes={meta.num_nodes} "
          f"tq={tq} tp={meta.total_prefix} depth={depth}", flush=True)
    assert meta.num_nodes > 3 and depth >= 2    # the case covers multi-level trees

    g = torch.Generator().manual_seed(9)
    q, k, v, dout = (torch.randn(tq, h, d, generator=g).bfloat16().to(cuda_device) for h in (hq, hkv, hkv, hq))
    qa, ka, va = (x.clone().requires_grad_(True) for x in (q, k, v))
    index = launch.prefix_index.to(cuda_device)
    out, _ = TPRPrefixAttention.apply(qa, ka, va, ka.index_select(0, index), va.index_select(0, index), meta, scale)
    out.backward(dout)
    torch.cuda.synchronize()

    spans = [(meta.cu_seqlens_q[i], meta.cu_seqlens_q[i + 1]) for i in range(meta.num_leaves)]
    seg_index = {seg: i for i, seg in enumerate(launch.segments)}
    parents = []
    for t, node_id in launch.segments:
        p = trees[t].get(node_id).parent_id
        parents.append(None if p is None else seg_index[(t, p)])
    qr, kr, vr = (x.float().clone().requires_grad_(True) for x in (q, k, v))
    ref = segment_visits(qr, kr, vr, spans, parents, scale)
    ref.backward(dout.float())

    print(f"  out: max_abs={max_abs(out, ref):.3e} cos={cosine(out, ref):.6f}", flush=True)
    assert max_abs(out, ref) <= BF16_FWD_MAX_ABS and cosine(out, ref) >= BF16_FWD_COS
    for label, a, b in (("dq", qa.grad, qr.grad), ("dk", ka.grad, kr.grad), ("dv", va.grad, vr.grad)):
        print(f"  {label}: cos={cosine(a, b):.6f}", flush=True)
        assert cosine(a, b) >= BF16_GRAD_COS


def test_forest_deeper_than_the_mfma_path_runs_on_the_simt_kernels(cuda_device):
    """A chain of 11 branchings (12 levels, beyond the MFMA path's 8 ancestors)
    lowered to one launch: the planner picks the SIMT kernels, and the result
    matches the per-segment visits."""
    from bridge_amd import TPRPrefixAttention
    from bridge_amd.topology import build_trajectory_trees, lower_forest
    from oracle.trie_oracle import segment_visits
    g = torch.Generator().manual_seed(4)
    spine = torch.randint(0, 1000, (12 * 24,), generator=g)
    # row i shares 24 (i + 1) tokens of the spine, then diverges for 16 tokens
    rows = [torch.cat([spine[:24 * (i + 1)], torch.randint(1000, 2000, (16,), generator=g)]) for i in range(11)]
    rows.append(spine.clone())
    trees = build_trajectory_trees([f"u_s_{i}" for i in range(len(rows))], {"input_ids": rows})
    launch = lower_forest(trees)
    meta = launch.meta
    depth = max(len(a) for a in meta.leaf_ancestors)
    hq, hkv, d = 4, 2, 128
    assert depth > 8
    assert meta.plan(hq, hkv, d, torch.bfloat16, cuda_device).path == "simt"
    print(f"[deep] segments={meta.num_leaves} depth={depth} tq={meta.total_q}", flush=True)
    scale = 1.0 / math.sqrt(d)
    q, k, v, dout = (torch.randn(meta.total_q, x, d, generator=g).bfloat16().to(cuda_device) for x in (hq, hkv, hkv, hq))
    qa, ka, va = (x.clone().requires_grad_(True) for x in (q, k, v))
    index = launch.prefix_index.to(cuda_device)
    out, _ = TPRPrefixAttention.apply(qa, ka, va, ka.index_select(0, index), va.index_select(0, index), meta, scale)
    out.backward(dout)
    torch.cuda.synchronize()
    spans = [(meta.cu_seqlens_q[i], meta.cu_seqlens_q[i + 1]) for i in range(meta.num_leaves)]
    seg_index = {seg: i for i, seg in enumerate(launch.segments)}
    parents = []
    for t, node_id in launch.segments:
        p = trees[t].get(node_id).parent_id
        parents.append(None if p is None else seg_index[(t, p)])
    qr, kr, vr = (x.float().clone().requires_grad_(True) for x in (q, k, v))
    ref = segment_visits(qr, kr, vr, spans, parents, scale)
    ref.backward(dout.float())
    print(f"  out: max_abs={max_abs(out, ref):.3e} cos={cosine(out, ref):.6f}", flush=True)
    assert max_abs(out, ref) <= BF16_FWD_MAX_ABS and cosine(out, ref) >= BF16_FWD_COS
    for label, a_, b_ in (("dq", qa.grad, qr.grad), ("dk", ka.grad, kr.grad), ("dv", va.grad, vr.grad)):
        print(f"  {label}: cos={cosine(a_, b_):.6f}", flush=True)
        assert cosine(a_, b_) >= BF16_GRAD_COS
