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
    from bridge_amd.topology import build_trajectory_trees, lower_forest
    keys, batch = _rollouts(3)
    trees = build_trajectory_trees(keys, batch)
    meta = lower_forest(trees).meta
    depth = max(len(a) for a in meta.leaf_ancestors)
    print(f"[forest] trees={len(trees)} segments={meta.num_leaves} prefix_nodes={meta.num_nodes} "
          f"tq={meta.total_q} tp={meta.total_prefix} depth={depth}", flush=True)
    assert meta.num_nodes > 3 and depth >= 2    # the case covers multi-level trees
    _check_forest(trees, 8, 2, 9, "forest", cuda_device)


def _check_forest(trees, hq, hkv, seed, label, cuda_device):
    """One launch over every segment of `trees` against the oracle's per-segment visits."""
    from bridge_amd import TPRPrefixAttention
    from bridge_amd.topology import lower_forest
    from oracle.trie_oracle import segment_visits
    launch = lower_forest(trees)
    meta = launch.meta
    d = 128
    scale = 1.0 / math.sqrt(d)
    g = torch.Generator().manual_seed(seed)
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
    print(f"[{label}] out: max_abs={max_abs(out, ref):.3e} cos={cosine(out, ref):.6f}", flush=True)
    assert max_abs(out, ref) <= BF16_FWD_MAX_ABS and cosine(out, ref) >= BF16_FWD_COS
    for name, a_, b_ in (("dq", qa.grad, qr.grad), ("dk", ka.grad, kr.grad), ("dv", va.grad, vr.grad)):
        print(f"  {name}: cos={cosine(a_, b_):.6f}", flush=True)
        assert cosine(a_, b_) >= BF16_GRAD_COS


def _max_key_runs(meta, hq, hkv, device):
    plan = meta.plan(hq, hkv, 128, torch.bfloat16, device)
    assert plan.path == "mfma"
    return int(plan.host[29])  # most key runs of any segment (plan header word)


def test_deep_spine_trie_is_one_key_run_per_segment(cuda_device):
    """A chain of 11 branchings (12 levels): the spine segments are internal
    nodes laid out one after the other, so every segment's ancestors form one
    key run and the launch keeps its run list in registers."""
    from bridge_amd.topology import build_trajectory_trees, lower_forest
    g = torch.Generator().manual_seed(4)
    spine = torch.randint(0, 1000, (12 * 24,), generator=g)
    # row i shares 24 (i + 1) tokens of the spine, then diverges for 16 tokens
    rows = [torch.cat([spine[:24 * (i + 1)], torch.randint(1000, 2000, (16,), generator=g)]) for i in range(11)]
    rows.append(spine.clone())
    trees = build_trajectory_trees([f"u_s_{i}" for i in range(len(rows))], {"input_ids": rows})
    meta = lower_forest(trees).meta
    assert max(len(a) for a in meta.leaf_ancestors) > 8
    assert _max_key_runs(meta, 4, 2, cuda_device) == 1
    _check_forest(trees, 4, 2, 5, "deep spine", cuda_device)


def test_deep_comb_trie_reads_its_key_runs_from_the_plan(cuda_device):
    """A spine with an internal side branch at each of 11 levels: each side
    branch sits between two spine segments in the prefix layout, so a segment
    at level i has i separate key runs (11 at most, beyond the 8 held in
    registers) and the forward / dQ kernels read the runs from the plan."""
    from bridge_amd.topology import build_trajectory_trees, lower_forest
    g = torch.Generator().manual_seed(4)
    spine = torch.randint(0, 1000, (12 * 24,), generator=g)
    rows = []
    for i in range(11):
        side = torch.randint(1000, 2000, (16,), generator=g)
        for _ in range(2):
            rows.append(torch.cat([spine[:24 * (i + 1)], side, torch.randint(2000, 3000, (8,), generator=g)]))
    rows.append(spine.clone())
    trees = build_trajectory_trees([f"u_s_{i}" for i in range(len(rows))], {"input_ids": rows})
    meta = lower_forest(trees).meta
    assert _max_key_runs(meta, 8, 2, cuda_device) == 11
    _check_forest(trees, 8, 2, 6, "deep comb", cuda_device)
