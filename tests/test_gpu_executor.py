"""GPU: the sibling-batched executor through the kernel against the reference's
per-sibling schedule on the oracle.

A two-layer model (bf16, GQA 8/2) runs a 3-level ragged segment tree at
head_dim 128 (the 32x32x16 MFMA kernels), and a 5-deep chain ending in five
sibling leaves at head_dim 256 (the 16x16x32 kernels), with
``BatchedLeafExecutor``: one launch per layer
for each run of sibling leaves, RoPE positions from the parent's end, the
path gradient added in-kernel into the PrefixKVStack's fp32 rows, and Pop
recomputes that inject it. The reference flow -- one leaf visit at a time
(fixed_topology_scheduler.py:142-158, segment_executor.py:239-444) -- runs
the same weights in fp64 on the CPU with the oracle's attention. Compared:
every parameter gradient, and the gradient relayed to every node at its Pop,
at the bf16 gradient tolerances (cosine >= 0.999, relative L2 <= 1e-2 for
the relayed prefix gradients)."""

from __future__ import annotations

import pytest
import torch

from bridge_amd.executor import BatchedLeafExecutor, ExecutionKind, build_segments
from bridge_amd.relay import PrefixKVStack

from _helpers import BF16_GRAD_COS, BF16_PREFIX_GRAD_REL_L2, cosine, rel_l2
from _oracle_backend import OracleStackBackend
from _toy_model import ToyModel

pytestmark = pytest.mark.gpu

TREES = {
    # name: (parents, lengths, head_dim, sibling runs the batched schedule visits, relayed nodes)
    "ragged_depth3": ({0: None, 1: 0, 2: 0, 3: 2, 4: 2, 5: 2, 6: 5, 7: 5, 8: 0, 9: 0, 10: 0, 11: 10},
                      {0: 300, 1: 200, 2: 150, 3: 90, 4: 170, 5: 64, 6: 33, 7: 100, 8: 256, 9: 77, 10: 40, 11: 129},
                      128, [(1,), (3, 4), (6, 7), (8, 9), (11,)], {0, 2, 5, 10}),
    # a 5-deep chain ending in five sibling leaves, a side branch with a leaf
    # before an internal sibling, at head_dim 256 (the 16x16x32 kernels)
    "deep_wide_d256": ({0: None, 1: 0, 2: 1, 3: 2, 4: 3, 5: 4, 6: 4, 7: 4, 8: 4, 9: 4, 10: 2, 11: 2, 12: 11},
                       {0: 130, 1: 64, 2: 97, 3: 40, 4: 128, 5: 70, 6: 150, 7: 33, 8: 64, 9: 101, 10: 58, 11: 80,
                        12: 66},
                       256, [(5, 6, 7, 8, 9), (10,), (12,)], {0, 1, 2, 3, 4, 11}),
}


@pytest.mark.parametrize("name", list(TREES))
def test_batched_tree_schedule_matches_per_sibling_oracle(name, cuda_device):
    parents, lengths, d, want_visits, want_relayed = TREES[name]
    gen = torch.Generator(device="cpu").manual_seed(11)
    tokens = {s: torch.randint(0, 64, (n,), generator=gen) for s, n in lengths.items()}
    segs = build_segments(parents, lengths)
    base = ToyModel(hq=8, hkv=2, d=d, hidden=256, layers=2, seed=5, dtype=torch.bfloat16)

    gpu = base.clone_to(torch.bfloat16, cuda_device)
    ex = BatchedLeafExecutor(segs, gpu.forward_fn(tokens), PrefixKVStack(sum(lengths.values())),
                             device=cuda_device)
    mine = ex.run(batch=True)
    torch.cuda.synchronize()
    visits = [st.segment_ids for st in mine.steps if st.kind is ExecutionKind.VISIT_LEAVES]
    print(f"[executor {name}] batched visits {visits}", flush=True)
    assert visits == want_visits

    ref_model = base.clone_to(torch.float64, "cpu")
    ref_ex = BatchedLeafExecutor(segs, ref_model.forward_fn(tokens), PrefixKVStack(sum(lengths.values())),
                                 backend_factory=OracleStackBackend)
    ref = ref_ex.run(batch=False)
    assert mine.leaf_trace() == ref.leaf_trace()

    g_mine, g_ref = gpu.grads(), ref_model.grads()
    for name in g_ref:
        c = cosine(g_mine[name], g_ref[name])
        print(f"  grad {name}: cos={c:.6f} rel_l2={rel_l2(g_mine[name], g_ref[name]):.3e}", flush=True)
        assert c >= BF16_GRAD_COS, name
    loss_mine = sum(v.item() for v in mine.losses.values())
    loss_ref = sum(v.item() for v in ref.losses.values())
    print(f"  loss {loss_mine:.4f} vs {loss_ref:.4f}", flush=True)
    assert abs(loss_mine - loss_ref) <= 1e-2 * abs(loss_ref)
    assert set(mine.relayed) == set(ref.relayed) == want_relayed
    for seg, layers in ref.relayed.items():
        for layer, (rk, rv) in layers.items():
            gk, gv = mine.relayed[seg][layer]
            for label, a, b in (("dK", gk, rk), ("dV", gv, rv)):
                c, r = cosine(a, b), rel_l2(a, b)
                print(f"  node {seg} layer {layer} relayed {label}: cos={c:.6f} rel_l2={r:.3e}", flush=True)
                assert c >= BF16_GRAD_COS and r <= BF16_PREFIX_GRAD_REL_L2, (seg, layer, label)
