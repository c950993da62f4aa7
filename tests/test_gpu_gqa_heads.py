"""GPU parity at the GQA ratios of the MFMA kernels' workgroup layouts, with
every head checked against the fp64 oracle.

The forward / dQ workgroup holds gcd(G, 8) query heads of one KV head
(G = Hq / Hkv), and the dK/dV kernel stages two heads per query block when G
is even, one when it is odd. The planner deals work items to the 8 XCDs by
KV head when Hkv is a multiple of 8, and over Hkv's share of them when Hkv
divides 8. The head pairs below cover those branches:

  (32, 8)  G=4: 4 heads per workgroup, two-head dK/dV stages, one KV head per XCD
  (16, 8)  G=2: 2 heads per workgroup, one KV head per XCD
  (32, 4)  G=8: 8 heads per workgroup (32 tokens), a KV head on two XCDs
  (28, 4)  G=7: 1 head per workgroup (256 tokens), one-head dK/dV stages

each on a ragged shared-prefix case and on a depth-3 tree, at head_dim 128
(32x32x16 MFMA kernels) and 256 (16x16x32), and with both dQ plans: the
default one that reads the dS store the dK/dV kernel writes, and the one
that recomputes the scores (recompute_dq=True; the plan the long-session
and ragged workloads fall back to when their store exceeds its budget)."""

from __future__ import annotations

import math

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

HEADS = [(32, 8), (16, 8), (32, 4), (28, 4)]


def _metas():
    from bridge_amd import TPRPrefixMeta as M
    return {
        # prefix 512, four siblings of ragged lengths (one shorter than a tile)
        "ragged": M.shared_prefix(512, [384, 131, 450, 71]),
        # root 256 -> 2 branches (128, 70) -> 2 leaves each
        "depth3": M(cu_seqlens_q=(0, 100, 227, 390, 450), node_offsets=(0, 256, 384, 454),
                    leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2))),
    }


@pytest.mark.parametrize("recompute_dq", [False, True], ids=["ds_store", "recompute"])
@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("case", ["ragged", "depth3"])
@pytest.mark.parametrize("hq,hkv", HEADS)
def test_every_head_matches_oracle(hq, hkv, case, d, recompute_dq, cuda_device):
    from bridge_amd import TPRPrefixAttention
    meta = _metas()[case]
    scale = 1.0 / math.sqrt(d)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device, recompute_dq=recompute_dq)
    print(f"[gqa {case}] hq={hq} hkv={hkv} d={d} recompute_dq={recompute_dq} tq={meta.total_q} "
          f"tp={meta.total_prefix} path={plan.path} shape={plan.mfma_shape} dq_from_ds={plan.dq_from_ds}", flush=True)
    assert plan.path == "mfma"
    assert plan.dq_from_ds == (not recompute_dq)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=7 * hq + hkv, device=cuda_device)
    tensors = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    out, lse = TPRPrefixAttention.apply(*tensors, meta, scale, None, recompute_dq)
    out.backward(dout)
    torch.cuda.synchronize()
    grads = [t.grad for t in tensors]
    ro, rl, rg = oracle(meta, q, k, v, pk, pv, dout, scale)

    # per head: out, lse and dq of every query head; dk, dv, dprefix_k/v of every KV head
    for h in range(hq):
        assert max_abs(out[:, h], ro[:, h]) <= BF16_FWD_MAX_ABS, f"out head {h}"
        assert cosine(out[:, h], ro[:, h]) >= BF16_FWD_COS, f"out head {h}"
        assert max_abs(lse[h], rl[h]) <= 1e-3, f"lse head {h}"
        assert cosine(grads[0][:, h], rg[0][:, h]) >= BF16_GRAD_COS, f"dq head {h}"
    for h in range(hkv):
        for label, g, r in zip(("dk", "dv", "dprefix_k", "dprefix_v"), grads[1:], rg[1:]):
            assert cosine(g[:, h], r[:, h]) >= BF16_GRAD_COS, f"{label} kv head {h}"
        for label, g, r in zip(("dprefix_k", "dprefix_v"), grads[3:], rg[3:]):
            assert rel_l2(g[:, h], r[:, h]) <= BF16_PREFIX_GRAD_REL_L2, f"{label} kv head {h}"
    print(f"  out cos={cosine(out, ro):.6f} dq cos={cosine(grads[0], rg[0]):.6f} "
          f"dpk rel_l2={rel_l2(grads[3], rg[3]):.3e}", flush=True)
