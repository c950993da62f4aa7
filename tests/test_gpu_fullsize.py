"""GPU parity at the benchmark configurations' full sizes.

The kernel runs on the whole workload (every head, every sibling); the fp32
oracle runs on the GPU for KV-head groups whose outputs and gradients depend
on that group alone, so the comparison is exact for them: out, lse and dq of
the group's query heads, dk/dv and the sibling-summed prefix dk/dv of its KV
head. The Qwen3-4B, long-session and ragged shapes check KV heads 0, 5 and 7
(the first and last query-head groups, and one between; the latter two run
the dQ kernel that recomputes the scores, their dS store being over its
budget); the turn tree KV head 5.
"""

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
    max_abs,
    oracle,
    rel_l2,
)

pytestmark = pytest.mark.gpu

HQ, HKV, D = 32, 8, 128
KVH = 5                                   # the checked KV-head group


def _configs():
    from bridge_amd import TPRPrefixMeta as M
    gen = torch.Generator(device="cpu").manual_seed(0)
    ragged = torch.randint(256, 8193, (16,), generator=gen).tolist()
    anc = tuple((0, 1 + i // 4) for i in range(16))
    return {
        "qwen3_4b": M.shared_prefix(4096, [4096] * 4),
        "long_session": M.shared_prefix(32768, [2048] * 8),
        "ragged_varlen": M.shared_prefix(8192, ragged),
        "turn_tree_depth3": M(tuple(1024 * i for i in range(17)), (0, 2048, 3072, 4096, 5120, 6144), anc),
    }


def _check_head_group(name, meta, hq, hkv, d, kvhs, device):
    from bridge_amd import TPRPrefixAttention
    scale = 1.0 / math.sqrt(d)
    gen = torch.Generator(device="cpu").manual_seed(2024)
    tq, tp = meta.total_q, meta.total_prefix
    shapes = [(tq, hq, d), (tq, hkv, d), (tq, hkv, d), (tp, hkv, d), (tp, hkv, d), (tq, hq, d)]
    q, k, v, pk, pv, dout = (torch.randn(s, generator=gen).to(torch.bfloat16).to(device) for s in shapes)
    print(f"[{name}] tq={tq} tp={tp} leaves={meta.num_leaves} hq={hq} hkv={hkv} d={d} "
          f"path={meta.plan(hq, hkv, d, torch.bfloat16, device).path}", flush=True)

    tensors = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    out, lse = TPRPrefixAttention.apply(*tensors, meta, scale)
    out.backward(dout)
    torch.cuda.synchronize()
    grads = [t.grad for t in tensors]

    for kvh in kvhs:
        _compare_group(meta, hq, hkv, kvh, scale, (q, k, v, pk, pv, dout), out, lse, grads, device)
    # every other head was computed too: finite everywhere
    for t in [out, lse, *grads]:
        assert torch.isfinite(t.float()).all()


def _compare_group(meta, hq, hkv, kvh, scale, inputs, out, lse, grads, device):
    """fp32 oracle of KV-head group kvh, on the GPU, against the kernel's outputs."""
    q, k, v, pk, pv, dout = inputs
    qh = slice(kvh * (hq // hkv), (kvh + 1) * (hq // hkv))
    kv = slice(kvh, kvh + 1)
    ro, rl, rg = oracle(meta, q[:, qh], k[:, kv], v[:, kv], pk[:, kv], pv[:, kv], dout[:, qh], scale,
                        compute_dtype=torch.float32, device=device)
    mine = [out[:, qh], lse[qh], grads[0][:, qh], grads[1][:, kv], grads[2][:, kv], grads[3][:, kv], grads[4][:, kv]]
    ref = [ro, rl, *rg]
    labels = ["out", "lse", "dq", "dk", "dv", "dprefix_k", "dprefix_v"]
    print(f"  KV head {kvh}:", flush=True)
    for label, a, b in zip(labels, mine, ref):
        print(f"    {label}: max_abs={max_abs(a, b):.3e} cos={cosine(a, b):.6f} rel_l2={rel_l2(a, b):.3e}", flush=True)
    assert max_abs(mine[0], ref[0]) <= BF16_FWD_MAX_ABS and cosine(mine[0], ref[0]) >= BF16_FWD_COS
    assert max_abs(mine[1], ref[1]) <= 1e-3
    for a, b in zip(mine[2:], ref[2:]):
        assert cosine(a, b) >= BF16_GRAD_COS
    for a, b in zip(mine[5:], ref[5:]):
        assert rel_l2(a, b) <= BF16_PREFIX_GRAD_REL_L2


@pytest.mark.parametrize("name", ["qwen3_4b", "long_session", "ragged_varlen", "turn_tree_depth3"])
def test_full_size_config_matches_oracle_on_head_groups(name, cuda_device):
    kvhs = (KVH,) if name == "turn_tree_depth3" else (0, KVH, HKV - 1)
    _check_head_group(name, _configs()[name], HQ, HKV, D, kvhs, cuda_device)


def test_qwen35_full_attention_shape_matches_oracle_on_one_head_group(cuda_device):
    """head_dim 256 (the 16-wide MFMA kernels) at the headline sequence shape: prefix
    4096 + 4 x 4096, GQA 8/2 -- the full-attention layers of the reference's
    Qwen3.5 hybrid test model (kv_channels=256). KV head 1, query heads 4..7."""
    from bridge_amd import TPRPrefixMeta
    _check_head_group("qwen35_d256", TPRPrefixMeta.shared_prefix(4096, [4096] * 4), 8, 2, 256, (1,), cuda_device)
