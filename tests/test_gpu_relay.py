"""GPU checks of the fp32 gradient relay.

* TPR_BWD_ACCUMULATE_PREFIX_F32: the backward adds the prefix gradient into
  caller fp32 buffers. Into zeros it gives the same gradient twice (bitwise,
  deterministic); into a prefilled buffer exactly prefill + that gradient (one
  fp32 add per element); dq/dk/dv are those of the ordinary backward; and the
  gradient matches the fp32 oracle -- on the head_dim-128 MFMA path with
  unsplit and with split (reduced) prefix tiles, on the 16-wide MFMA path
  (head_dim 64, and 256 with split tiles), and on the SIMT paths (fp32, and
  bf16 at head_dim 96).
* A DFS through PrefixKVStack with TPRKernelBackend.from_stack relays every
  node's gradient (fp32, summed over two sibling batches for the root) to the
  values of the oracle's whole-tree backward -- the reference's relay
  (kv_stack.py:156-203, prefix_state.py:546-573) end to end.
"""

from __future__ import annotations

import math

import pytest
import torch

from _helpers import (
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


def _run_backward(meta, q, k, v, pk, pv, dout, scale, accumulators=None):
    from bridge_amd import prefix_attention_backward, prefix_attention_forward
    out, lse = prefix_attention_forward(q, k, v, pk, pv, meta, scale)
    grads = prefix_attention_backward(q, k, v, pk, pv, out, lse, dout, meta, scale,
                                      prefix_grad_accumulators=accumulators)
    torch.cuda.synchronize()
    return grads


@pytest.mark.parametrize("case", ["mfma_unsplit", "mfma_split", "simt_fp32", "mfma16_bf16_d64", "mfma16_split_d256",
                                  "simt_bf16_d96"])
def test_accumulate_mode_adds_the_prefix_gradient(case, cuda_device):
    from bridge_amd import TPRPrefixMeta
    if case == "mfma_unsplit":
        meta, hq, hkv, d, dtype = TPRPrefixMeta.shared_prefix(300, [100, 37, 64]), 8, 2, 128, torch.bfloat16
    elif case == "mfma_split":
        # 80 query blocks on every prefix tile: the planner splits each into 2 chunks
        # whose fp32 partials a reduction item sums (4 partial slots)
        meta, hq, hkv, d, dtype = TPRPrefixMeta.shared_prefix(256, [300] * 16), 4, 1, 128, torch.bfloat16
        stat_bytes = (64 + 2 * ((hq * meta.total_q + 63) // 64 * 64)) * 4   # constants + lse and -delta rows
        compact = meta.plan(hq, hkv, d, dtype, cuda_device, recompute_dq=True)  # no dS store
        assert compact.workspace_bytes == stat_bytes + 4 * 2 * 128 * 128 * 4
    elif case == "simt_fp32":
        meta, hq, hkv, d, dtype = TPRPrefixMeta.shared_prefix(96, [40, 17, 33]), 4, 2, 64, torch.float32
    elif case == "mfma16_bf16_d64":  # bf16 with head_dim 64: the 16-wide MFMA kernels
        meta, hq, hkv, d, dtype = TPRPrefixMeta.shared_prefix(96, [40, 17, 33]), 4, 2, 64, torch.bfloat16
    elif case == "mfma16_split_d256":  # head_dim 256 with split prefix tiles (partials + reduction)
        meta, hq, hkv, d, dtype = TPRPrefixMeta.shared_prefix(100, [1300, 1300, 70, 2400]), 4, 1, 256, torch.bfloat16
        assert int(meta.plan(hq, hkv, d, dtype, cuda_device).host[25]) > 0
    else:  # bf16 with head_dim 96 runs the SIMT kernels
        meta, hq, hkv, d, dtype = TPRPrefixMeta.shared_prefix(96, [40, 17, 33]), 4, 2, 96, torch.bfloat16
    scale = 1.0 / math.sqrt(d)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, dtype, 31, cuda_device)
    print(f"[{case}] tq={meta.total_q} tp={meta.total_prefix} path={meta.plan(hq, hkv, d, dtype, cuda_device).path}",
          flush=True)

    base = _run_backward(meta, q, k, v, pk, pv, dout, scale)
    zeros = [torch.zeros(pk.shape, dtype=torch.float32, device=cuda_device) for _ in range(2)]
    acc1 = _run_backward(meta, q, k, v, pk, pv, dout, scale, zeros)
    zeros2 = [torch.zeros(pk.shape, dtype=torch.float32, device=cuda_device) for _ in range(2)]
    acc2 = _run_backward(meta, q, k, v, pk, pv, dout, scale, zeros2)
    gen = torch.Generator(device="cpu").manual_seed(7)
    prefill = [torch.randn(pk.shape, generator=gen).to(cuda_device) for _ in range(2)]
    filled = [t.clone() for t in prefill]
    acc3 = _run_backward(meta, q, k, v, pk, pv, dout, scale, filled)

    # the accumulators are what is returned for the prefix, and were written in place
    assert acc1[3] is zeros[0] and acc1[4] is zeros[1] and acc3[3] is filled[0]
    for i in range(3):  # dq, dk, dv unchanged by the mode
        assert torch.equal(acc1[i], base[i])
    for j in (3, 4):
        assert torch.equal(acc1[j], acc2[j]), "accumulation is deterministic"
        assert torch.equal(acc3[j], prefill[j - 3] + acc1[j]), "one fp32 add per element"
        if dtype == torch.float32:
            assert torch.equal(acc1[j], base[j])
        else:  # the ordinary path rounds the same fp32 sum to bf16 once
            assert torch.equal(acc1[j].bfloat16(), base[j])

    ref = oracle(meta, q, k, v, pk, pv, dout, scale, compute_dtype=torch.float32, device=cuda_device)[2]
    for j, label in ((3, "dprefix_k"), (4, "dprefix_v")):
        print(f"  {label}: cos={cosine(acc1[j], ref[j]):.6f} rel_l2={rel_l2(acc1[j], ref[j]):.3e} "
              f"max_abs={max_abs(acc1[j], ref[j]):.3e}", flush=True)
        if dtype == torch.float32:
            assert max_abs(acc1[j], ref[j]) <= FP32_TOL
        else:
            assert cosine(acc1[j], ref[j]) >= BF16_GRAD_COS
            assert rel_l2(acc1[j], ref[j]) <= BF16_PREFIX_GRAD_REL_L2


def test_accumulators_are_validated(cuda_device):
    from bridge_amd import TPRPrefixAttention, TPRPrefixMeta
    meta = TPRPrefixMeta.shared_prefix(64, [32])
    q, k, v, pk, pv, _ = make_inputs(meta, 4, 1, 128, torch.bfloat16, 3, cuda_device)
    good = torch.zeros(pk.shape, dtype=torch.float32, device=cuda_device)
    with pytest.raises(ValueError, match="float32"):
        TPRPrefixAttention.apply(q, k, v, pk, pv, meta, None, (good.bfloat16(), good))
    with pytest.raises(ValueError, match="shape"):
        TPRPrefixAttention.apply(q, k, v, pk, pv, meta, None, (good[1:], good))
    with pytest.raises(TypeError, match="pair"):
        TPRPrefixAttention.apply(q, k, v, pk, pv, meta, None, (good,))
    with pytest.raises(ValueError, match="must not require grad"):
        TPRPrefixAttention.apply(q, k, v, pk.clone().requires_grad_(True), pv, meta, None, (good, good))


def test_dfs_through_the_stack_relays_the_oracles_node_gradients(cuda_device):
    """root(256) -> a(128) -> leaves [100, 64, 37]; root -> b(64) -> leaves [80, 50].
    Each child's leaves run as one batched visit through the stack; the root's
    gradient sums the two visits in fp32."""
    from bridge_amd import PrefixKVStack, StackSegment, TPRKernelBackend, TPRPrefixMeta
    hq, hkv, d = 8, 2, 128
    scale = 1.0 / math.sqrt(d)
    node_len = [256, 128, 64]                       # root, a, b
    groups = [(1, [100, 64, 37]), (2, [80, 50])]    # (parent node, leaf lengths)
    lengths = [s for _, ls in groups for s in ls]
    anc = tuple((0, n) for n, ls in groups for _ in ls)
    cu = [0]
    for s in lengths:
        cu.append(cu[-1] + s)
    offs = [0, 256, 384, 448]
    meta = TPRPrefixMeta(tuple(cu), tuple(offs), anc)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, 41, cuda_device)
    ro, _, rg = oracle(meta, q, k, v, pk, pv, dout, scale, compute_dtype=torch.float32, device=cuda_device)

    def node_kv(n):
        return {1: (pk[offs[n]:offs[n + 1]].unsqueeze(1), pv[offs[n]:offs[n + 1]].unsqueeze(1))}

    stack = PrefixKVStack(1024)
    stack.push(StackSegment(0, None, node_len[0], 0, 0), node_kv(0))
    got, dq, dk, dv, outs = {}, [], [], [], []
    row = 0
    for n, ls in groups:
        stack.push(StackSegment(n, 0, node_len[n], node_len[0], node_len[0]), node_kv(n))
        backend = TPRKernelBackend.from_stack(stack, ls)
        rows = slice(row, row + sum(ls))
        qs = q[rows].unsqueeze(1).clone().requires_grad_(True)
        ks = k[rows].unsqueeze(1).clone().requires_grad_(True)
        vs = v[rows].unsqueeze(1).clone().requires_grad_(True)
        out = backend.attention(1, qs, ks, vs, softmax_scale=scale)
        out.backward(dout[rows].reshape(out.shape))
        torch.cuda.synchronize()
        outs.append(out.detach().reshape(-1, hq, d))
        dq.append(qs.grad[:, 0])
        dk.append(ks.grad[:, 0])
        dv.append(vs.grad[:, 0])
        got[n] = [t.clone() for t in stack.get_new_kv_gradients(n)[1]]
        stack.pop(n)
        row += sum(ls)
    got[0] = [t.clone() for t in stack.get_new_kv_gradients(0)[1]]
    stack.pop(0)
    stack.assert_empty()

    assert cosine(torch.cat(outs), ro) >= 0.9999
    for label, mine, ref in (("dq", dq, rg[0]), ("dk", dk, rg[1]), ("dv", dv, rg[2])):
        c = cosine(torch.cat(mine), ref)
        print(f"  {label}: cos={c:.6f}", flush=True)
        assert c >= BF16_GRAD_COS
    for n in range(3):
        a, b = offs[n], offs[n + 1]
        for j, label in ((0, "dK"), (1, "dV")):
            mine, ref = got[n][j][:, 0], rg[3 + j][a:b]
            print(f"  node {n} {label}: cos={cosine(mine, ref):.6f} rel_l2={rel_l2(mine, ref):.3e}", flush=True)
            assert mine.dtype == torch.float32
            assert cosine(mine, ref) >= BF16_GRAD_COS
            assert rel_l2(mine, ref) <= BF16_PREFIX_GRAD_REL_L2
