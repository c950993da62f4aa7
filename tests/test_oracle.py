"""Pins of the CPU oracle against the reference's own known-answer tests,
closed forms, brute force and independent library routines (CPU only)."""

import math

import pytest
import torch

from _helpers import random_key_mask
from oracle.tpr_oracle import (
    Tree,
    block_reference,
    finalize_attention_result,
    fp32_reference,
    merge_attention,
    prefix_attention,
    tree_autograd,
    tree_backward,
    tree_forward,
    visible_pairs,
)


# ---- tests/models/mcore/tpr/unit/test_fa_fp32_reference.py:9-37 ----------
@pytest.mark.parametrize("heads", [2, 4])
@pytest.mark.parametrize("scale", [None, 0.7])
def test_fp32_reference_matches_per_query_float64(heads, scale):
    gen = torch.Generator().manual_seed(44)
    shapes = {"q": (3, 1, heads, 4), "k": (3, 1, 2, 4), "v": (3, 1, 2, 4),
              "pk": (2, 1, 2, 4), "pv": (2, 1, 2, 4)}
    entry = {n: torch.randn(s, generator=gen) for n, s in shapes.items()}
    entry["scale"] = scale
    upstream = torch.randn(3, 1, heads * 4, generator=gen)
    actual = fp32_reference(entry, upstream)
    inputs = {n: entry[n].double().requires_grad_() for n in shapes}
    rows = []
    for t in range(3):
        cols = []
        for h in range(heads):
            kvh = h // (heads // 2)
            keys = torch.cat((inputs["pk"][:, 0, kvh], inputs["k"][:t + 1, 0, kvh]))
            vals = torch.cat((inputs["pv"][:, 0, kvh], inputs["v"][:t + 1, 0, kvh]))
            sc = keys @ inputs["q"][t, 0, h] * (0.5 if scale is None else scale)
            cols.append(sc.softmax(0) @ vals)
        rows.append(torch.cat(cols))
    output = torch.stack(rows).unsqueeze(1)
    grads = torch.autograd.grad(output, tuple(inputs.values()), grad_outputs=upstream.double())
    expected = {"output": output, **dict(zip(shapes, grads))}
    for name, exp in expected.items():
        assert actual[name].dtype == torch.float32
        torch.testing.assert_close(actual[name].double(), exp, atol=2e-6, rtol=2e-5)


# ---- same file :40-50, closed form ---------------------------------------
def test_closed_form_future_values_are_masked():
    q = torch.ones(3, 1, 1, 1)
    k = torch.zeros_like(q)
    pk = torch.zeros(2, 1, 1, 1)
    v = torch.tensor([3.0, 6.0, 100.0]).reshape_as(q).requires_grad_()
    pv = torch.tensor([0.0, 0.0]).reshape_as(pk).requires_grad_()
    out = prefix_attention(q, k, v, pk, pv, None)
    torch.testing.assert_close(out[:, 0, 0], torch.tensor([1.0, 2.25, 21.8]))
    dv, dpv = torch.autograd.grad(out[0].sum(), (v, pv))
    torch.testing.assert_close(dv.flatten(), torch.tensor([1 / 3, 0.0, 0.0]))
    torch.testing.assert_close(dpv.flatten(), torch.tensor([1 / 3, 1 / 3]))


def test_tree_forward_matches_closed_form_and_lse():
    # same closed form through the packed-tree path: lse of row t is log(P + t + 1)
    q = torch.ones(3, 1, 1)
    k = torch.zeros(3, 1, 1)
    v = torch.tensor([3.0, 6.0, 100.0]).reshape(3, 1, 1)
    pk = torch.zeros(2, 1, 1)
    pv = torch.zeros(2, 1, 1)
    out, lse = tree_forward(q, k, v, pk, pv, Tree.single(2, [3]))
    torch.testing.assert_close(out[:, 0, 0], torch.tensor([1.0, 2.25, 21.8], dtype=torch.float64))
    torch.testing.assert_close(lse[0], torch.log(torch.tensor([3.0, 4.0, 5.0], dtype=torch.float64)))


# ---- tests/models/mcore/tpr/unit/test_ring_merge_probe.py:9-32 -----------
@pytest.mark.parametrize("causal", [False, True])
def test_block_reference_gqa_and_statistics(causal):
    q = torch.zeros(3, 4, 2)
    k = torch.zeros(3, 2, 2)
    v = torch.arange(12.0).reshape(3, 2, 2)
    out, maximum, total = block_reference(q, k, v, scale=0.5, causal=causal)
    for t in range(3):
        visible = t + 1 if causal else 3
        torch.testing.assert_close(out[t], v[:visible].mean(0).repeat_interleave(2, dim=0))
        torch.testing.assert_close(total[t], torch.full((4,), float(visible)))
    assert torch.count_nonzero(maximum) == 0


def test_block_reference_explicit_mask_and_fully_masked_guard():
    q = torch.zeros(2, 1, 1)
    k = torch.zeros(3, 1, 1)
    v = torch.tensor([2.0, 4.0, 100.0]).reshape(3, 1, 1)
    mask = torch.tensor([[False, True, True], [False, False, True]])
    out, _, total = block_reference(q, k, v, scale=1.0, causal=False, mask=mask)
    torch.testing.assert_close(out.flatten(), torch.tensor([2.0, 3.0]))
    torch.testing.assert_close(total.flatten(), torch.tensor([1.0, 2.0]))
    with pytest.raises(ValueError, match="fully-masked"):
        block_reference(q, k, v, scale=1.0, causal=False, mask=torch.ones_like(mask))


# ---- parallel/test_ring_cp_attention_contract.py:188-243 ------------------
def test_merge_known_answer():
    t, h, d = 4, 2, 8
    prev = (torch.zeros(t, h, d), torch.zeros(t, h), torch.ones(t, h))
    cur = (torch.ones(t, h, d), torch.zeros(t, h), torch.ones(t, h))
    out, m, l = merge_attention(prev, cur)
    torch.testing.assert_close(out, torch.full((t, h, d), 0.5))
    torch.testing.assert_close(m, torch.zeros(t, h))
    torch.testing.assert_close(l, torch.full((t, h), 2.0))


@pytest.mark.parametrize("blocks", [1, 5, 8])
def test_merge_of_equal_stat_bf16_blocks_is_fp32_mean(blocks):
    gen = torch.Generator().manual_seed(44)
    values = [torch.randn(4, 2, 8, generator=gen).bfloat16() for _ in range(blocks)]
    merged = None
    for val in values:
        merged = merge_attention(merged, (val, torch.zeros(4, 2), torch.ones(4, 2)))
        assert all(x.dtype == torch.float32 for x in merged)
    expected = torch.stack([x.float() for x in values]).mean(0)
    torch.testing.assert_close(merged[0], expected, atol=2e-7, rtol=2e-6)
    final = finalize_attention_result(merged, dtype=torch.bfloat16)
    assert final[0].dtype == torch.bfloat16 and final[0].is_contiguous()
    torch.testing.assert_close(final[0], merged[0].bfloat16(), atol=0, rtol=0)


def test_prefix_block_merged_with_causal_block_equals_dense():
    # FULL prefix block + CAUSAL current block, merged, == dense prefix attention
    gen = torch.Generator().manual_seed(3)
    q = torch.randn(5, 4, 8, generator=gen, dtype=torch.float64)
    k, v = (torch.randn(5, 2, 8, generator=gen, dtype=torch.float64) for _ in range(2))
    pk, pv = (torch.randn(7, 2, 8, generator=gen, dtype=torch.float64) for _ in range(2))
    b1 = block_reference(q, pk, pv, scale=0.3, causal=False)
    b2 = block_reference(q, k, v, scale=0.3, causal=True)
    merged = merge_attention(tuple(x.double() for x in b1), tuple(x.double() for x in b2))
    dense = prefix_attention(q[:, None], k[:, None], v[:, None], pk[:, None], pv[:, None], 0.3)
    torch.testing.assert_close(merged[0].reshape(5, -1).double(), dense[:, 0], atol=1e-6, rtol=1e-6)
    out, lse = tree_forward(q, k, v, pk, pv, Tree.single(7, [5]), 0.3)
    torch.testing.assert_close(lse.T, (merged[1] + torch.log(merged[2])).double(), atol=1e-6, rtol=1e-6)


# ---- independent library check: SDPA in fp64 with an explicit mask --------
def test_tree_forward_matches_sdpa_fp64():
    gen = torch.Generator().manual_seed(5)
    hq, hkv, d = 4, 2, 16
    tree = Tree(cu_seqlens_q=[0, 6, 9], node_offsets=[0, 5, 9], ancestors=[[0, 1], [0]])
    tq, tp = 9, 9
    q = torch.randn(tq, hq, d, generator=gen, dtype=torch.float64)
    k, v = (torch.randn(tq, hkv, d, generator=gen, dtype=torch.float64) for _ in range(2))
    pk, pv = (torch.randn(tp, hkv, d, generator=gen, dtype=torch.float64) for _ in range(2))
    out, _ = tree_forward(q, k, v, pk, pv, tree, 0.4)
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        rows = tree.prefix_rows(s)
        keys = torch.cat((pk[rows], k[a:b])).repeat_interleave(2, 1).transpose(0, 1)
        vals = torch.cat((pv[rows], v[a:b])).repeat_interleave(2, 1).transpose(0, 1)
        plen = len(rows)
        allowed = torch.arange(plen + b - a)[None, :] <= plen + torch.arange(b - a)[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            q[a:b].transpose(0, 1), keys, vals, attn_mask=allowed, scale=0.4)
        torch.testing.assert_close(out[a:b], ref.transpose(0, 1), atol=1e-12, rtol=1e-12)


# ---- explicit backward vs autograd and finite differences -----------------
def _random_tree_inputs(seed, tree, hq=4, hkv=2, d=8, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    tq = tree.cu_seqlens_q[-1]
    tp = tree.node_offsets[-1]
    q = torch.randn(tq, hq, d, generator=gen, dtype=dtype)
    k, v = (torch.randn(tq, hkv, d, generator=gen, dtype=dtype) for _ in range(2))
    pk, pv = (torch.randn(tp, hkv, d, generator=gen, dtype=dtype) for _ in range(2))
    dout = torch.randn(tq, hq, d, generator=gen, dtype=dtype)
    return q, k, v, pk, pv, dout


TREES = {
    "single": Tree.single(5, [4, 3]),
    "no_prefix": Tree.single(0, [3, 5]),
    "depth3": Tree(cu_seqlens_q=[0, 3, 5, 9, 10], node_offsets=[0, 4, 6, 9],
                   ancestors=[[0, 1], [0, 1], [0, 2], [0, 2]]),
}


@pytest.mark.parametrize("name", sorted(TREES))
def test_explicit_backward_matches_reference_style_autograd(name):
    tree = TREES[name]
    q, k, v, pk, pv, dout = _random_tree_inputs(11, tree)
    out, lse = tree_forward(q, k, v, pk, pv, tree, 0.35)
    grads = tree_backward(q, k, v, pk, pv, tree, dout, 0.35, out=out, lse=lse)
    ref = tree_autograd(q, k, v, pk, pv, tree, dout, 0.35)
    torch.testing.assert_close(out, ref[0], atol=1e-12, rtol=1e-10)
    for mine, theirs in zip(grads, ref[1:]):
        torch.testing.assert_close(mine, theirs, atol=1e-11, rtol=1e-9)


def test_explicit_backward_finite_differences():
    tree = TREES["depth3"]
    q, k, v, pk, pv, dout = _random_tree_inputs(12, tree, hq=2, hkv=1, d=4)
    grads = tree_backward(q, k, v, pk, pv, tree, dout, 0.6)
    tensors = [q, k, v, pk, pv]
    gen = torch.Generator().manual_seed(0)
    eps = 1e-6
    for t_idx, tensor in enumerate(tensors):
        for _ in range(4):
            flat = torch.randint(0, tensor.numel(), (1,), generator=gen).item()
            plus = [x.clone() for x in tensors]
            minus = [x.clone() for x in tensors]
            plus[t_idx].view(-1)[flat] += eps
            minus[t_idx].view(-1)[flat] -= eps
            fp = (tree_forward(*plus, tree, 0.6)[0] * dout).sum()
            fm = (tree_forward(*minus, tree, 0.6)[0] * dout).sum()
            numeric = (fp - fm) / (2 * eps)
            assert abs(numeric.item() - grads[t_idx].view(-1)[flat].item()) < 1e-6


# ---- unit/test_kv_stack.py:79-120 and unit/test_segment_executor.py:291-325 --
def test_multilevel_prefix_gradient_split_per_ancestor():
    # leaf gradients of cat(root, middle) split back to each node unchanged
    tree = Tree(cu_seqlens_q=[0, 4], node_offsets=[0, 6, 9], ancestors=[[0, 1]])
    q, k, v, pk, pv, dout = _random_tree_inputs(21, tree)
    _, _, _, dpk, dpv = tree_backward(q, k, v, pk, pv, tree, dout)
    flat = Tree.single(9, [4])
    _, _, _, dpk_flat, dpv_flat = tree_backward(q, k, v, pk, pv, flat, dout)
    torch.testing.assert_close(dpk, dpk_flat)
    torch.testing.assert_close(dpv, dpv_flat)


def test_sibling_prefix_gradient_is_sum_of_single_leaf_runs():
    tree = Tree.single(6, [5, 3, 4])
    q, k, v, pk, pv, dout = _random_tree_inputs(22, tree)
    batched = tree_backward(q, k, v, pk, pv, tree, dout)
    acc_k = torch.zeros_like(pk)
    acc_v = torch.zeros_like(pv)
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        single = Tree.single(6, [b - a])
        g = tree_backward(q[a:b], k[a:b], v[a:b], pk, pv, single, dout[a:b])
        torch.testing.assert_close(batched[0][a:b], g[0])
        torch.testing.assert_close(batched[1][a:b], g[1])
        acc_k += g[3]
        acc_v += g[4]
    torch.testing.assert_close(batched[3], acc_k)
    torch.testing.assert_close(batched[4], acc_v)


def test_sibling_sum_known_answer_two_plus_three():
    # kv_stack test: prefix grads 2 and 3 from two siblings accumulate to 5.
    # With q = 0 every visible key gets weight 1/count, so d(sum out)/dpv is
    # count-normalised; choose dout so each sibling contributes a constant.
    tree = Tree.single(2, [1, 1])
    q = torch.zeros(2, 1, 1, dtype=torch.float64)
    k = torch.zeros(2, 1, 1, dtype=torch.float64)
    v = torch.zeros(2, 1, 1, dtype=torch.float64)
    pk = torch.zeros(2, 1, 1, dtype=torch.float64)
    pv = torch.zeros(2, 1, 1, dtype=torch.float64)
    dout = torch.tensor([6.0, 9.0], dtype=torch.float64).reshape(2, 1, 1)  # 3 visible keys each
    _, _, _, _, dpv = tree_backward(q, k, v, pk, pv, tree, dout)
    torch.testing.assert_close(dpv.flatten(), torch.tensor([5.0, 5.0], dtype=torch.float64))


def test_visible_pairs_matches_closed_form():
    assert visible_pairs(Tree.single(512, [512, 512])) == 786944
    assert visible_pairs(Tree.single(4096, [4096] * 4)) == 100671488
    assert visible_pairs(Tree.single(32768, [2048] * 8)) == 553656320
    root, branch, leaf = 2048, 1024, 1024
    anc = [[0, 1 + b] for b in range(4) for _ in range(4)]
    tree = Tree([i * leaf for i in range(17)], [0, root] + [root + (b + 1) * branch for b in range(4)], anc)
    assert visible_pairs(tree) == 58728448


# ---- masked forms: the custom-mask mode of rectangular_attention.py:112-122 --
def _sdpa_tree(q, k, v, pk, pv, tree, dout, scale, mask):
    """Per leaf, torch's scaled_dot_product_attention in fp64 with the mask's
    complement as attn_mask, gradients by autograd (summed over leaves)."""
    ins = [t.detach().clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    qa, ka, va, pka, pva = ins
    group = q.shape[1] // k.shape[1]
    outs = []
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        rows = torch.tensor(tree.prefix_rows(s), dtype=torch.long)
        keys = torch.cat((pka[rows], ka[a:b])).repeat_interleave(group, 1).transpose(0, 1)
        vals = torch.cat((pva[rows], va[a:b])).repeat_interleave(group, 1).transpose(0, 1)
        allowed = ~mask[a:b, :keys.shape[1]]
        outs.append(torch.nn.functional.scaled_dot_product_attention(
            qa[a:b].transpose(0, 1), keys, vals, attn_mask=allowed, scale=scale).transpose(0, 1))
    out = torch.cat(outs)
    (out * dout).sum().backward()
    return out.detach(), [t.grad for t in ins]


@pytest.mark.parametrize("name", sorted(TREES))
def test_masked_tree_matches_sdpa_fp64_values_and_gradients(name):
    tree = TREES[name]
    q, k, v, pk, pv, dout = _random_tree_inputs(31, tree)
    mask = random_key_mask(tree, torch.Generator().manual_seed(3))
    # the mask shows some query a later key of its own suffix (not causal)
    later = [(r, c) for s in range(tree.num_leaves) for r in range(*tree.leaf_range(s))
             for c in range(len(tree.prefix_rows(s)) + r - tree.leaf_range(s)[0] + 1,
                            len(tree.prefix_rows(s)) + tree.leaf_range(s)[1] - tree.leaf_range(s)[0])
             if not mask[r, c]]
    assert later
    out, lse = tree_forward(q, k, v, pk, pv, tree, 0.45, mask=mask)
    grads = tree_backward(q, k, v, pk, pv, tree, dout, 0.45, out=out, lse=lse, mask=mask)
    ref, ref_grads = _sdpa_tree(q, k, v, pk, pv, tree, dout, 0.45, mask)
    torch.testing.assert_close(out, ref, atol=1e-12, rtol=1e-12)
    for mine, theirs in zip(grads, ref_grads):
        torch.testing.assert_close(mine, theirs, atol=1e-11, rtol=1e-9)
    # lse: torch.logsumexp of the visible scaled scores
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        rows = tree.prefix_rows(s)
        keys = torch.cat((pk[rows], k[a:b])).repeat_interleave(2, 1)
        sc = torch.einsum("thd,khd->htk", q[a:b], keys) * 0.45
        sc = sc.masked_fill(mask[a:b, :keys.shape[0]][None], float("-inf"))
        torch.testing.assert_close(lse[:, a:b], torch.logsumexp(sc, -1), atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("name", sorted(TREES))
def test_causal_mask_gives_the_unmasked_tree(name):
    tree = TREES[name]
    q, k, v, pk, pv, dout = _random_tree_inputs(32, tree)
    lens = [len(tree.prefix_rows(s)) + tree.leaf_range(s)[1] - tree.leaf_range(s)[0] for s in range(tree.num_leaves)]
    mask = torch.ones(tree.cu_seqlens_q[-1], max(lens), dtype=torch.bool)
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        plen = len(tree.prefix_rows(s))
        for i in range(b - a):
            mask[a + i, :plen + i + 1] = False
    plain = tree_backward(q, k, v, pk, pv, tree, dout, 0.4)
    masked = tree_backward(q, k, v, pk, pv, tree, dout, 0.4, mask=mask)
    for x, y in zip(plain, masked):
        torch.testing.assert_close(x, y, atol=0, rtol=0)
    assert torch.equal(tree_forward(q, k, v, pk, pv, tree, 0.4)[1], tree_forward(q, k, v, pk, pv, tree, 0.4,
                                                                                 mask=mask)[1])


def test_physical_padding_mask_equals_logical_attention():
    """equivalence/test_rectangular_attention_npu.py:149-284 on the oracle, in
    fp64: Q 63 + 1 padding row and KV 127 + 1 padding row (prefix 64), GQA
    4/2, D 64. With the padding key hidden (and the padding query seeing keys
    up to position 126), the logical rows' output and gradients equal the
    unpadded causal attention, the padding rows get zero gradient (their
    upstream gradient is zero); with the padding query row hidden entirely its
    output is 0 and its lse -inf."""
    gen = torch.Generator().manual_seed(2027)
    sq, skv, hq, hkv, d = 63, 127, 4, 2, 64
    p = skv - sq
    q, k, v = (torch.randn(n, h, d, generator=gen, dtype=torch.float64) for n, h in ((sq, hq), (skv, hkv), (skv, hkv)))
    dout = torch.randn(sq, hq, d, generator=gen, dtype=torch.float64)
    pq, pk_, pv_ = (torch.cat((t, torch.randn(1, *t.shape[1:], generator=gen, dtype=torch.float64))) for t in (q, k, v))
    pdout = torch.cat((dout, torch.zeros(1, hq, d, dtype=torch.float64)))
    logical = tree_backward(q, k[p:], v[p:], k[:p], v[:p], Tree.single(p, [sq]), dout, d ** -0.5)
    logical_out, _ = tree_forward(q, k[p:], v[p:], k[:p], v[:p], Tree.single(p, [sq]), d ** -0.5)
    query_positions = torch.arange(64, 128).clamp_max(126)
    key_positions = torch.arange(128).clamp_max(126)
    key_valid = torch.arange(128) < skv
    physical = ~key_valid[None, :] | (key_positions[None, :] > query_positions[:, None])
    invalid_row = physical | (torch.arange(64) >= sq)[:, None]
    tree = Tree.single(p, [sq + 1])
    for mask in (physical, invalid_row):
        args = (pq, pk_[p:], pv_[p:], pk_[:p], pv_[:p], tree)
        out, lse = tree_forward(*args, d ** -0.5, mask=mask)
        dq, dk, dv, dpk, dpv = tree_backward(*args, pdout, d ** -0.5, out=out, lse=lse, mask=mask)
        torch.testing.assert_close(out[:sq], logical_out, atol=1e-12, rtol=1e-12)
        torch.testing.assert_close(dq[:sq], logical[0], atol=1e-12, rtol=1e-12)
        torch.testing.assert_close(torch.cat((dpk, dk[:sq])), torch.cat((logical[3], logical[1])), atol=1e-12,
                                   rtol=1e-12)
        torch.testing.assert_close(torch.cat((dpv, dv[:sq])), torch.cat((logical[4], logical[2])), atol=1e-12,
                                   rtol=1e-12)
        for g in (dq[sq:], dk[sq:], dv[sq:]):
            assert torch.count_nonzero(g) == 0
    assert torch.count_nonzero(out[sq:]) == 0 and bool(torch.isneginf(lse[:, sq:]).all())
