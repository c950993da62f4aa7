"""PrefixKVStack: the reference's KVStack contract (unit/test_kv_stack.py), the
zero-copy path views, and a DFS over a tree whose relayed gradients match the
oracle's whole-tree backward. CPU only: the stack is device-agnostic."""

from __future__ import annotations

import pytest
import torch

from bridge_amd import PastKVAnchors, PrefixKVStack, StackSegment


def _segment(segment_id, parent_id, length, prefix_length):
    return StackSegment(segment_id, parent_id, length, prefix_length, prefix_length)


def _kv(length, *, layers=(1, 2), value=1.0, requires_grad=False, dtype=torch.float32):
    # the fixture of unit/test_kv_stack.py:31-39
    return {
        layer: (
            torch.full((length, 1, 2, 4), value + layer, dtype=dtype, requires_grad=requires_grad),
            torch.full((length, 1, 2, 4), value + 10 + layer, dtype=dtype, requires_grad=requires_grad),
        )
        for layer in layers
    }


# ---- unit/test_kv_stack.py:42-52 ----------------------------------------------------
def test_single_segment_push_pop_and_empty_assertion():
    stack = PrefixKVStack(4096)
    entry = stack.push(_segment(0, None, 3, 0), _kv(3))
    assert stack.top() is entry
    assert stack.segment_ids == (0,)
    assert stack.prefix_length == 3
    assert stack.pop(0) is entry
    stack.assert_empty()


# ---- unit/test_kv_stack.py:55-63 ----------------------------------------------------
def test_multilevel_past_kv_is_the_path_in_order():
    stack = PrefixKVStack(4096)
    stack.push(_segment(0, None, 1024, 0), _kv(1024, value=0))
    stack.push(_segment(1, 0, 512, 1024), _kv(512, value=100))
    past = stack.build_past_key_values()
    assert past[1][0].shape == (1536, 1, 2, 4)
    torch.testing.assert_close(past[1][0][:1024], _kv(1024, value=0)[1][0])
    torch.testing.assert_close(past[1][0][1024:], _kv(512, value=100)[1][0])
    torch.testing.assert_close(past[2][1][1024:], _kv(512, value=100)[2][1])


def test_past_kv_is_a_view_of_the_stack_buffers_at_every_depth():
    stack = PrefixKVStack(64)
    stack.push(_segment(0, None, 5, 0), _kv(5, value=0))
    first = stack.build_past_key_values()[1][0]
    stack.push(_segment(1, 0, 7, 5), _kv(7, value=3))
    second = stack.build_past_key_values()[1][0]
    # both are views starting at the same buffer row: no concatenation copy
    assert first.data_ptr() == second.data_ptr()
    assert first.untyped_storage().data_ptr() == second.untyped_storage().data_ptr()
    assert second.shape[0] == 12
    grads = stack.past_gradient_accumulators()[1][0]
    assert grads.dtype == torch.float32 and grads.shape == (12, 2, 4) and grads.is_contiguous()
    assert stack.build_past_key_values()[1][0][:, 0].is_contiguous()


# ---- unit/test_kv_stack.py:66-77 ----------------------------------------------------
def test_past_anchors_are_leaf_tensors():
    stack = PrefixKVStack(16)
    cached = _kv(2)
    stack.push(_segment(0, None, 2, 0), cached)
    anchors = stack.build_past_anchors()
    key_anchor, value_anchor = anchors.key_values[1]
    assert isinstance(anchors, PastKVAnchors)
    assert anchors.prefix_length == 2
    assert key_anchor.requires_grad and key_anchor.is_leaf and key_anchor.grad_fn is None
    assert value_anchor.requires_grad and value_anchor.is_leaf and value_anchor.grad_fn is None
    assert key_anchor is not cached[1][0]
    torch.testing.assert_close(key_anchor, cached[1][0])


# ---- unit/test_kv_stack.py:80-98 ----------------------------------------------------
def test_full_past_gradient_is_split_across_multilevel_segments():
    stack = PrefixKVStack(2048)
    stack.push(_segment(0, None, 1024, 0), _kv(1024))
    stack.push(_segment(1, 0, 512, 1024), _kv(512))
    anchors = stack.build_past_anchors()
    for layer, (key, value) in anchors.key_values.items():
        factor = float(layer)
        (key * factor).sum().backward(retain_graph=True)
        (value * (factor + 10)).sum().backward()
    stack.accumulate_anchor_gradients(anchors)
    for layer in (1, 2):
        root_dk, root_dv = stack.get_new_kv_gradients(0)[layer]
        middle_dk, middle_dv = stack.get_new_kv_gradients(1)[layer]
        assert root_dk.shape == (1024, 1, 2, 4) and middle_dk.shape == (512, 1, 2, 4)
        torch.testing.assert_close(root_dk, torch.full_like(root_dk, float(layer)))
        torch.testing.assert_close(middle_dk, torch.full_like(middle_dk, float(layer)))
        torch.testing.assert_close(root_dv, torch.full_like(root_dv, float(layer + 10)))
        torch.testing.assert_close(middle_dv, torch.full_like(middle_dv, float(layer + 10)))


# ---- unit/test_kv_stack.py:101-120 (the 2 + 3 = 5 sibling sum) -------------------------
def test_sibling_gradients_accumulate_into_shared_prefix():
    stack = PrefixKVStack(2048)
    root = _segment(0, None, 1024, 0)
    stack.push(root, _kv(1024))
    for child, factor in ((_segment(1, 0, 512, 1024), 2.0), (_segment(2, 0, 256, 1024), 3.0)):
        stack.push(child, _kv(child.length))
        stack.pop(child.segment_id)
        anchors = stack.build_past_anchors()
        for key, value in anchors.key_values.values():
            (key * factor).sum().backward(retain_graph=True)
            (value * factor).sum().backward()
        stack.accumulate_anchor_gradients(anchors)
    for key_grad, value_grad in stack.get_new_kv_gradients(0).values():
        assert key_grad.shape[0] == 1024 and key_grad.dtype == torch.float32
        torch.testing.assert_close(key_grad, torch.full_like(key_grad, 5.0))
        torch.testing.assert_close(value_grad, torch.full_like(value_grad, 5.0))


def test_bf16_state_accumulates_in_fp32():
    # the reference adds in the K/V dtype (prefix_state.py:565-573); the stack
    # keeps fp32 rows: 256 + 1 + 1 stays 258 (bf16 would round each step to 256)
    stack = PrefixKVStack(8)
    entry = stack.push(_segment(0, None, 2, 0), _kv(2, layers=(1,), dtype=torch.bfloat16))
    for g in (256.0, 1.0, 1.0):
        full = torch.full((2, 1, 2, 4), g, dtype=torch.bfloat16)
        entry.accumulate(1, full, full)
    dk, dv = stack.get_new_kv_gradients(0)[1]
    assert dk.dtype == torch.float32
    torch.testing.assert_close(dk, torch.full_like(dk, 258.0))
    torch.testing.assert_close(dv, torch.full_like(dv, 258.0))


# ---- unit/test_kv_stack.py:123-134 --------------------------------------------------------
def test_stale_anchor_and_missing_gradient_are_rejected():
    stack = PrefixKVStack(16)
    stack.push(_segment(0, None, 2, 0), _kv(2))
    anchors = stack.build_past_anchors()
    stack.push(_segment(1, 0, 1, 2), _kv(1))
    with pytest.raises(RuntimeError, match="stale"):
        stack.accumulate_anchor_gradients(anchors)
    stack.pop(1)
    with pytest.raises(RuntimeError, match="gradient is missing"):
        stack.accumulate_anchor_gradients(anchors)


# ---- unit/test_kv_stack.py:137-147 --------------------------------------------------------
def test_stack_rejects_wrong_parent_position_duplicate_and_non_lifo_pop():
    stack = PrefixKVStack(16)
    root = _segment(0, None, 2, 0)
    stack.push(root, _kv(2))
    with pytest.raises(RuntimeError, match="already"):
        stack.push(root, _kv(2))
    with pytest.raises(ValueError, match="stack prefix length"):
        stack.push(_segment(1, 0, 1, 3), _kv(1))
    with pytest.raises(ValueError, match="expected parent"):
        stack.push(_segment(1, 5, 1, 2), _kv(1))
    stack.push(_segment(1, 0, 1, 2), _kv(1))
    with pytest.raises(RuntimeError, match="stack top"):
        stack.pop(0)


# ---- unit/test_kv_stack.py:150-166 --------------------------------------------------------
@pytest.mark.parametrize(
    "key_values,match",
    [
        (_kv(2, requires_grad=True), "graph-free"),
        (_kv(3), "sequence length"),
        (_kv(2, layers=(1,)), "KV layers"),
    ],
)
def test_invalid_cached_kv_is_rejected(key_values, match):
    stack = PrefixKVStack(16)
    if tuple(key_values) == (1,):
        stack.push(_segment(0, None, 1, 0), _kv(1))
        segment = _segment(1, 0, 2, 1)
    else:
        segment = _segment(0, None, 2, 0)
    with pytest.raises(ValueError, match=match):
        stack.push(segment, key_values)


def test_gradient_checks_follow_the_reference():
    # prefix_state.py:551-559: shape, device and dtype must match the segment's K/V
    stack = PrefixKVStack(8)
    entry = stack.push(_segment(0, None, 2, 0), _kv(2, layers=(1,)))
    with pytest.raises(ValueError, match="shape mismatch"):
        entry.accumulate(1, torch.ones(3, 1, 2, 4), torch.ones(3, 1, 2, 4))
    with pytest.raises(ValueError, match="dtype mismatch"):
        entry.accumulate(1, torch.ones(2, 1, 2, 4, dtype=torch.float64), torch.ones(2, 1, 2, 4, dtype=torch.float64))
    with pytest.raises(KeyError, match="no KV for layer 2"):
        entry.accumulate(2, torch.ones(2, 1, 2, 4), torch.ones(2, 1, 2, 4))


def test_capacity_and_shape_checks():
    stack = PrefixKVStack(4)
    stack.push(_segment(0, None, 3, 0), _kv(3))
    with pytest.raises(ValueError, match="capacity"):
        stack.push(_segment(1, 0, 2, 3), _kv(2))
    bad = {layer: (k[:, :, :1], v[:, :, :1]) for layer, (k, v) in _kv(1).items()}
    with pytest.raises(ValueError, match="non-sequence shape"):
        stack.push(_segment(1, 0, 1, 3), bad)
    with pytest.raises(ValueError, match="positive"):
        PrefixKVStack(0)


# ---- unit/test_kv_stack.py:169-181 --------------------------------------------------------
def test_pop_releases_child_state_and_empty_stack_has_no_past():
    stack = PrefixKVStack(16)
    assert not stack.build_past_key_values()
    assert not stack.build_past_anchors().key_values
    stack.push(_segment(0, None, 2, 0), _kv(2))
    stack.push(_segment(1, 0, 1, 2), _kv(1))
    child = stack.pop(1)
    assert stack.segment_ids == (0,)
    with pytest.raises(KeyError, match="not on"):
        stack.get(child.segment.segment_id)
    with pytest.raises(RuntimeError, match="released"):
        child.key_values


def test_pushed_rows_start_with_a_zero_gradient_after_reuse():
    stack = PrefixKVStack(16)
    stack.push(_segment(0, None, 2, 0), _kv(2))
    child = stack.push(_segment(1, 0, 3, 2), _kv(3))
    child.accumulate(1, torch.ones(3, 1, 2, 4), torch.ones(3, 1, 2, 4))
    stack.pop(1)
    stack.push(_segment(2, 0, 3, 2), _kv(3, value=7))
    dk, _ = stack.get_new_kv_gradients(2)[1]
    assert torch.count_nonzero(dk) == 0
    torch.testing.assert_close(stack.get(2).key_values[1][0], _kv(3, value=7)[1][0])


def test_dfs_over_a_tree_relays_the_oracles_node_gradients():
    """Leaves visited through the stack (anchors + the oracle's attention +
    accumulate_anchor_gradients) give every node the gradient of the oracle's
    whole-tree backward: root -> {a -> 2 leaves, b -> 1 leaf}."""
    from oracle.tpr_oracle import Tree, prefix_attention, tree_backward
    g = torch.Generator().manual_seed(5)
    hq, hkv, d, scale = 4, 2, 8, 0.4
    lens = {"root": 6, "a": 3, "b": 4}
    leaves = [("a", 5), ("a", 2), ("b", 4)]
    node_ids = {"root": 0, "a": 1, "b": 2}
    offs = [0, 6, 9, 13]
    tree = Tree([0, 5, 7, 11], offs, [[0, 1], [0, 1], [0, 2]])
    r = lambda *s: torch.randn(*s, generator=g, dtype=torch.float64)  # noqa: E731
    pk, pv = r(13, hkv, d), r(13, hkv, d)
    q, k, v, dout = r(11, hq, d), r(11, hkv, d), r(11, hkv, d), r(11, hq, d)
    _, _, _, dpk, dpv = tree_backward(q, k, v, pk, pv, tree, dout, scale)

    stack = PrefixKVStack(32)
    kv_of = lambda n: {1: (pk[offs[node_ids[n]]:offs[node_ids[n] + 1]].unsqueeze(1),  # noqa: E731
                           pv[offs[node_ids[n]]:offs[node_ids[n] + 1]].unsqueeze(1))}
    stack.push(_segment(0, None, 6, 0), kv_of("root"))
    got = {}
    row = 0
    for child in ("a", "b"):
        stack.push(_segment(node_ids[child], 0, lens[child], 6), kv_of(child))
        for parent, length in leaves:
            if parent != child:
                continue
            anchors = stack.build_past_anchors()
            ak, av = anchors.key_values[1]
            qs, ks, vs = (t[row:row + length].unsqueeze(1) for t in (q, k, v))
            out = prefix_attention(qs, ks, vs, ak, av, scale)
            out.backward(dout[row:row + length].reshape(out.shape))
            stack.accumulate_anchor_gradients(anchors)
            row += length
        # views are valid while the segment is on the stack: copy before the pop
        got[child] = [t.clone() for t in stack.get_new_kv_gradients(node_ids[child])[1]]
        stack.pop(node_ids[child])
    got["root"] = [t.clone() for t in stack.get_new_kv_gradients(0)[1]]
    stack.pop(0)
    stack.assert_empty()
    for name, n in node_ids.items():
        a, b = offs[n], offs[n + 1]
        torch.testing.assert_close(got[name][0][:, 0].double(), dpk[a:b], rtol=1e-5, atol=1e-6)
        torch.testing.assert_close(got[name][1][:, 0].double(), dpv[a:b], rtol=1e-5, atol=1e-6)
