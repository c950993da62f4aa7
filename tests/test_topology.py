"""Rollout tries and their one-launch lowering (bridge_amd.topology), on the CPU.

* The reference's own trie tests (unit/test_trajectory_tree.py,
  unit/test_trajectory_tree_turn.py), restated.
* The radix builder against the oracle's one-token trie (the reference's
  algorithm) on random batches: identical trees, field by field.
* The lowering: packed tokens / positions reconstruct the rows, and the
  oracle's tree attention on the lowered layout (prefix = k[prefix_index],
  gradient folded back) equals the per-segment visits of the tree, outputs
  and gradients, in fp64.
"""

from __future__ import annotations

import random

import pytest
import torch

from bridge_amd.topology import (
    QWEN3_IM_END_TOKEN_ID as EOT,
    build_prompt_sibling_trees,
    build_trajectory_trees,
    build_trajectory_trees_turn,
    lower_forest,
    lower_tree,
)


def _make_batch(rows):
    return {"input_ids": [torch.tensor(r, dtype=torch.long) for r in rows]}


def _tokens(tree, node_id, batch):
    ref = tree.get(node_id).segment
    return batch["input_ids"][ref.row][ref.start:ref.end].tolist()


def _paths_reconstruct(trees, data):
    # unit/test_trajectory_tree_turn.py:37-52
    covered = {}
    for tree in trees:
        def visit(node_id, path):
            node = tree.get(node_id)
            merged = path + _tokens(tree, node_id, data)
            for row in node.terminal_rows:
                assert row not in covered
                assert merged == data["input_ids"][row].tolist()
                covered[row] = True
            for child_id in node.children:
                visit(child_id, merged)
        visit(tree.root_id, [])
    assert set(covered) == set(range(len(data["input_ids"])))


# ---- unit/test_trajectory_tree.py:23-171 -------------------------------------------------
def test_builds_multilevel_compressed_trie_from_complete_input_ids():
    batch = _make_batch([[1, 2, 3, 4, 5], [1, 2, 3, 4, 6], [1, 2, 3, 7]])
    (tree,) = build_trajectory_trees(["uid-a_0_0", "uid-a_1_0", "uid-a_2_0"], batch)
    root = tree.get(tree.root_id)
    assert tree.uid == "uid-a" and tree.member_rows == (0, 1, 2)
    assert (root.segment.start, root.segment.end) == (0, 3)
    assert _tokens(tree, root.node_id, batch) == [1, 2, 3]
    assert root.member_rows == (0, 1, 2) and root.terminal_rows == () and len(root.children) == 2
    shared_4, direct_7 = tree.get(root.children[0]), tree.get(root.children[1])
    assert _tokens(tree, shared_4.node_id, batch) == [4]
    assert shared_4.member_rows == (0, 1) and shared_4.terminal_rows == ()
    assert [_tokens(tree, c, batch) for c in shared_4.children] == [[5], [6]]
    assert _tokens(tree, direct_7.node_id, batch) == [7]
    assert direct_7.member_rows == (2,) and direct_7.terminal_rows == (2,) and direct_7.children == ()


def test_compression_is_not_limited_by_prompt_boundary():
    prompts = [torch.tensor([1, 2, 3]), torch.tensor([1, 2, 3])]
    responses = [torch.tensor([4, 5, 6]), torch.tensor([4, 5, 7])]
    batch = {"prompts": prompts, "responses": responses,
             "input_ids": [torch.cat((prompts[0], responses[0])), torch.cat((prompts[1], responses[1]))]}
    (tree,) = build_trajectory_trees(["u_0_0", "u_1_0"], batch)
    root = tree.get(tree.root_id)
    assert (root.segment.start, root.segment.end) == (0, 5)
    assert _tokens(tree, root.node_id, batch) == [1, 2, 3, 4, 5]


def test_terminal_rows_preserve_sequence_that_ends_inside_another_path():
    batch = _make_batch([[1, 2, 3], [1, 2, 3, 4, 5]])
    (tree,) = build_trajectory_trees(["u_0_0", "u_1_0"], batch)
    root = tree.get(tree.root_id)
    assert _tokens(tree, root.node_id, batch) == [1, 2, 3]
    assert root.member_rows == (0, 1) and root.terminal_rows == (0,) and len(root.children) == 1
    child = tree.get(root.children[0])
    assert _tokens(tree, child.node_id, batch) == [4, 5]
    assert child.member_rows == (1,) and child.terminal_rows == (1,)


def test_uid_is_only_candidate_partition_not_prefix_definition():
    batch = _make_batch([[1, 2, 3], [9, 8], [1, 2, 4]])
    trees = build_trajectory_trees(["u1_0_0", "u1_1_0", "u1_2_0"], batch)
    assert len(trees) == 2 and [t.uid for t in trees] == ["u1", "u1"]
    assert trees[0].member_rows == (0, 2) and trees[1].member_rows == (1,)
    assert trees[0].get(trees[0].root_id).segment.start == 0
    assert trees[1].get(trees[1].root_id).segment.start == 0


def test_multiple_uids_remain_separate_candidate_groups_in_first_seen_order():
    batch = _make_batch([[1, 2, 3], [1, 2, 9], [1, 2, 4]])
    trees = build_trajectory_trees(["u1_0_0", "u2_0_0", "u1_1_0"], batch)
    assert [t.uid for t in trees] == ["u1", "u2"]
    assert trees[0].member_rows == (0, 2) and trees[1].member_rows == (1,)


def test_exact_duplicate_trajectories_keep_distinct_logical_terminal_rows():
    batch = _make_batch([[1, 2, 3], [1, 2, 3]])
    (tree,) = build_trajectory_trees(["u_0_0", "u_1_0"], batch)
    root = tree.get(tree.root_id)
    assert _tokens(tree, root.node_id, batch) == [1, 2, 3]
    assert root.member_rows == (0, 1) and root.terminal_rows == (0, 1) and root.children == ()


def test_old_builder_name_is_a_compatibility_alias():
    batch = _make_batch([[1, 2, 3, 4], [1, 2, 3, 5]])
    keys = ["u_0_0", "u_1_0"]
    assert build_prompt_sibling_trees(keys, batch) == build_trajectory_trees(keys, batch)


def test_rejects_duplicate_keys_and_empty_sequences():
    with pytest.raises(ValueError, match="duplicate trajectory key"):
        build_trajectory_trees(["u_0_0", "u_0_0"], _make_batch([[1], [2]]))
    with pytest.raises(ValueError, match="must not be empty"):
        build_trajectory_trees(["u_0_0"], {"input_ids": [torch.tensor([], dtype=torch.long)]})
    with pytest.raises(ValueError, match="key format"):
        build_trajectory_trees(["nokey"], _make_batch([[1]]))
    with pytest.raises(ValueError, match="integer dtype"):
        build_trajectory_trees(["u_0_0"], {"input_ids": [torch.tensor([1.0])]})


# ---- the radix builder against the reference's one-token trie ----------------------------
def _random_batch(seed, n_uids=3, rows_per_uid=6, vocab=5):
    rng = random.Random(seed)
    keys, rows = [], []
    for u in range(n_uids):
        pool = []
        for i in range(rows_per_uid):
            if pool and rng.random() < 0.7:
                base = rng.choice(pool)
                cut = rng.randint(1, len(base))
                row = base[:cut] + [rng.randrange(vocab) for _ in range(rng.randint(0, 6))]
                if rng.random() < 0.15:
                    row = list(base)          # exact duplicate
            else:
                row = [rng.randrange(vocab) for _ in range(rng.randint(1, 9))]
            pool.append(row)
            keys.append(f"uid{u}_s_{i}")
            rows.append(row)
    order = list(range(len(rows)))
    rng.shuffle(order)                          # interleave the uid groups
    return [keys[i] for i in order], [rows[i] for i in order]


def test_oracle_token_trie_reproduces_the_reference_known_answers():
    # unit/test_trajectory_tree.py:23-50, :83-100 and :138-151 applied to the oracle itself
    from oracle.trie_oracle import token_trie
    rows = [[1, 2, 3, 4, 5], [1, 2, 3, 4, 6], [1, 2, 3, 7]]
    ((uid, index, root_id, nodes),) = token_trie([("a", [0, 1, 2])], rows)
    assert (uid, index, root_id) == ("a", 0, 0)
    parent, (row, start, end), members, terminals, children = nodes[0]
    assert (parent, (start, end), members, terminals) == (None, (0, 3), (0, 1, 2), ())
    shared4, direct7 = nodes[children[0]], nodes[children[1]]
    assert shared4[1][1:] == (3, 4) and shared4[2] == (0, 1) and shared4[3] == ()
    assert [rows[nodes[c][1][0]][nodes[c][1][1]:nodes[c][1][2]] for c in shared4[4]] == [[5], [6]]
    assert direct7[1][1:] == (3, 4) and direct7[2] == (2,) and direct7[3] == (2,) and direct7[4] == ()
    ((_, _, _, nodes),) = token_trie([("u", [0, 1])], [[1, 2, 3], [1, 2, 3, 4, 5]])
    assert nodes[0][1][1:] == (0, 3) and nodes[0][3] == (0,) and nodes[nodes[0][4][0]][1][1:] == (3, 5)
    ((_, _, _, nodes),) = token_trie([("u", [0, 1])], [[1, 2, 3], [1, 2, 3]])
    assert nodes[0][2] == (0, 1) and nodes[0][3] == (0, 1) and nodes[0][4] == ()
    trees = token_trie([("u1", [0, 2])], [[1, 2, 3], [9, 8], [1, 2, 4]])
    assert len(trees) == 1 and trees[0][3][0][2] == (0, 2)


@pytest.mark.parametrize("seed", range(12))
def test_radix_builder_equals_the_one_token_trie(seed):
    from oracle.trie_oracle import token_trie
    keys, rows = _random_batch(seed)
    batch = _make_batch(rows)
    trees = build_trajectory_trees(keys, batch)
    groups = {}
    for r, key in enumerate(keys):
        groups.setdefault(key.rsplit("_", 2)[0], []).append(r)
    expected = token_trie(list(groups.items()), rows)
    assert len(trees) == len(expected)
    for tree, (uid, index, root_id, nodes) in zip(trees, expected):
        assert (tree.uid, tree.tree_index, tree.root_id) == (uid, index, root_id)
        assert set(tree.nodes) == set(nodes)
        for node_id, (parent, (row, start, end), members, terminals, children) in nodes.items():
            n = tree.get(node_id)
            assert n.parent_id == parent
            assert (n.segment.row, n.segment.start, n.segment.end) == (row, start, end)
            assert n.member_rows == members and n.terminal_rows == terminals and n.children == children
    _paths_reconstruct(trees, batch)


@pytest.mark.parametrize("seed", range(12))
def test_turn_builder_equals_the_unit_trie(seed):
    """The radix-based turn builder against the reference's unit trie restated
    in the oracle, field by field, on random batches with message ends,
    prompts and several minimum unit lengths."""
    from oracle.trie_oracle import turn_trie
    rng = random.Random(seed)
    end = 7
    groups_n = rng.randint(1, 3)
    keys, rows, prompts = [], [], []
    for gi in range(groups_n):
        base_prompt = [rng.randint(0, 9) for _ in range(rng.randint(1, 12))]
        turns = [[rng.randint(0, 9) for _ in range(rng.randint(1, 6))] + [end] for _ in range(rng.randint(0, 4))]
        for _ in range(rng.randint(1, 5)):
            row = list(base_prompt)
            prompt_len = len(row)
            for t in turns[:rng.randint(0, len(turns))]:
                row += t
            row += [rng.randint(0, 9) for _ in range(rng.randint(0, 8))]
            if rng.random() < 0.3:
                row += [end]
            keys.append(f"g{gi}_tpr_{len(keys)}")
            rows.append(row)
            prompts.append(prompt_len)
    for min_len in (1, 2, 5, 128):
        batch = {"input_ids": [torch.tensor(r) for r in rows], "prompts": [torch.tensor(r[:p]) for r, p in zip(rows, prompts)]}
        trees = build_trajectory_trees_turn(keys, batch, min_segment_tokens=min_len, end_token_id=end)
        groups = {}
        for r, key in enumerate(keys):
            groups.setdefault(key.rsplit("_", 2)[0], []).append(r)
        expected = turn_trie(list(groups.items()), rows, prompts, min_len, end)
        assert len(trees) == len(expected)
        for tree, (uid, index, root_id, nodes) in zip(trees, expected):
            assert (tree.uid, tree.tree_index, tree.root_id) == (uid, index, root_id)
            assert set(tree.nodes) == set(nodes)
            for node_id, (parent, (row, start, stop), members, terminals, children) in nodes.items():
                n = tree.get(node_id)
                assert n.parent_id == parent
                assert (n.segment.row, n.segment.start, n.segment.end) == (row, start, stop), (seed, min_len, node_id)
                assert n.member_rows == members and n.terminal_rows == terminals and n.children == children


def test_oracle_turn_trie_reproduces_the_reference_known_answers():
    # unit/test_trajectory_tree_turn.py:64-172 applied to the oracle: complete
    # shared turns share a node, a short partial message does not
    from oracle.trie_oracle import turn_trie
    end = 151645
    prompt = [1, 2, 3]
    rows = [prompt + [10, 11, end] + [20, 21], prompt + [10, 11, end] + [30], prompt + [10, 12, end]]
    ((_, _, root, nodes),) = turn_trie([("s", [0, 1, 2])], rows, [3, 3, 3], 2, end)
    parent, (row, start, stop), members, terminals, children = nodes[root]
    assert (start, stop) == (0, 3) and members == (0, 1, 2) and len(children) == 2
    shared = nodes[children[0]]
    assert shared[1][1:] == (3, 6) and shared[2] == (0, 1) and len(shared[4]) == 2
    assert nodes[children[1]][1][1:] == (3, 6) and nodes[children[1]][2] == (2,)


def test_radix_builder_handles_long_rows():
    # 8 rollouts of 20k tokens sharing a 12k-token prompt and pairwise longer prefixes
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, 1000, (12000,), generator=g)
    rows = []
    for i in range(8):
        shared = torch.randint(0, 1000, (3000,), generator=torch.Generator().manual_seed(100 + i // 2))
        rows.append(torch.cat([prompt, shared, torch.randint(0, 1000, (5000,), generator=g)]))
    trees = build_trajectory_trees([f"u_s_{i}" for i in range(8)], {"input_ids": rows})
    (tree,) = trees
    root = tree.get(tree.root_id)
    assert root.segment.length >= 12000 and len(root.children) == 4
    assert all(len(tree.get(c).children) == 2 for c in root.children)
    _paths_reconstruct(trees, {"input_ids": rows})


# ---- unit/test_trajectory_tree_turn.py:64-172 --------------------------------------------
KEYS = ("same_tpr_0", "same_tpr_1", "same_tpr_2")


def _turn_batch(inputs, prompt_lengths=None):
    value = {"input_ids": [torch.tensor(t, dtype=torch.long) for t in inputs]}
    if prompt_lengths is not None:
        value["prompts"] = [torch.tensor(t[:n], dtype=torch.long) for t, n in zip(inputs, prompt_lengths)]
    return value


def _count(trees):
    return sum(len(t.nodes) for t in trees)


def test_turn_short_partial_shared_message_is_not_pushed():
    prompt = [11, 12, 13, 14]
    common_partial = [21, 22, 23, 24, 25, 26, 27, 28, 29]
    data = _turn_batch([prompt + common_partial + [31, EOT], prompt + common_partial + [32, EOT],
                        prompt + [33, EOT]], prompt_lengths=[len(prompt)] * 3)
    exact = build_trajectory_trees(KEYS, data)
    turned = build_trajectory_trees_turn(KEYS, data, min_segment_tokens=2)
    _paths_reconstruct(turned, data)
    assert _count(exact) > _count(turned)
    assert len(turned) == 1
    tree = turned[0]
    root = tree.get(tree.root_id)
    assert root.segment.end == len(prompt) and len(root.children) == 3
    assert all(not tree.get(k).children for k in root.children)


def test_turn_complete_turns_share_and_short_complete_turns_coalesce():
    prompt = [11, 12, 13, 14]
    t1 = [7] * 140 + [EOT]
    t2, t3 = [8, 9, EOT], [10, 11, EOT]
    data = _turn_batch([prompt + t1 + t2 + t3 + [12, EOT], prompt + t1 + t2 + t3 + [13, EOT],
                        prompt + t1 + [14, EOT]], prompt_lengths=[4] * 3)
    trees = build_trajectory_trees_turn(KEYS, data, min_segment_tokens=128)
    _paths_reconstruct(trees, data)
    assert len(trees) == 1
    tree = trees[0]
    assert tree.get(tree.root_id).segment.end == len(prompt) + len(t1)
    assert not any(node.children and node.segment.length in (3, 6) for node in tree.nodes.values())


def test_turn_no_full_shared_turn_leaves_independent_trees():
    data = _turn_batch([[1, 2, 3, 4, 5, 6, EOT], [1, 2, 3, 4, 5, 7, EOT]])
    trees = build_trajectory_trees_turn(("one_tpr_0", "one_tpr_1"), data)
    assert len(trees) == 2 and all(len(t.nodes) == 1 for t in trees)
    _paths_reconstruct(trees, data)


def test_turn_terminal_row_and_duplicates_remain_exact():
    shared = [1, 2, 3, EOT]
    data = _turn_batch([shared, shared + [4, 5, EOT], shared])
    trees = build_trajectory_trees_turn(KEYS, data, min_segment_tokens=2)
    _paths_reconstruct(trees, data)
    assert len(trees) == 1
    assert trees[0].get(trees[0].root_id).terminal_rows == (0, 2)


def test_turn_separate_uids_false_boundary_and_wrong_prompt():
    data = _turn_batch([[1, 2, EOT, 3, EOT], [1, 2, EOT, 4, EOT]])
    assert len(build_trajectory_trees_turn(("a_tpr_0", "b_tpr_1"), data)) == 2
    data = _turn_batch([[1, 2, 3, 4], [1, 2, 3, 5]])
    trees = build_trajectory_trees_turn(("a_tpr_0", "a_tpr_1"), data)
    assert len(trees) == 2
    _paths_reconstruct(trees, data)
    bad = _turn_batch([[1, 2, 3, 4]], prompt_lengths=[2])
    bad["prompts"][0][0] = 999
    with pytest.raises(ValueError, match="not an exact input prefix"):
        build_trajectory_trees_turn(["x_tpr_0"], bad)
    with pytest.raises(ValueError, match="min_segment_tokens"):
        build_trajectory_trees_turn(["x_tpr_0"], data, min_segment_tokens=0)


# ---- lowering ------------------------------------------------------------------------------
def test_lowering_packs_segments_in_preorder_with_positions_and_sources():
    batch = _make_batch([[1, 2, 3, 4, 5], [1, 2, 3, 4, 6], [1, 2, 3, 7], [9, 9]])
    trees = build_trajectory_trees(["u_s_0", "u_s_1", "u_s_2", "u_s_3"], batch)
    launch = lower_forest(trees)
    meta = launch.meta
    # tree 0: root [1,2,3] -> {4 -> {5, 6}, 7}; tree 1: [9, 9]
    assert meta.cu_seqlens_q == (0, 3, 4, 5, 6, 7, 9)
    assert meta.node_offsets == (0, 3, 4)             # internal: root [1,2,3], [4]
    assert meta.leaf_ancestors == ((), (0,), (0, 1), (0, 1), (0,), ())
    assert launch.positions.tolist() == [0, 1, 2, 3, 4, 4, 3, 0, 1]
    assert launch.gather_tokens(batch).tolist() == [1, 2, 3, 4, 5, 6, 7, 9, 9]
    assert launch.prefix_index.tolist() == [0, 1, 2, 3]
    assert launch.segments[0] == (0, trees[0].root_id) and launch.segments[-1] == (1, trees[1].root_id)
    single = lower_tree(trees[1])
    assert single.meta.node_offsets == (0,) and single.meta.leaf_ancestors == ((),)


@pytest.mark.parametrize("seed", range(4))
def test_lowered_launch_equals_the_per_segment_visits(seed):
    """The oracle's tree attention on the lowered layout == the reference's
    per-segment visits, outputs and all gradients (fp64)."""
    from _helpers import tree_of
    from oracle.tpr_oracle import tree_backward, tree_forward
    from oracle.trie_oracle import segment_visits
    keys, rows = _random_batch(seed + 100, n_uids=2, rows_per_uid=5)
    batch = _make_batch(rows)
    trees = build_trajectory_trees(keys, batch)
    launch = lower_forest(trees)
    meta = launch.meta
    tq, hq, hkv, d, scale = meta.total_q, 4, 2, 8, 0.35
    g = torch.Generator().manual_seed(seed)
    q, k, v, dout = (torch.randn(tq, h, d, generator=g, dtype=torch.float64) for h in (hq, hkv, hkv, hq))

    # lowered: prefix = k[prefix_index]; the prefix gradient folds back onto k, v
    pk, pv = launch.prefix_of(k), launch.prefix_of(v)
    out, lse = tree_forward(q, k, v, pk, pv, tree_of(meta), scale)
    dq, dk, dv, dpk, dpv = tree_backward(q, k, v, pk, pv, tree_of(meta), dout, scale, out=out, lse=lse)
    dk_total, dv_total = launch.fold_prefix_grad(dk, dpk), launch.fold_prefix_grad(dv, dpv)

    # per-segment visits over the same packed rows
    spans = [(meta.cu_seqlens_q[i], meta.cu_seqlens_q[i + 1]) for i in range(meta.num_leaves)]
    seg_index = {seg: i for i, seg in enumerate(launch.segments)}
    parents = []
    for t, node_id in launch.segments:
        p = trees[t].get(node_id).parent_id
        parents.append(None if p is None else seg_index[(t, p)])
    qa, ka, va = (x.clone().requires_grad_(True) for x in (q, k, v))
    ref = segment_visits(qa, ka, va, spans, parents, scale)
    ref.backward(dout)
    torch.testing.assert_close(out, ref.detach())
    torch.testing.assert_close(dq, qa.grad)
    torch.testing.assert_close(dk_total, ka.grad)
    torch.testing.assert_close(dv_total, va.grad)
