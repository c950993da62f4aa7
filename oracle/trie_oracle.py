"""CPU oracle of the rollout trie -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, as the checker of
``bridge_amd.topology``; the product never does.

``token_trie`` restates the reference's exact-trie builder in the plain form
it has there (trajectory_tree.py:126-245): one trie node per token, children
keyed by token id in insertion order, member rows appended as rows pass, the
row's last node recording it as a terminal row; then each real root (first
token) is compressed by following single-child chains of equal membership
with no terminal rows, numbering nodes in preorder. The result is plain
tuples, so tests compare it field by field with ``bridge_amd.topology``.

Pins: ``token_trie`` reproduces the known answers of the reference's own
trie tests (unit/test_trajectory_tree.py:23-151, in tests/test_topology.py);
``segment_visits`` is built on ``prefix_attention`` (pinned in
tests/test_oracle.py) and is checked against the oracle's independent
``tree_forward`` / ``tree_backward`` formulation on lowered layouts.

``segment_visits`` restates what the reference's executor computes for a
tree, one segment at a time (segment_executor.py visit order, kv_stack.py:139-154
path order): each segment's queries attend to the concatenated K/V of its
ancestors in full and to its own K/V causally.
"""

from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import torch

from .tpr_oracle import prefix_attention

Node = Tuple[int | None, Tuple[int, int, int], Tuple[int, ...], Tuple[int, ...], Tuple[int, ...]]


class _TokenNode:
    __slots__ = ("position", "members", "terminals", "children")

    def __init__(self, position: int):
        self.position = position
        self.members: List[int] = []
        self.terminals: List[int] = []
        self.children: Dict[int, "_TokenNode"] = {}


def _compress(first: _TokenNode, parent: int | None, out: Dict[int, Node]) -> int:
    start = first.position
    cur = first
    while not cur.terminals and len(cur.children) == 1:
        nxt = next(iter(cur.children.values()))
        if cur.members != nxt.members:
            break
        cur = nxt
    node_id = len(out)
    out[node_id] = None
    kids = tuple(_compress(c, node_id, out) for c in cur.children.values())
    out[node_id] = (parent, (cur.members[0], start, cur.position + 1), tuple(cur.members), tuple(cur.terminals), kids)
    return node_id


def token_trie(groups: Sequence[Tuple[str, Sequence[int]]], rows: Sequence[Sequence[int]]):
    """[(uid, tree_index, root_id, {node_id: (parent, (row, start, end), members, terminals, children)})]
    for uid groups given as (uid, member rows in row order)."""
    trees = []
    for uid, members in groups:
        dummy = _TokenNode(-1)
        for row in members:
            node = dummy
            for position, token in enumerate(rows[row]):
                child = node.children.get(int(token))
                if child is None:
                    child = _TokenNode(position)
                    node.children[int(token)] = child
                child.members.append(row)
                node = child
            node.terminals.append(row)
        for index, real_root in enumerate(dummy.children.values()):
            nodes: Dict[int, Node] = {}
            root_id = _compress(real_root, None, nodes)
            trees.append((uid, index, root_id, nodes))
    return trees


def segment_visits(q, k, v, spans, parents, scale):
    """Per-segment visits of a tree laid out segment by segment.

    ``spans[s]`` = rows [a, b) of segment s in q/k/v ([T, H, D] tensors),
    ``parents[s]`` = its parent segment or None; returns out [T, Hq, D].
    Gradients flow to q, k, v through autograd (every segment's K/V rows are
    the same tensor rows whether read as its own keys or as a descendant's
    prefix)."""
    outs = [None] * len(spans)
    for s, (a, b) in enumerate(spans):
        path, p = [], parents[s]
        while p is not None:
            path.append(p)
            p = parents[p]
        rows = [i for n in reversed(path) for i in range(*spans[n])]
        idx = torch.tensor(rows, dtype=torch.long, device=k.device)
        pk = k.index_select(0, idx).unsqueeze(1)
        pv = v.index_select(0, idx).unsqueeze(1)
        o = prefix_attention(q[a:b].unsqueeze(1), k[a:b].unsqueeze(1), v[a:b].unsqueeze(1), pk, pv, scale)
        outs[s] = o.reshape(b - a, q.shape[1], q.shape[2])
    return torch.cat(outs, 0)
