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

``turn_trie`` restates the reference's message-unit trie
(trajectory_tree_turn.py:46-186) in its plain form: each row is cut into
units after every end-of-message token and at the prompt end (a boundary
closer than ``min_segment_tokens`` to the previous kept one is dropped,
except the row end), one trie node per unit keyed by the unit's tokens under
its parent, then compressed and numbered like ``token_trie``.

Pins: ``token_trie`` reproduces the known answers of the reference's own
trie tests (unit/test_trajectory_tree.py:23-151, in tests/test_topology.py);
``turn_trie`` those of its turn-trie tests (unit/test_trajectory_tree_turn.py:64-172);
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


def _units(tokens: Sequence[int], prompt_length, min_segment_tokens: int, end_token_id: int):
    """[(unit tokens, end position)] of one row (trajectory_tree_turn.py:46-75)."""
    length = len(tokens)
    candidates = {i + 1 for i, t in enumerate(tokens) if int(t) == end_token_id}
    if prompt_length is not None and 0 < prompt_length < length:
        candidates.add(prompt_length)
    candidates.add(length)
    previous, units = 0, []
    for end in sorted(candidates):
        if end < length and end - previous < min_segment_tokens:
            continue
        units.append((tuple(int(t) for t in tokens[previous:end]), end))
        previous = end
    return units


class _UnitNode:
    __slots__ = ("position", "members", "terminals", "children")

    def __init__(self, end: int):
        self.position = end - 1          # last token of the unit, as in _TokenNode
        self.members: List[int] = []
        self.terminals: List[int] = []
        self.children: Dict[tuple, "_UnitNode"] = {}


def _compress_units(first: "_UnitNode", parent, start: int, out: Dict[int, Node]) -> int:
    cur = first
    while not cur.terminals and len(cur.children) == 1:
        nxt = next(iter(cur.children.values()))
        if cur.members != nxt.members:
            break
        cur = nxt
    node_id = len(out)
    out[node_id] = None
    kids = tuple(_compress_units(c, node_id, cur.position + 1, out) for c in cur.children.values())
    out[node_id] = (parent, (first.members[0], start, cur.position + 1), tuple(cur.members), tuple(cur.terminals), kids)
    return node_id


def turn_trie(groups: Sequence[Tuple[str, Sequence[int]]], rows: Sequence[Sequence[int]], prompt_lengths,
              min_segment_tokens: int, end_token_id: int):
    """The ``token_trie`` result format for the message-unit trie."""
    trees = []
    for uid, members in groups:
        dummy = _UnitNode(0)
        for row in members:
            node = dummy
            plen = None if prompt_lengths is None else prompt_lengths[row]
            for unit, end in _units(rows[row], plen, min_segment_tokens, end_token_id):
                child = node.children.get(unit)
                if child is None:
                    child = _UnitNode(end)
                    node.children[unit] = child
                child.members.append(row)
                node = child
            node.terminals.append(row)
        for index, real_root in enumerate(dummy.children.values()):
            nodes: Dict[int, Node] = {}
            root_id = _compress_units(real_root, None, 0, nodes)
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
