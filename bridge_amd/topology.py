"""Rollout topology: token-exact tries and their lowering to one kernel launch.

The reference turns a training batch into compressed tries of the rollouts
that share token prefixes -- ``build_trajectory_trees``
(trajectory_tree.py:126-314, exact tokens) or ``build_trajectory_trees_turn``
(trajectory_tree_turn.py:32-186, Qwen3 ChatML message units) -- and lowers
each tree to a ``SegmentPlan`` of segments with ``position_start =
prefix_length = segment start`` (tree_plan_builder.py:179-193), which its
executor then visits one segment at a time, building RoPE for positions
``[P, P + b)`` of each (rope.py:71-119).

Here the same tries are built (same node ids, children order, member and
terminal rows) by a radix insertion that compares whole token spans with
numpy instead of walking one token at a time, and ``lower_tree`` /
``lower_forest`` turn one tree (or a forest) into the packed metadata of ONE
launch per layer that runs every segment:

  * query segments = every segment of every tree, in DFS preorder (children
    in insertion order), packed back to back: ``meta.cu_seqlens_q``;
  * prefix nodes = the internal segments, in the same order:
    ``meta.node_offsets``; each query segment's ancestors, root first:
    ``meta.leaf_ancestors`` -- in preorder every node's descendants form one
    contiguous run of query segments, as the kernel's tree contract needs;
  * ``positions`` = each packed token's absolute position (its RoPE position),
    ``source_rows`` = the batch row it is read from (the SegmentRef row);
  * ``prefix_index`` = the packed row of every prefix-node row, so the prefix
    K/V of a layer are ``k[prefix_index]`` and the prefix gradient folds back
    with ``dk.index_add_(0, prefix_index, dprefix_k)``.

Each segment then attends to its ancestors in full and to itself causally --
the visit of the reference's executor -- with all segments and all levels in
one launch.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from types import MappingProxyType
from typing import Any, Dict, List, Mapping, Optional, Sequence, Tuple

import numpy as np
import torch

from .meta import TPRPrefixMeta

__all__ = [
    "QWEN3_IM_END_TOKEN_ID",
    "SegmentRef",
    "TrajectoryNode",
    "TrajectoryTree",
    "TreeLaunch",
    "build_trajectory_trees",
    "build_prompt_sibling_trees",
    "build_trajectory_trees_turn",
    "lower_tree",
    "lower_forest",
]

QWEN3_IM_END_TOKEN_ID = 151645  # <|im_end|> (trajectory_tree_turn.py:32)


def _is_int(value) -> bool:
    return isinstance(value, int) and not isinstance(value, bool)


@dataclass(frozen=True)
class SegmentRef:
    """Rows [start, end) of one batch row (trajectory_tree.py:26-43)."""

    row: int
    start: int
    end: int

    def __post_init__(self):
        if not _is_int(self.row) or self.row < 0:
            raise ValueError(f"row must be a non-negative integer, got {self.row!r}")
        if not _is_int(self.start) or self.start < 0:
            raise ValueError(f"start must be a non-negative integer, got {self.start!r}")
        if not _is_int(self.end) or self.end <= self.start:
            raise ValueError(f"end must be an integer > start, got {self.end!r}")

    @property
    def length(self) -> int:
        return self.end - self.start


@dataclass(frozen=True)
class TrajectoryNode:
    """One compressed segment of a trie (trajectory_tree.py:46-72)."""

    node_id: int
    parent_id: Optional[int]
    segment: SegmentRef
    member_rows: Tuple[int, ...]
    terminal_rows: Tuple[int, ...]
    children: Tuple[int, ...]

    def __post_init__(self):
        if not _is_int(self.node_id) or self.node_id < 0:
            raise ValueError(f"node_id must be a non-negative integer, got {self.node_id!r}")
        if self.parent_id is not None and (not _is_int(self.parent_id) or self.parent_id < 0
                                           or self.parent_id == self.node_id):
            raise ValueError(f"invalid parent_id {self.parent_id!r} for node {self.node_id}")
        if not self.member_rows:
            raise ValueError(f"node {self.node_id} must contain at least one member row")
        if len(set(self.member_rows)) != len(self.member_rows):
            raise ValueError(f"node {self.node_id} member_rows must be unique")
        if not set(self.terminal_rows).issubset(self.member_rows):
            raise ValueError(f"node {self.node_id} terminal_rows must be a subset of member_rows")


@dataclass(frozen=True)
class TrajectoryTree:
    """A trie whose root starts at token position 0 (trajectory_tree.py:75-124)."""

    uid: str
    tree_index: int
    root_id: int
    member_rows: Tuple[int, ...]
    nodes: Mapping[int, TrajectoryNode]

    def __post_init__(self):
        nodes = dict(self.nodes)
        if self.root_id not in nodes:
            raise ValueError(f"root_id {self.root_id} does not exist")
        root = nodes[self.root_id]
        if root.parent_id is not None:
            raise ValueError("trajectory tree root must not have a parent")
        if root.segment.start != 0:
            raise ValueError("trajectory tree executable root must start at token position 0")
        if root.member_rows != self.member_rows:
            raise ValueError("trajectory tree member_rows must match root member_rows")
        for node_id, node in nodes.items():
            if node_id != node.node_id:
                raise ValueError(f"node mapping key {node_id} does not match node_id {node.node_id}")
            if node.parent_id is not None and node.parent_id not in nodes:
                raise ValueError(f"node {node_id} has missing parent {node.parent_id}")
            for child_id in node.children:
                if child_id not in nodes:
                    raise ValueError(f"node {node_id} has missing child {child_id}")
                child = nodes[child_id]
                if child.parent_id != node_id:
                    raise ValueError(f"node {node_id} child {child_id} has inconsistent parent")
                if child.segment.start != node.segment.end:
                    raise ValueError(f"node {child_id} must start at parent {node_id} end {node.segment.end}, "
                                     f"got {child.segment.start}")
        object.__setattr__(self, "nodes", MappingProxyType(nodes))

    @property
    def key(self) -> str:
        return f"{self.uid}:{self.tree_index}"

    def get(self, node_id: int) -> TrajectoryNode:
        try:
            return self.nodes[node_id]
        except KeyError as exc:
            raise KeyError(f"unknown trajectory node {node_id}") from exc

    def preorder(self) -> Tuple[int, ...]:
        """Node ids in DFS preorder, children in insertion order."""
        order, todo = [], [self.root_id]
        while todo:
            n = todo.pop()
            order.append(n)
            todo.extend(reversed(self.nodes[n].children))
        return tuple(order)


# ---- batch parsing (trajectory_tree.py:136-175) ------------------------------------
def _rows(batch: Any, name: str) -> list:
    try:
        value = batch[name]
    except Exception as exc:
        raise ValueError(f"training batch is missing required field {name!r}") from exc
    if isinstance(value, (list, tuple)):
        return list(value)
    unbind = getattr(value, "unbind", None)
    if callable(unbind):
        return list(unbind())
    raise TypeError(f"field {name!r} does not expose row-wise values: {type(value)!r}")


def _as_token_array(value: Any, *, row: int) -> np.ndarray:
    if not isinstance(value, torch.Tensor):
        raise TypeError(f"input_ids[{row}] must be a torch.Tensor, got {type(value)!r}")
    if value.ndim != 1:
        raise ValueError(f"input_ids[{row}] must be 1-D, got shape={tuple(value.shape)}")
    if value.numel() == 0:
        raise ValueError(f"input_ids[{row}] must not be empty")
    if value.dtype == torch.bool or torch.is_floating_point(value) or torch.is_complex(value):
        raise ValueError(f"input_ids[{row}] must use an integer dtype, got {value.dtype}")
    tokens = value.detach().cpu().to(torch.int64).numpy()
    if (tokens < 0).any():
        raise ValueError(f"input_ids[{row}] must contain non-negative token ids")
    return tokens


def _parse_key(key: str) -> Tuple[str, str, int]:
    if not isinstance(key, str):
        raise TypeError(f"trajectory key must be str, got {type(key)!r}")
    fields = key.rsplit("_", 2)
    if len(fields) != 3 or not fields[0] or not fields[1]:
        raise ValueError(f"unexpected trajectory key format: {key!r}")
    try:
        index = int(fields[2])
    except ValueError as exc:
        raise ValueError(f"trajectory key has non-integer index: {key!r}") from exc
    return fields[0], fields[1], index


def _group_rows(keys: Sequence[str]) -> Dict[str, List[int]]:
    seen, groups = set(), {}
    for row, key in enumerate(keys):
        if key in seen:
            raise ValueError(f"duplicate trajectory key: {key!r}")
        seen.add(key)
        uid, _, _ = _parse_key(key)
        groups.setdefault(uid, []).append(row)
    return groups


# ---- radix trie ---------------------------------------------------------------------
@dataclass
class _Radix:
    start: int
    end: int
    src: int                     # first row through this span (its tokens are the span's)
    members: List[int] = field(default_factory=list)
    terminals: List[int] = field(default_factory=list)
    children: Dict[Any, "_Radix"] = field(default_factory=dict)   # insertion-ordered


def _first_mismatch(a: np.ndarray, b: np.ndarray) -> int:
    """Length of the common prefix of two equal-length arrays."""
    diff = np.flatnonzero(a != b)
    return int(diff[0]) if diff.size else int(a.size)


def _insert_tokens(root: _Radix, row: int, tokens: np.ndarray, all_tokens: List[np.ndarray]) -> None:
    """Insert one row into the radix trie. Spans end only where a row ends or
    rows branch, so every node is one maximal chain of the reference's
    one-token trie (trajectory_tree.py:178-194, compressed as in :197-245)."""
    length = int(tokens.size)
    node, pos = root, 0
    while True:
        if pos == length:
            node.terminals.append(row)
            return
        child = node.children.get(int(tokens[pos]))
        if child is None:
            node.children[int(tokens[pos])] = _Radix(pos, length, row, [row], [row])
            return
        span = all_tokens[child.src][child.start:child.end]
        m = min(length, child.end) - pos
        common = _first_mismatch(tokens[pos:pos + m], span[:m])
        if common < child.end - pos:
            # split the child at pos + common: the upper part is shared with `row`
            cut = pos + common
            lower = _Radix(cut, child.end, child.src, child.members, child.terminals, child.children)
            child.end = cut
            child.members = list(lower.members)
            child.terminals = []
            child.children = {int(all_tokens[child.src][cut]): lower}
        child.members.append(row)
        node, pos = child, child.end


def _emit(root: _Radix, nodes: Dict[int, TrajectoryNode]) -> int:
    """Assign node ids in preorder, children in insertion order (the numbering
    of trajectory_tree.py:197-245), without recursion."""
    ids: Dict[int, int] = {}
    order: List[Tuple[_Radix, Optional[int]]] = []
    todo: List[Tuple[_Radix, Optional[int]]] = [(root, None)]
    while todo:
        node, parent = todo.pop()
        ids[id(node)] = len(order)
        order.append((node, parent))
        todo.extend((c, ids[id(node)]) for c in reversed(list(node.children.values())))
    base = len(nodes)
    for node, parent in order:
        nid = base + ids[id(node)]
        nodes[nid] = TrajectoryNode(nid, None if parent is None else base + parent,
                                    SegmentRef(row=node.members[0], start=node.start, end=node.end),
                                    tuple(node.members), tuple(node.terminals),
                                    tuple(base + ids[id(c)] for c in node.children.values()))
    return base


def build_trajectory_trees(keys: Sequence[str], batch: Any) -> Tuple[TrajectoryTree, ...]:
    """Token-exact compressed tries of each uid group (trajectory_tree.py:248-301).

    Rows of one uid that share no first token become separate trees; a row
    that ends inside another's path is a terminal row of an internal node;
    duplicate rows share a path and are all terminal rows of its last node.
    """
    keys = list(keys)
    if not keys:
        return ()
    input_rows = _rows(batch, "input_ids")
    if len(keys) != len(input_rows):
        raise ValueError(f"keys/batch row mismatch: keys={len(keys)} rows={len(input_rows)}")
    groups = _group_rows(keys)
    tokens = [_as_token_array(value, row=row) for row, value in enumerate(input_rows)]
    trees = []
    for uid, rows in groups.items():
        dummy = _Radix(0, 0, -1)
        for row in rows:
            _insert_tokens(dummy, row, tokens[row], tokens)
        for tree_index, real_root in enumerate(dummy.children.values()):
            nodes: Dict[int, TrajectoryNode] = {}
            root_id = _emit(real_root, nodes)
            trees.append(TrajectoryTree(uid, tree_index, root_id, nodes[root_id].member_rows, nodes))
    return tuple(trees)


def build_prompt_sibling_trees(keys: Sequence[str], batch: Any) -> Tuple[TrajectoryTree, ...]:
    """The reference's older name for ``build_trajectory_trees`` (trajectory_tree.py:304-314)."""
    return build_trajectory_trees(keys, batch)


# ---- turn-unit trie (trajectory_tree_turn.py) ----------------------------------------------
def _unit_ends(tokens: np.ndarray, *, prompt_length: Optional[int], min_segment_tokens: int,
               end_token_id: int) -> np.ndarray:
    """Token positions where a row's units end (the unit rule of
    trajectory_tree_turn.py:46-75): after every end-of-message token and at
    the prompt end, dropping a boundary closer than ``min_segment_tokens`` to
    the one kept before it; the row's end always closes the last unit."""
    length = int(tokens.size)
    cuts = np.flatnonzero(tokens == end_token_id) + 1
    if prompt_length is not None and 0 < prompt_length < length:
        cuts = np.union1d(cuts, [prompt_length])
    kept, previous = [], 0
    for end in cuts.tolist():
        if end < length and end - previous >= min_segment_tokens:
            kept.append(end)
            previous = end
    kept.append(length)
    return np.asarray(kept, dtype=np.int64)


def build_trajectory_trees_turn(keys: Sequence[str], batch: Any, *, min_segment_tokens: int = 128,
                                end_token_id: int = QWEN3_IM_END_TOKEN_ID) -> Tuple[TrajectoryTree, ...]:
    """Tries that share only complete message units (trajectory_tree_turn.py:120-186).

    Each row is cut into units, every distinct unit (its exact tokens) gets
    an integer id, and the rows' id sequences go through the same radix trie
    as the token-exact builder: rows share a node while they share whole
    units, and a node ends where rows branch or end. Node spans are mapped
    back from unit indices to token positions (equal unit prefixes end at
    equal positions).
    """
    if not _is_int(min_segment_tokens) or min_segment_tokens < 1:
        raise ValueError("min_segment_tokens must be a positive integer")
    if not _is_int(end_token_id) or end_token_id < 0:
        raise ValueError("end_token_id must be a non-negative integer")
    keys = list(keys)
    if not keys:
        return ()
    inputs = _rows(batch, "input_ids")
    if len(inputs) != len(keys):
        raise ValueError("turn builder input rows and trajectory keys disagree")
    try:
        prompts = _rows(batch, "prompts")
    except (ValueError, KeyError):
        prompts = None
    if prompts is not None and len(prompts) != len(keys):
        raise ValueError("turn builder prompt rows and trajectory keys disagree")
    unit_id: Dict[bytes, int] = {}
    ends, seqs = [], []
    for row in range(len(keys)):
        tokens = _as_token_array(inputs[row], row=row)
        prompt_length = None
        if prompts is not None:
            prompt = _as_token_array(prompts[row], row=row)
            prompt_length = int(prompt.size)
            if prompt_length > tokens.size or not np.array_equal(tokens[:prompt_length], prompt):
                raise ValueError(f"turn builder prompt is not an exact input prefix for row={row}")
        cut = _unit_ends(tokens, prompt_length=prompt_length, min_segment_tokens=min_segment_tokens,
                         end_token_id=end_token_id)
        starts = np.concatenate(([0], cut[:-1]))
        seqs.append(np.asarray([unit_id.setdefault(tokens[a:b].tobytes(), len(unit_id))
                                for a, b in zip(starts.tolist(), cut.tolist())], dtype=np.int64))
        ends.append(cut)
    forest = []
    for uid, rows in _group_rows(keys).items():
        dummy = _Radix(0, 0, -1)
        for row in rows:
            _insert_tokens(dummy, row, seqs[row], seqs)
        for tree_index, real_root in enumerate(dummy.children.values()):
            unit_nodes: Dict[int, TrajectoryNode] = {}
            root_id = _emit(real_root, unit_nodes)
            nodes = {}
            for nid, nd in unit_nodes.items():
                e = ends[nd.segment.row]
                span = SegmentRef(row=nd.segment.row, start=int(e[nd.segment.start - 1]) if nd.segment.start else 0,
                                  end=int(e[nd.segment.end - 1]))
                nodes[nid] = TrajectoryNode(nid, nd.parent_id, span, nd.member_rows, nd.terminal_rows, nd.children)
            forest.append(TrajectoryTree(uid, tree_index, root_id, nodes[root_id].member_rows, nodes))
    return tuple(forest)


# ---- lowering to one launch ---------------------------------------------------------------
@dataclass(frozen=True)
class TreeLaunch:
    """Packed metadata of one launch that runs every segment of a forest.

    ``segments[i]`` = (tree index, node id) of query segment i;
    ``prefix_segments[j]`` = (tree index, node id) of prefix node j (the
    internal segments); ``positions`` / ``source_rows`` / ``prefix_index`` as
    in the module docstring.
    """

    meta: TPRPrefixMeta
    segments: Tuple[Tuple[int, int], ...]
    prefix_segments: Tuple[Tuple[int, int], ...]
    positions: torch.Tensor      # int64 [total_q]
    source_rows: torch.Tensor    # int64 [total_q]
    prefix_index: torch.Tensor   # int64 [total_prefix]

    def gather_tokens(self, batch: Any) -> torch.Tensor:
        """input_ids of the packed layout (int64 [total_q])."""
        rows = _rows(batch, "input_ids")
        flat = torch.cat([torch.as_tensor(r).to(torch.int64).cpu() for r in rows])
        starts = torch.tensor([0] + [int(torch.as_tensor(r).numel()) for r in rows[:-1]], dtype=torch.int64).cumsum(0)
        return flat[starts[self.source_rows] + self.positions]

    def prefix_of(self, packed: torch.Tensor) -> torch.Tensor:
        """The prefix-node rows of a packed ``[total_q, ...]`` tensor (K or V)."""
        return packed.index_select(0, self.prefix_index.to(packed.device))

    def fold_prefix_grad(self, grad: torch.Tensor, prefix_grad: torch.Tensor) -> torch.Tensor:
        """Add a prefix-node gradient back onto the packed rows it came from."""
        return grad.index_add(0, self.prefix_index.to(grad.device), prefix_grad.to(grad.dtype))


def lower_forest(trees: Sequence[TrajectoryTree]) -> TreeLaunch:
    """One launch for every segment of every tree (see the module docstring)."""
    if not trees:
        raise ValueError("lower_forest needs at least one tree")
    cu, node_off, anc = [0], [0], []
    segments, prefix_segments = [], []
    positions, source_rows, prefix_index = [], [], []
    for t_index, tree in enumerate(trees):
        if not isinstance(tree, TrajectoryTree):
            raise TypeError(f"trees must hold TrajectoryTree objects, got {type(tree).__name__}")
        order = tree.preorder()
        packed_start: Dict[int, int] = {}
        for node_id in order:
            seg = tree.nodes[node_id].segment
            packed_start[node_id] = cu[-1]
            cu.append(cu[-1] + seg.length)
            segments.append((t_index, node_id))
            positions.append(torch.arange(seg.start, seg.end, dtype=torch.int64))
            source_rows.append(torch.full((seg.length,), seg.row, dtype=torch.int64))
        node_index: Dict[int, int] = {}
        for node_id in order:
            node = tree.nodes[node_id]
            if node.children:
                node_index[node_id] = len(prefix_segments)
                prefix_segments.append((t_index, node_id))
                node_off.append(node_off[-1] + node.segment.length)
                start = packed_start[node_id]
                prefix_index.append(torch.arange(start, start + node.segment.length, dtype=torch.int64))
        for node_id in order:
            path, p = [], tree.nodes[node_id].parent_id
            while p is not None:
                path.append(node_index[p])
                p = tree.nodes[p].parent_id
            anc.append(tuple(reversed(path)))
    meta = TPRPrefixMeta(tuple(cu), tuple(node_off), tuple(anc))
    cat = lambda xs: torch.cat(xs) if xs else torch.zeros(0, dtype=torch.int64)  # noqa: E731
    return TreeLaunch(meta, tuple(segments), tuple(prefix_segments), cat(positions), cat(source_rows),
                      cat(prefix_index))


def lower_tree(tree: TrajectoryTree) -> TreeLaunch:
    """``lower_forest`` of one tree."""
    return lower_forest([tree])
