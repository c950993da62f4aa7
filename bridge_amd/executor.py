"""Sibling-batched tree execution: the reference's Push / Pop / leaf-visit
schedule with each parent's adjacent leaves run as one kernel launch per layer.

The reference executes a segment tree as a DFS event stream
(``SegmentPlan.dfs_events``, segment_plan.py:266-275: Push(seg), the
children's events in insertion order, Pop(seg)). Its scheduler turns every
adjacent (Push L, Pop L) of a childless segment L into one physical
``visit_leaf`` (fixed_topology_scheduler.py:142-158, 200-210), and the
executor visits those leaves one at a time (segment_executor.py:327-444):
forward over the leaf's tokens against the concatenated path K/V, loss,
backward, and the path's K/V gradient added to every ancestor
(kv_stack.py:175-203). Pop(seg) then recomputes seg with its gradient graph
and injects the gradient relayed to its K/V (segment_executor.py:239-325).

Here a maximal run of adjacent leaf pairs under one parent becomes one
``VISIT_LEAVES`` step: the siblings' tokens are packed along the sequence
axis, each sibling's RoPE positions run from the parent's end P to P + S_i
(rope.py:71-119, position_start = prefix_length, segment_plan.py:193-197),
and one ``TPRKernelBackend`` launch per layer attends every sibling to the
shared path and causally to itself. The kernel adds the path's gradient,
summed over the siblings in sibling order, into the ``PrefixKVStack``'s fp32
rows. Flattening the steps (one ``visit_leaf`` per leaf of a batch, in order)
gives back the reference's physical trace exactly; only the launch grouping
changes.

The model is the caller's: ``forward_fn(segments, position_ids, backend)``
runs it over the packed tokens of ``segments`` with ``backend`` as the
attention backend of every layer (the seam of attention.py:141-148) and
returns ``(loss, new_key_values)``, ``new_key_values`` being ``{layer: (K, V)}``
``[sum S, 1, Hkv, D]``: the post-RoPE keys and the values its attention layers
recorded (attention.py:169-171).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from typing import Callable, Dict, Mapping, Optional, Sequence, Tuple

import torch

from .backend import TPRKernelBackend
from .relay import PrefixKVStack, StackSegment

__all__ = ["SegmentEventKind", "SegmentEvent", "ExecutionKind", "ExecutionStep", "ScheduleResult",
           "build_segments", "dfs_events", "batch_leaf_visits", "BatchedLeafExecutor"]


class SegmentEventKind(str, Enum):
    PUSH = "push"
    POP = "pop"


@dataclass(frozen=True)
class SegmentEvent:
    kind: SegmentEventKind
    segment_id: int


class ExecutionKind(str, Enum):
    PUSH = "push"
    POP = "pop"
    VISIT_LEAVES = "visit_leaves"


@dataclass(frozen=True)
class ExecutionStep:
    """PUSH / POP of ``segment_ids[0]``, or one batched visit of the leaves
    ``segment_ids`` (all children of ``parent_id``, adjacent in the DFS)."""

    kind: ExecutionKind
    segment_ids: Tuple[int, ...]
    parent_id: Optional[int] = None


@dataclass
class ScheduleResult:
    steps: Tuple[ExecutionStep, ...]
    losses: Dict[Tuple[int, ...], torch.Tensor] = field(default_factory=dict)  # visit / pop -> loss (detached)
    relayed: Dict[int, Dict[int, Tuple[torch.Tensor, torch.Tensor]]] = field(default_factory=dict)
    # popped segment -> {layer: (dK, dV)} fp32, the gradient relayed to its K/V by its descendants

    def leaf_trace(self) -> Tuple[Tuple[str, int], ...]:
        """The reference scheduler's physical trace: one visit_leaf per leaf."""
        out = []
        for st in self.steps:
            if st.kind is ExecutionKind.VISIT_LEAVES:
                out.extend(("visit_leaf", s) for s in st.segment_ids)
            else:
                out.append((st.kind.value, st.segment_ids[0]))
        return tuple(out)


def build_segments(parents: Mapping[int, Optional[int]], lengths: Mapping[int, int]) -> Dict[int, StackSegment]:
    """Segments with the reference's derived fields: a child's prefix_length
    and position_start are its parent's end (segment_plan.py:193-197).
    ``parents`` is in insertion order (the children order of the DFS)."""
    roots = [s for s, p in parents.items() if p is None]
    if len(roots) != 1:
        raise ValueError(f"segment tree must have exactly one root, got {roots}")
    children = _children_of(parents)
    out: Dict[int, StackSegment] = {}
    stack = [(roots[0], 0)]
    while stack:
        seg, start = stack.pop()
        length = int(lengths[seg])
        out[seg] = StackSegment(seg, parents[seg], length, start, start)
        for c in reversed(children[seg]):
            stack.append((c, start + length))
    if len(out) != len(parents):
        raise ValueError("segment tree is not connected")
    return {s: out[s] for s in parents}


def _children_of(parents: Mapping[int, Optional[int]]) -> Dict[int, list]:
    children: Dict[int, list] = {s: [] for s in parents}
    for s, p in parents.items():
        if p is not None:
            if p not in children:
                raise ValueError(f"segment {s} has missing parent {p}")
            children[p].append(s)
    return children


def dfs_events(segments: Mapping[int, StackSegment]) -> Tuple[SegmentEvent, ...]:
    """Push(seg), its children's events in insertion order, Pop(seg)
    (segment_plan.py:266-275), on an explicit stack."""
    parents = {s: seg.parent_id for s, seg in segments.items()}
    children = _children_of(parents)
    root = next(s for s, p in parents.items() if p is None)
    events = []
    stack = [(root, False)]
    while stack:
        seg, done = stack.pop()
        if done:
            events.append(SegmentEvent(SegmentEventKind.POP, seg))
            continue
        events.append(SegmentEvent(SegmentEventKind.PUSH, seg))
        stack.append((seg, True))
        for c in reversed(children[seg]):
            stack.append((c, False))
    return tuple(events)


def batch_leaf_visits(events: Sequence[SegmentEvent], segments: Mapping[int, StackSegment], *,
                      batch: bool = True) -> Tuple[ExecutionStep, ...]:
    """Lower an event stream to execution steps.

    An adjacent (Push L, Pop L) of a childless L is a leaf visit
    (fixed_topology_scheduler.py:200-210); with ``batch``, a maximal run of
    leaf visits under one parent is one VISIT_LEAVES step, otherwise each is
    its own. The stream must keep the stack discipline the reference's
    ``validate_events`` checks (segment_plan.py:277-313)."""
    parents = {s: seg.parent_id for s, seg in segments.items()}
    children = _children_of(parents)
    _validate_events(events, parents, children)
    steps = []
    i = 0
    while i < len(events):
        ev = events[i]
        nxt = events[i + 1] if i + 1 < len(events) else None
        is_leaf = (ev.kind is SegmentEventKind.PUSH and nxt is not None and nxt.kind is SegmentEventKind.POP
                   and nxt.segment_id == ev.segment_id and not children[ev.segment_id])
        if is_leaf:
            parent = parents[ev.segment_id]
            last = steps[-1] if steps else None
            if (batch and last is not None and last.kind is ExecutionKind.VISIT_LEAVES
                    and last.parent_id == parent):
                steps[-1] = ExecutionStep(ExecutionKind.VISIT_LEAVES, last.segment_ids + (ev.segment_id,), parent)
            else:
                steps.append(ExecutionStep(ExecutionKind.VISIT_LEAVES, (ev.segment_id,), parent))
            i += 2
            continue
        kind = ExecutionKind.PUSH if ev.kind is SegmentEventKind.PUSH else ExecutionKind.POP
        steps.append(ExecutionStep(kind, (ev.segment_id,), parents[ev.segment_id]))
        i += 1
    return tuple(steps)


def _validate_events(events, parents, children) -> None:
    # the stack discipline of SegmentPlan.validate_events (segment_plan.py:277-313)
    stack, pushed, popped = [], set(), set()
    for ev in events:
        if not isinstance(ev, SegmentEvent):
            raise TypeError(f"events must contain SegmentEvent objects, got {type(ev).__name__}")
        if ev.segment_id not in parents:
            raise KeyError(f"unknown segment_id {ev.segment_id}")
        if ev.kind is SegmentEventKind.PUSH:
            if ev.segment_id in pushed:
                raise ValueError(f"segment {ev.segment_id} is pushed more than once")
            expected = stack[-1] if stack else None
            if parents[ev.segment_id] != expected:
                raise ValueError(f"cannot push segment {ev.segment_id}: expected parent on stack "
                                 f"{parents[ev.segment_id]}, got {expected}")
            stack.append(ev.segment_id)
            pushed.add(ev.segment_id)
        else:
            if not stack or stack[-1] != ev.segment_id:
                raise ValueError(f"cannot pop segment {ev.segment_id}: current stack is {stack}")
            if any(c not in popped for c in children[ev.segment_id]):
                raise ValueError(f"cannot pop segment {ev.segment_id} before all children")
            stack.pop()
            popped.add(ev.segment_id)
    if stack or pushed != set(parents) or popped != set(parents):
        raise ValueError(f"incomplete event stream: stack={stack}, unpushed={sorted(set(parents) - pushed)}, "
                         f"unpopped={sorted(set(parents) - popped)}")


ForwardFn = Callable[[Tuple[StackSegment, ...], torch.Tensor, object],
                     Tuple[torch.Tensor, Mapping[int, Tuple[torch.Tensor, torch.Tensor]]]]


class BatchedLeafExecutor:
    """Runs execution steps against a ``PrefixKVStack``.

    ``backend_factory(stack, suffix_lengths)`` makes the attention backend of
    one step; the default, ``TPRKernelBackend.from_stack``, attends to the
    stack's path and adds the path's gradient into the stack's fp32 rows.
    """

    def __init__(self, segments: Mapping[int, StackSegment], forward_fn: ForwardFn, stack: PrefixKVStack, *,
                 backend_factory: Callable = TPRKernelBackend.from_stack, device: Optional[torch.device] = None):
        self.segments = dict(segments)
        self.forward_fn = forward_fn
        self.stack = stack
        self.backend_factory = backend_factory
        self.device = device

    # -- steps ------------------------------------------------------------------------
    def position_ids(self, segs: Sequence[StackSegment]) -> torch.Tensor:
        """Each segment's positions [position_start, position_start + length),
        concatenated in order (rope.py:71-119 with offset = prefix_length)."""
        return torch.cat([torch.arange(s.position_start, s.position_start + s.length, device=self.device)
                          for s in segs])

    def _check_top(self, segs: Sequence[StackSegment], what: str) -> None:
        top = self.stack.top().segment_id if len(self.stack) else None
        for s in segs:
            if s.parent_id != top:
                raise RuntimeError(f"cannot {what} segment {s.segment_id}: expected parent on stack "
                                   f"{s.parent_id}, got {top}")
            if s.prefix_length != self.stack.prefix_length:
                raise RuntimeError(f"cannot {what} segment {s.segment_id}: stack prefix length is "
                                   f"{self.stack.prefix_length}, got {s.prefix_length}")

    def push(self, seg_id: int) -> None:
        """Graph-free forward of the segment; its K/V go on the stack (segment_executor.py:208-237)."""
        seg = self.segments[seg_id]
        self._check_top([seg], "push")
        backend = self.backend_factory(self.stack, (seg.length,))
        with torch.no_grad():
            _, new_kv = self.forward_fn((seg,), self.position_ids([seg]), backend)
        self.stack.push(seg, {layer: (k.detach(), v.detach()) for layer, (k, v) in new_kv.items()})

    def visit_leaves(self, leaf_ids: Sequence[int]) -> torch.Tensor:
        """One packed forward + backward of sibling leaves (segment_executor.py:327-444,
        batched). Returns the detached loss."""
        segs = tuple(self.segments[s] for s in leaf_ids)
        self._check_top(segs, "visit")
        backend = self.backend_factory(self.stack, tuple(s.length for s in segs))
        with torch.enable_grad():
            loss, _ = self.forward_fn(segs, self.position_ids(segs), backend)
            if not isinstance(loss, torch.Tensor) or loss.numel() != 1:
                raise TypeError("forward_fn must return a scalar loss")
            loss.backward()
        return loss.detach()

    def pop(self, seg_id: int) -> Tuple[torch.Tensor, Dict[int, Tuple[torch.Tensor, torch.Tensor]]]:
        """Recompute the segment with its graph and inject the gradient relayed
        to its K/V (segment_executor.py:239-325). Returns (loss, relayed)."""
        entry = self.stack.top()
        if entry.segment_id != seg_id:
            raise RuntimeError(f"cannot pop segment {seg_id}: stack top is {entry.segment_id}")
        relayed = {layer: (gk.clone(), gv.clone()) for layer, (gk, gv) in entry.gradients.items()}
        self.stack.pop(seg_id)
        seg = self.segments[seg_id]
        backend = self.backend_factory(self.stack, (seg.length,))
        with torch.enable_grad():
            loss, new_kv = self.forward_fn((seg,), self.position_ids([seg]), backend)
            roots, grads = [loss], [None]
            for layer, (k, v) in new_kv.items():
                gk, gv = relayed[layer]
                roots.extend((k, v))
                grads.extend((gk.to(k.dtype).reshape(k.shape), gv.to(v.dtype).reshape(v.shape)))
            torch.autograd.backward(roots, grad_tensors=grads)
        return loss.detach(), relayed

    # -- the whole schedule ---------------------------------------------------------------
    def run(self, events: Optional[Sequence[SegmentEvent]] = None, *, batch: bool = True) -> ScheduleResult:
        """Execute a DFS event stream (default: the segments' own DFS) with
        leaf visits batched per parent (``batch``) or one at a time."""
        self.stack.assert_empty()
        steps = batch_leaf_visits(dfs_events(self.segments) if events is None else tuple(events),
                                  self.segments, batch=batch)
        result = ScheduleResult(steps)
        for st in steps:
            if st.kind is ExecutionKind.PUSH:
                self.push(st.segment_ids[0])
            elif st.kind is ExecutionKind.VISIT_LEAVES:
                result.losses[st.segment_ids] = self.visit_leaves(st.segment_ids)
            else:
                loss, relayed = self.pop(st.segment_ids[0])
                result.losses[st.segment_ids] = loss
                result.relayed[st.segment_ids[0]] = relayed
        self.stack.assert_empty()
        return result
