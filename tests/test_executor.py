"""CPU tests of the sibling-batched tree executor (bridge_amd/executor.py).

* The event lowering reproduces the reference scheduler: an adjacent
  (Push L, Pop L) of a childless L is one leaf visit
  (fixed_topology_scheduler.py:142-158, 200-210) and everything else is a
  push or pop, in the DFS order of segment_plan.py:266-275; batching merges
  only runs of adjacent leaf visits under one parent, so flattening the
  batches gives back the reference's physical trace.
* End to end on the CPU, with the oracle as the attention backend: the
  batched schedule's parameter gradients equal the one-leaf-at-a-time
  schedule's, and both equal the gradient of the sum over segments of each
  segment's loss computed densely over its whole root path (what the
  Push/Pop relay reconstructs, segment_executor.py:208-444)."""

from __future__ import annotations

import pytest
import torch

from bridge_amd.executor import (
    BatchedLeafExecutor,
    ExecutionKind,
    SegmentEvent,
    SegmentEventKind,
    batch_leaf_visits,
    build_segments,
    dfs_events,
)
from bridge_amd.relay import PrefixKVStack

from _oracle_backend import OracleStackBackend
from _toy_model import ToyModel

# A 3-level ragged plan: root 0 -> [leaf 1, node 2 -> [leaves 3, 4, node 5 -> [leaves 6, 7]],
# leaf 8, leaf 9, node 10 -> [leaf 11]]
PARENTS = {0: None, 1: 0, 2: 0, 3: 2, 4: 2, 5: 2, 6: 5, 7: 5, 8: 0, 9: 0, 10: 0, 11: 10}
LENGTHS = {0: 37, 1: 20, 2: 18, 3: 11, 4: 25, 5: 9, 6: 14, 7: 6, 8: 30, 9: 7, 10: 12, 11: 16}


def _reference_trace(events, children):
    """The reference scheduler's physical execution trace, restated
    (fixed_topology_scheduler.py:110-158 with _is_direct_leaf_pair :200-210)."""
    out, i = [], 0
    while i < len(events):
        ev, nxt = events[i], events[i + 1] if i + 1 < len(events) else None
        if (ev.kind is SegmentEventKind.PUSH and nxt is not None and nxt.kind is SegmentEventKind.POP
                and nxt.segment_id == ev.segment_id and not children[ev.segment_id]):
            out.append(("visit_leaf", ev.segment_id))
            i += 2
            continue
        out.append((ev.kind.value, ev.segment_id))
        i += 1
    return tuple(out)


def test_segments_carry_the_references_derived_positions():
    segs = build_segments(PARENTS, LENGTHS)
    assert segs[0].prefix_length == 0 and segs[1].prefix_length == 37
    assert segs[3].position_start == 37 + 18 and segs[6].prefix_length == 37 + 18 + 9
    assert segs[11].prefix_length == 37 + 12
    assert all(s.prefix_length == s.position_start for s in segs.values())


def test_dfs_events_follow_insertion_order():
    events = dfs_events(build_segments(PARENTS, LENGTHS))
    assert [(e.kind.value[1], e.segment_id) for e in events[:8]] == [
        ("u", 0), ("u", 1), ("o", 1), ("u", 2), ("u", 3), ("o", 3), ("u", 4), ("o", 4)]
    assert events[-1] == SegmentEvent(SegmentEventKind.POP, 0)
    assert len(events) == 2 * len(PARENTS)


def test_leaf_batches_reproduce_the_reference_trace():
    segs = build_segments(PARENTS, LENGTHS)
    events = dfs_events(segs)
    children = {s: [c for c, p in PARENTS.items() if p == s] for s in PARENTS}
    ref = _reference_trace(events, children)
    steps = batch_leaf_visits(events, segs)
    flat = []
    for st in steps:
        if st.kind is ExecutionKind.VISIT_LEAVES:
            flat.extend(("visit_leaf", s) for s in st.segment_ids)
        else:
            flat.append((st.kind.value, st.segment_ids[0]))
    assert tuple(flat) == ref
    visits = [(st.parent_id, st.segment_ids) for st in steps if st.kind is ExecutionKind.VISIT_LEAVES]
    # adjacent leaves of one parent are batched; a node between them splits the run
    assert visits == [(0, (1,)), (2, (3, 4)), (5, (6, 7)), (0, (8, 9)), (10, (11,))]
    unbatched = batch_leaf_visits(events, segs, batch=False)
    assert all(len(st.segment_ids) == 1 for st in unbatched)
    assert tuple((("visit_leaf" if st.kind is ExecutionKind.VISIT_LEAVES else st.kind.value), st.segment_ids[0])
                 for st in unbatched) == ref


def test_invalid_event_streams_are_rejected():
    segs = build_segments(PARENTS, LENGTHS)
    events = list(dfs_events(segs))
    with pytest.raises(ValueError, match="before all children"):
        cut = events.index(SegmentEvent(SegmentEventKind.PUSH, 2)) + 1
        batch_leaf_visits(events[:cut] + [SegmentEvent(SegmentEventKind.POP, 2)], segs)
    with pytest.raises(ValueError, match="incomplete"):
        batch_leaf_visits(events[:-1], segs)
    with pytest.raises(ValueError, match="expected parent"):
        batch_leaf_visits([SegmentEvent(SegmentEventKind.PUSH, 3)] + events, segs)


def _tokens(seed=0):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return {s: torch.randint(0, 64, (n,), generator=gen) for s, n in LENGTHS.items()}


def _run_executor(model, tokens, batch):
    segs = build_segments(PARENTS, LENGTHS)
    stack = PrefixKVStack(sum(LENGTHS.values()))
    ex = BatchedLeafExecutor(segs, model.forward_fn(tokens), stack, backend_factory=OracleStackBackend)
    for p in model.params.values():
        p.grad = None
    result = ex.run(batch=batch)
    return result, model.grads()


def test_batched_schedule_equals_per_leaf_schedule_and_dense_paths():
    tokens = _tokens()
    model = ToyModel(hq=4, hkv=2, d=16, hidden=32, layers=2, seed=3)
    batched, g_batched = _run_executor(model, tokens, True)
    single, g_single = _run_executor(model, tokens, False)
    assert batched.leaf_trace() == single.leaf_trace()
    # dense reference: every segment's loss over its whole root path
    for p in model.params.values():
        p.grad = None
    total = 0
    for s in PARENTS:
        path, cur = [], s
        while cur is not None:
            path.append(cur)
            cur = PARENTS[cur]
        ids = torch.cat([tokens[x] for x in reversed(path)])
        total = total + model.dense_path_loss(ids, LENGTHS[s])
    total.backward()
    g_dense = model.grads()
    loss_b = sum(v.item() for v in batched.losses.values())
    assert abs(loss_b - total.item()) <= 1e-9 * abs(total.item())
    for name in g_dense:
        scale = g_dense[name].abs().max().item()
        # fp64 model; the stack relays gradients through fp32 rows
        assert (g_batched[name] - g_dense[name]).abs().max().item() <= 1e-5 * scale, name
        assert (g_single[name] - g_dense[name]).abs().max().item() <= 1e-5 * scale, name
    # the gradient relayed to every node at its pop is the same either way
    assert set(batched.relayed) == {0, 2, 5, 10}
    for seg, layers in batched.relayed.items():
        for layer, (gk, gv) in layers.items():
            rk, rv = single.relayed[seg][layer]
            assert torch.allclose(gk, rk, rtol=1e-5, atol=1e-7 * rk.abs().max().item())
            assert torch.allclose(gv, rv, rtol=1e-5, atol=1e-7 * rv.abs().max().item())


def test_positions_of_a_batched_visit_start_at_the_parents_end():
    segs = build_segments(PARENTS, LENGTHS)
    ex = BatchedLeafExecutor(segs, None, PrefixKVStack(8), backend_factory=OracleStackBackend)
    pos = ex.position_ids([segs[6], segs[7]])
    start = 37 + 18 + 9
    assert pos.tolist() == list(range(start, start + 14)) + list(range(start, start + 6))
