"""Zero-copy prefix-state relay: the K/V path stack with fp32 gradient buffers.

The reference's ``KVStack`` (kv_stack.py:70-212) keeps one ``KVPrefixState``
(prefix_state.py:371-573) per segment on the active root-to-leaf DFS path, and
at every leaf visit
  * concatenates the path's K/V per layer (``build_past_key_values``,
    kv_stack.py:139-154: one ``torch.cat`` of the whole prefix per visit),
  * wraps the result in detached leaves (``build_past_anchors``,
    kv_stack.py:156-173), and after the backward
  * slices the leaves' gradients per ancestor and adds them, in the K/V dtype,
    to each ancestor's buffer (``accumulate_anchor_gradients`` kv_stack.py:175-
    203 -> ``accumulate_layer_gradients`` prefix_state.py:546-573, a bf16
    ``add_`` for bf16 K/V).

``PrefixKVStack`` keeps the same stack discipline and checks, but stores the
path in place: each layer owns one K and one V buffer of ``capacity`` rows,
and a pushed segment's K/V is copied once into the rows that follow its
parent's. The path is then always the leading ``prefix_length`` rows, so
``build_past_key_values`` returns views (no copy, at any depth), and the
gradient buffers are fp32 rows beside them. ``TPRKernelBackend.from_stack``
hands both to the kernel, whose backward adds each prefix row's gradient --
already summed over the siblings in a fixed order -- into the fp32 rows
(``TPR_BWD_ACCUMULATE_PREFIX_F32``): no anchors, no per-ancestor slicing, no
bf16 rounding between contributions. The anchor API is kept for callers that
produce prefix gradients through autograd (views again; the add is one fp32
``add_`` over the whole path).

Views returned by the stack stay valid while their segments are on it; a
popped segment's rows are reused by the next push.
"""

from __future__ import annotations

from dataclasses import dataclass
from types import MappingProxyType
from typing import Dict, Mapping, Optional, Tuple

import torch

__all__ = ["StackSegment", "PastKVSlice", "PastKVAnchors", "PrefixKVStack", "StackEntry"]

KVPair = Tuple[torch.Tensor, torch.Tensor]


def _validate_segment_id(segment_id, field_name: str = "segment_id") -> None:
    # segment_plan.py:35-40
    if not isinstance(segment_id, int) or isinstance(segment_id, bool) or segment_id < 0:
        raise ValueError(f"{field_name} must be a non-negative integer, got {segment_id!r}")


def _validate_layer_number(layer_number) -> None:
    # prefix_state.py:37-39
    if not isinstance(layer_number, int) or isinstance(layer_number, bool) or layer_number <= 0:
        raise ValueError(f"layer_number must be a positive integer, got {layer_number!r}")


@dataclass(frozen=True)
class StackSegment:
    """The fields of a ``SegmentSpec`` (segment_plan.py:67-114) the stack checks.

    Any object with these attributes (the reference's ``SegmentSpec`` among
    them) can be pushed.
    """

    segment_id: int
    parent_id: Optional[int]
    length: int
    prefix_length: int
    position_start: int

    def __post_init__(self):
        _validate_segment_id(self.segment_id)
        if self.parent_id is not None:
            _validate_segment_id(self.parent_id, "parent_id")
            if self.parent_id == self.segment_id:
                raise ValueError(f"segment {self.segment_id} cannot be its own parent")
        for name in ("length", "prefix_length", "position_start"):
            value = getattr(self, name)
            if not isinstance(value, int) or isinstance(value, bool) or value < (1 if name == "length" else 0):
                raise ValueError(f"{name} must be a {'positive' if name == 'length' else 'non-negative'} "
                                 f"integer, got {value!r}")


@dataclass(frozen=True)
class PastKVSlice:
    """Rows [start, end) of the path that belong to one segment (kv_stack.py:35-41)."""

    segment_id: int
    start: int
    end: int


@dataclass(frozen=True)
class PastKVAnchors:
    """Leaf tensors over the path K/V plus what relays their gradients (kv_stack.py:44-55)."""

    key_values: Mapping[int, KVPair]
    slices: Tuple[PastKVSlice, ...]
    stack_signature: Tuple[int, ...]

    @property
    def prefix_length(self) -> int:
        return 0 if not self.slices else self.slices[-1].end


class StackEntry:
    """One segment on the stack: its rows of the path buffers."""

    __slots__ = ("segment", "start", "_stack", "_released")

    def __init__(self, segment, start: int, stack: "PrefixKVStack"):
        self.segment = segment
        self.start = start
        self._stack = stack
        self._released = False

    @property
    def segment_id(self) -> int:
        return self.segment.segment_id

    @property
    def end(self) -> int:
        return self.start + self.segment.length

    @property
    def released(self) -> bool:
        return self._released

    def _live(self) -> None:
        if self._released:
            raise RuntimeError(f"KV prefix state for segment {self.segment_id} has been released")

    @property
    def key_values(self) -> Mapping[int, KVPair]:
        """``{layer: (K, V)}`` views ``[length, 1, Hkv, D]`` of the segment's rows."""
        self._live()
        return MappingProxyType({layer: (k[self.start:self.end], v[self.start:self.end])
                                 for layer, (k, v) in self._stack._kv.items()})

    @property
    def gradients(self) -> Mapping[int, KVPair]:
        """``{layer: (dK, dV)}`` fp32 views ``[length, 1, Hkv, D]`` of the gradient
        relayed to the segment so far."""
        self._live()
        return MappingProxyType({layer: (gk[self.start:self.end].unsqueeze(1), gv[self.start:self.end].unsqueeze(1))
                                 for layer, (gk, gv) in self._stack._grad.items()})

    def accumulate(self, layer_number: int, key_grad: torch.Tensor, value_grad: torch.Tensor) -> None:
        """Add a gradient of the segment's K/V (prefix_state.py:546-573), in fp32."""
        self._live()
        self._stack._accumulate_rows(self.segment_id, layer_number, self.start, self.end, key_grad, value_grad)


class PrefixKVStack:
    """``KVStack`` (kv_stack.py:70-212) over per-layer path buffers of ``capacity`` rows."""

    def __init__(self, capacity: int):
        if not isinstance(capacity, int) or isinstance(capacity, bool) or capacity <= 0:
            raise ValueError(f"capacity must be a positive integer, got {capacity!r}")
        self._capacity = capacity
        self._entries: list = []
        self._by_id: Dict[int, StackEntry] = {}
        self._kv: Dict[int, KVPair] = {}     # layer -> (K, V) [capacity, 1, Hkv, D]
        self._grad: Dict[int, KVPair] = {}   # layer -> (dK, dV) fp32 [capacity, Hkv, D]
        self._layers: Tuple[int, ...] = ()

    # -- stack state -------------------------------------------------------------
    def __len__(self) -> int:
        return len(self._entries)

    @property
    def capacity(self) -> int:
        return self._capacity

    @property
    def segment_ids(self) -> Tuple[int, ...]:
        return tuple(e.segment_id for e in self._entries)

    @property
    def prefix_length(self) -> int:
        return self._entries[-1].end if self._entries else 0

    @property
    def layer_numbers(self) -> Tuple[int, ...]:
        return self._layers

    def top(self) -> StackEntry:
        if not self._entries:
            raise RuntimeError("KV stack is empty")
        return self._entries[-1]

    def get(self, segment_id: int) -> StackEntry:
        try:
            return self._by_id[segment_id]
        except KeyError as exc:
            raise KeyError(f"segment {segment_id} is not on the KV stack") from exc

    def assert_empty(self) -> None:
        if self._entries or self._by_id:
            raise RuntimeError(f"KV stack is not empty: {self.segment_ids}")

    # -- push / pop --------------------------------------------------------------
    def push(self, segment, key_values: Mapping[int, KVPair]) -> StackEntry:
        """Copy the segment's graph-free K/V into the rows after its parent's.

        The checks are those of PrefixStateStack.push_state
        (prefix_state.py:651-689), KVPrefixState (prefix_state.py:388-425) and
        KVStack.push (kv_stack.py:105-131).
        """
        for name in ("segment_id", "parent_id", "length", "prefix_length", "position_start"):
            if not hasattr(segment, name):
                raise TypeError(f"segment must have {name} (a SegmentSpec or StackSegment), "
                                f"got {type(segment).__name__}")
        seg_id, length = segment.segment_id, segment.length
        _validate_segment_id(seg_id)
        if not isinstance(length, int) or isinstance(length, bool) or length <= 0:
            raise ValueError(f"sequence_length must be positive, got {length!r}")
        if seg_id in self._by_id:
            raise RuntimeError(f"segment {seg_id} is already on the KV stack")
        expected_parent = self._entries[-1].segment_id if self._entries else None
        if segment.parent_id != expected_parent:
            raise ValueError(f"cannot push segment {seg_id}: expected parent {expected_parent}, "
                             f"got {segment.parent_id}")
        start = self.prefix_length
        if segment.prefix_length != start or segment.position_start != start:
            raise ValueError(f"cannot push segment {seg_id}: stack prefix length is {start}, "
                             f"got prefix_length={segment.prefix_length}, position_start={segment.position_start}")
        if start + length > self._capacity:
            raise ValueError(f"cannot push segment {seg_id}: path of {start + length} rows exceeds the stack "
                             f"capacity of {self._capacity}")
        pairs = self._validate_key_values(seg_id, length, key_values)
        if not self._kv:
            self._allocate(pairs)
        else:
            for layer, (key, _) in pairs.items():
                buf = self._kv[layer][0]
                if key.shape[1:] != buf.shape[1:]:
                    raise ValueError(f"layer {layer} KV non-sequence shape differs across segments")
                if key.device != buf.device or key.dtype != buf.dtype:
                    raise ValueError(f"layer {layer} KV device or dtype differs across segments")
        end = start + length
        for layer, (key, value) in pairs.items():
            kbuf, vbuf = self._kv[layer]
            kbuf[start:end].copy_(key)
            vbuf[start:end].copy_(value)
            gk, gv = self._grad[layer]
            gk[start:end].zero_()
            gv[start:end].zero_()
        entry = StackEntry(segment, start, self)
        self._entries.append(entry)
        self._by_id[seg_id] = entry
        return entry

    def pop(self, segment_id: int) -> StackEntry:
        """Remove the top segment; its rows (and views of them) are free for reuse."""
        if not self._entries:
            raise RuntimeError("cannot pop an empty KV stack")
        if self._entries[-1].segment_id != segment_id:
            raise RuntimeError(f"cannot pop segment {segment_id}: stack top is {self._entries[-1].segment_id}")
        entry = self._entries.pop()
        del self._by_id[segment_id]
        entry._released = True
        return entry

    # -- the path ------------------------------------------------------------------
    def build_past_key_values(self) -> Mapping[int, KVPair]:
        """``{layer: (K, V)}`` views ``[prefix_length, 1, Hkv, D]`` of the whole path,
        root first (the order of kv_stack.py:139-154), without a copy."""
        p = self.prefix_length
        if p == 0:
            return MappingProxyType({})
        return MappingProxyType({layer: (k[:p], v[:p]) for layer, (k, v) in self._kv.items()})

    def past_gradient_accumulators(self) -> Mapping[int, KVPair]:
        """``{layer: (dK, dV)}`` fp32 views ``[prefix_length, Hkv, D]`` of the path's
        gradient rows: what ``TPRPrefixAttention`` adds the prefix gradient into."""
        p = self.prefix_length
        if p == 0:
            return MappingProxyType({})
        return MappingProxyType({layer: (gk[:p], gv[:p]) for layer, (gk, gv) in self._grad.items()})

    def build_past_anchors(self) -> PastKVAnchors:
        """Detached leaves over the path K/V (kv_stack.py:156-173), as views."""
        anchors = {layer: (k.detach().requires_grad_(True), v.detach().requires_grad_(True))
                   for layer, (k, v) in self.build_past_key_values().items()}
        slices = tuple(PastKVSlice(e.segment_id, e.start, e.end) for e in self._entries)
        return PastKVAnchors(MappingProxyType(anchors), slices, self.segment_ids)

    def accumulate_anchor_gradients(self, anchors: PastKVAnchors) -> None:
        """Add the anchors' gradients to the path's fp32 rows (kv_stack.py:175-203)."""
        if not isinstance(anchors, PastKVAnchors):
            raise TypeError(f"anchors must be PastKVAnchors, got {type(anchors).__name__}")
        if anchors.stack_signature != self.segment_ids:
            raise RuntimeError(f"past KV anchors are stale: built for {anchors.stack_signature}, "
                               f"current stack is {self.segment_ids}")
        if not self._entries:
            if anchors.key_values or anchors.slices:
                raise RuntimeError("empty stack received non-empty past KV anchors")
            return
        if tuple(anchors.key_values) != self._layers:
            raise RuntimeError(f"past KV anchor layers must be {self._layers}, got {tuple(anchors.key_values)}")
        p = self.prefix_length
        for layer, (key_anchor, value_anchor) in anchors.key_values.items():
            if key_anchor.grad is None or value_anchor.grad is None:
                raise RuntimeError(f"layer {layer} past KV anchor gradient is missing")
            self._accumulate_rows(None, layer, 0, p, key_anchor.grad, value_anchor.grad)

    def get_new_kv_gradients(self, segment_id: int) -> Mapping[int, KVPair]:
        """The fp32 gradient relayed to a segment on the stack (kv_stack.py:205-206)."""
        return self.get(segment_id).gradients

    # -- internals -------------------------------------------------------------------
    def _validate_key_values(self, seg_id: int, length: int, key_values) -> Dict[int, KVPair]:
        # prefix_state.py:388-425 and the layer check of kv_stack.py:113-118
        if not isinstance(key_values, Mapping) or not key_values:
            raise ValueError("key_values must be a non-empty mapping")
        pairs: Dict[int, KVPair] = {}
        ref = None
        for layer, pair in key_values.items():
            _validate_layer_number(layer)
            if not isinstance(pair, tuple) or len(pair) != 2:
                raise TypeError(f"layer {layer} KV must be a (key, value) tuple")
            key, value = pair
            if not isinstance(key, torch.Tensor) or not isinstance(value, torch.Tensor):
                raise TypeError(f"layer {layer} K/V must be torch tensors")
            if key.ndim != 4 or value.ndim != 4:
                raise ValueError(f"layer {layer} K/V must have shape [sequence, batch, heads, head_dim], "
                                 f"got K={tuple(key.shape)}, V={tuple(value.shape)}")
            if key.shape != value.shape:
                raise ValueError(f"layer {layer} K/V shapes must match, got K={key.shape}, V={value.shape}")
            if key.shape[0] != length:
                raise ValueError(f"layer {layer} KV local sequence length must be {length}, got {key.shape[0]}")
            if key.shape[1] != 1:
                raise ValueError(f"layer {layer} KV batch size must be 1, got {key.shape[1]}")
            if key.device != value.device or key.dtype != value.dtype:
                raise ValueError(f"layer {layer} K/V device and dtype must match, "
                                 f"got K=({key.device}, {key.dtype}), V=({value.device}, {value.dtype})")
            if key.requires_grad or value.requires_grad or key.grad_fn is not None or value.grad_fn is not None:
                raise ValueError(f"layer {layer} cached K/V must be detached and graph-free")
            if ref is None:
                ref = (key.device, key.dtype)
            elif (key.device, key.dtype) != ref:
                raise ValueError("all KV layers in a prefix state must use the same device and dtype")
            pairs[layer] = (key, value)
        pairs = dict(sorted(pairs.items()))
        if self._layers and tuple(pairs) != self._layers:
            raise ValueError(f"segment {seg_id} KV layers must be {self._layers}, got {tuple(pairs)}")
        return pairs

    def _allocate(self, pairs: Dict[int, KVPair]) -> None:
        for layer, (key, _) in pairs.items():
            shape = (self._capacity,) + tuple(key.shape[1:])
            self._kv[layer] = (torch.empty(shape, dtype=key.dtype, device=key.device),
                               torch.empty(shape, dtype=key.dtype, device=key.device))
            gshape = (self._capacity, key.shape[2], key.shape[3])
            self._grad[layer] = (torch.zeros(gshape, dtype=torch.float32, device=key.device),
                                 torch.zeros(gshape, dtype=torch.float32, device=key.device))
        self._layers = tuple(pairs)

    def _accumulate_rows(self, seg_id, layer, start, end, key_grad, value_grad) -> None:
        who = "path" if seg_id is None else f"segment {seg_id}"
        if layer not in self._grad:
            raise KeyError(f"{who} has no KV for layer {layer}")
        gk, gv = self._grad[layer]
        kbuf = self._kv[layer][0]
        expected = (end - start,) + tuple(kbuf.shape[1:])
        for name, g in (("dK", key_grad), ("dV", value_grad)):
            if not isinstance(g, torch.Tensor):
                raise TypeError(f"{who} layer {layer} {name} must be a torch tensor")
            if tuple(g.shape) != expected:
                raise ValueError(f"{who} layer {layer} gradient shape mismatch: expected {expected}, "
                                 f"got {name}={tuple(g.shape)}")
            if g.device != kbuf.device:
                raise ValueError(f"{who} layer {layer} gradient device mismatch")
            if g.dtype != kbuf.dtype:  # prefix_state.py:558-559 (the sum itself is kept in fp32)
                raise ValueError(f"{who} layer {layer} gradient dtype mismatch")
        gk[start:end].add_(key_grad.detach().reshape(end - start, *gk.shape[1:]).float())
        gv[start:end].add_(value_grad.detach().reshape(end - start, *gv.shape[1:]).float())
