"""A TPRAttentionBackend for the reference's model seam, on one GPU.

The reference's ``TPRSelfAttention._tree_forward`` hands attention to
``context.attention_backend.attention(layer_number, query, new_key,
new_value, *, softmax_scale)`` whenever a backend is set (attention.py:141-148),
under the ``TPRAttentionBackend`` protocol of context.py:35-58, and checks that
``parallel_size`` equals the configured context-parallel size
(attention.py:262-270) -- 1 on one GPU.

``TPRKernelBackend`` implements that protocol with ``parallel_size = 1``. It
holds the parent's per-layer prefix K/V -- the ``past_key_values`` a
``TPRAttentionContext`` carries (context.py:104, 163-175), ``{layer: (K, V)}``
with K, V ``[P, 1, Hkv, D]`` -- and the lengths of the sibling leaves executed
together. ``attention`` takes those siblings' tokens packed in sibling order
along the sequence axis (``[sum S_i, 1, H, D]``, the layout of one model
forward over the concatenated siblings) and returns ``[sum S_i, 1, Hq * D]``:
each sibling attends to the whole prefix and causally to its own tokens,
never to another sibling's, in one kernel launch per layer.

With one sibling this is the per-leaf visit of segment_executor.py:327-444;
with all of a parent's leaf children it is the batched leaf visit that
replaces the reference's sibling loop. The prefix K/V are autograd inputs:
their gradient is the sum over the siblings, accumulated in fp32 inside the
kernel in sibling order and cast once, in place of the per-sibling bf16
``add_`` of prefix_state.py:546-573.

``TPRKernelBackend.from_stack`` takes the prefix from a ``PrefixKVStack``
instead: the path K/V are views of the stack's buffers, and the kernel adds
the prefix gradient straight into the stack's fp32 gradient rows, so the
prefix K/V get no autograd gradient (the relay of kv_stack.py:156-203 without
anchors).
"""

from __future__ import annotations

from typing import Mapping, Optional, Sequence, Tuple

import torch

from .meta import TPRPrefixMeta, ds_store_budget_bytes
from .prefix_attention import TPRPrefixAttention

__all__ = ["TPRKernelBackend"]

KVPair = Tuple[torch.Tensor, torch.Tensor]


def _validate_layer_number(layer_number) -> None:
    # context.py:59-61
    if not isinstance(layer_number, int) or isinstance(layer_number, bool) or layer_number <= 0:
        raise ValueError(f"layer_number must be a positive integer, got {layer_number!r}")


def _validate_kv_pair(layer_number: int, key, value, *, expected_sequence_length: int, kind: str) -> None:
    # the checks of context.py:64-96 on a layer's K/V pair
    if not isinstance(key, torch.Tensor) or not isinstance(value, torch.Tensor):
        raise TypeError(f"layer {layer_number} {kind} K/V must be torch tensors")
    if key.ndim != 4 or value.ndim != 4:
        raise ValueError(f"layer {layer_number} {kind} K/V must have shape [sequence, batch, heads, head_dim], "
                         f"got K={tuple(key.shape)}, V={tuple(value.shape)}")
    if key.shape != value.shape:
        raise ValueError(f"layer {layer_number} {kind} K/V shapes must match, "
                         f"got K={tuple(key.shape)}, V={tuple(value.shape)}")
    if key.shape[0] != expected_sequence_length:
        raise ValueError(f"layer {layer_number} {kind} KV sequence length must be {expected_sequence_length}, "
                         f"got {key.shape[0]}")
    if key.shape[1] != 1:
        raise ValueError(f"layer {layer_number} {kind} KV batch size must be 1, got {key.shape[1]}")
    if key.device != value.device or key.dtype != value.dtype:
        raise ValueError(f"layer {layer_number} {kind} K/V device and dtype must match, "
                         f"got K=({key.device}, {key.dtype}), V=({value.device}, {value.dtype})")


class TPRKernelBackend:
    """``TPRAttentionBackend`` (context.py:35-58) with ``parallel_size = 1``.

    ``prefix_key_values``: ``{layer_number: (K, V)}``, K and V ``[P, 1, Hkv,
    D]`` (empty mapping when P = 0); ``suffix_lengths``: the token counts of
    the sibling leaves whose tokens are packed, in this order, into each
    ``attention`` call. ``ds_store_budget``: bytes the backward's dS store
    may take per layer call (``TPRPrefixAttention``; None = the library
    default of 8 GiB, 0 = none). The store is transient -- allocated by each
    layer's backward and released after it.
    """

    def __init__(self, prefix_key_values: Mapping[int, KVPair], suffix_lengths: Sequence[int], *,
                 prefix_length: Optional[int] = None,
                 prefix_grad_accumulators: Optional[Mapping[int, KVPair]] = None,
                 ds_store_budget: Optional[int] = None):
        lengths = tuple(suffix_lengths)
        if not lengths or any(not isinstance(s, int) or isinstance(s, bool) or s <= 0 for s in lengths):
            raise ValueError(f"suffix_lengths must be positive integers, got {suffix_lengths!r}")
        pairs = dict(prefix_key_values)
        if prefix_length is None:
            prefix_length = next(iter(pairs.values()))[0].shape[0] if pairs else 0
        if not isinstance(prefix_length, int) or isinstance(prefix_length, bool) or prefix_length < 0:
            raise ValueError(f"prefix_length must be a non-negative integer, got {prefix_length!r}")
        if prefix_length == 0 and pairs:
            raise ValueError("prefix_key_values must be empty when prefix_length is 0")  # context.py:128-129
        for layer_number, pair in pairs.items():
            _validate_layer_number(layer_number)
            if not isinstance(pair, tuple) or len(pair) != 2:
                raise TypeError(f"layer {layer_number} past KV must be a (key, value) tuple")
            _validate_kv_pair(layer_number, *pair, expected_sequence_length=prefix_length, kind="past")
        accumulators = dict(prefix_grad_accumulators) if prefix_grad_accumulators is not None else None
        if accumulators is not None and set(accumulators) != set(pairs):
            raise ValueError(f"prefix_grad_accumulators layers {sorted(accumulators)} must match the past KV "
                             f"layers {sorted(pairs)}")
        self._prefix = pairs
        self._accumulators = accumulators
        self._prefix_length = prefix_length
        self._lengths = lengths
        self._meta = TPRPrefixMeta.shared_prefix(prefix_length, lengths)
        self._ds_store_budget = ds_store_budget_bytes(ds_store_budget)

    @classmethod
    def from_stack(cls, stack, suffix_lengths: Sequence[int], *,
                   ds_store_budget: Optional[int] = None) -> "TPRKernelBackend":
        """The siblings under the top of a ``PrefixKVStack``: prefix = the stack's
        path (views), prefix gradient added into the stack's fp32 rows."""
        return cls(stack.build_past_key_values(), suffix_lengths, prefix_length=stack.prefix_length,
                   prefix_grad_accumulators=stack.past_gradient_accumulators() if stack.prefix_length else None,
                   ds_store_budget=ds_store_budget)

    # -- the protocol ---------------------------------------------------------
    @property
    def global_prefix_length(self) -> int:
        return self._prefix_length

    @property
    def global_suffix_length(self) -> int:
        return sum(self._lengths)

    @property
    def local_suffix_length(self) -> int:
        return sum(self._lengths)  # one rank holds every suffix token

    @property
    def parallel_size(self) -> int:
        return 1

    def attention(self, layer_number: int, query: torch.Tensor, new_key: torch.Tensor, new_value: torch.Tensor, *,
                  softmax_scale: Optional[float]) -> torch.Tensor:
        """``[sum S_i, 1, Hq, D]`` query and ``[sum S_i, 1, Hkv, D]`` new K/V of the
        packed siblings -> ``[sum S_i, 1, Hq * D]``."""
        _validate_layer_number(layer_number)
        _validate_kv_pair(layer_number, new_key, new_value, expected_sequence_length=self.local_suffix_length,
                          kind="new")
        if not isinstance(query, torch.Tensor) or query.ndim != 4 or query.shape[1] != 1:
            raise ValueError(f"layer {layer_number} query must have shape [sequence, 1, heads, head_dim], "
                             f"got {tuple(getattr(query, 'shape', ()))}")
        if query.shape[0] != self.local_suffix_length:
            raise ValueError(f"layer {layer_number} query sequence length must be {self.local_suffix_length}, "
                             f"got {query.shape[0]}")
        if self._prefix_length:
            try:
                past_key, past_value = self._prefix[layer_number]
            except KeyError as exc:
                raise KeyError(f"missing past KV for layer {layer_number}") from exc  # context.py:232-235
        else:
            past_key = new_key.new_empty((0,) + tuple(new_key.shape[1:]))
            past_value = past_key
        accumulators = None
        if self._accumulators is not None and self._prefix_length:
            accumulators = self._accumulators[layer_number]
        out, _ = TPRPrefixAttention.apply(query[:, 0], new_key[:, 0], new_value[:, 0], past_key[:, 0],
                                          past_value[:, 0], self._meta, softmax_scale, accumulators, False,
                                          self._ds_store_budget)
        return out.reshape(query.shape[0], 1, query.shape[2] * query.shape[3])

    # -- packing helpers --------------------------------------------------------
    def pack(self, per_sibling: Sequence[torch.Tensor]) -> torch.Tensor:
        """Concatenate per-sibling ``[S_i, ...]`` tensors in sibling order."""
        if len(per_sibling) != len(self._lengths) or any(t.shape[0] != s for t, s in zip(per_sibling, self._lengths)):
            raise ValueError(f"expected {len(self._lengths)} tensors of lengths {self._lengths}, "
                             f"got {[tuple(t.shape) for t in per_sibling]}")
        return torch.cat(list(per_sibling), dim=0)

    def unpack(self, packed: torch.Tensor) -> Tuple[torch.Tensor, ...]:
        """Split a packed ``[sum S_i, ...]`` tensor back into the siblings' views."""
        if packed.shape[0] != self.local_suffix_length:
            raise ValueError(f"expected {self.local_suffix_length} packed rows, got {packed.shape[0]}")
        return tuple(torch.split(packed, list(self._lengths), dim=0))
