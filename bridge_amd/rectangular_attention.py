"""Drop-in for the reference's single-sequence operator
``rectangular_causal_attention`` (verl/models/mcore/tpr/rectangular_attention.py:125-209).

Same signature, argument meaning, validation and exception types
(``_validate_inputs`` :51-83, ``_validate_attention_mask`` :86-109,
device / pre_tokens / scale checks :165-172, output shape check :206-208);
the device check names a ROCm GPU where the reference names an NPU.

Key/value carry the external prefix in front of the suffix, exactly as the
reference's caller builds them (attention.py:150-158): the prefix length is
``Skv - Sq`` and, without ``attention_mask``, the mask is right-down causal
(key j visible to query i iff j <= Skv - Sq + i; the reference's sparse mode
3). The call is one leaf under one prefix node of the sibling-batched
``TPRPrefixAttention``.

A physical ``attention_mask`` (bool ``[Sq, Skv]``, True = excluded) is the
sole visibility rule, as in the reference's custom-mask mode (sparse mode 0
with the token window open, :112-122): it may hide padding rows and columns
or show more than the causal mask. It runs on the masked (SIMT) kernels,
except a mask equal to the right-down causal one, which takes the unmasked
kernels. A query row the mask hides entirely gets output 0 and no gradient.
"""

from __future__ import annotations

import math
from functools import lru_cache

import torch
from torch import Tensor

from .meta import TPRPrefixMeta
from .prefix_attention import TPRPrefixAttention

__all__ = ["rectangular_causal_attention"]

_DEFAULT_PRE_TOKENS = 2**31 - 1


def _validate_inputs(query: Tensor, key: Tensor, value: Tensor, dropout_p: float) -> tuple[int, int, int, int]:
    for name, tensor in (("query", query), ("key", key), ("value", value)):
        if tensor.ndim != 4:
            raise ValueError(f"{name} must have shape [sequence, batch, heads, head_dim], got {tensor.shape}")
    query_length, batch_size, query_heads, head_dim = query.shape
    kv_length, key_batch_size, key_heads, key_head_dim = key.shape
    if value.shape != key.shape:
        raise ValueError(f"key and value must have identical shapes, got key={key.shape}, value={value.shape}")
    if batch_size != 1 or key_batch_size != 1:
        raise ValueError(f"rectangular attention requires batch size 1, got Q={batch_size}, KV={key_batch_size}")
    if query_length <= 0 or kv_length <= 0:
        raise ValueError(f"sequence lengths must be positive, got Q={query_length}, KV={kv_length}")
    if query_length > kv_length:
        raise ValueError(f"query length cannot exceed KV length, got Q={query_length}, KV={kv_length}")
    if query_heads <= 0 or key_heads <= 0 or head_dim <= 0:
        raise ValueError(f"head counts and head_dim must be positive, got Q={query.shape}, KV={key.shape}")
    if key_head_dim != head_dim:
        raise ValueError(f"Q and KV head dimensions must match, got Q={head_dim}, KV={key_head_dim}")
    if query_heads % key_heads != 0:
        raise ValueError(f"query head count must be divisible by KV head count, got Q={query_heads}, KV={key_heads}")
    if query.dtype != key.dtype or query.dtype != value.dtype:
        raise ValueError(f"Q, K, and V dtypes must match, got Q={query.dtype}, K={key.dtype}, V={value.dtype}")
    if query.device != key.device or query.device != value.device:
        raise ValueError(f"Q, K, and V devices must match, got Q={query.device}, K={key.device}, V={value.device}")
    if not query.is_floating_point():
        raise ValueError(f"Q, K, and V must use a floating-point dtype, got {query.dtype}")
    if dropout_p != 0.0:
        raise ValueError(f"rectangular attention requires dropout_p=0, got {dropout_p}")
    return query_length, kv_length, query_heads, head_dim


def _validate_attention_mask(attention_mask, *, query_length: int, kv_length: int, device: torch.device) -> None:
    if attention_mask is None:
        return
    if not isinstance(attention_mask, Tensor):
        raise TypeError(f"attention_mask must be a torch.Tensor or None, got {type(attention_mask).__name__}")
    if attention_mask.dtype != torch.bool:
        raise ValueError(f"attention_mask must use torch.bool, got {attention_mask.dtype}")
    if attention_mask.device != device:
        raise ValueError(f"attention_mask must be on {device}, got {attention_mask.device}")
    expected = (query_length, kv_length)
    if tuple(attention_mask.shape) != expected:
        raise ValueError(f"attention_mask must have shape {expected}, got {tuple(attention_mask.shape)}")


def _right_down_causal_mask(query_length: int, kv_length: int, device) -> Tensor:
    """True = excluded: key j is hidden from query i iff j > kv_length - query_length + i."""
    cols = torch.arange(kv_length, device=device)
    rows = torch.arange(query_length, device=device)
    return cols[None, :] > (kv_length - query_length + rows[:, None])


@lru_cache(maxsize=256)
def _single_leaf_meta(prefix_length: int, query_length: int) -> TPRPrefixMeta:
    return TPRPrefixMeta.shared_prefix(prefix_length, [query_length])


def rectangular_causal_attention(
    query: Tensor,
    key: Tensor,
    value: Tensor,
    *,
    softmax_scale: float | None = None,
    dropout_p: float = 0.0,
    pre_tokens: int = _DEFAULT_PRE_TOKENS,
    inner_precise: int = 0,
    attention_mask: Tensor | None = None,
) -> Tensor:
    """Differentiable right-down rectangular causal attention on one sequence.

    query ``[Sq, 1, Hq, D]`` (post-RoPE), key/value ``[Skv, 1, Hkv, D]``
    including the external prefix; returns ``[Sq, 1, Hq * D]``.
    ``inner_precise`` is accepted for signature compatibility (accumulation
    is always fp32). ``attention_mask``: an optional physical ``[Sq, Skv]``
    bool mask, True = excluded, which replaces the causal rule.
    """
    query_length, kv_length, query_heads, head_dim = _validate_inputs(query, key, value, dropout_p)
    _validate_attention_mask(attention_mask, query_length=query_length, kv_length=kv_length, device=query.device)
    if query.device.type != "cuda":
        raise RuntimeError(f"rectangular_causal_attention requires a ROCm GPU tensor, got device {query.device}")
    if pre_tokens < 0:
        raise ValueError(f"pre_tokens must be non-negative, got {pre_tokens}")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(head_dim)
    if not math.isfinite(softmax_scale) or softmax_scale <= 0:
        raise ValueError(f"softmax_scale must be finite and positive, got {softmax_scale}")
    if pre_tokens < kv_length:
        raise NotImplementedError("a preceding-token window shorter than the KV length is not supported")
    if attention_mask is not None and torch.equal(
            attention_mask, _right_down_causal_mask(query_length, kv_length, attention_mask.device)):
        attention_mask = None  # the causal mask itself: the unmasked kernels

    prefix_length = kv_length - query_length
    q = query.squeeze(1)
    k = key.squeeze(1)
    v = value.squeeze(1)
    meta = _single_leaf_meta(prefix_length, query_length)
    # one leaf: the mask's columns cat(prefix, suffix) are the leaf's key sequence
    output, _ = TPRPrefixAttention.apply(q[:, :, :], k[prefix_length:], v[prefix_length:],
                                         k[:prefix_length], v[:prefix_length], meta, softmax_scale,
                                         None, False, None, attention_mask)
    expected_shape = (query_length, query_heads, head_dim)
    if tuple(output.shape) != expected_shape:
        raise RuntimeError(f"unexpected attention output shape: expected {expected_shape}, got {tuple(output.shape)}")
    return output.reshape(query_length, 1, query_heads * head_dim)
