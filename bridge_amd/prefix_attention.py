"""Sibling-batched prefix-reuse attention as a torch.autograd.Function.

``TPRPrefixAttention.apply(q, k, v, prefix_k, prefix_v, meta, softmax_scale)``
returns ``(out, lse)``:

* q ``[Tq, Hq, D]``, k/v ``[Tq, Hkv, D]``: the N leaf suffixes packed by
  ``meta.cu_seqlens_q`` (TND, rectangular_attention.py:179-181);
* prefix_k/prefix_v ``[Tp, Hkv, D]``: the shared prefix nodes packed by
  ``meta.node_offsets``;
* out ``[Tq, Hq, D]`` (input dtype) and lse ``[Hq, Tq]`` float32 (natural log of
  the scaled-score normaliser, the quantity max + log(sum) of
  _ring_merge_probe.py:25-27; it is not differentiable).

Backward returns dq, dk, dv and dprefix_k/dprefix_v, where each node's
gradient is the sum over all its descendant leaves in leaf order -- the
sibling relay of kv_stack.py:175-203 / prefix_state.py:546-573, reduced on the
GPU without atomics.

For one leaf under one node this equals the reference's
rectangular_causal_attention(q, cat(prefix_k, k), cat(prefix_v, v))
(rectangular_attention.py:125-209); see ``bridge_amd.rectangular_attention``.

``attention_mask`` (optional, bool ``[Tq, L]``, True = hidden) replaces the
causal rule by a physical key mask, the reference's custom-mask mode
(rectangular_attention.py:112-122): row r is query row r, column c is key c
of that row's leaf key sequence cat(ancestor nodes root first, own suffix),
and L is at least ``meta.max_keys()``. Masked calls run on the SIMT kernels.
A query row that sees no key gets output 0 and zero gradients.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from . import _lib
from .meta import TPRPrefixMeta, ds_store_budget_bytes

__all__ = ["TPRPrefixAttention", "tpr_prefix_attention"]

_SUPPORTED = (torch.bfloat16, torch.float32)


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def _stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


_MAX_ROW_BYTES = 1 << 25


def _rows(t: torch.Tensor) -> torch.Tensor:
    """``t`` itself when the kernels can read it through a row stride (heads
    and head_dim packed, rows 16-byte aligned: a slice of a fused
    [tokens, (Hq + 2 Hkv) * D] projection is one), else a packed copy."""
    _, h, d = t.shape
    es = t.element_size()
    rs = t.stride(0)
    if ((t.stride(2) == 1 or d == 1) and (t.stride(1) == d or h == 1) and rs >= h * d and (rs * es) % 16 == 0
            and rs * es <= _MAX_ROW_BYTES and t.data_ptr() % 16 == 0):
        return t
    return t.contiguous()


def _row_stride(t: torch.Tensor) -> int:
    """Row stride (elements) for the ABI: 0 when packed."""
    _, h, d = t.shape
    return 0 if t.shape[0] <= 1 or t.stride(0) == h * d else t.stride(0)


def _inputs(q, k, v, prefix_k, prefix_v):
    """q, k, v as strided row views where possible; the prefix packed."""
    return _rows(q), _rows(k), _rows(v), prefix_k.contiguous(), prefix_v.contiguous()


def _empty(t: torch.Tensor) -> torch.Tensor:
    return torch.empty(t.shape, dtype=t.dtype, device=t.device)


def validate(q, k, v, prefix_k, prefix_v, meta: TPRPrefixMeta, softmax_scale):
    """Contract checks with the reference's exception types and wording
    (rectangular_attention.py:51-83, 165-172). Returns the resolved scale."""
    for name, t in (("query", q), ("key", k), ("value", v), ("prefix_key", prefix_k), ("prefix_value", prefix_v)):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor, got {type(t).__name__}")
        if t.ndim != 3:
            raise ValueError(f"{name} must have shape [tokens, heads, head_dim], got {tuple(t.shape)}")
    if not isinstance(meta, TPRPrefixMeta):
        raise TypeError(f"meta must be a TPRPrefixMeta, got {type(meta).__name__}")
    tq, hq, d = q.shape
    if k.shape != v.shape:
        raise ValueError(f"key and value must have identical shapes, got key={tuple(k.shape)}, value={tuple(v.shape)}")
    if prefix_k.shape != prefix_v.shape:
        raise ValueError("prefix key and value must have identical shapes, "
                         f"got key={tuple(prefix_k.shape)}, value={tuple(prefix_v.shape)}")
    hkv = k.shape[1]
    if k.shape[0] != tq:
        raise ValueError(f"suffix key length must equal query length, got Q={tq}, KV={k.shape[0]}")
    if k.shape[2] != d or prefix_k.shape[2] != d:
        raise ValueError(f"Q and KV head dimensions must match, got Q={d}, KV={k.shape[2]}, prefix={prefix_k.shape[2]}")
    if prefix_k.shape[1] != hkv:
        raise ValueError(f"prefix KV head count must match suffix KV heads, got {prefix_k.shape[1]} vs {hkv}")
    if hq <= 0 or hkv <= 0 or d <= 0:
        raise ValueError(f"head counts and head_dim must be positive, got Q={tuple(q.shape)}, KV={tuple(k.shape)}")
    if hq % hkv != 0:
        raise ValueError(f"query head count must be divisible by KV head count, got Q={hq}, KV={hkv}")
    dtypes = {q.dtype, k.dtype, v.dtype, prefix_k.dtype, prefix_v.dtype}
    if len(dtypes) != 1:
        raise ValueError(f"Q, K, and V dtypes must match, got Q={q.dtype}, K={k.dtype}, V={v.dtype}, "
                         f"prefix K={prefix_k.dtype}, prefix V={prefix_v.dtype}")
    devices = {q.device, k.device, v.device, prefix_k.device, prefix_v.device}
    if len(devices) != 1:
        raise ValueError(f"Q, K, and V devices must match, got {sorted(str(x) for x in devices)}")
    if not q.is_floating_point():
        raise ValueError(f"Q, K, and V must use a floating-point dtype, got {q.dtype}")
    if q.dtype not in _SUPPORTED:
        raise ValueError(f"prefix attention supports torch.bfloat16 and torch.float32, got {q.dtype}")
    if tq != meta.total_q:
        raise ValueError(f"query rows ({tq}) must equal meta.total_q ({meta.total_q})")
    if prefix_k.shape[0] != meta.total_prefix:
        raise ValueError(f"prefix rows ({prefix_k.shape[0]}) must equal meta.total_prefix ({meta.total_prefix})")
    if q.device.type != "cuda":
        raise RuntimeError(f"tpr_prefix_attention requires a ROCm GPU (cuda) tensor, got device {q.device}")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)
    softmax_scale = float(softmax_scale)
    if not math.isfinite(softmax_scale) or softmax_scale <= 0:
        raise ValueError(f"softmax_scale must be finite and positive, got {softmax_scale}")
    return softmax_scale


def check_mask(attention_mask, q: torch.Tensor, meta: TPRPrefixMeta) -> Optional[torch.Tensor]:
    """The physical key mask as the kernels read it (uint8 rows, nonzero =
    hidden), or None. Exception types and wording follow the reference's
    _validate_attention_mask (rectangular_attention.py:86-109)."""
    if attention_mask is None:
        return None
    if not isinstance(attention_mask, torch.Tensor):
        raise TypeError(f"attention_mask must be a torch.Tensor or None, got {type(attention_mask).__name__}")
    if attention_mask.dtype != torch.bool:
        raise ValueError(f"attention_mask must use torch.bool, got {attention_mask.dtype}")
    if attention_mask.device != q.device:
        raise ValueError(f"attention_mask must be on {q.device}, got {attention_mask.device}")
    keys = meta.max_keys()
    if attention_mask.ndim != 2 or attention_mask.shape[0] != meta.total_q or attention_mask.shape[1] < keys:
        raise ValueError(f"attention_mask must have shape [{meta.total_q}, L] with L >= {keys} (query rows, "
                         f"longest leaf key sequence), got {tuple(attention_mask.shape)}")
    return attention_mask.contiguous().view(torch.uint8)


def _mask_args(mask: Optional[torch.Tensor]) -> Tuple[Optional[int], int]:
    """(pointer, row stride in bytes) of a checked mask for the ABI."""
    if mask is None:
        return None, 0
    return _ptr(mask), int(mask.shape[1])


def _forward(q, k, v, prefix_k, prefix_v, meta, scale, mask=None):
    plan = meta.plan(q.shape[1], k.shape[1], q.shape[2], q.dtype, q.device, masked=mask is not None)
    out = _empty(q)
    lse = torch.empty((q.shape[1], q.shape[0]), dtype=torch.float32, device=q.device)
    if q.shape[0] == 0:
        return out, lse
    lib = _lib.load()
    params = _lib.TprFwdParams(
        _lib.ABI_VERSION, 0, scale, 0.0,
        plan.host.data_ptr(), plan.device.data_ptr(),
        _ptr(q), _ptr(k), _ptr(v), _ptr(prefix_k), _ptr(prefix_v), _ptr(out), _ptr(lse),
        _row_stride(q), _row_stride(k), _row_stride(v), *_mask_args(mask))
    _lib.check(lib.tpr_attn_fwd(ctypes.byref(params), ctypes.c_void_p(_stream_handle(q.device))), "tpr_attn_fwd")
    return out, lse


def _check_accumulators(accumulators, prefix_k) -> Tuple[torch.Tensor, torch.Tensor]:
    """fp32 [total_prefix, Hkv, D] pair on prefix_k's device, contiguous."""
    if not isinstance(accumulators, (tuple, list)) or len(accumulators) != 2:
        raise TypeError("prefix_grad_accumulators must be a (dprefix_k, dprefix_v) pair of fp32 tensors")
    for name, t in zip(("dprefix_k", "dprefix_v"), accumulators):
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"prefix_grad_accumulators {name} must be a torch tensor")
        if t.dtype != torch.float32:
            raise ValueError(f"prefix_grad_accumulators {name} must be float32, got {t.dtype}")
        if tuple(t.shape) != tuple(prefix_k.shape):
            raise ValueError(f"prefix_grad_accumulators {name} must have shape {tuple(prefix_k.shape)}, "
                             f"got {tuple(t.shape)}")
        if t.device != prefix_k.device:
            raise RuntimeError(f"prefix_grad_accumulators {name} must be on {prefix_k.device}, got {t.device}")
        if not t.is_contiguous():
            raise ValueError(f"prefix_grad_accumulators {name} must be contiguous")
    return accumulators[0], accumulators[1]


def _workspace(meta, q, k, budget, ws, masked=False):
    """(plan, workspace) of the backward. A plan with a dS store whose
    workspace cannot be allocated falls back to the plan without one (a few
    MB), which gives the same gradients with a slower dQ."""
    plan = meta.plan(q.shape[1], k.shape[1], q.shape[2], q.dtype, q.device, ds_store_budget=budget, masked=masked)
    if ws is not None or not plan.workspace_bytes:
        return plan, ws
    try:
        return plan, torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=q.device)
    except torch.OutOfMemoryError:
        if not plan.dq_from_ds:
            raise
    plan = meta.plan(q.shape[1], k.shape[1], q.shape[2], q.dtype, q.device, ds_store_budget=0)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=q.device) if plan.workspace_bytes else None
    return plan, ws


def _backward(q, k, v, prefix_k, prefix_v, out, lse, dout, meta, scale, *, phases=None, buffers=None,
              prefix_grad_accumulators=None, ds_store_budget=None, mask=None):
    """Enqueue the backward. ``buffers`` may supply preallocated dq, dk, dv,
    dprefix_k, dprefix_v and delta tensors; ``phases`` is a mask of
    _lib.TPR_BWD_* bits (default: all). With ``prefix_grad_accumulators`` (a
    pair of fp32 tensors shaped like prefix_k) the prefix gradients are added
    into that pair by the kernels (TPR_BWD_ACCUMULATE_PREFIX_F32), which is
    also what is returned for them. ``ds_store_budget``: the plan's dS store
    budget in bytes (TPRPrefixMeta.plan; None = the library default).
    ``mask``: the forward's key mask as check_mask returns it, or None."""
    b = dict(buffers or {})
    dq = b.get("dq") if b.get("dq") is not None else _empty(q)
    dk = b.get("dk") if b.get("dk") is not None else _empty(k)
    dv = b.get("dv") if b.get("dv") is not None else _empty(v)
    for name, t in (("dq", dq), ("dk", dk), ("dv", dv)):
        if not t.is_contiguous():
            raise ValueError(f"buffer {name} must be contiguous (gradients are written packed)")
    flags = 0
    if prefix_grad_accumulators is not None:
        dpk, dpv = _check_accumulators(prefix_grad_accumulators, prefix_k)
        flags = _lib.TPR_BWD_ACCUMULATE_PREFIX_F32
    else:
        dpk = b.get("dprefix_k") if b.get("dprefix_k") is not None else torch.empty_like(prefix_k)
        dpv = b.get("dprefix_v") if b.get("dprefix_v") is not None else torch.empty_like(prefix_v)
    if q.shape[0] == 0:
        if flags:
            return dq, dk, dv, dpk, dpv
        return dq, dk, dv, dpk.zero_(), dpv.zero_()
    delta = b.get("delta") if b.get("delta") is not None else torch.empty_like(lse)
    plan, ws = _workspace(meta, q, k, ds_store_budget, b.get("workspace"), masked=mask is not None)
    lib = _lib.load()
    params = _lib.TprBwdParams(
        _lib.ABI_VERSION, flags, scale, 0.0,
        plan.host.data_ptr(), plan.device.data_ptr(),
        _ptr(q), _ptr(k), _ptr(v), _ptr(prefix_k), _ptr(prefix_v), _ptr(out), _ptr(dout), _ptr(lse),
        _ptr(delta), _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dpk), _ptr(dpv), _ptr(ws), plan.workspace_bytes,
        _row_stride(q), _row_stride(k), _row_stride(v), *_mask_args(mask))
    mask = phases if phases is not None else (_lib.TPR_BWD_DELTA | _lib.TPR_BWD_DKDV | _lib.TPR_BWD_DQ)
    _lib.check(lib.tpr_attn_bwd_phases(ctypes.byref(params), int(mask), ctypes.c_void_p(_stream_handle(q.device))),
               "tpr_attn_bwd")
    return dq, dk, dv, dpk, dpv


class TPRPrefixAttention(torch.autograd.Function):
    """(q, k, v, prefix_k, prefix_v, meta, softmax_scale, prefix_grad_accumulators,
    recompute_dq, ds_store_budget, attention_mask) -> (out, lse).

    With ``prefix_grad_accumulators`` = (dK, dV), fp32 tensors shaped like
    prefix_k, the backward adds the prefix gradients into them (the relay of
    prefix_state.py:546-573, in fp32 and inside the kernel) and gives
    prefix_k / prefix_v no autograd gradient; they must then not require one.

    Memory: the backward's workspace holds, besides a few MB of statistics,
    the dS store when the plan has one -- 2 bytes per visible (query, key)
    pair and query head, 6.5 GB at the Qwen3-4B layer shape (prefix 4096 +
    4 x 4096, GQA 32/8) -- which makes dQ one matrix product instead of three.
    ``ds_store_budget`` caps it in bytes: None = the library default (8 GiB),
    0 = no store (``recompute_dq=True`` is the same). If the workspace of a
    plan with a store cannot be allocated, the backward falls back to the plan
    without one (same gradients, slower dQ).

    ``attention_mask``: an optional physical key mask (module docstring),
    which replaces the causal rule.
    """

    @staticmethod
    def forward(ctx, q, k, v, prefix_k, prefix_v, meta, softmax_scale=None, prefix_grad_accumulators=None,
                recompute_dq=False, ds_store_budget=None, attention_mask=None):
        scale = validate(q, k, v, prefix_k, prefix_v, meta, softmax_scale)
        mask = check_mask(attention_mask, q, meta)
        budget = ds_store_budget_bytes(ds_store_budget, recompute_dq)
        if prefix_grad_accumulators is not None:
            if prefix_k.requires_grad or prefix_v.requires_grad:
                raise ValueError("prefix_k/prefix_v must not require grad when prefix_grad_accumulators is given")
            _check_accumulators(prefix_grad_accumulators, prefix_k)
        q, k, v, prefix_k, prefix_v = _inputs(q, k, v, prefix_k, prefix_v)
        out, lse = _forward(q, k, v, prefix_k, prefix_v, meta, scale, mask)
        ctx.save_for_backward(q, k, v, prefix_k, prefix_v, out, lse)
        ctx.mask = mask
        ctx.meta = meta
        ctx.scale = scale
        ctx.accumulators = prefix_grad_accumulators
        ctx.ds_store_budget = budget
        ctx.mark_non_differentiable(lse)
        return out, lse

    @staticmethod
    def backward(ctx, dout, _dlse):
        q, k, v, prefix_k, prefix_v, out, lse = ctx.saved_tensors
        if dout is None:
            dout = torch.zeros_like(out)
        dout = dout.contiguous()
        dq, dk, dv, dpk, dpv = _backward(q, k, v, prefix_k, prefix_v, out, lse, dout, ctx.meta, ctx.scale,
                                         prefix_grad_accumulators=ctx.accumulators,
                                         ds_store_budget=ctx.ds_store_budget, mask=ctx.mask)
        if ctx.accumulators is not None:
            dpk = dpv = None
        return dq, dk, dv, dpk, dpv, None, None, None, None, None, None


def tpr_prefix_attention(q, k, v, prefix_k, prefix_v, meta: TPRPrefixMeta, softmax_scale=None, *,
                         prefix_grad_accumulators=None, recompute_dq=False, ds_store_budget=None,
                         attention_mask=None):
    """Functional form of TPRPrefixAttention; returns (out, lse)."""
    return TPRPrefixAttention.apply(q, k, v, prefix_k, prefix_v, meta, softmax_scale, prefix_grad_accumulators,
                                    recompute_dq, ds_store_budget, attention_mask)


def prefix_attention_forward(q, k, v, prefix_k, prefix_v, meta: TPRPrefixMeta, softmax_scale=None, *,
                             attention_mask=None):
    """Forward only, no autograd graph: (out, lse)."""
    scale = validate(q, k, v, prefix_k, prefix_v, meta, softmax_scale)
    mask = check_mask(attention_mask, q, meta)
    q, k, v, prefix_k, prefix_v = _inputs(q, k, v, prefix_k, prefix_v)
    return _forward(q, k, v, prefix_k, prefix_v, meta, scale, mask)


def prefix_attention_backward(q, k, v, prefix_k, prefix_v, out, lse, dout, meta: TPRPrefixMeta,
                              softmax_scale=None, *, phases=None, buffers=None, prefix_grad_accumulators=None,
                              recompute_dq=False, ds_store_budget=None, attention_mask=None):
    """Backward only: (dq, dk, dv, dprefix_k, dprefix_v) from saved out/lse.

    ``phases`` selects backward phases (mask of TPR_BWD_DELTA / _DKDV / _DQ,
    or _DKDV_TILES then _DKDV_REDUCE for the two steps of _DKDV; the delta
    phase must have run before the others, with the same ``delta`` and
    ``workspace``); ``buffers`` may hold preallocated outputs, the fp32
    ``delta`` scratch and the ``workspace``, keyed by name.
    ``prefix_grad_accumulators``: a (dK, dV) pair of fp32 tensors shaped like
    prefix_k into which the prefix gradients are added (and returned).
    ``ds_store_budget`` (bytes; None = the library default) or
    ``recompute_dq=True`` (= budget 0) select the plan (TPRPrefixMeta.plan);
    with a dS store the dQ phase reads what the dK/dV phase wrote, and a
    ``workspace`` given in ``buffers`` must be of that plan's size.
    ``attention_mask``: the forward's physical key mask, if it had one."""
    scale = validate(q, k, v, prefix_k, prefix_v, meta, softmax_scale)
    mask = check_mask(attention_mask, q, meta)
    tensors = [*_inputs(q, k, v, prefix_k, prefix_v), *(t.contiguous() for t in (out, lse, dout))]
    return _backward(*tensors[:7], tensors[7], meta, scale, phases=phases, buffers=buffers,
                     prefix_grad_accumulators=prefix_grad_accumulators,
                     ds_store_budget=ds_store_budget_bytes(ds_store_budget, recompute_dq), mask=mask)
