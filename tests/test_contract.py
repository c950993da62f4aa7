"""CPU tests of the drop-in's input contract, mirroring the reference's
tests/models/mcore/tpr/unit/test_rectangular_attention_contract.py (same
mutations, same exception types and message fragments)."""

import pytest
import torch

from bridge_amd import TPRPrefixAttention, TPRPrefixMeta, rectangular_causal_attention
from bridge_amd.rectangular_attention import _validate_attention_mask, _validate_inputs


def _qkv(query_length=3, kv_length=9, query_heads=4, kv_heads=2, head_dim=8):
    query = torch.randn(query_length, 1, query_heads, head_dim)
    key = torch.randn(kv_length, 1, kv_heads, head_dim)
    return query, key, torch.randn_like(key)


def test_contract_accepts_rectangular_gqa_shapes():
    assert _validate_inputs(*_qkv(), dropout_p=0.0) == (3, 9, 4, 8)


@pytest.mark.parametrize(
    ("mutation", "match"),
    [
        (lambda q, k, v: (q[:, :, :, :-1], k, v), "head dimensions"),
        (lambda q, k, v: (q, k[:, :, :1], v), "identical shapes"),
        (lambda q, k, v: (q.repeat(1, 2, 1, 1), k, v), "batch size 1"),
        (lambda q, k, v: (q, k.to(torch.float64), v), "dtypes must match"),
        (lambda q, k, v: (q[:, :, :3], k, v), "divisible"),
        (lambda q, k, v: (q.repeat(4, 1, 1, 1), k, v), "cannot exceed"),
        (lambda q, k, v: (q[0], k, v), r"\[sequence, batch, heads, head_dim\]"),
    ],
)
def test_contract_rejects_incompatible_inputs(mutation, match):
    with pytest.raises(ValueError, match=match):
        _validate_inputs(*mutation(*_qkv()), dropout_p=0.0)


def test_contract_rejects_attention_dropout():
    with pytest.raises(ValueError, match="dropout_p=0"):
        _validate_inputs(*_qkv(), dropout_p=0.1)


def test_contract_accepts_physical_bool_attention_mask():
    q, k, _ = _qkv()
    _validate_attention_mask(torch.zeros(q.shape[0], k.shape[0], dtype=torch.bool), query_length=q.shape[0],
                             kv_length=k.shape[0], device=q.device)


@pytest.mark.parametrize(("mask", "match"), [(torch.zeros(3, 9), "torch.bool"),
                                             (torch.zeros(3, 8, dtype=torch.bool), "shape")])
def test_contract_rejects_invalid_physical_attention_mask(mask, match):
    with pytest.raises(ValueError, match=match):
        _validate_attention_mask(mask, query_length=3, kv_length=9, device=torch.device("cpu"))


def test_contract_rejects_non_tensor_mask():
    with pytest.raises(TypeError, match="torch.Tensor or None"):
        _validate_attention_mask([[False]], query_length=1, kv_length=1, device=torch.device("cpu"))


def test_public_adapter_fails_clearly_off_gpu():
    with pytest.raises(RuntimeError, match="requires a ROCm GPU tensor"):
        rectangular_causal_attention(*_qkv())


def test_public_adapter_checks_mask_before_device():
    q, k, v = _qkv()
    with pytest.raises(ValueError, match="torch.bool"):
        rectangular_causal_attention(q, k, v, attention_mask=torch.zeros(3, 9))


def _packed(meta, hq=4, hkv=2, d=8, dtype=torch.float32):
    return (torch.randn(meta.total_q, hq, d, dtype=dtype), torch.randn(meta.total_q, hkv, d, dtype=dtype),
            torch.randn(meta.total_q, hkv, d, dtype=dtype), torch.randn(meta.total_prefix, hkv, d, dtype=dtype),
            torch.randn(meta.total_prefix, hkv, d, dtype=dtype))


def test_function_rejects_cpu_tensors_with_device_message():
    meta = TPRPrefixMeta.shared_prefix(5, [3, 2])
    with pytest.raises(RuntimeError, match="requires a ROCm GPU"):
        TPRPrefixAttention.apply(*_packed(meta), meta, None)


@pytest.mark.parametrize(
    ("mutate", "exc", "match"),
    [
        (lambda t: (t[0][:, :3], *t[1:]), ValueError, "divisible"),
        (lambda t: (t[0], t[1][:, :1], *t[2:]), ValueError, "identical shapes"),
        (lambda t: (t[0], t[1], t[2], t[3][:-1], t[4][:-1]), ValueError, "meta.total_prefix"),
        (lambda t: (t[0][:-1], t[1][:-1], t[2][:-1], t[3], t[4]), ValueError, "meta.total_q"),
        (lambda t: tuple(x.double() for x in t), ValueError, "bfloat16 and torch.float32"),
        (lambda t: (t[0], t[1].bfloat16(), *t[2:]), ValueError, "dtypes must match"),
        (lambda t: (t[0][..., :4], *t[1:]), ValueError, "head dimensions"),
        (lambda t: (t[0].unsqueeze(1), *t[1:]), ValueError, "tokens, heads, head_dim"),
    ],
)
def test_function_contract(mutate, exc, match):
    meta = TPRPrefixMeta.shared_prefix(5, [3, 2])
    with pytest.raises(exc, match=match):
        TPRPrefixAttention.apply(*mutate(_packed(meta)), meta, None)
