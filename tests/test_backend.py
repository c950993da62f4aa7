"""CPU checks of TPRKernelBackend: the TPRAttentionBackend protocol
(context.py:35-58) as the reference's context validates it
(context.py:132-162), and the argument errors of its attention call
(context.py:59-96). No GPU work."""

from __future__ import annotations

import pytest
import torch

from bridge_amd import TPRKernelBackend

P, HKV, HQ, D = 6, 2, 4, 16


def _prefix(layers=(1, 2), p=P):
    return {n: (torch.zeros(p, 1, HKV, D), torch.zeros(p, 1, HKV, D)) for n in layers}


def test_protocol_surface_as_the_reference_context_checks_it():
    backend = TPRKernelBackend(_prefix(), [3, 5])
    for name in ("global_prefix_length", "global_suffix_length", "local_suffix_length", "parallel_size",
                 "attention"):
        assert hasattr(backend, name)
    assert callable(backend.attention)
    assert backend.global_prefix_length == P
    assert backend.global_suffix_length == backend.local_suffix_length == 8
    assert backend.parallel_size == 1


def test_prefix_length_zero_needs_no_past_kv():
    backend = TPRKernelBackend({}, [4])
    assert backend.global_prefix_length == 0
    with pytest.raises(ValueError, match="must be empty"):
        TPRKernelBackend(_prefix(), [4], prefix_length=0)


@pytest.mark.parametrize("lengths", [[], [0], [3, -1], [2.0]])
def test_suffix_lengths_must_be_positive_integers(lengths):
    with pytest.raises(ValueError, match="suffix_lengths"):
        TPRKernelBackend(_prefix(), lengths)


def test_past_kv_is_validated_like_the_reference_context():
    with pytest.raises(ValueError, match="layer_number"):
        TPRKernelBackend({0: (torch.zeros(P, 1, HKV, D), torch.zeros(P, 1, HKV, D))}, [2])
    with pytest.raises(TypeError, match="tuple"):
        TPRKernelBackend({1: [torch.zeros(P, 1, HKV, D), torch.zeros(P, 1, HKV, D)]}, [2])
    with pytest.raises(ValueError, match="batch size must be 1"):
        TPRKernelBackend({1: (torch.zeros(P, 2, HKV, D), torch.zeros(P, 2, HKV, D))}, [2])
    with pytest.raises(ValueError, match="shapes must match"):
        TPRKernelBackend({1: (torch.zeros(P, 1, HKV, D), torch.zeros(P, 1, HKV, D + 1))}, [2])
    with pytest.raises(ValueError, match="sequence length must be 5"):
        TPRKernelBackend({1: (torch.zeros(P, 1, HKV, D), torch.zeros(P, 1, HKV, D))}, [2], prefix_length=5)


def test_attention_argument_errors():
    backend = TPRKernelBackend(_prefix(), [3, 5])
    q = torch.zeros(8, 1, HQ, D)
    k = torch.zeros(8, 1, HKV, D)
    with pytest.raises(ValueError, match="layer_number"):
        backend.attention(True, q, k, k, softmax_scale=None)
    with pytest.raises(ValueError, match="sequence length must be 8"):
        backend.attention(1, q, k[:7], k[:7], softmax_scale=None)
    with pytest.raises(ValueError, match="query sequence length must be 8"):
        backend.attention(1, q[:7], k, k, softmax_scale=None)
    with pytest.raises(KeyError, match="missing past KV for layer 3"):
        backend.attention(3, q, k, k, softmax_scale=None)
    # the kernel runs on the GPU only
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        backend.attention(1, q, k, k, softmax_scale=None)


def test_pack_and_unpack_keep_sibling_order():
    backend = TPRKernelBackend(_prefix(), [3, 5])
    a, b = torch.arange(3.0), torch.arange(5.0) + 10
    packed = backend.pack([a, b])
    assert packed.tolist() == a.tolist() + b.tolist()
    ua, ub = backend.unpack(packed)
    assert torch.equal(ua, a) and torch.equal(ub, b)
    with pytest.raises(ValueError):
        backend.pack([b, a])
