"""GPU: the reference's operator equivalence tests, restated for the drop-in.

They mirror tests/models/mcore/tpr/equivalence/test_rectangular_attention_npu.py
of the reference (NPU-only there): the same shapes, seeds, dtype and
tolerances, with inputs drawn from a CPU generator (the NPU's generator is
not available here, so the draws differ) and the fp32 math of the
reference's dense oracle (_reference, :25-38; oracle/tpr_oracle.py::
prefix_attention here)."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _right_down_mask(query_length, kv_length, device):
    """True = masked: key j is hidden from query i iff j > P + i (the reference's :40-44)."""
    prefix_length = kv_length - query_length
    query_positions = torch.arange(query_length, device=device) + prefix_length
    key_positions = torch.arange(kv_length, device=device)
    return key_positions.unsqueeze(0) > query_positions.unsqueeze(1)


def _inputs(seed, sq, skv, hq, hkv, d, device):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(sq, 1, hq, d, generator=g).bfloat16()
    k = torch.randn(skv, 1, hkv, d, generator=g).bfloat16()
    v = torch.randn(skv, 1, hkv, d, generator=g).bfloat16()
    dout = torch.randn(sq, 1, hq * d, generator=g).bfloat16()
    return [t.to(device) for t in (q, k, v)], dout.to(device)


def _fp32_reference(q, k, v, dout, scale):
    """Dense fp32 attention over [prefix; suffix] with the right-down mask, and its gradients."""
    from oracle.tpr_oracle import prefix_attention
    p = k.shape[0] - q.shape[0]
    qc, kc, vc = (t.detach().float().cpu().requires_grad_(True) for t in (q, k, v))
    out = prefix_attention(qc, kc[p:], vc[p:], kc[:p], vc[:p], scale)
    out.backward(dout.float().cpu())
    return out.detach(), [t.grad for t in (qc, kc, vc)]


def _fused_backward_reference(q, k, v, dout, out, scale):
    """Gradients as a fused attention backward computes them: P from the exact
    lse, and delta = rowsum(dO * O) from the bf16 output O the forward
    returned. The reference's backward passes that output in the same way
    (npu_fusion_attention_grad(attention_in=...), ring_attention.py:709-737,
    with the output cast to the input dtype at :633-636)."""
    from bridge_amd import TPRPrefixMeta
    from oracle.tpr_oracle import tree_backward, tree_forward
    from _helpers import tree_of
    sq, _, hq, d = q.shape
    p = k.shape[0] - sq
    tree = tree_of(TPRPrefixMeta.shared_prefix(p, [sq]))
    qt, kt, vt = (t.detach().double().cpu()[:, 0] for t in (q, k, v))
    args = (qt, kt[p:], vt[p:], kt[:p], vt[:p])
    _, lse = tree_forward(*args, tree, scale)
    o = out.detach().double().cpu().view(sq, hq, d)
    dq, dk, dv, dpk, dpv = tree_backward(*args, tree, dout.detach().double().cpu().view(sq, hq, d), scale,
                                         out=o, lse=lse)
    return [dq.unsqueeze(1), torch.cat([dpk, dk]).unsqueeze(1), torch.cat([dpv, dv]).unsqueeze(1)]


@pytest.mark.parametrize(("prefix_length", "suffix_length"), [(0, 3), (6, 3), (32, 1)])
def test_rectangular_attention_matches_reference_forward_and_backward(prefix_length, suffix_length, cuda_device):
    """The reference's :54-85: H=2, D=64, bf16; output against the fp32 oracle
    at 5e-3. Gradients at 5e-3 against the fused-backward reference (delta
    from the returned bf16 output, as the reference's kernel computes it),
    and against the exact fp32 gradients at the reference's gradient
    tolerance of :137-146 (6e-3 / 2e-2): with delta from a bf16 output the
    exact gradients can differ by more than 5e-3 (0.009 on this draw)."""
    from bridge_amd import rectangular_causal_attention
    heads, head_dim = 2, 64
    scale = head_dim ** -0.5
    (q, k, v), dout = _inputs(1234, suffix_length, prefix_length + suffix_length, heads, heads, head_dim,
                              cuda_device)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = rectangular_causal_attention(qa, ka, va, softmax_scale=scale)
    out.backward(dout)
    torch.cuda.synchronize()
    ref, ref_grads = _fp32_reference(q, k, v, dout, scale)
    torch.testing.assert_close(out.float().cpu(), ref, atol=5e-3, rtol=5e-3)
    fused = _fused_backward_reference(q, k, v, dout, out, scale)
    for mine, same_algorithm, exact in zip((qa.grad, ka.grad, va.grad), fused, ref_grads):
        torch.testing.assert_close(mine.double().cpu(), same_algorithm, atol=5e-3, rtol=5e-3)
        torch.testing.assert_close(mine.float().cpu(), exact, atol=6e-3, rtol=2e-2)
    if prefix_length:
        assert ka.grad[:prefix_length].float().norm() > 0
        assert va.grad[:prefix_length].float().norm() > 0


def test_explicit_causal_mask_matches_sparse_mode_3_forward_and_backward(cuda_device):
    """The reference's :88-146: the explicit right-down mask and the default
    (sparse mode 3) give the same attention, both within 6e-3 / 1e-2 (out)
    and 6e-3 / 2e-2 (grads) of the fp32 oracle; 63 x 127, 4 heads, D=64."""
    from bridge_amd import rectangular_causal_attention
    query_length, kv_length, heads, head_dim = 63, 127, 4, 64
    scale = head_dim ** -0.5
    (q, k, v), dout = _inputs(2026, query_length, kv_length, heads, heads, head_dim, cuda_device)
    ref, ref_grads = _fp32_reference(q, k, v, dout, scale)
    for mask in (None, _right_down_mask(query_length, kv_length, cuda_device)):
        qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
        out = rectangular_causal_attention(qa, ka, va, softmax_scale=scale, attention_mask=mask)
        out.backward(dout)
        torch.cuda.synchronize()
        torch.testing.assert_close(out.float().cpu(), ref, atol=6e-3, rtol=1e-2)
        for mine, theirs in zip((qa.grad, ka.grad, va.grad), ref_grads):
            torch.testing.assert_close(mine.float().cpu(), theirs, atol=6e-3, rtol=2e-2)


def test_physical_padding_mask_matches_logical_attention_forward_and_backward(cuda_device):
    """The reference's :149-284: Q 63 + 1 and KV 127 + 1 physical rows, GQA
    4/2, D 64, bf16. The padding key is hidden by a custom mask (the padding
    query sees keys up to position 126), or, with ``inner_precise=2`` there,
    the padding query row is hidden entirely. Against the logical call (63 x
    127, causal mask): output within 6e-3 / 1e-2, gradients of the logical
    rows within 6e-3 / 2e-2, the padding rows' gradients zero, and the fully
    hidden row's output zero -- the reference's assertions. The masked calls
    run on the masked SIMT kernels, the logical one on the 16x16x32 MFMA
    kernels."""
    from bridge_amd import rectangular_causal_attention
    lq, lkv, hq, hkv, d = 63, 127, 4, 2, 64
    scale = d ** -0.5
    g = torch.Generator().manual_seed(2027)
    logical = [torch.randn(n, 1, h, d, generator=g).bfloat16().to(cuda_device)
               for n, h in ((lq, hq), (lkv, hkv), (lkv, hkv))]
    physical = [torch.cat((t, torch.randn(1, *t.shape[1:], generator=g).bfloat16().to(cuda_device))) for t in logical]
    grad_output = torch.randn(lq, 1, hq * d, generator=g).bfloat16().to(cuda_device)
    physical_grad_output = torch.cat((grad_output, torch.zeros_like(grad_output[:1])))
    query_positions = torch.arange(64, 128, device=cuda_device).clamp_max(126)
    key_positions = torch.arange(128, device=cuda_device).clamp_max(126)
    key_valid = torch.arange(128, device=cuda_device) < lkv
    physical_mask = torch.logical_or(~key_valid.unsqueeze(0), key_positions.unsqueeze(0) > query_positions.unsqueeze(1))
    invalid_row_mask = torch.logical_or(physical_mask, (torch.arange(64, device=cuda_device) >= lq).unsqueeze(1))

    la = [t.clone().requires_grad_(True) for t in logical]
    logical_output = rectangular_causal_attention(*la, softmax_scale=scale,
                                                  attention_mask=_right_down_mask(lq, lkv, cuda_device))
    logical_output.backward(grad_output)
    runs = []
    for mask, precise in ((physical_mask, 0), (invalid_row_mask, 2)):
        pa = [t.clone().requires_grad_(True) for t in physical]
        out = rectangular_causal_attention(*pa, softmax_scale=scale, attention_mask=mask, inner_precise=precise)
        out.backward(physical_grad_output)
        runs.append((out, pa))
    torch.cuda.synchronize()
    torch.testing.assert_close(runs[0][0][:lq].float(), logical_output.float(), atol=6e-3, rtol=1e-2)
    for _, inputs in runs:
        for phys, log in zip(inputs, la):
            torch.testing.assert_close(phys.grad[:log.shape[0]].float(), log.grad.float(), atol=6e-3, rtol=2e-2)
            torch.testing.assert_close(phys.grad[log.shape[0]:], torch.zeros_like(phys.grad[log.shape[0]:]))
    invalid_row_output = runs[1][0]
    torch.testing.assert_close(invalid_row_output[:lq].float(), logical_output.float(), atol=6e-3, rtol=1e-2)
    torch.testing.assert_close(invalid_row_output[lq:], torch.zeros_like(invalid_row_output[lq:]))


def test_physical_mask_against_the_fp32_oracle(cuda_device):
    """A physical mask that shows later keys too (not a causal mask), through
    the drop-in: output and gradients within the reference's bf16 tolerances
    (6e-3 / 1e-2, grads 6e-3 / 2e-2) of the fp64 oracle with the same mask."""
    from bridge_amd import TPRPrefixMeta, rectangular_causal_attention
    from oracle.tpr_oracle import tree_backward, tree_forward
    from _helpers import random_key_mask, tree_of
    sq, skv, hq, hkv, d = 40, 100, 4, 2, 64
    p = skv - sq
    scale = d ** -0.5
    (q, k, v), dout = _inputs(2028, sq, skv, hq, hkv, d, cuda_device)
    tree = tree_of(TPRPrefixMeta.shared_prefix(p, [sq]))
    mask = random_key_mask(tree, torch.Generator().manual_seed(7))
    assert mask.shape == (sq, skv)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = rectangular_causal_attention(qa, ka, va, softmax_scale=scale, attention_mask=mask.to(cuda_device))
    out.backward(dout)
    torch.cuda.synchronize()
    qt, kt, vt = (t.double().cpu()[:, 0] for t in (q, k, v))
    args = (qt, kt[p:], vt[p:], kt[:p], vt[:p], tree)
    ro, lse = tree_forward(*args, scale, mask=mask)
    dq, dk, dv, dpk, dpv = tree_backward(*args, dout.double().cpu().view(sq, hq, d), scale, out=ro, lse=lse,
                                         mask=mask)
    torch.testing.assert_close(out.double().cpu().view(sq, hq, d), ro, atol=6e-3, rtol=1e-2)
    for mine, theirs in ((qa.grad[:, 0], dq), (ka.grad[:, 0], torch.cat((dpk, dk))),
                         (va.grad[:, 0], torch.cat((dpv, dv)))):
        torch.testing.assert_close(mine.double().cpu(), theirs, atol=6e-3, rtol=2e-2)
