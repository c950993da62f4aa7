"""GPU checks of the dS store (bf16, head_dim 128 and 256): the dK/dV kernel
stores every dS block it computes and the dQ kernel (mfma_dqs, m16_dqs)
computes dQ = scale dS K from them, instead of recomputing S and dP.

* dK, dV and the prefix gradients are those of the recomputing plan bit for
  bit (the same dK/dV kernel, the stores only add writes);
* dQ matches the recomputing dQ and the fp32 oracle within the bf16 bars;
* cases: GQA ratios 1, 3, 4 and 8 (2, 1 or 4 heads per dK/dV stage, 1 to 8
  heads per dQ workgroup), a depth-3 tree with ragged leaves (partial 64-key
  halves at every segment end, dK/dV waves past a segment's end that store
  nothing), split prefix tiles (partial-slot chunks each storing their blocks),
  suffixes shorter than one query block, and q/k/v read through a row stride;
* the backward run phase by phase (delta, dK/dV tiles, reduction, dQ: the
  order bench.py times) equals the one-call backward bitwise.
"""

from __future__ import annotations

import pytest
import torch

from _helpers import BF16_GRAD_COS, cosine, make_inputs, oracle, rel_l2

pytestmark = pytest.mark.gpu


def _cases():
    from bridge_amd import TPRPrefixMeta as M
    return {
        "gqa4": (M.shared_prefix(300, [100, 37, 64, 200]), 8, 2),
        "gqa1": (M.shared_prefix(200, [129, 64]), 4, 4),
        "gqa3": (M.shared_prefix(150, [257, 20]), 6, 2),
        "gqa8": (M.shared_prefix(130, [70, 300]), 16, 2),
        "depth3_ragged": (M(cu_seqlens_q=(0, 33, 98, 138, 155, 420), node_offsets=(0, 130, 200, 270),
                            leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2), (0,))), 8, 2),
        "split_prefix": (M.shared_prefix(256, [300] * 16), 4, 1),
        "no_prefix": (M.shared_prefix(0, [200, 5]), 8, 1),
    }


def _backward(meta, q, k, v, pk, pv, out, lse, dout, scale, recompute, phases=None):
    from bridge_amd import prefix_attention_backward
    grads = prefix_attention_backward(q, k, v, pk, pv, out, lse, dout, meta, scale, recompute_dq=recompute,
                                      phases=phases)
    torch.cuda.synchronize()
    return grads


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("case", list(_cases()))
def test_ds_store_backward_matches_recomputed_dq_and_oracle(case, d, cuda_device):
    from bridge_amd import prefix_attention_forward
    meta, hq, hkv = _cases()[case]
    scale = 0.09
    assert meta.plan(hq, hkv, d, torch.bfloat16, cuda_device).dq_from_ds
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=5, device=cuda_device)
    print(f"ds_store case={case} d={d} hq={hq} hkv={hkv} tq={meta.total_q} tp={meta.total_prefix}", flush=True)
    out, lse = prefix_attention_forward(q, k, v, pk, pv, meta, scale)
    ds = _backward(meta, q, k, v, pk, pv, out, lse, dout, scale, recompute=False)
    rc = _backward(meta, q, k, v, pk, pv, out, lse, dout, scale, recompute=True)
    for name, a, b in zip(("dk", "dv", "dprefix_k", "dprefix_v"), ds[1:], rc[1:]):
        assert torch.equal(a, b), f"{name} differs between the dS-store and recomputing plans"
    assert torch.isfinite(ds[0].float()).all()
    assert rel_l2(ds[0], rc[0]) < 1e-2 and cosine(ds[0], rc[0]) > 0.9999
    ref = oracle(meta, q, k, v, pk, pv, dout, scale)
    assert cosine(ds[0], ref[2][0]) > BF16_GRAD_COS
    assert rel_l2(ds[0], ref[2][0]) < 2e-2


def test_ds_store_phase_by_phase_equals_one_call(cuda_device):
    from bridge_amd import _lib, prefix_attention_forward
    meta, hq, hkv = _cases()["split_prefix"]
    d, scale = 128, 0.09
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=9, device=cuda_device)
    out, lse = prefix_attention_forward(q, k, v, pk, pv, meta, scale)
    one = _backward(meta, q, k, v, pk, pv, out, lse, dout, scale, recompute=False)
    from bridge_amd import prefix_attention_backward
    plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device)
    buffers = {"delta": torch.empty_like(lse),
               "workspace": torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=cuda_device)}
    outs = None
    for ph in (_lib.TPR_BWD_DELTA, _lib.TPR_BWD_DKDV_TILES, _lib.TPR_BWD_DKDV_REDUCE, _lib.TPR_BWD_DQ):
        outs = prefix_attention_backward(q, k, v, pk, pv, out, lse, dout, meta, scale, phases=ph,
                                         buffers={**buffers, **(dict(zip(("dq", "dk", "dv", "dprefix_k",
                                                                          "dprefix_v"), outs)) if outs else {})})
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv", "dprefix_k", "dprefix_v"), outs, one):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("d", [128, 256])
def test_ds_store_reads_strided_inputs(d, cuda_device):
    """q/k/v as slices of one fused projection: the dS-store backward equals
    that of packed copies bit for bit."""
    from bridge_amd import tpr_prefix_attention
    meta, hq, hkv = _cases()["depth3_ragged"]
    scale, tq = 0.09, meta.total_q
    gen = torch.Generator(device="cpu").manual_seed(3)
    width = (hq + 2 * hkv) * d
    base = torch.randn(tq, width, generator=gen).to(torch.bfloat16).to(cuda_device)
    pk, pv = (torch.randn(meta.total_prefix, hkv, d, generator=gen).to(torch.bfloat16).to(cuda_device)
              for _ in range(2))
    dout = torch.randn(tq, hq, d, generator=gen).to(torch.bfloat16).to(cuda_device)
    fused = base.clone().requires_grad_(True)
    views = (fused[:, :hq * d].view(tq, hq, d), fused[:, hq * d:(hq + hkv) * d].view(tq, hkv, d),
             fused[:, (hq + hkv) * d:].view(tq, hkv, d))
    tpr_prefix_attention(*views, pk, pv, meta, scale)[0].backward(dout)
    packed = [t.detach().contiguous().requires_grad_(True) for t in views]
    tpr_prefix_attention(*packed, pk, pv, meta, scale)[0].backward(dout)
    torch.cuda.synchronize()
    grads = (fused.grad[:, :hq * d].reshape(tq, hq, d), fused.grad[:, hq * d:(hq + hkv) * d].reshape(tq, hkv, d),
             fused.grad[:, (hq + hkv) * d:].reshape(tq, hkv, d))
    for name, a, p in zip(("dq", "dk", "dv"), grads, packed):
        assert torch.equal(a, p.grad), name


@pytest.mark.parametrize("recompute", [False, True])
def test_autograd_backward_follows_the_recompute_flag(recompute, cuda_device):
    """tpr_prefix_attention(..., recompute_dq=...) backward equals the direct
    backward of the same plan bit for bit (head_dim 128, GQA 4)."""
    from bridge_amd import prefix_attention_backward, tpr_prefix_attention
    meta, hq, hkv = _cases()["gqa4"]
    d, scale = 128, 0.09
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=13, device=cuda_device)
    leaves = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    out, lse = tpr_prefix_attention(*leaves, meta, scale, recompute_dq=recompute)
    out.backward(dout)
    torch.cuda.synchronize()
    direct = prefix_attention_backward(q, k, v, pk, pv, out.detach(), lse, dout, meta, scale, recompute_dq=recompute)
    torch.cuda.synchronize()
    for name, leaf, ref in zip(("dq", "dk", "dv", "dprefix_k", "dprefix_v"), leaves, direct):
        assert torch.equal(leaf.grad, ref), name


def test_backward_falls_back_to_recomputing_dq_when_the_store_does_not_fit_in_memory(cuda_device):
    """The autograd backward whose dS store workspace cannot be allocated
    (the allocator capped 160 MB above what it holds, so the 419 MB store
    fails and the gradients plus the 1 MB recomputing workspace fit) runs the plan
    without a store: its gradients equal those of recompute_dq=True bitwise."""
    from bridge_amd import TPRPrefixMeta, tpr_prefix_attention
    meta, hq, hkv, d = TPRPrefixMeta.shared_prefix(1024, [1024] * 4), 32, 8, 128
    plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device)
    small = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device, ds_store_budget=0)
    assert plan.dq_from_ds and plan.workspace_bytes - small.workspace_bytes == 800 * 32 * 16384
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=17, device=cuda_device)
    grads = {}
    for label, recompute in (("recompute", True), ("fallback", False)):
        leaves = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
        out, _ = tpr_prefix_attention(*leaves, meta, 0.09, recompute_dq=recompute)
        torch.cuda.synchronize()
        total = torch.cuda.get_device_properties(cuda_device).total_memory
        if label == "fallback":
            torch.cuda.empty_cache()
            cap = torch.cuda.memory_reserved(cuda_device) + (160 << 20)
            torch.cuda.set_per_process_memory_fraction(cap / total, cuda_device)
        try:
            out.backward(dout)
            torch.cuda.synchronize()
        finally:
            torch.cuda.set_per_process_memory_fraction(1.0, cuda_device)
        grads[label] = [t.grad for t in leaves]
    print(f"fallback: store {plan.workspace_bytes} B, recomputing workspace {small.workspace_bytes} B", flush=True)
    for a, b in zip(grads["fallback"], grads["recompute"]):
        assert torch.equal(a, b)
