"""GPU checks of TPRKernelBackend (the model seam, parallel_size 1): one
launch for all siblings equals the per-sibling visits, and the prefix
gradient is the sum of the siblings' -- the reference invariant of
test_segment_executor.py:291-325 -- and both match the fp32 oracle."""

from __future__ import annotations

import math

import pytest
import torch

from _helpers import BF16_FWD_COS, BF16_FWD_MAX_ABS, BF16_GRAD_COS, BF16_PREFIX_GRAD_REL_L2, cosine, max_abs, rel_l2

pytestmark = pytest.mark.gpu


def _inputs(lengths, p, hq, hkv, d, device, seed=11):
    g = torch.Generator(device="cpu").manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g).bfloat16().to(device)  # noqa: E731
    qs = [r(s, 1, hq, d) for s in lengths]
    ks = [r(s, 1, hkv, d) for s in lengths]
    vs = [r(s, 1, hkv, d) for s in lengths]
    dos = [r(s, 1, hq * d) for s in lengths]
    return qs, ks, vs, dos, r(p, 1, hkv, d), r(p, 1, hkv, d)


def test_batched_visit_equals_per_sibling_visits_and_the_oracle(cuda_device):
    from bridge_amd import TPRKernelBackend
    from oracle.tpr_oracle import prefix_attention
    lengths, p, hq, hkv, d = [100, 37, 64], 200, 8, 2, 128
    scale = 1.0 / math.sqrt(d)
    qs, ks, vs, dos, pk0, pv0 = _inputs(lengths, p, hq, hkv, d, cuda_device)

    # batched: one backend for all three siblings, one launch per layer
    pk, pv = pk0.clone().requires_grad_(True), pv0.clone().requires_grad_(True)
    batched = TPRKernelBackend({1: (pk, pv)}, lengths)
    q, k, v = (batched.pack(x).requires_grad_(True) for x in (qs, ks, vs))
    out = batched.attention(1, q, k, v, softmax_scale=scale)
    assert out.shape == (sum(lengths), 1, hq * d)
    out.backward(batched.pack(dos))
    torch.cuda.synchronize()

    # per sibling: the reference's loop of single-leaf visits
    single_outs, single_dq, pk_sum, pv_sum = [], [], 0, 0
    for i, s in enumerate(lengths):
        pki, pvi = pk0.clone().requires_grad_(True), pv0.clone().requires_grad_(True)
        qi, ki, vi = (x[i].clone().requires_grad_(True) for x in (qs, ks, vs))
        oi = TPRKernelBackend({1: (pki, pvi)}, [s]).attention(1, qi, ki, vi, softmax_scale=scale)
        oi.backward(dos[i])
        single_outs.append(oi.detach())
        single_dq.append(qi.grad)
        pk_sum = pk_sum + pki.grad.float()
        pv_sum = pv_sum + pvi.grad.float()
    torch.cuda.synchronize()

    # same per-sibling results, and the batched prefix gradient is the sum of the siblings'
    assert torch.equal(out.detach(), torch.cat(single_outs))
    assert torch.equal(q.grad, torch.cat(single_dq))
    assert cosine(pk.grad, pk_sum) >= 0.99999 and rel_l2(pk.grad, pk_sum) <= 5e-3
    assert cosine(pv.grad, pv_sum) >= 0.99999 and rel_l2(pv.grad, pv_sum) <= 5e-3

    # fp32 oracle of each sibling against [prefix; suffix], prefix grads summed
    ref_pk = ref_pv = 0
    for i, s in enumerate(lengths):
        a, b = sum(lengths[:i]), sum(lengths[:i + 1])
        tq, tk, tv = (x[i].double().cpu().requires_grad_(True) for x in (qs, ks, vs))
        tpk, tpv = (x.double().cpu().requires_grad_(True) for x in (pk0, pv0))
        ro = prefix_attention(tq, tk, tv, tpk, tpv, scale)
        ro.backward(dos[i].double().cpu())
        assert max_abs(out[a:b], ro) <= BF16_FWD_MAX_ABS and cosine(out[a:b], ro) >= BF16_FWD_COS
        assert cosine(q.grad[a:b], tq.grad) >= BF16_GRAD_COS
        assert cosine(k.grad[a:b], tk.grad) >= BF16_GRAD_COS and cosine(v.grad[a:b], tv.grad) >= BF16_GRAD_COS
        ref_pk, ref_pv = ref_pk + tpk.grad, ref_pv + tpv.grad
    assert rel_l2(pk.grad, ref_pk) <= BF16_PREFIX_GRAD_REL_L2 and rel_l2(pv.grad, ref_pv) <= BF16_PREFIX_GRAD_REL_L2


def test_backend_without_prefix(cuda_device):
    from bridge_amd import TPRKernelBackend
    from oracle.tpr_oracle import prefix_attention
    lengths, hq, hkv, d = [48, 80], 4, 1, 128
    qs, ks, vs, dos, _, _ = _inputs(lengths, 0, hq, hkv, d, cuda_device, seed=3)
    backend = TPRKernelBackend({}, lengths)
    out = backend.attention(1, backend.pack(qs), backend.pack(ks), backend.pack(vs), softmax_scale=None)
    for i, o in enumerate(backend.unpack(out)):
        empty = torch.zeros(0, 1, hkv, d, dtype=torch.float64)
        ro = prefix_attention(qs[i].double().cpu(), ks[i].double().cpu(), vs[i].double().cpu(), empty, empty, None)
        assert max_abs(o, ro) <= BF16_FWD_MAX_ABS and cosine(o, ro) >= BF16_FWD_COS
