"""GPU checks of the q/k/v row strides (TprFwdParams / TprBwdParams
q_row_stride, k_row_stride, v_row_stride).

q, k and v taken as slices of one fused [tokens, (Hq + 2 Hkv) * D]
projection, or from rows padded by 16 bytes, reach the kernels without a
copy; out, lse and every gradient (into the fused projection through
autograd) equal those of packed copies of the same values bit for bit, on
each kernel path: head_dim 128 (32x32x16 MFMA), 64 and 256 (16x16x32 MFMA),
at 128 and 256 with both dQ plans (the dS store, and recomputing), and the
SIMT kernels (fp32, and bf16 at head_dim 96). The leaves mix full and
partial 64-row tiles and suffixes longer than one dK/dV tile, so both copy
forms of each kernel (whole tiles and the clamped tail) read through the
stride.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

CASES = {  # name: (hq, hkv, head_dim, dtype, recompute_dq)
    "mfma_d128": (8, 2, 128, torch.bfloat16, False),
    "mfma_d128_recompute": (8, 2, 128, torch.bfloat16, True),
    "mfma16_d64": (8, 2, 64, torch.bfloat16, False),
    "mfma16_d256": (4, 2, 256, torch.bfloat16, False),
    "mfma16_d256_recompute": (4, 2, 256, torch.bfloat16, True),
    "simt_fp32_d64": (4, 2, 64, torch.float32, False),
    "simt_bf16_d96": (4, 2, 96, torch.bfloat16, False),
}


def _run(meta, q, k, v, pk, pv, dout, scale, recompute_dq):
    from bridge_amd import tpr_prefix_attention
    out, lse = tpr_prefix_attention(q, k, v, pk, pv, meta, scale, recompute_dq=recompute_dq)
    out.backward(dout)
    torch.cuda.synchronize()
    return out.detach(), lse


@pytest.mark.parametrize("layout", ["fused_qkv", "padded_rows"])
@pytest.mark.parametrize("case", list(CASES))
def test_strided_views_equal_packed_copies_bitwise(case, layout, cuda_device):
    from bridge_amd import TPRPrefixMeta
    from bridge_amd.prefix_attention import _row_stride, _rows
    hq, hkv, d, dtype, recompute_dq = CASES[case]
    meta = TPRPrefixMeta.shared_prefix(300, [200, 37, 64, 130])
    tq, scale = meta.total_q, 0.7 / d ** 0.5
    gen = torch.Generator(device="cpu").manual_seed(11)
    width = (hq + 2 * hkv) * d
    pad = 16 // torch.tensor([], dtype=dtype).element_size() if layout == "padded_rows" else 0
    base = torch.randn(tq, width + pad, generator=gen).to(dtype).to(cuda_device)
    pk, pv = (torch.randn(meta.total_prefix, hkv, d, generator=gen).to(dtype).to(cuda_device) for _ in range(2))
    dout = torch.randn(tq, hq, d, generator=gen).to(dtype).to(cuda_device)
    print(f"strides case={case} layout={layout} hq={hq} hkv={hkv} d={d} tq={tq}", flush=True)

    fused = base.clone().requires_grad_(True)
    q = fused[:, :hq * d].view(tq, hq, d)
    k = fused[:, hq * d:(hq + hkv) * d].view(tq, hkv, d)
    v = fused[:, (hq + hkv) * d:width].view(tq, hkv, d)
    for t in (q, k, v):  # the kernels read the views in place
        assert _rows(t) is t and _row_stride(t) == width + pad
    out_s, lse_s = _run(meta, q, k, v, pk, pv, dout, scale, recompute_dq)

    packed = [base[:, a:b].reshape(tq, -1, d).contiguous().requires_grad_(True)
              for a, b in ((0, hq * d), (hq * d, (hq + hkv) * d), ((hq + hkv) * d, width))]
    out_p, lse_p = _run(meta, *packed, pk, pv, dout, scale, recompute_dq)

    assert torch.equal(out_s, out_p)
    assert torch.equal(lse_s, lse_p)
    grad = fused.grad
    assert torch.equal(grad[:, :hq * d].reshape(tq, hq, d), packed[0].grad)
    assert torch.equal(grad[:, hq * d:(hq + hkv) * d].reshape(tq, hkv, d), packed[1].grad)
    assert torch.equal(grad[:, (hq + hkv) * d:width].reshape(tq, hkv, d), packed[2].grad)
    assert not grad[:, width:].any()  # padding untouched
    assert torch.isfinite(out_s.float()).all() and out_s.float().abs().sum() > 0
