"""GPU parity of the HIP kernels (through the C ABI) against the fp64 CPU oracle."""

from __future__ import annotations

import math

import pytest
import torch

from _helpers import (
    BF16_FWD_COS,
    BF16_FWD_MAX_ABS,
    BF16_GRAD_COS,
    BF16_PREFIX_GRAD_REL_L2,
    FP32_TOL,
    cosine,
    make_inputs,
    max_abs,
    oracle,
    rel_l2,
)

pytestmark = pytest.mark.gpu


def _meta_cases():
    from bridge_amd import TPRPrefixMeta as M
    return {
        # name: (meta, hq, hkv)
        "shared_prefix_gqa4": (M.shared_prefix(200, [100, 37]), 8, 2),
        "no_prefix": (M.shared_prefix(0, [70, 33]), 4, 1),
        "tile_aligned": (M.shared_prefix(128, [64, 64, 128]), 8, 2),
        "mha": (M.shared_prefix(96, [80]), 2, 2),
        "gqa2": (M.shared_prefix(64, [90]), 4, 2),
        "gqa3": (M.shared_prefix(70, [45, 20]), 6, 2),
        "depth3_tree": (M(cu_seqlens_q=(0, 33, 98, 138, 155), node_offsets=(0, 130, 200, 270),
                          leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2))), 8, 2),
        "unused_node": (M(cu_seqlens_q=(0, 40), node_offsets=(0, 10, 30), leaf_ancestors=((0,),)), 4, 1),
        "empty_leaf": (M.shared_prefix(50, [0, 60, 0]), 4, 1),
        # 12 nested nodes of ragged lengths laid out root first: every leaf's
        # ancestors form one key run
        "deep_chain_one_run": (M(cu_seqlens_q=(0, 50, 179, 243), node_offsets=_offsets(_DEEP_LENS),
                                 leaf_ancestors=(tuple(range(12)), tuple(range(9)), tuple(range(3)))), 8, 2),
        # the same chain laid out deepest node first: 12, 9 and 3 separate key
        # runs, more than the forward / dQ kernels hold in registers
        "deep_run_list": (M(cu_seqlens_q=(0, 50, 179, 243), node_offsets=_offsets(_DEEP_LENS[::-1]),
                            leaf_ancestors=(tuple(range(11, -1, -1)), tuple(range(11, 2, -1)),
                                            tuple(range(11, 8, -1)))), 8, 2),
        # suffix dK/dV tiles paired with their mirrors: 3 tiles (a pair and a
        # lone middle tile), 2 tiles with a 1-key mirror, 4 tiles (two pairs),
        # 1 tile, 3 tiles with a 4-key last tile
        "paired_suffix_tiles": (M.shared_prefix(100, [333, 129, 400, 64, 260]), 8, 2),
    }


_DEEP_LENS = (29, 66, 2, 40, 17, 90, 5, 33, 64, 1, 70, 13)


def _offsets(lens):
    out = [0]
    for n in lens:
        out.append(out[-1] + n)
    return tuple(out)


CASES = ["shared_prefix_gqa4", "no_prefix", "tile_aligned", "mha", "gqa2", "gqa3", "depth3_tree",
         "unused_node", "empty_leaf", "deep_chain_one_run", "deep_run_list", "paired_suffix_tiles"]
KEY_RUNS = {"deep_chain_one_run": 1, "deep_run_list": 12}   # plan header word 29: most runs of a leaf


def _run(meta, q, k, v, pk, pv, dout, scale):
    from bridge_amd import TPRPrefixAttention
    tensors = [t.clone().requires_grad_(True) for t in (q, k, v, pk, pv)]
    out, lse = TPRPrefixAttention.apply(*tensors, meta, scale)
    out.backward(dout)
    torch.cuda.synchronize()
    return out.detach(), lse.detach(), [t.grad for t in tensors]


def _report(name, out, lse, grads, ref):
    ro, rl, rg = ref
    lines = [f"[{name}] out max_abs={max_abs(out, ro):.3e} cos={cosine(out, ro):.6f} "
             f"lse max_abs={max_abs(lse, rl):.3e}"]
    for label, g, r in zip(("dq", "dk", "dv", "dpk", "dpv"), grads, rg):
        lines.append(f"  {label}: cos={cosine(g, r):.6f} rel_l2={rel_l2(g, r):.3e} max_abs={max_abs(g, r):.3e}")
    print("\n".join(lines), flush=True)


@pytest.mark.parametrize("name", CASES)
def test_mfma_bf16_matches_oracle(name, cuda_device):
    meta, hq, hkv = _meta_cases()[name]
    d = 128
    scale = 1.0 / math.sqrt(d)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=1234, device=cuda_device)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device)
    assert plan.path == "mfma"
    if name in KEY_RUNS:
        assert int(plan.host[29]) == KEY_RUNS[name]
    out, lse, grads = _run(meta, q, k, v, pk, pv, dout, scale)
    ref = oracle(meta, q, k, v, pk, pv, dout, scale)
    _report(name, out, lse, grads, ref)
    ro, rl, rg = ref
    assert max_abs(out, ro) <= BF16_FWD_MAX_ABS
    assert cosine(out, ro) >= BF16_FWD_COS
    assert max_abs(lse, rl) <= 1e-3
    for g, r in zip(grads, rg):
        assert cosine(g, r) >= BF16_GRAD_COS
    for g, r in zip(grads[3:], rg[3:]):
        assert rel_l2(g, r) <= BF16_PREFIX_GRAD_REL_L2
    if name == "unused_node":
        assert torch.count_nonzero(grads[3][10:]) == 0 and torch.count_nonzero(grads[4][10:]) == 0
    # every 128-key dK/dV tile of every leaf on its own: a tile written by the
    # wrong item, or not at all, hides in a whole-tensor cosine but has a
    # relative error near 1 (the bound leaves room for a tile of one key,
    # whose few dS values may cancel)
    for s, (a, b) in enumerate(zip(meta.cu_seqlens_q[:-1], meta.cu_seqlens_q[1:])):
        for k0 in range(a, b, 128):
            for g, r in zip(grads[1:3], rg[1:3]):
                assert rel_l2(g[k0:min(b, k0 + 128)], r[k0:min(b, k0 + 128)]) <= 0.1, (s, k0 - a)


def test_fp32_plumbing_config_matches_oracle(cuda_device):
    """P=512, 2 sibling suffixes of 512, 4 heads MHA, D=64, fp32 (tolerance 1e-4)."""
    from bridge_amd import TPRPrefixMeta
    meta = TPRPrefixMeta.shared_prefix(512, [512, 512])
    hq = hkv = 4
    d = 64
    scale = 1.0 / math.sqrt(d)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.float32, seed=7, device=cuda_device)
    assert meta.plan(hq, hkv, d, torch.float32, cuda_device).path == "simt"
    out, lse, grads = _run(meta, q, k, v, pk, pv, dout, scale)
    ref = oracle(meta, q, k, v, pk, pv, dout, scale)
    _report("fp32_config1", out, lse, grads, ref)
    ro, rl, rg = ref
    assert max_abs(out, ro) <= FP32_TOL
    assert max_abs(lse, rl) <= FP32_TOL
    for g, r in zip(grads, rg):
        assert max_abs(g, r) <= FP32_TOL


def _simt_cases():
    from bridge_amd import TPRPrefixMeta as M
    tree = _meta_cases()["depth3_tree"][0]
    return {
        # name: (meta, hq, hkv, head_dim, dtype)
        "bf16_d64": (M.shared_prefix(100, [70, 40]), 8, 2, 64, torch.bfloat16),
        "bf16_d96": (M.shared_prefix(77, [50, 33]), 6, 2, 96, torch.bfloat16),
        # the full-attention layers of the reference's Qwen3.5 hybrid test model:
        # 8 query heads, 2 KV heads, head_dim 256
        "bf16_d256_qwen35": (M.shared_prefix(150, [90, 61]), 8, 2, 256, torch.bfloat16),
        "bf16_d200_tree": (tree, 4, 1, 200, torch.bfloat16),
        "fp32_d128_tree": (tree, 8, 2, 128, torch.float32),
        "fp32_d256": (M.shared_prefix(64, [50, 17]), 4, 2, 256, torch.float32),
        "fp32_deep_run_list": (_meta_cases()["deep_run_list"][0], 8, 2, 64, torch.float32),
        "bf16_d256_empty_leaf": (M.shared_prefix(50, [0, 60, 0]), 4, 1, 256, torch.bfloat16),
    }


@pytest.mark.parametrize("name", ["bf16_d64", "bf16_d96", "bf16_d256_qwen35", "bf16_d200_tree",
                                  "fp32_d128_tree", "fp32_d256", "fp32_deep_run_list", "bf16_d256_empty_leaf"])
def test_simt_matches_oracle(name, cuda_device):
    meta, hq, hkv, d, dtype = _simt_cases()[name]
    scale = 1.0 / math.sqrt(d)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, dtype, seed=3, device=cuda_device)
    # bf16 at head_dim 64 and 256 runs on the 16-wide MFMA kernels, the rest on SIMT
    plan = meta.plan(hq, hkv, d, dtype, cuda_device)
    if dtype == torch.bfloat16 and d in (64, 256):
        assert plan.path == "mfma" and plan.mfma_shape == "16x16x32"
    else:
        assert plan.path == "simt" and plan.mfma_shape is None
    out, lse, grads = _run(meta, q, k, v, pk, pv, dout, scale)
    ref = oracle(meta, q, k, v, pk, pv, dout, scale)
    _report(f"{plan.path}{plan.mfma_shape or ''}_{name}", out, lse, grads, ref)
    ro, rl, rg = ref
    if dtype == torch.float32:
        assert max_abs(out, ro) <= FP32_TOL and max_abs(lse, rl) <= FP32_TOL
        for g, r in zip(grads, rg):
            assert max_abs(g, r) <= FP32_TOL
        return
    assert max_abs(out, ro) <= BF16_FWD_MAX_ABS and cosine(out, ro) >= BF16_FWD_COS
    assert max_abs(lse, rl) <= 1e-3
    for g, r in zip(grads, rg):
        assert cosine(g, r) >= BF16_GRAD_COS
    for g, r in zip(grads[3:], rg[3:]):
        assert rel_l2(g, r) <= BF16_PREFIX_GRAD_REL_L2


def test_mfma_is_deterministic(cuda_device):
    meta, hq, hkv = _meta_cases()["depth3_tree"]
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, 128, torch.bfloat16, seed=99, device=cuda_device)
    first = _run(meta, q, k, v, pk, pv, dout, None)
    second = _run(meta, q, k, v, pk, pv, dout, None)
    assert torch.equal(first[0], second[0]) and torch.equal(first[1], second[1])
    for a, b in zip(first[2], second[2]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("d", [128, 256])  # 256: the reference's Qwen3.5 full-attention head size
def test_rectangular_shim_matches_reference_oracle(d, cuda_device):
    from bridge_amd import rectangular_causal_attention
    from oracle.tpr_oracle import prefix_attention
    gen = torch.Generator().manual_seed(44)
    sq, skv, hq, hkv = 40, 100, 8, 2
    q = torch.randn(sq, 1, hq, d, generator=gen).bfloat16()
    k = torch.randn(skv, 1, hkv, d, generator=gen).bfloat16()
    v = torch.randn(skv, 1, hkv, d, generator=gen).bfloat16()
    g = torch.randn(sq, 1, hq * d, generator=gen).bfloat16()
    qd, kd, vd = (t.to(cuda_device).requires_grad_(True) for t in (q, k, v))
    out = rectangular_causal_attention(qd, kd, vd)
    assert out.shape == (sq, 1, hq * d) and out.dtype == torch.bfloat16
    out.backward(g.to(cuda_device))
    qc, kc, vc = (t.double().requires_grad_(True) for t in (q, k, v))
    p = skv - sq
    ref = prefix_attention(qc, kc[p:], vc[p:], kc[:p], vc[:p], None)
    ref.backward(g.double())
    assert max_abs(out, ref) <= BF16_FWD_MAX_ABS and cosine(out, ref) >= BF16_FWD_COS
    for mine, theirs in ((qd.grad, qc.grad), (kd.grad, kc.grad), (vd.grad, vc.grad)):
        assert cosine(mine, theirs) >= BF16_GRAD_COS


@pytest.mark.parametrize("name,prefix,suffixes,hq,hkv", [
    ("split_prefix_tiles", 300, [4100, 4100, 100, 4200], 8, 2),
    ("split_suffix_tile", 64, [16500], 4, 1),
])
def test_mfma_split_tiles_match_oracle(name, prefix, suffixes, hq, hkv, cuda_device):
    """dK/dV tiles whose query range is split into fp32 partials + ordered reduction."""
    from bridge_amd import TPRPrefixMeta
    meta = TPRPrefixMeta.shared_prefix(prefix, suffixes)
    d = 128
    scale = 1.0 / math.sqrt(d)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device)
    assert plan.path == "mfma" and plan.workspace_bytes > 0
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=5, device=cuda_device)
    out, lse, grads = _run(meta, q, k, v, pk, pv, dout, scale)
    # larger shapes: the oracle runs in fp32 on the GPU
    ref = oracle(meta, q, k, v, pk, pv, dout, scale, compute_dtype=torch.float32, device=cuda_device)
    _report(name, out, lse, grads, ref)
    ro, rl, rg = ref
    assert max_abs(out, ro) <= BF16_FWD_MAX_ABS and cosine(out, ro) >= BF16_FWD_COS
    for g, r in zip(grads, rg):
        assert cosine(g, r) >= BF16_GRAD_COS
    for g, r in zip(grads[3:], rg[3:]):
        assert rel_l2(g, r) <= BF16_PREFIX_GRAD_REL_L2
