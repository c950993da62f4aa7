"""The allocation-free backward entry point, tpr_attn_bwd_noalloc, through the C
ABI: its outputs must equal tpr_attn_bwd's (with a caller-allocated
workspace) bit for bit -- the same kernels run, only the workspace differs --
on two calls in a row, the second smaller, so the static scratch is reused
with the first call's contents still in it."""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from bridge_amd import TPRPrefixMeta, _lib
from bridge_amd.prefix_attention import prefix_attention_forward

from _helpers import make_inputs


def _ptr(t):
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _bwd_params(plan, scale, tensors, outs, ws):
    q, k, v, pk, pv, out, lse, dout = tensors
    delta, dq, dk, dv, dpk, dpv = outs
    return _lib.TprBwdParams(
        _lib.ABI_VERSION, 0, scale, 0.0, plan.host.data_ptr(), plan.device.data_ptr(),
        _ptr(q), _ptr(k), _ptr(v), _ptr(pk), _ptr(pv), _ptr(out), _ptr(dout), _ptr(lse), _ptr(delta),
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dpk), _ptr(dpv), _ptr(ws), 0 if ws is None else ws.numel())


def _fresh_outputs(q, k, v, pk, pv, lse):
    # NaN-filled, so an element a call failed to write cannot match
    return [torch.full_like(t, float("nan")) for t in (lse, q, k, v, pk, pv)]


def test_noalloc_rejects_a_plan_beyond_its_scratch_before_any_launch():
    """A plan needing more workspace than the static scratch is refused on the
    host (no device call is made, so this runs without a GPU)."""
    lib = _lib.load()
    cap = lib.tpr_attn_bwd_noalloc_max_workspace_bytes()
    assert cap == 64 << 20
    gen = torch.Generator(device="cpu").manual_seed(0)
    ragged = torch.randint(256, 8193, (16,), generator=gen).tolist()
    plan = TPRPrefixMeta.shared_prefix(8192, ragged).plan(32, 8, 128, torch.bfloat16, torch.device("cpu"))
    assert plan.workspace_bytes > cap
    b = _lib.TprBwdParams()
    b.abi_version = _lib.ABI_VERSION
    b.softmax_scale = 0.1
    b.plan_host = b.plan_device = plan.host.data_ptr()
    assert lib.tpr_attn_bwd_noalloc(ctypes.byref(b), None) == _lib.TPR_ERR_UNSUPPORTED
    assert b"static scratch" in lib.tpr_attn_last_error()


@pytest.mark.gpu
def test_noalloc_backward_equals_the_workspace_backward(cuda_device):
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda_device).cuda_stream)
    # first: split prefix tiles (fp32 partial slots + ordered reduction in the
    # workspace), dQ recomputed (its dS store would not fit the scratch);
    # second, smaller: stat rows and a dS store, in the same scratch
    cases = [(TPRPrefixMeta.shared_prefix(300, [4100, 4100, 100, 4200]), 8, 2, True),
             (TPRPrefixMeta.shared_prefix(200, [100, 37]), 8, 2, False)]
    for i, (meta, hq, hkv, recompute) in enumerate(cases):
        d = 128
        scale = 1.0 / math.sqrt(d)
        plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device, recompute_dq=recompute)
        assert plan.dq_from_ds != recompute
        print(f"[noalloc call {i}] tq={meta.total_q} tp={meta.total_prefix} hq={hq} hkv={hkv} "
              f"workspace_bytes={plan.workspace_bytes} slots={int(plan.host[25])} dS store={plan.dq_from_ds}",
              flush=True)
        assert plan.path == "mfma" and 0 < plan.workspace_bytes <= lib.tpr_attn_bwd_noalloc_max_workspace_bytes()
        if i == 0:
            assert int(plan.host[25]) > 0  # the first call uses partial slots
        q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=31 + i, device=cuda_device)
        out, lse = prefix_attention_forward(q, k, v, pk, pv, meta, scale)
        tensors = (q, k, v, pk, pv, out, lse, dout)

        ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=cuda_device)
        ref = _fresh_outputs(q, k, v, pk, pv, lse)
        p = _bwd_params(plan, scale, tensors, ref, ws)
        _lib.check(lib.tpr_attn_bwd(ctypes.byref(p), stream), "tpr_attn_bwd")

        mine = _fresh_outputs(q, k, v, pk, pv, lse)
        p = _bwd_params(plan, scale, tensors, mine, None)   # workspace fields are ignored
        _lib.check(lib.tpr_attn_bwd_noalloc(ctypes.byref(p), stream), "tpr_attn_bwd_noalloc")
        torch.cuda.synchronize()
        for label, a, b in zip(("delta", "dq", "dk", "dv", "dprefix_k", "dprefix_v"), mine, ref):
            assert torch.isfinite(b.float()).all(), label
            assert torch.equal(a, b), f"call {i}: {label} differs"
        print(f"  bitwise equal: delta dq dk dv dprefix_k dprefix_v", flush=True)


@pytest.mark.gpu
def test_noalloc_backward_replays_from_a_captured_graph(cuda_device):
    """tpr_attn_bwd_noalloc captured into a torch.cuda.CUDAGraph after one call
    outside capture (which looks up the scratch address): every replay, with
    eager work and synchronisation between replays, equals tpr_attn_bwd
    bitwise. The backward's kernels fill every workspace element they read,
    so no memset node is needed."""
    lib = _lib.load()
    meta, hq, hkv, d = TPRPrefixMeta.shared_prefix(200, [100, 37]), 8, 2, 128
    scale = 1.0 / math.sqrt(d)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, cuda_device)
    assert plan.dq_from_ds and plan.workspace_bytes <= lib.tpr_attn_bwd_noalloc_max_workspace_bytes()
    print(f"[noalloc graph] tq={meta.total_q} tp={meta.total_prefix} workspace_bytes={plan.workspace_bytes}",
          flush=True)
    q, k, v, pk, pv, dout = make_inputs(meta, hq, hkv, d, torch.bfloat16, seed=41, device=cuda_device)
    out, lse = prefix_attention_forward(q, k, v, pk, pv, meta, scale)
    tensors = (q, k, v, pk, pv, out, lse, dout)
    ws = torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=cuda_device)
    ref = _fresh_outputs(q, k, v, pk, pv, lse)
    p_ref = _bwd_params(plan, scale, tensors, ref, ws)
    _lib.check(lib.tpr_attn_bwd(ctypes.byref(p_ref), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
               "tpr_attn_bwd")
    mine = _fresh_outputs(q, k, v, pk, pv, lse)
    p = _bwd_params(plan, scale, tensors, mine, None)
    _lib.check(lib.tpr_attn_bwd_noalloc(ctypes.byref(p), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
               "tpr_attn_bwd_noalloc (outside capture)")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(lib.tpr_attn_bwd_noalloc(ctypes.byref(p),
                                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
                   "tpr_attn_bwd_noalloc (captured)")
    for rep in range(3):
        for t in mine:
            t.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for label, a, b in zip(("delta", "dq", "dk", "dv", "dprefix_k", "dprefix_v"), mine, ref):
            assert torch.equal(a, b), f"replay {rep}: {label} differs"
        print(f"  replay {rep}: bitwise equal", flush=True)
