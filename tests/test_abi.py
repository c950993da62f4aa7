"""CPU checks of the C ABI: libtpr_attn.so loads, exports every function
include/tpr_attn.h declares, the ctypes mirrors match the C struct layouts,
and argument errors come back as status codes with messages (host code only,
no GPU work is launched)."""

from __future__ import annotations

import ctypes
import os
import re
import shutil
import subprocess

import pytest

from bridge_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tpr_attn.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(tpr_attn_\w+)\s*\(", text, re.M)))


def test_library_loads_and_reports_abi_version():
    lib = _lib.load()
    assert lib.tpr_attn_abi_version() == _lib.ABI_VERSION == 6


def test_every_declared_symbol_is_exported_and_bound():
    declared = _declared_functions()
    assert declared == sorted(_lib.EXPORTED_SYMBOLS)
    lib = ctypes.CDLL(_lib.library_path())
    for name in declared:
        assert hasattr(lib, name), name


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_ctypes_structs_match_c_layout(tmp_path):
    structs = {"TprTreeDesc": _lib.TprTreeDesc, "TprFwdParams": _lib.TprFwdParams,
               "TprBwdParams": _lib.TprBwdParams}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for sname, cls in structs.items():
        lines.append(f'  printf("{sname} size %zu\\n", sizeof({sname}));')
        for fname, _ in cls._fields_:
            lines.append(f'  printf("{sname}.{fname} %zu\\n", offsetof({sname}, {fname}));')
    lines.append("  return 0; }")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-o", str(exe), str(src)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], check=True, stdout=subprocess.PIPE,
                                                                 text=True).stdout.splitlines())
    for sname, cls in structs.items():
        assert int(got[f"{sname} size"]) == ctypes.sizeof(cls), sname
        for fname, _ in cls._fields_:
            assert int(got[f"{sname}.{fname}"]) == getattr(cls, fname).offset, f"{sname}.{fname}"


def test_null_params_and_bad_version_fail_with_messages():
    lib = _lib.load()
    assert lib.tpr_attn_fwd(None, None) == _lib.TPR_ERR_INVALID_ARGUMENT
    assert b"must not be NULL" in lib.tpr_attn_last_error()
    p = _lib.TprFwdParams()
    p.abi_version = 99
    assert lib.tpr_attn_fwd(ctypes.byref(p), None) == _lib.TPR_ERR_INVALID_ARGUMENT
    assert b"abi_version" in lib.tpr_attn_last_error()
    b = _lib.TprBwdParams()
    b.abi_version = _lib.ABI_VERSION
    assert lib.tpr_attn_bwd(ctypes.byref(b), None) == _lib.TPR_ERR_INVALID_ARGUMENT
    assert b"plan" in lib.tpr_attn_last_error()
    assert lib.tpr_attn_bwd_phases(ctypes.byref(b), 32, None) == _lib.TPR_ERR_INVALID_ARGUMENT
    assert b"phases" in lib.tpr_attn_last_error()


def test_bad_scale_is_rejected_before_any_launch():
    import torch

    from bridge_amd import TPRPrefixMeta
    lib = _lib.load()
    plan = TPRPrefixMeta.shared_prefix(8, [4]).plan(4, 2, 128, torch.bfloat16, torch.device("cpu"))
    for scale in (0.0, -1.0, float("inf"), float("nan")):
        p = _lib.TprFwdParams(_lib.ABI_VERSION, 0, scale, 0.0, plan.host.data_ptr(), plan.host.data_ptr())
        assert lib.tpr_attn_fwd(ctypes.byref(p), None) == _lib.TPR_ERR_INVALID_ARGUMENT
        assert b"softmax_scale" in lib.tpr_attn_last_error()


def test_missing_tensor_pointer_is_rejected():
    import torch

    from bridge_amd import TPRPrefixMeta
    lib = _lib.load()
    plan = TPRPrefixMeta.shared_prefix(8, [4]).plan(4, 2, 128, torch.bfloat16, torch.device("cpu"))
    p = _lib.TprFwdParams(_lib.ABI_VERSION, 0, 0.1, 0.0, plan.host.data_ptr(), plan.host.data_ptr())
    assert lib.tpr_attn_fwd(ctypes.byref(p), None) == _lib.TPR_ERR_INVALID_ARGUMENT
    assert b"q must not be NULL" in lib.tpr_attn_last_error()


def test_plan_capacity_and_workspace_queries():
    import torch

    from bridge_amd import TPRPrefixMeta
    plan = TPRPrefixMeta.shared_prefix(4096, [4096] * 4).plan(32, 8, 128, torch.bfloat16, torch.device("cpu"))
    lib = _lib.load()
    assert lib.tpr_attn_bwd_workspace_bytes(ctypes.c_void_p(plan.host.data_ptr())) == plan.workspace_bytes > 0
    assert lib.tpr_attn_bwd_workspace_bytes(None) == 0


def test_misaligned_workspace_is_rejected_before_any_launch():
    """The MFMA backward needs a 256-byte aligned workspace; the check runs on
    the host before anything is enqueued (the pointers below are never
    dereferenced)."""
    import torch

    from bridge_amd import TPRPrefixMeta
    lib = _lib.load()
    plan = TPRPrefixMeta.shared_prefix(64, [64]).plan(4, 2, 128, torch.bfloat16, torch.device("cpu"))
    need = plan.workspace_bytes
    assert need > 0
    b = _lib.TprBwdParams()
    b.abi_version = _lib.ABI_VERSION
    b.softmax_scale = 0.1
    b.plan_host = b.plan_device = plan.host.data_ptr()
    fake = 1 << 20
    for name in ("q", "k", "v", "prefix_k", "prefix_v", "out", "dout", "lse", "delta", "dq", "dk", "dv",
                 "dprefix_k", "dprefix_v"):
        setattr(b, name, fake)
        fake += 1 << 20
    b.workspace = fake + 16
    b.workspace_bytes = need + 256
    assert lib.tpr_attn_bwd(ctypes.byref(b), None) == _lib.TPR_ERR_INVALID_ARGUMENT
    assert b"256-byte aligned" in lib.tpr_attn_last_error()


def _fake_fwd_params(plan):
    p = _lib.TprFwdParams(_lib.ABI_VERSION, 0, 0.1, 0.0, plan.host.data_ptr(), plan.host.data_ptr())
    fake = 1 << 20
    for name in ("q", "k", "v", "prefix_k", "prefix_v", "out", "lse"):
        setattr(p, name, fake)
        fake += 1 << 20
    return p


def test_bad_row_strides_are_rejected_before_any_launch():
    """q/k/v row strides: 0 (packed) or at least the packed stride, rows a
    multiple of 16 bytes, at most 32 MiB. The checks run on the host before
    anything is enqueued (the pointers below are never dereferenced)."""
    import torch

    from bridge_amd import TPRPrefixMeta
    lib = _lib.load()
    for dtype, d, elem in ((torch.bfloat16, 128, 2), (torch.bfloat16, 64, 2), (torch.float32, 96, 4)):
        hq, hkv = 4, 2
        plan = TPRPrefixMeta.shared_prefix(8, [4]).plan(hq, hkv, d, dtype, torch.device("cpu"))
        cases = [("q_row_stride", hq * d - 8, "at least"), ("k_row_stride", hkv * d - 8, "at least"),
                 ("v_row_stride", hkv * d + 8 // elem + 1, "16 bytes"), ("q_row_stride", (1 << 25) // elem + 8,
                                                                        "32 MiB")]
        for field, value, words in cases:
            p = _fake_fwd_params(plan)
            setattr(p, field, value)
            assert lib.tpr_attn_fwd(ctypes.byref(p), None) != 0, (dtype, field, value)
            msg = lib.tpr_attn_last_error()
            assert field.encode() in msg and words.encode() in msg, msg
        b = _lib.TprBwdParams()
        b.abi_version = _lib.ABI_VERSION
        b.softmax_scale = 0.1
        b.plan_host = b.plan_device = plan.host.data_ptr()
        b.k_row_stride = hkv * d - 8
        assert lib.tpr_attn_bwd(ctypes.byref(b), None) != 0
        assert b"k_row_stride" in lib.tpr_attn_last_error() or b"must not be NULL" in lib.tpr_attn_last_error()


def test_key_mask_rules_are_checked_before_any_launch():
    """A key mask needs a TPR_PLAN_MASKED plan, such a plan needs a mask, and
    the mask rows must hold the longest key sequence (prefix 8 + suffix 4 =
    12 bytes here). The checks run on the host before anything is enqueued
    (the pointers below are never dereferenced)."""
    import torch

    from bridge_amd import TPRPrefixMeta
    lib = _lib.load()
    meta = TPRPrefixMeta.shared_prefix(8, [4])
    plain = meta.plan(4, 2, 128, torch.bfloat16, torch.device("cpu"))
    masked = meta.plan(4, 2, 128, torch.bfloat16, torch.device("cpu"), masked=True)
    assert not plain.masked and masked.masked and masked.path == "simt" and masked.workspace_bytes == 0
    cases = [(plain, 1 << 30, 0, b"TPR_PLAN_MASKED"), (masked, None, 0, b"must not be NULL"),
             (masked, 1 << 30, 11, b"at least 12")]
    for plan, mask, stride, words in cases:
        p = _fake_fwd_params(plan)
        p.mask, p.mask_row_stride = mask, stride
        assert lib.tpr_attn_fwd(ctypes.byref(p), None) == _lib.TPR_ERR_INVALID_ARGUMENT
        assert words in lib.tpr_attn_last_error(), (words, lib.tpr_attn_last_error())
        b = _lib.TprBwdParams()
        b.abi_version = _lib.ABI_VERSION
        b.softmax_scale = 0.1
        b.plan_host = b.plan_device = plan.host.data_ptr()
        fake = 1 << 20
        for name in ("q", "k", "v", "prefix_k", "prefix_v", "out", "dout", "lse", "delta", "dq", "dk", "dv",
                     "dprefix_k", "dprefix_v", "workspace"):
            setattr(b, name, fake)
            fake += 1 << 20
        b.workspace_bytes = plan.workspace_bytes
        b.mask, b.mask_row_stride = mask, stride
        assert lib.tpr_attn_bwd(ctypes.byref(b), None) == _lib.TPR_ERR_INVALID_ARGUMENT
        assert words in lib.tpr_attn_last_error(), (words, lib.tpr_attn_last_error())


def test_fused_projection_views_pass_through_with_their_row_stride():
    """Slices of one [tokens, (Hq + 2 Hkv) * D] projection reach the kernels
    as views with the projection's row stride; layouts the kernels cannot read
    (head stride not D, misaligned rows) are copied packed."""
    import torch

    from bridge_amd.prefix_attention import _inputs, _row_stride, _rows
    t, hq, hkv, d = 10, 4, 2, 64
    qkv = torch.zeros(t, (hq + 2 * hkv) * d, dtype=torch.bfloat16)
    q = qkv[:, :hq * d].view(t, hq, d)
    k = qkv[:, hq * d:(hq + hkv) * d].view(t, hkv, d)
    v = qkv[:, (hq + hkv) * d:].view(t, hkv, d)
    pk = torch.zeros(3, hkv, d, dtype=torch.bfloat16)
    q2, k2, v2, pk2, pv2 = _inputs(q, k, v, pk, pk)
    for a, b in ((q, q2), (k, k2), (v, v2)):
        assert b.data_ptr() == a.data_ptr() and _row_stride(b) == (hq + 2 * hkv) * d
    assert _row_stride(pk2) == 0
    assert _row_stride(torch.zeros(t, hq, d)) == 0
    heads_strided = torch.zeros(t, hq, 2 * d, dtype=torch.bfloat16)[:, :, :d]
    assert _rows(heads_strided).is_contiguous()
    odd_rows = torch.zeros(t * (hq * d + 4), dtype=torch.bfloat16).as_strided((t, hq, d), (hq * d + 4, d, 1))
    assert _rows(odd_rows).is_contiguous()
    head_major = torch.zeros(hq, t, d, dtype=torch.bfloat16).transpose(0, 1)
    assert _rows(head_major).is_contiguous()

