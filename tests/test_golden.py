"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every committed fixture.
GPU: the HIP kernels match the fixtures to the bf16 / fp32 tolerances."""

from __future__ import annotations

import glob
import os

import numpy as np
import pytest
import torch

from _helpers import BF16_FWD_COS, BF16_FWD_MAX_ABS, BF16_GRAD_COS, FP32_TOL, cosine, max_abs
from oracle.tpr_oracle import Tree, tree_backward, tree_forward

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))
NAMES = ("q", "k", "v", "prefix_k", "prefix_v", "dout")
OUTS = ("out", "lse", "dq", "dk", "dv", "dprefix_k", "dprefix_v")


def _load(path):
    z = np.load(path)  # allow_pickle defaults to False
    bf16 = "q_bf16_bits" in z.files
    tensors = {}
    for n in NAMES:
        if bf16:
            tensors[n] = torch.from_numpy(z[n + "_bf16_bits"].copy()).view(torch.bfloat16)
        else:
            tensors[n] = torch.from_numpy(z[n].copy())
    tree = Tree(z["cu_seqlens_q"].tolist(), z["node_offsets"].tolist(), z["leaf_ancestors"].tolist())
    expected = {k: torch.from_numpy(z[k].copy()) for k in OUTS}
    return tensors, tree, float(z["scale"][0]), expected, bf16, z["heads"].tolist()


def test_golden_fixtures_exist():
    assert len(GOLDEN) >= 2


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_reproduces_golden(path):
    tensors, tree, scale, expected, _, _ = _load(path)
    x = [tensors[n].double() for n in NAMES[:5]]
    out, lse = tree_forward(*x, tree, scale)
    grads = tree_backward(*x, tree, tensors["dout"].double(), scale, out=out, lse=lse)
    for key, val in zip(OUTS, (out, lse, *grads)):
        torch.testing.assert_close(val.float(), expected[key], atol=1e-6, rtol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_kernels_match_golden(path, cuda_device):
    from bridge_amd import TPRPrefixAttention, TPRPrefixMeta
    tensors, tree, scale, expected, bf16, _ = _load(path)
    meta = TPRPrefixMeta(tuple(tree.cu_seqlens_q), tuple(tree.node_offsets),
                         tuple(tuple(a) for a in tree.ancestors))
    dev = {n: t.to(cuda_device) for n, t in tensors.items()}
    inputs = [dev[n].clone().requires_grad_(True) for n in NAMES[:5]]
    out, lse = TPRPrefixAttention.apply(*inputs, meta, scale)
    out.backward(dev["dout"])
    torch.cuda.synchronize()
    got = {"out": out, "lse": lse, **{k: t.grad for k, t in zip(OUTS[2:], inputs)}}
    for key in OUTS:
        g, e = got[key].detach().float().cpu(), expected[key]
        if bf16:
            if key == "out":
                assert max_abs(g, e) <= BF16_FWD_MAX_ABS and cosine(g, e) >= BF16_FWD_COS
            elif key == "lse":
                assert max_abs(g, e) <= 1e-3
            else:
                assert cosine(g, e) >= BF16_GRAD_COS, key
        else:
            assert max_abs(g, e) <= FP32_TOL, key
