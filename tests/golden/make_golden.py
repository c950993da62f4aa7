"""Write the golden fixtures under tests/golden/ from the CPU oracle (fp64).

Each fixture holds seeded inputs (stored exactly: bf16 bit patterns or fp32)
and the oracle's fp64 outputs: out, lse, dq, dk, dv, dprefix_k, dprefix_v,
plus the packed tree metadata. Expected outputs are the fp64 results
rounded to fp32. Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle.tpr_oracle import Tree, tree_backward, tree_forward  # noqa: E402

CASES = {
    # depth-3 tree: root node 0, branch nodes 1 and 2, two leaves under each branch
    "tree_depth3_bf16_d128": dict(cu=[0, 17, 50, 70, 100], nodes=[0, 70, 100, 140],
                                  anc=[[0, 1], [0, 1], [0, 2], [0, 2]], hq=4, hkv=1, d=128,
                                  dtype="bf16", scale=None, seed=101),
    # two siblings under one shared prefix, GQA 2, ragged, fp32
    "siblings_fp32_d64": dict(cu=[0, 40, 73], nodes=[0, 90], anc=[[0], [0]], hq=4, hkv=2, d=64,
                              dtype="fp32", scale=0.11, seed=102),
}


def make(name, spec):
    gen = torch.Generator().manual_seed(spec["seed"])
    tq, tp = spec["cu"][-1], spec["nodes"][-1]
    hq, hkv, d = spec["hq"], spec["hkv"], spec["d"]
    shapes = {"q": (tq, hq, d), "k": (tq, hkv, d), "v": (tq, hkv, d), "prefix_k": (tp, hkv, d),
              "prefix_v": (tp, hkv, d), "dout": (tq, hq, d)}
    tensors = {}
    for key, shape in shapes.items():
        t = torch.randn(shape, generator=gen)
        tensors[key] = t.bfloat16() if spec["dtype"] == "bf16" else t.float()
    tree = Tree(spec["cu"], spec["nodes"], spec["anc"])
    x = [tensors[n].double() for n in ("q", "k", "v", "prefix_k", "prefix_v")]
    out, lse = tree_forward(*x, tree, spec["scale"])
    grads = tree_backward(*x, tree, tensors["dout"].double(), spec["scale"], out=out, lse=lse)
    arrays = {
        "cu_seqlens_q": np.array(spec["cu"], dtype=np.int32),
        "node_offsets": np.array(spec["nodes"], dtype=np.int32),
        "leaf_ancestors": np.array(spec["anc"], dtype=np.int32),
        "heads": np.array([hq, hkv, d], dtype=np.int32),
        "scale": np.array([spec["scale"] if spec["scale"] is not None else d ** -0.5], dtype=np.float64),
        # expected outputs: fp64 oracle results stored as fp32
        "out": out.float().numpy(), "lse": lse.float().numpy(),
    }
    for key, g in zip(("dq", "dk", "dv", "dprefix_k", "dprefix_v"), grads):
        arrays[key] = g.float().numpy()
    for key, t in tensors.items():
        if spec["dtype"] == "bf16":
            arrays[key + "_bf16_bits"] = t.view(torch.int16).numpy()
        else:
            arrays[key] = t.numpy()
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    print(name, {k: v.shape for k, v in arrays.items()})


if __name__ == "__main__":
    for case, spec in CASES.items():
        make(case, spec)
