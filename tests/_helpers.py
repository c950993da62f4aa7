"""Shared helpers for the parity tests: seeded inputs, the oracle call, metrics."""

from __future__ import annotations

import torch

from oracle.tpr_oracle import Tree, tree_backward, tree_forward

# parity tolerances: bf16 kernels against the fp32 oracle
BF16_FWD_MAX_ABS = 2e-2
BF16_FWD_COS = 0.9999
BF16_GRAD_COS = 0.999
BF16_PREFIX_GRAD_REL_L2 = 1e-2
FP32_TOL = 1e-4


def tree_of(meta) -> Tree:
    return Tree(list(meta.cu_seqlens_q), list(meta.node_offsets), [list(a) for a in meta.leaf_ancestors])


def make_inputs(meta, hq, hkv, d, dtype, seed, device):
    """N(0,1) q, k, v, prefix_k, prefix_v, dout from a CPU generator, cast, then moved."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    tq, tp = meta.total_q, meta.total_prefix
    shapes = [(tq, hq, d), (tq, hkv, d), (tq, hkv, d), (tp, hkv, d), (tp, hkv, d), (tq, hq, d)]
    return [torch.randn(s, generator=gen).to(dtype).to(device) for s in shapes]


def oracle(meta, q, k, v, pk, pv, dout, scale, compute_dtype=torch.float64, device="cpu", mask=None):
    tree = tree_of(meta)
    args = [t.detach().to(device) for t in (q, k, v, pk, pv)]
    if mask is not None:
        mask = mask.to(device)
    out, lse = tree_forward(*args, tree, scale, compute_dtype=compute_dtype, mask=mask)
    grads = tree_backward(*args, tree, dout.detach().to(device), scale, compute_dtype=compute_dtype, out=out, lse=lse,
                          mask=mask)
    return out, lse, grads


def random_key_mask(tree, gen, hidden=0.4, empty_rows=()):
    """bool [Tq, L] (True = hidden) over each row's leaf key sequence: about
    ``hidden`` of the keys hidden at random -- so rows see later suffix keys
    too -- every row keeping at least one key except those in ``empty_rows``,
    which see none. L is the longest key sequence of any leaf."""
    lens = [len(tree.prefix_rows(s)) + tree.leaf_range(s)[1] - tree.leaf_range(s)[0]
            for s in range(tree.num_leaves)]
    mask = torch.rand(tree.cu_seqlens_q[-1], max(lens), generator=gen) < hidden
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        for r in range(a, b):
            mask[r, torch.randint(0, lens[s], (1,), generator=gen).item()] = False
    for r in empty_rows:
        mask[r] = True
    return mask


def max_abs(a, b) -> float:
    if a.numel() == 0:
        return 0.0
    return (a.double().cpu() - b.double().cpu()).abs().max().item()


def cosine(a, b) -> float:
    a = a.double().flatten().cpu()
    b = b.double().flatten().cpu()
    if a.numel() == 0:
        return 1.0
    na, nb = a.norm(), b.norm()
    if na == 0 and nb == 0:
        return 1.0
    return (a @ b / (na * nb).clamp_min(1e-300)).item()


def rel_l2(a, b) -> float:
    a = a.double().flatten().cpu()
    b = b.double().flatten().cpu()
    if b.norm() == 0:
        return a.norm().item()
    return ((a - b).norm() / b.norm()).item()
