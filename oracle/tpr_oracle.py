"""CPU oracle for prefix-reuse (TPR) attention -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the timed
CPU baseline). The product path (``bridge_amd``) never imports it and fails
loudly when its HIP library is missing.

It restates, in fresh code, the reference's fp32 math for the hot path:

* ``prefix_attention`` / ``fp32_reference`` -- the dense fp32 oracle of
  tests/models/mcore/tpr/parallel/_fa_fp32_reference.py:12-40
  (key j visible to query i iff j <= P + i; contiguous GQA query-head groups;
  default scale D**-0.5; gradients by autograd).
* ``block_reference`` -- block statistics of
  tests/models/mcore/tpr/parallel/_ring_merge_probe.py:9-29 (out, max, sum in
  the scaled-score domain; LSE = max + log(sum), natural log).
* ``merge_attention`` / ``finalize_attention_result`` -- the fp32 online
  softmax merge of verl/models/mcore/tpr/parallel/ring_attention.py:588-636,
  with statistics kept as [T, H] (one lane of the reference's [T, H, 8]).
* ``tree_forward`` / ``tree_backward`` -- the sibling/tree generalisation the
  kernel implements: every leaf attends to cat(ancestor node KV in root ->
  parent order, own suffix KV) (verl/models/mcore/tpr/kv_stack.py:139-154),
  and each node's gradient is the sum over its descendant leaves in leaf
  order (kv_stack.py:175-203 split per ancestor slice, prefix_state.py:546-573
  sibling accumulation; here the sum is kept in the compute dtype instead of
  the reference's bf16 ``add_``).
* ``tree_forward`` / ``tree_backward`` with ``mask`` -- the reference's
  custom-mask mode (rectangular_attention.py:112-122, sparse mode 0): a
  physical bool mask [Tq, L] (True = excluded; column c = key c of the
  row's leaf sequence cat(ancestors, suffix)) is the only visibility rule; a
  row that sees no key gets out 0, lse -inf and no gradient (the fully-masked
  padding row of equivalence/test_rectangular_attention_npu.py:149-284).
* ``tree_autograd`` -- the same tree computed the reference's way: one dense
  ``prefix_attention`` per leaf on freshly concatenated anchors, gradients by
  autograd, anchor gradients split per ancestor and summed in leaf order.

Parity pins (each is a test in tests/test_oracle.py):
  closed-form KAT of _fa_fp32_reference (tests/.../unit/test_fa_fp32_reference.py:40-50),
  fp64 per-query brute force (same file :9-37), block-statistics KATs
  (unit/test_ring_merge_probe.py:9-32), merge KATs
  (parallel/test_ring_cp_attention_contract.py:188-243), multi-level split and
  sibling sum invariants (unit/test_kv_stack.py:79-120), batched-tree ==
  sum of single-leaf runs (unit/test_segment_executor.py:291-325),
  torch scaled_dot_product_attention in fp64 with an explicit mask, and
  central finite differences of the explicit backward. The masked forms:
  scaled_dot_product_attention in fp64 (values and autograd gradients) with
  random masks that show later suffix keys, the causal mask giving the
  unmasked result, and the reference's padding equivalence (a masked padding
  row and column leave the logical rows' results unchanged, the padding
  gets zero gradient, a fully masked row zero output).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Sequence

import torch

__all__ = [
    "prefix_attention",
    "fp32_reference",
    "block_reference",
    "merge_attention",
    "finalize_attention_result",
    "Tree",
    "tree_forward",
    "tree_backward",
    "tree_autograd",
    "visible_pairs",
]


# --------------------------------------------------------------------------
# Single-sequence oracle (_fa_fp32_reference.py:12-40)
# --------------------------------------------------------------------------

def prefix_attention(q, k, v, pk, pv, scale):
    """Dense prefix + causal attention. [S,1,H,D] inputs -> [S,1,Hq*D].

    Follows _fa_fp32_reference.py:12-28: the key sequence is cat(pk, k); query
    i sees every prefix key and current keys j <= i; query head h uses KV head
    h // (Hq // Hkv).
    """
    if q.ndim != 4 or q.shape[1] != 1:
        raise ValueError("q must be [S, 1, Hq, D]")
    if k.shape != v.shape or pk.shape != pv.shape:
        raise ValueError("K/V and prefix K/V shapes must match")
    if k.shape[0] != q.shape[0] or k.shape[1:] != pk.shape[1:]:
        raise ValueError("suffix K/V length must equal Q length and share [1, Hkv, D] with the prefix")
    if q.shape[-1] != k.shape[-1] or q.shape[2] % k.shape[2] != 0:
        raise ValueError("head_dim mismatch or Hq not divisible by Hkv")
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    if not (math.isfinite(scale) and scale > 0):
        raise ValueError("scale must be finite and positive")
    group = q.shape[2] // k.shape[2]
    prefix_len, length = pk.shape[0], q.shape[0]
    keys = torch.cat((pk, k), 0)[:, 0].repeat_interleave(group, dim=1)      # [L, Hq, D]
    values = torch.cat((pv, v), 0)[:, 0].repeat_interleave(group, dim=1)
    qh = q[:, 0].transpose(0, 1)                                            # [Hq, S, D]
    scores = torch.matmul(qh, keys.permute(1, 2, 0).contiguous()) * scale   # [Hq, S, L]
    col = torch.arange(prefix_len + length, device=q.device)
    row = torch.arange(length, device=q.device)
    visible = col[None, :] <= prefix_len + row[:, None]
    probs = scores.masked_fill(~visible, float("-inf")).softmax(-1)
    out = torch.matmul(probs, values.transpose(0, 1).contiguous())          # [Hq, S, D]
    return out.transpose(0, 1).reshape(length, 1, -1)


def fp32_reference(entry, upstream):
    """fp32 output and autograd gradients, as _fa_fp32_reference.py:31-40."""
    names = ("q", "k", "v", "pk", "pv")
    with torch.enable_grad():
        inputs = {n: entry[n].detach().to("cpu", torch.float32).clone().requires_grad_(True) for n in names}
        output = prefix_attention(**inputs, scale=entry.get("scale"))
        grads = torch.autograd.grad(output, tuple(inputs.values()),
                                    grad_outputs=upstream.detach().cpu().float())
    return {"output": output.detach(), **{n: g.detach() for n, g in zip(names, grads)}}


# --------------------------------------------------------------------------
# Block statistics and merge (_ring_merge_probe.py:9-29, ring_attention.py:588-636)
# --------------------------------------------------------------------------

def block_reference(query, key, value, *, scale, causal, mask=None):
    """One attention block over TND tensors [T,H,D] -> (out [Tq,Hq,D], max [Tq,Hq], sum [Tq,Hq]).

    ``causal`` is right-down causal (query i sees key j iff
    j <= Tk - Tq + i); ``mask`` (bool [Tq,Tk], True = excluded) overrides it.
    Rows with no visible key are rejected, as in _ring_merge_probe.py:21-24.
    """
    q, k, v = (x.detach().float() for x in (query, key, value))
    group = q.shape[1] // k.shape[1]
    if group * k.shape[1] != q.shape[1]:
        raise ValueError("query heads must be a multiple of KV heads")
    k = k.repeat_interleave(group, dim=1)
    v = v.repeat_interleave(group, dim=1)
    tq, tk = q.shape[0], k.shape[0]
    scores = torch.matmul(q.transpose(0, 1), k.permute(1, 2, 0).contiguous()) * scale  # [H,Tq,Tk]
    excluded = torch.zeros(tq, tk, dtype=torch.bool, device=q.device)
    if mask is not None:
        excluded |= mask.to(q.device)
    elif causal:
        excluded |= torch.arange(tk, device=q.device)[None, :] > (tk - tq + torch.arange(tq, device=q.device)[:, None])
    if bool(excluded.all(-1).any()):
        raise ValueError("fully-masked query row in an attention block")
    scores = scores.masked_fill(excluded, float("-inf"))
    maximum = scores.amax(-1)                              # [H,Tq]
    weights = torch.exp(scores - maximum[..., None])
    total = weights.sum(-1)
    out = torch.matmul(weights / total[..., None], v.transpose(0, 1).contiguous())
    return out.transpose(0, 1).contiguous(), maximum.T.contiguous(), total.T.contiguous()


def merge_attention(previous, current):
    """fp32 online-softmax merge of two (out [T,H,D], max [T,H], sum [T,H]) blocks.

    ring_attention.py:588-630: m = max(m1, m2); l_i' = l_i * exp(m_i - m);
    l = l1' + l2'; out = (l1'/l) out1 + (l2'/l) out2. ``previous`` may be None.
    """
    current = tuple(t.float() for t in current)
    if previous is None:
        return current
    o1, m1, l1 = (t.float() for t in previous)
    o2, m2, l2 = current
    m = torch.maximum(m1, m2)
    l1s = l1 * torch.exp(m1 - m)
    l2s = l2 * torch.exp(m2 - m)
    l = l1s + l2s
    out = o1 * (l1s / l)[..., None] + o2 * (l2s / l)[..., None]
    return out, m, l


def finalize_attention_result(result, *, dtype):
    """Single final cast of the merged fp32 output (ring_attention.py:633-636)."""
    out, maximum, total = result
    return out.to(dtype).contiguous(), maximum, total


# --------------------------------------------------------------------------
# Tree / sibling generalisation
# --------------------------------------------------------------------------

@dataclass(frozen=True)
class Tree:
    """Packed tree metadata.

    cu_seqlens_q[N+1]: leaf suffix offsets; node_offsets[M+1]: node offsets in
    the packed prefix; ancestors[s]: node ids of leaf s, root first.
    """

    cu_seqlens_q: Sequence[int]
    node_offsets: Sequence[int]
    ancestors: Sequence[Sequence[int]]

    @property
    def num_leaves(self) -> int:
        return len(self.cu_seqlens_q) - 1

    @property
    def num_nodes(self) -> int:
        return len(self.node_offsets) - 1

    def leaf_range(self, s):
        return int(self.cu_seqlens_q[s]), int(self.cu_seqlens_q[s + 1])

    def node_range(self, n):
        return int(self.node_offsets[n]), int(self.node_offsets[n + 1])

    def prefix_rows(self, s):
        """Row indices of leaf s's prefix, root -> parent (kv_stack.py:139-154)."""
        rows = []
        for n in self.ancestors[s]:
            a, b = self.node_range(n)
            rows.extend(range(a, b))
        return rows

    @staticmethod
    def single(prefix_len: int, suffix_lens: Sequence[int]) -> "Tree":
        """One shared prefix node (possibly empty) and N sibling leaves."""
        cu = [0]
        for s in suffix_lens:
            cu.append(cu[-1] + int(s))
        if prefix_len > 0:
            return Tree(cu, [0, int(prefix_len)], [[0] for _ in suffix_lens])
        return Tree(cu, [0], [[] for _ in suffix_lens])


def visible_pairs(tree: Tree) -> int:
    """Sum over leaves of S_i * P_i + S_i (S_i + 1) / 2 (visible (q, k) pairs per head)."""
    total = 0
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        length = b - a
        total += length * len(tree.prefix_rows(s)) + length * (length + 1) // 2
    return total


def _leaf_kv(tree, s, k, v, pk, pv):
    a, b = tree.leaf_range(s)
    rows = torch.tensor(tree.prefix_rows(s), dtype=torch.long, device=k.device)
    keys = torch.cat((pk.index_select(0, rows), k[a:b]), 0)
    values = torch.cat((pv.index_select(0, rows), v[a:b]), 0)
    return keys, values, rows.numel()


def _head_groups(hq, hkv, heads_per_chunk):
    group = hq // hkv
    kv_per_chunk = max(1, heads_per_chunk // group)
    for h0 in range(0, hkv, kv_per_chunk):
        yield h0, min(hkv, h0 + kv_per_chunk)


def _visible(tree: Tree, s, plen, mask, device):
    """[S, plen + S] bool: keys of leaf s each query row sees -- the causal
    rule j <= plen + i, or the complement of the physical ``mask`` rows."""
    a, b = tree.leaf_range(s)
    if mask is not None:
        return ~mask[a:b, :plen + b - a].to(device)
    col = torch.arange(plen + b - a, device=device)
    return col[None, :] <= plen + torch.arange(b - a, device=device)[:, None]


def tree_forward(q, k, v, pk, pv, tree: Tree, scale=None, *, compute_dtype=torch.float64,
                 heads_per_chunk=64, mask=None):
    """Forward over a packed tree. Returns (out [Tq,Hq,D] compute_dtype, lse [Hq,Tq] compute_dtype).

    Chunked over leaves and KV-head groups to bound memory; each chunk is the
    dense masked softmax of prefix_attention. ``mask`` (bool [Tq, L], True =
    excluded) replaces the causal rule; rows that see no key get out 0 and
    lse -inf.
    """
    tq, hq, d = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    scale = d ** -0.5 if scale is None else float(scale)
    cd = compute_dtype
    out = torch.zeros(tq, hq, d, dtype=cd, device=q.device)
    lse = torch.full((hq, tq), float("-inf"), dtype=cd, device=q.device)
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        if b == a:
            continue
        keys, values, plen = _leaf_kv(tree, s, k, v, pk, pv)
        visible = _visible(tree, s, plen, mask, q.device)
        for g0, g1 in _head_groups(hq, hkv, heads_per_chunk):
            qs = q[a:b, g0 * group:g1 * group].to(cd).transpose(0, 1)                     # [h,S,D]
            ks = keys[:, g0:g1].to(cd).repeat_interleave(group, 1).permute(1, 2, 0).contiguous()
            vs = values[:, g0:g1].to(cd).repeat_interleave(group, 1).transpose(0, 1).contiguous()
            sc = torch.matmul(qs, ks) * scale
            sc = sc.masked_fill(~visible, float("-inf"))
            m = sc.amax(-1, keepdim=True)
            m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))  # a row that sees no key: w = 0
            w = torch.exp(sc - m)
            l = w.sum(-1, keepdim=True)
            o = torch.matmul(w / torch.where(l > 0, l, torch.ones_like(l)), vs)
            out[a:b, g0 * group:g1 * group] = o.transpose(0, 1)
            lse[g0 * group:g1 * group, a:b] = (m + torch.log(l))[..., 0]
    return out, lse


def tree_backward(q, k, v, pk, pv, tree: Tree, dout, scale=None, *, compute_dtype=torch.float64,
                  heads_per_chunk=64, out=None, lse=None, mask=None):
    """Explicit backward over a packed tree: returns (dq, dk, dv, dpk, dpv) in compute_dtype.

    Per (leaf, KV-head group): P = exp(scale*QK^T - lse), dV = P^T dO,
    dP = dO V^T, dS = P * (dP - rowsum(dO*O)), dQ = scale*dS K,
    dK = scale*dS^T Q. Prefix gradients of leaf s are split back to each
    ancestor node's rows and added in leaf order. ``mask`` as in
    tree_forward (P is 0 wherever the key is hidden).
    """
    tq, hq, d = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    scale = d ** -0.5 if scale is None else float(scale)
    cd = compute_dtype
    if out is None or lse is None:
        out, lse = tree_forward(q, k, v, pk, pv, tree, scale, compute_dtype=cd, heads_per_chunk=heads_per_chunk,
                                mask=mask)
    dq = torch.zeros(tq, hq, d, dtype=cd, device=q.device)
    dk = torch.zeros(k.shape, dtype=cd, device=q.device)
    dv = torch.zeros(v.shape, dtype=cd, device=q.device)
    dpk = torch.zeros(pk.shape, dtype=cd, device=q.device)
    dpv = torch.zeros(pv.shape, dtype=cd, device=q.device)
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        if b == a:
            continue
        keys, values, plen = _leaf_kv(tree, s, k, v, pk, pv)
        rows = torch.tensor(tree.prefix_rows(s), dtype=torch.long, device=q.device)
        visible = _visible(tree, s, plen, mask, q.device)
        for g0, g1 in _head_groups(hq, hkv, heads_per_chunk):
            hs = slice(g0 * group, g1 * group)
            qs = q[a:b, hs].to(cd).transpose(0, 1)                                            # [h,S,D]
            dos = dout[a:b, hs].to(cd).transpose(0, 1)
            os_ = out[a:b, hs].to(cd).transpose(0, 1)
            ks = keys[:, g0:g1].to(cd).repeat_interleave(group, 1).transpose(0, 1).contiguous()  # [h,L,D]
            vs = values[:, g0:g1].to(cd).repeat_interleave(group, 1).transpose(0, 1).contiguous()
            sc = torch.matmul(qs, ks.transpose(1, 2).contiguous()) * scale
            p = torch.exp(sc - lse[hs, a:b].to(cd)[..., None]).masked_fill(~visible, 0.0)
            dvh = torch.matmul(p.transpose(1, 2).contiguous(), dos)                          # [h,L,D]
            dp = torch.matmul(dos, vs.transpose(1, 2).contiguous())
            delta = (dos * os_).sum(-1, keepdim=True)
            ds = p * (dp - delta)
            dq[a:b, hs] = (torch.matmul(ds, ks) * scale).transpose(0, 1)
            dkh = torch.matmul(ds.transpose(1, 2).contiguous(), qs) * scale                   # [h,L,D]
            # sum the query heads of each KV group
            dkh = dkh.reshape(g1 - g0, group, -1, d).sum(1).transpose(0, 1)                  # [L,hkv,D]
            dvh = dvh.reshape(g1 - g0, group, -1, d).sum(1).transpose(0, 1)
            dk[a:b, g0:g1] += dkh[plen:]
            dv[a:b, g0:g1] += dvh[plen:]
            if plen:
                dpk[:, g0:g1].index_add_(0, rows, dkh[:plen])
                dpv[:, g0:g1].index_add_(0, rows, dvh[:plen])
    return dq, dk, dv, dpk, dpv


def tree_autograd(q, k, v, pk, pv, tree: Tree, dout, scale=None, *, dtype=torch.float64):
    """Reference-style execution: one leaf at a time with fresh anchors.

    For each leaf: build cat(ancestor KV) anchors (kv_stack.py:156-173), run
    prefix_attention, backprop dout with autograd, then split the anchor
    gradient per ancestor slice (kv_stack.py:175-203) and accumulate into each
    node in leaf order (prefix_state.py:565-573). Returns (out [Tq,Hq,D], dq,
    dk, dv, dpk, dpv) in ``dtype``.
    """
    tq, hq, d = q.shape
    out = torch.zeros(tq, hq, d, dtype=dtype)
    dq = torch.zeros(tq, hq, d, dtype=dtype)
    dk = torch.zeros(k.shape, dtype=dtype)
    dv = torch.zeros(v.shape, dtype=dtype)
    node_grads: dict[int, list] = {}
    for s in range(tree.num_leaves):
        a, b = tree.leaf_range(s)
        rows = tree.prefix_rows(s)
        with torch.enable_grad():
            qs = q[a:b].detach().to(dtype).unsqueeze(1).clone().requires_grad_(True)
            ks = k[a:b].detach().to(dtype).unsqueeze(1).clone().requires_grad_(True)
            vs = v[a:b].detach().to(dtype).unsqueeze(1).clone().requires_grad_(True)
            idx = torch.tensor(rows, dtype=torch.long)
            pka = pk.detach().to(dtype).index_select(0, idx).unsqueeze(1).clone().requires_grad_(True)
            pva = pv.detach().to(dtype).index_select(0, idx).unsqueeze(1).clone().requires_grad_(True)
            o = prefix_attention(qs, ks, vs, pka, pva, scale)
            g = torch.autograd.grad(o, (qs, ks, vs, pka, pva), grad_outputs=dout[a:b].to(dtype).reshape(o.shape))
        out[a:b] = o.detach().reshape(b - a, hq, d)
        dq[a:b], dk[a:b], dv[a:b] = g[0][:, 0], g[1][:, 0], g[2][:, 0]
        offset = 0
        for n in tree.ancestors[s]:
            na, nb = tree.node_range(n)
            sl = slice(offset, offset + nb - na)
            offset += nb - na
            if n not in node_grads:
                node_grads[n] = [g[3][sl, 0].clone(), g[4][sl, 0].clone()]
            else:
                node_grads[n][0].add_(g[3][sl, 0])
                node_grads[n][1].add_(g[4][sl, 0])
    dpk = torch.zeros(pk.shape, dtype=dtype)
    dpv = torch.zeros(pv.shape, dtype=dtype)
    for n, (gk, gv) in node_grads.items():
        na, nb = tree.node_range(n)
        dpk[na:nb] = gk
        dpv[na:nb] = gv
    return out, dq, dk, dv, dpk, dpv
