"""An attention backend over a PrefixKVStack computed by the CPU oracle (test
infrastructure): the same protocol and relay as TPRKernelBackend.from_stack --
each packed sibling attends to the stack's path and causally to itself, and
the path's gradient is added into the stack's fp32 rows -- with the dense
oracle (_fa_fp32_reference.py:12-40 restated) in place of the kernel."""

from __future__ import annotations

import torch

from oracle.tpr_oracle import prefix_attention


class _AddPathGradient(torch.autograd.Function):
    """Identity on the path K/V; the backward adds their gradient into the
    stack's fp32 rows (what the kernel's accumulate mode does)."""

    @staticmethod
    def forward(ctx, pk, pv, acc_k, acc_v):
        ctx.acc = (acc_k, acc_v)
        return pk.view_as(pk), pv.view_as(pv)

    @staticmethod
    def backward(ctx, gk, gv):
        acc_k, acc_v = ctx.acc
        acc_k.add_(gk.reshape(acc_k.shape).float())
        acc_v.add_(gv.reshape(acc_v.shape).float())
        return None, None, None, None


class OracleStackBackend:
    def __init__(self, stack, suffix_lengths):
        self.stack = stack
        self.lengths = tuple(suffix_lengths)

    @property
    def global_prefix_length(self):
        return self.stack.prefix_length

    @property
    def global_suffix_length(self):
        return sum(self.lengths)

    @property
    def local_suffix_length(self):
        return sum(self.lengths)

    @property
    def parallel_size(self):
        return 1

    def attention(self, layer_number, query, new_key, new_value, *, softmax_scale):
        p = self.stack.prefix_length
        if p:
            pk, pv = self.stack.build_past_key_values()[layer_number]
            acc_k, acc_v = self.stack.past_gradient_accumulators()[layer_number]
            pk, pv = _AddPathGradient.apply(pk.detach().requires_grad_(True), pv.detach().requires_grad_(True),
                                            acc_k, acc_v)
        else:
            pk = pv = new_key[:0]
        outs, off = [], 0
        for s in self.lengths:
            sl = slice(off, off + s)
            outs.append(prefix_attention(query[sl], new_key[sl], new_value[sl], pk, pv, softmax_scale))
            off += s
        return torch.cat(outs, 0)
