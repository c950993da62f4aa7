"""bridge_amd -- MI355X-native prefix-reuse (TPR) attention.

Sibling rollouts attend to one shared external prefix K/V (or a tree of
shared prefix segments) plus their own causal suffix K/V, in one gfx950 HIP
launch per pass (libtpr_attn.so, C ABI in include/tpr_attn.h).

Public API:
  TPRPrefixMeta                 packed sibling / varlen / tree metadata
  TPRPrefixAttention            autograd.Function (q, k, v, prefix_k, prefix_v, meta, scale) -> (out, lse)
  tpr_prefix_attention          functional form
  rectangular_causal_attention  drop-in for the reference's single-sequence operator
  TPRKernelBackend              TPRAttentionBackend (parallel_size 1) for the model seam: one
                                launch per layer for all sibling leaves of a parent
  PrefixKVStack                 zero-copy K/V path stack with fp32 gradient relay (KVStack)
  topology                      rollout tries (exact / Qwen3 turn units) and their one-launch lowering
"""

from .meta import LaunchPlan, TPRPrefixMeta
from .prefix_attention import (
    TPRPrefixAttention,
    prefix_attention_backward,
    prefix_attention_forward,
    tpr_prefix_attention,
)
from .backend import TPRKernelBackend
from .relay import PastKVAnchors, PastKVSlice, PrefixKVStack, StackSegment
from . import topology
from .rectangular_attention import rectangular_causal_attention

__all__ = [
    "LaunchPlan",
    "TPRPrefixMeta",
    "TPRPrefixAttention",
    "tpr_prefix_attention",
    "prefix_attention_forward",
    "prefix_attention_backward",
    "rectangular_causal_attention",
    "TPRKernelBackend",
    "PrefixKVStack",
    "StackSegment",
    "PastKVAnchors",
    "PastKVSlice",
]
