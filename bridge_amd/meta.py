"""Sibling / varlen / tree metadata for prefix-reuse attention, and its launch plan.

A prefix tree is lowered to three packed arrays (the kernel's view of the
reference's SegmentPlan, verl/models/mcore/tpr/segment_plan.py:67-313):

* ``cu_seqlens_q[N+1]``  -- offsets of the N leaf suffixes ("siblings") packed
  padding-free in q/k/v (TND layout, rectangular_attention.py:179-181);
* ``node_offsets[M+1]``  -- offsets of the M shared prefix segments ("nodes")
  packed in prefix_k/prefix_v;
* ``leaf_ancestors[N]``  -- for every leaf, the node ids of its path, root
  first (the concatenation order of KVStack.build_past_key_values,
  kv_stack.py:139-154).

Leaves are numbered in DFS order so that every node's descendant leaves form a
contiguous range; the planner (native, ``tpr_attn_plan``) checks that and
every other structural rule, then emits the per-kernel work lists.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Mapping, Optional, Sequence, Tuple

import ctypes
import torch

from . import _lib

__all__ = ["TPRPrefixMeta", "LaunchPlan"]

# header word indices of the plan blob (bridge_amd/csrc/tpr_common.h)
_PF_PATH = 11
_PF_N_FWD = 19
_PF_N_DKDV = 21
_PF_TOTAL_WORDS = 27
_PF_DS_SLOTS = 30
_PF_MASK_COLS = 32

DS_STORE_DEFAULT_BYTES = 8 << 30  # the library's default dS store budget (TPR_DS_STORE_DEFAULT_BYTES)


def ds_store_budget_bytes(ds_store_budget: Optional[int], recompute_dq: bool = False) -> Optional[int]:
    """The dS store budget a plan is built with: None (the library default),
    or a byte count >= 0 (0: no store)."""
    if recompute_dq:
        return 0
    if ds_store_budget is None:
        return None
    if isinstance(ds_store_budget, bool) or not isinstance(ds_store_budget, int) or ds_store_budget < 0:
        raise ValueError(f"ds_store_budget must be None or a non-negative integer, got {ds_store_budget!r}")
    return ds_store_budget


@dataclass(frozen=True)
class LaunchPlan:
    """A plan blob in host and device memory for one (heads, head_dim, dtype, device)."""

    host: torch.Tensor     # int32, CPU
    device: torch.Tensor   # int32, on the compute device
    workspace_bytes: int

    @property
    def path(self) -> str:
        """Kernel path: "mfma" (bf16 matrix-core kernels: head_dim 64, 128 and
        256) or "simt" (fp32, and bf16 with other head sizes)."""
        return "mfma" if int(self.host[_PF_PATH]) in (1, 2) else "simt"

    @property
    def mfma_shape(self) -> Optional[str]:
        """The MFMA instruction the kernels are built on: "32x32x16" (bf16,
        head_dim 128), "16x16x32" (bf16, head_dim 64 and 256), None off the
        MFMA path."""
        return {1: "32x32x16", 2: "16x16x32"}.get(int(self.host[_PF_PATH]))

    @property
    def dq_from_ds(self) -> bool:
        """Whether the backward stores dS and computes dQ from it (bf16
        head_dim 128 and 256 when the store fits the plan's dS store budget);
        the workspace then holds the store."""
        return int(self.host[_PF_DS_SLOTS]) > 0

    @property
    def masked(self) -> bool:
        """Whether the plan is for calls with a physical key mask (built with
        ``masked=True``; SIMT kernels, the mask the only visibility rule)."""
        return int(self.host[_PF_MASK_COLS]) > 0

    @property
    def num_forward_items(self) -> int:
        return int(self.host[_PF_N_FWD])

    @property
    def num_dkdv_items(self) -> int:
        return int(self.host[_PF_N_DKDV])


def _int_list(values, name) -> Tuple[int, ...]:
    if isinstance(values, torch.Tensor):
        values = values.detach().cpu().tolist()
    out = []
    for v in values:
        if isinstance(v, bool) or int(v) != v:
            raise TypeError(f"{name} must contain integers, got {v!r}")
        out.append(int(v))
    return tuple(out)


@dataclass(frozen=True)
class TPRPrefixMeta:
    cu_seqlens_q: Tuple[int, ...]
    node_offsets: Tuple[int, ...]
    leaf_ancestors: Tuple[Tuple[int, ...], ...]
    _plans: Dict[tuple, LaunchPlan] = field(default_factory=dict, init=False, repr=False, compare=False)

    def __post_init__(self):
        object.__setattr__(self, "cu_seqlens_q", _int_list(self.cu_seqlens_q, "cu_seqlens_q"))
        object.__setattr__(self, "node_offsets", _int_list(self.node_offsets, "node_offsets"))
        anc = tuple(_int_list(a, "leaf_ancestors") for a in self.leaf_ancestors)
        object.__setattr__(self, "leaf_ancestors", anc)
        if len(self.cu_seqlens_q) < 2:
            raise ValueError("cu_seqlens_q must hold at least one leaf (N+1 >= 2 entries)")
        if len(self.node_offsets) < 1:
            raise ValueError("node_offsets must hold at least one entry")
        if len(anc) != self.num_leaves:
            raise ValueError(f"leaf_ancestors must have one entry per leaf ({self.num_leaves}), got {len(anc)}")

    # ---- constructors ------------------------------------------------------
    @classmethod
    def shared_prefix(cls, prefix_length: int, suffix_lengths: Sequence[int]) -> "TPRPrefixMeta":
        """N sibling suffixes under one shared prefix (prefix_length may be 0)."""
        cu = [0]
        for s in suffix_lengths:
            cu.append(cu[-1] + int(s))
        if prefix_length < 0:
            raise ValueError(f"prefix_length must be non-negative, got {prefix_length}")
        if prefix_length == 0:
            return cls(tuple(cu), (0,), tuple(() for _ in suffix_lengths))
        return cls(tuple(cu), (0, int(prefix_length)), tuple((0,) for _ in suffix_lengths))

    @classmethod
    def from_segment_tree(cls, parents: Mapping[int, Optional[int]], lengths: Mapping[int, int]
                          ) -> Tuple["TPRPrefixMeta", Tuple[int, ...], Tuple[int, ...]]:
        """Lower a rooted segment tree to packed metadata.

        ``parents[seg]`` is the parent segment id (None for the root) and
        ``lengths[seg]`` the token count, as in SegmentSpec (segment_plan.py:67-122).
        Children are visited in insertion order (segment_plan.py:266-275).
        Childless segments become leaves (suffixes, DFS order), the others
        nodes (shared prefixes, DFS preorder). Returns (meta, node_segment_ids,
        leaf_segment_ids) giving the packing order of prefix_k/v and q/k/v.
        """
        roots = [s for s, p in parents.items() if p is None]
        if len(roots) != 1:
            raise ValueError(f"segment tree must have exactly one root, got {roots}")
        children: Dict[int, list] = {s: [] for s in parents}
        for s, p in parents.items():
            if p is not None:
                if p not in children:
                    raise ValueError(f"segment {s} has missing parent {p}")
                children[p].append(s)
        nodes, leaves, paths = [], [], []
        node_index: Dict[int, int] = {}
        # DFS preorder on an explicit stack (a chain of thousands of segments
        # must not hit Python's recursion limit); children are pushed in
        # reverse so they are visited in insertion order.
        stack = [(roots[0], ())]
        while stack:
            seg, path = stack.pop()
            if children[seg]:
                node_index[seg] = len(nodes)
                nodes.append(seg)
                below = path + (node_index[seg],)
                for c in reversed(children[seg]):
                    stack.append((c, below))
            else:
                leaves.append(seg)
                paths.append(path)

        if len(nodes) + len(leaves) != len(parents):
            raise ValueError("segment tree is not connected")
        node_offsets = [0]
        for s in nodes:
            node_offsets.append(node_offsets[-1] + int(lengths[s]))
        cu = [0]
        for s in leaves:
            cu.append(cu[-1] + int(lengths[s]))
        return cls(tuple(cu), tuple(node_offsets), tuple(paths)), tuple(nodes), tuple(leaves)

    # ---- properties --------------------------------------------------------
    @property
    def num_leaves(self) -> int:
        return len(self.cu_seqlens_q) - 1

    @property
    def num_nodes(self) -> int:
        return len(self.node_offsets) - 1

    @property
    def max_depth(self) -> int:
        return max((len(a) for a in self.leaf_ancestors), default=0)

    @property
    def total_q(self) -> int:
        return self.cu_seqlens_q[-1]

    @property
    def total_prefix(self) -> int:
        return self.node_offsets[-1]

    def prefix_length(self, leaf: int) -> int:
        return sum(self.node_offsets[n + 1] - self.node_offsets[n] for n in self.leaf_ancestors[leaf])

    def suffix_lengths(self) -> Tuple[int, ...]:
        return tuple(b - a for a, b in zip(self.cu_seqlens_q[:-1], self.cu_seqlens_q[1:]))

    def max_keys(self) -> int:
        """Longest key sequence of any leaf (ancestor prefix + own suffix):
        the least column count of a key mask."""
        return max((self.prefix_length(i) + s for i, s in enumerate(self.suffix_lengths())), default=0)

    def visible_pairs(self) -> int:
        """Sum over leaves of S_i * P_i + S_i (S_i + 1) / 2 (per query head)."""
        return sum(s * self.prefix_length(i) + s * (s + 1) // 2 for i, s in enumerate(self.suffix_lengths()))

    # ---- launch plan -------------------------------------------------------
    def plan(self, num_q_heads: int, num_kv_heads: int, head_dim: int, dtype: torch.dtype,
             device: torch.device, *, recompute_dq: bool = False,
             ds_store_budget: Optional[int] = None, masked: bool = False) -> LaunchPlan:
        """Build (once per configuration) the native launch plan and upload it.

        ``ds_store_budget``: bytes the backward's dS store may take (bf16
        head_dim 128 and 256). With a store, the dK/dV kernel writes every dS
        block, 2 bytes per visible (query, key) pair and query head, and the
        dQ kernel computes dQ = scale dS K from them instead of recomputing S
        and dP (one matrix product instead of three); without one the
        workspace is a few MB. ``None``: the library default,
        ``DS_STORE_DEFAULT_BYTES`` (8 GiB; the Qwen3-4B layer shape, prefix
        4096 + 4 x 4096 at GQA 32/8, needs 6.5 GB); ``0``: no store.
        ``recompute_dq=True`` is the same as ``ds_store_budget=0``.

        ``masked=True``: the plan for calls that pass a physical key mask,
        which is then the only visibility rule (the reference's custom-mask
        mode); it runs the SIMT kernels, for any dtype and head size, with
        no dS store."""
        if dtype == torch.bfloat16:
            code = _lib.TPR_DTYPE_BF16
        elif dtype == torch.float32:
            code = _lib.TPR_DTYPE_FP32
        else:
            raise ValueError(f"prefix attention supports torch.bfloat16 and torch.float32, got {dtype}")
        budget = ds_store_budget_bytes(ds_store_budget, recompute_dq)
        masked = bool(masked)
        flags = _lib.TPR_PLAN_MASKED if masked else 0
        key = (num_q_heads, num_kv_heads, head_dim, code, str(device), budget, masked)
        cached = self._plans.get(key)
        if cached is not None:
            return cached
        lib = _lib.load()
        depth = self.max_depth
        anc = [n for a in self.leaf_ancestors for n in (list(a) + [-1] * (depth - len(a)))]
        cu = (ctypes.c_int32 * len(self.cu_seqlens_q))(*self.cu_seqlens_q)
        no = (ctypes.c_int32 * len(self.node_offsets))(*self.node_offsets)
        an = (ctypes.c_int32 * max(1, len(anc)))(*anc) if anc else (ctypes.c_int32 * 1)(-1)
        desc = _lib.TprTreeDesc(self.num_leaves, self.num_nodes, depth, num_q_heads, num_kv_heads, head_dim,
                                code, flags, ctypes.cast(cu, ctypes.c_void_p), ctypes.cast(no, ctypes.c_void_p),
                                ctypes.cast(an, ctypes.c_void_p),
                                _lib.TPR_DS_STORE_DEFAULT if budget is None else budget)
        words = ctypes.c_int64(0)
        _lib.check(lib.tpr_attn_plan(ctypes.byref(desc), None, 0, ctypes.byref(words)), "tpr_attn_plan")
        host = torch.empty(int(words.value), dtype=torch.int32)
        _lib.check(lib.tpr_attn_plan(ctypes.byref(desc), ctypes.c_void_p(host.data_ptr()), host.numel(),
                                     ctypes.byref(words)), "tpr_attn_plan")
        if device.type == "cpu":
            dev = host
        else:
            dev = host.to(device, non_blocking=False)
        ws = int(lib.tpr_attn_bwd_workspace_bytes(ctypes.c_void_p(host.data_ptr())))
        plan = LaunchPlan(host, dev, ws)
        self._plans[key] = plan
        return plan
