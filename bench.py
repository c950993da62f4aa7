#!/usr/bin/env python3
"""Prefix-reuse (TPR) attention benchmark on one MI355X.

A step is one forward + backward pass of sibling-batched prefix attention
over the whole workload (inputs already resident in HBM). Default workload:
the Qwen3-4B attention-layer shape -- GQA 32/8, head_dim 128, bf16, one
shared prefix of 4096 tokens and 4 sibling suffixes of 4096 tokens, N(0,1)
synthetic inputs, scale 1/sqrt(128).

Throughput is algorithmic: only visible (query, key) pairs count,
V_i = S_i * P_i + S_i (S_i + 1) / 2 per query head, and
fwd = 4 Hq D sum(V_i), fwd+bwd = 14 Hq D sum(V_i) FLOP.

Prints one JSON line (rank 0). ``--gpus N`` with N > 1 exits: this build
runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

import torch

BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3    # MI355X fp32 (matrix and vector)
HBM_PEAK_GBS = 8000.0


def workload(name: str):
    """(description, meta, hq, hkv, d, dtype) for a named workload."""
    from bridge_amd import TPRPrefixMeta
    if name == "qwen3-4b":
        return ("Qwen3-4B attention layer: prefix 4096 + 4 x 4096 sibling suffixes, GQA 32/8, d128, bf16",
                TPRPrefixMeta.shared_prefix(4096, [4096] * 4), 32, 8, 128, torch.bfloat16)
    if name == "qwen3-4b-1sibling":   # prefix-traffic probe: the headline shape with one sibling
        return ("Qwen3-4B attention layer, one sibling: prefix 4096 + 1 x 4096, GQA 32/8, d128, bf16",
                TPRPrefixMeta.shared_prefix(4096, [4096]), 32, 8, 128, torch.bfloat16)
    if name == "qwen3-4b-noprefix":   # prefix-traffic probe: the headline siblings without the prefix
        return ("Qwen3-4B attention layer, no prefix: 4 x 4096 causal suffixes, GQA 32/8, d128, bf16",
                TPRPrefixMeta.shared_prefix(0, [4096] * 4), 32, 8, 128, torch.bfloat16)
    if name == "plumbing-fp32":
        return ("plumbing: prefix 512 + 2 x 512 suffixes, 4 heads MHA, d64, fp32",
                TPRPrefixMeta.shared_prefix(512, [512] * 2), 4, 4, 64, torch.float32)
    if name == "long-session":
        return ("long agent session: prefix 32768 + 8 x 2048 suffixes, GQA 32/8, d128, bf16",
                TPRPrefixMeta.shared_prefix(32768, [2048] * 8), 32, 8, 128, torch.bfloat16)
    if name == "ragged":
        g = torch.Generator(device="cpu").manual_seed(0)
        lens = torch.randint(256, 8193, (16,), generator=g).tolist()
        return (f"ragged varlen: prefix 8192 + 16 suffixes U[256,8192] (seed 0), GQA 32/8, d128, bf16",
                TPRPrefixMeta.shared_prefix(8192, lens), 32, 8, 128, torch.bfloat16)
    if name == "qwen35-attn":   # head_dim 256: the 16-wide MFMA kernels
        return ("Qwen3.5 hybrid full-attention layer: prefix 4096 + 4 x 4096 sibling suffixes, GQA 8/2, d256, bf16",
                TPRPrefixMeta.shared_prefix(4096, [4096] * 4), 8, 2, 256, torch.bfloat16)
    if name == "head64":   # head_dim 64 (the reference's operator-test head size) at the headline sequence shape
        return ("head_dim 64: prefix 4096 + 4 x 4096 sibling suffixes, GQA 32/8, d64, bf16",
                TPRPrefixMeta.shared_prefix(4096, [4096] * 4), 32, 8, 64, torch.bfloat16)
    if name == "turn-tree":
        anc = tuple((0, 1 + i // 4) for i in range(16))
        meta = TPRPrefixMeta(tuple(1024 * i for i in range(17)), (0, 2048, 3072, 4096, 5120, 6144), anc)
        return ("turn-boundary tree depth 3: root 2048 -> 4 x 1024 -> 16 leaves x 1024, GQA 32/8, d128, bf16",
                meta, 32, 8, 128, torch.bfloat16)
    raise SystemExit(f"unknown workload {name!r}")


def traffic_bytes(workload_name: str, kernel: str):
    """HBM bytes (read + write) per launch of `kernel`, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary of this workload (scaled by the
    copy-probe calibration), or None when there is none."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return None
    entry = data.get("per_launch", {}).get(kernel) if data.get("workload") == workload_name else None
    return None if entry is None else int(entry["read_bytes"] + entry["write_bytes"])


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_threads() -> int:
    """Host threads the CPU baseline may use: the CPUs this process may run on,
    capped by OMP_NUM_THREADS when the environment sets it (a shared GPU host
    may give a job only a share of its cores)."""
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS", "")
    if cap.isdigit() and int(cap) > 0:
        usable = min(usable, int(cap))
    return max(1, usable)


def cpu_baseline(meta, hq: int, hkv: int, d: int, reps: int = 3, max_siblings: int = 4):
    """The reference's CPU fp32 path, timed on a bounded sample: the first
    ``max_siblings`` siblings of the workload, one KV-head group (its Hq/Hkv
    query heads), run one sibling after another as the reference's executor
    visits leaves (dense fp32 prefix attention + autograd per sibling, prefix
    gradients summed in sibling order)."""
    from oracle.tpr_oracle import prefix_attention
    threads = cpu_threads()
    torch.set_num_threads(threads)
    g = torch.Generator(device="cpu").manual_seed(0)
    heads = hq // hkv
    nsib = min(max_siblings, meta.num_leaves)
    sibs = []
    for i in range(nsib):
        s, p = meta.suffix_lengths()[i], meta.prefix_length(i)
        sibs.append((p, [torch.randn(s, 1, heads, d, generator=g), torch.randn(s, 1, 1, d, generator=g),
                         torch.randn(s, 1, 1, d, generator=g), torch.randn(s, 1, heads * d, generator=g)]))
    plen = max(p for p, _ in sibs)
    pk = torch.randn(plen, 1, 1, d, generator=g)
    pv = torch.randn(plen, 1, 1, d, generator=g)
    scale = 1.0 / math.sqrt(d)
    times = []
    for i in range(reps + 1):
        t0 = time.perf_counter()
        dpk = dpv = None
        for p, (q, k, v, dout) in sibs:
            tensors = [q.clone().requires_grad_(True), k.clone().requires_grad_(True),
                       v.clone().requires_grad_(True), pk[:p].clone().requires_grad_(True),
                       pv[:p].clone().requires_grad_(True)]
            out = prefix_attention(*tensors, scale)
            grads = torch.autograd.grad(out, tensors, grad_outputs=dout)
            dpk = grads[3] if dpk is None else dpk + grads[3]
            dpv = grads[4] if dpv is None else dpv + grads[4]
        dt = time.perf_counter() - t0
        if i > 0:
            times.append(dt)
    pairs = sum(s * p + s * (s + 1) // 2 for p, s in
                ((p, t[0].shape[0]) for p, t in sibs))
    flops = 14.0 * heads * d * pairs
    med = statistics.median(times)
    return {
        "value": round(flops / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "cpu_count": os.cpu_count(),
        "threads": torch.get_num_threads(),
        "cpu_model": cpu_model(),
        "kind": "port",
        "sample": (f"{nsib} of {meta.num_leaves} siblings x 1 KV-head group ({heads} query heads of {hq}), "
                   f"fp32 dense prefix attention + autograd per sibling, prefix grads summed in sibling order; "
                   f"median of {reps} after 1 warmup, {med:.2f} s per rep"),
    }


def relay_bench(args) -> int:
    """One leaf-batch visit (fwd + bwd, one layer) under a two-segment path --
    root 2048 + branch 2048 tokens, 4 sibling leaves of 4096, Qwen3-4B layer
    dims -- two ways:
      reference flow: torch.cat of the path K/V, detached anchors, the kernel
        with autograd prefix gradients (bf16), then the per-ancestor split and
        bf16 add_ (kv_stack.py:139-203, prefix_state.py:546-573);
      relay flow: PrefixKVStack views and the kernel adding the prefix
        gradient into the stack's fp32 rows (TPR_BWD_ACCUMULATE_PREFIX_F32).
    Also times the reference flow's relay operations alone (cat + split/add)."""
    from bridge_amd import PrefixKVStack, StackSegment, TPRPrefixAttention, TPRPrefixMeta
    device = torch.device("cuda", 0)
    hq, hkv, d, seg, lengths = 32, 8, 128, 2048, [4096] * 4
    scale = 1.0 / math.sqrt(d)
    meta = TPRPrefixMeta.shared_prefix(2 * seg, lengths)
    gen = torch.Generator(device=device).manual_seed(99)
    r = lambda *shape: torch.randn(*shape, device=device, generator=gen).bfloat16()  # noqa: E731
    tq = sum(lengths)
    q, k, v, dout = r(tq, hq, d), r(tq, hkv, d), r(tq, hkv, d), r(tq, hq, d)
    seg_kv = [{1: (r(seg, 1, hkv, d), r(seg, 1, hkv, d))} for _ in range(2)]
    seg_grad = [(torch.zeros(seg, 1, hkv, d, dtype=torch.bfloat16, device=device),
                 torch.zeros(seg, 1, hkv, d, dtype=torch.bfloat16, device=device)) for _ in range(2)]
    stack = PrefixKVStack(2 * seg)
    stack.push(StackSegment(0, None, seg, 0, 0), seg_kv[0])
    stack.push(StackSegment(1, 0, seg, seg, seg), seg_kv[1])
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))

    def reference_relay_ops_forward():
        past_k = torch.cat([s[1][0] for s in seg_kv], 0)
        past_v = torch.cat([s[1][1] for s in seg_kv], 0)
        return past_k.detach().requires_grad_(True), past_v.detach().requires_grad_(True)

    def reference_relay_ops_backward(gk, gv):
        for i in range(2):
            seg_grad[i][0].add_(gk[i * seg:(i + 1) * seg])
            seg_grad[i][1].add_(gv[i * seg:(i + 1) * seg])

    def reference_visit():
        ak, av = reference_relay_ops_forward()
        out, _ = TPRPrefixAttention.apply(qa, ka, va, ak[:, 0], av[:, 0], meta, scale)
        out.backward(dout)
        reference_relay_ops_backward(ak.grad, av.grad)

    def relay_visit():
        pk, pv = stack.build_past_key_values()[1]
        acc = stack.past_gradient_accumulators()[1]
        out, _ = TPRPrefixAttention.apply(qa, ka, va, pk[:, 0], pv[:, 0], meta, scale, acc)
        out.backward(dout)

    gk_fixed = r(2 * seg, 1, hkv, d)

    def relay_ops_only():
        ak, av = reference_relay_ops_forward()
        reference_relay_ops_backward(gk_fixed, gk_fixed)

    def timed(fn, n):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        return statistics.median(times)

    ref_ms = timed(reference_visit, args.steps)
    relay_ms = timed(relay_visit, args.steps)
    ref_again_ms = timed(reference_visit, args.steps)
    ops_ms = timed(relay_ops_only, args.steps)
    row_bytes = hkv * d * 2
    print(json.dumps({
        "metric": "leaf-batch visit ms (fwd+bwd, one layer), reference relay flow vs PrefixKVStack relay",
        "reference_flow_ms": round(statistics.mean([ref_ms, ref_again_ms]), 4),
        "relay_flow_ms": round(relay_ms, 4),
        "reference_relay_ops_ms": round(ops_ms, 4),
        "reference_relay_ops_bytes": 2 * (2 * 2 * seg * row_bytes) + 2 * (3 * 2 * seg * row_bytes),
        "relay_flow_copies_per_visit": 0,
        "config": {"path_segments": [seg, seg], "siblings": len(lengths), "suffix_tokens": tq,
                   "q_heads": hq, "kv_heads": hkv, "head_dim": d, "dtype": "bf16", "layers": 1},
        "steps": args.steps, "warmup": args.warmup,
    }), flush=True)
    return 0


def tree_launch_bench(args) -> int:
    """A depth-3 rollout tree -- 16 rollouts of 2048 shared + 1024 shared by 4
    + 1024 own tokens, Qwen3-4B layer dims -- built with build_trajectory_trees
    from synthetic token rows and run (fwd + bwd, one layer) two ways:
      one launch: lower_tree's packing, every segment at once;
      per segment: the reference executor's order, one visit per segment with
        the concatenated path K/V as its prefix (kv_stack.py:139-154).
    Both do the same visible pairs; reports ms and TFLOP/s of each, and the
    host time of the trie build + lowering."""
    from bridge_amd import TPRPrefixAttention, TPRPrefixMeta
    from bridge_amd.topology import build_trajectory_trees, lower_tree
    device = torch.device("cuda", 0)
    hq, hkv, d = 32, 8, 128
    scale = 1.0 / math.sqrt(d)
    g = torch.Generator().manual_seed(5)
    root = torch.randint(0, 150000, (2048,), generator=g)
    branches = [torch.randint(0, 150000, (1024,), generator=g) for _ in range(4)]
    rows = [torch.cat([root, branches[i // 4], torch.randint(0, 150000, (1024,), generator=g)]) for i in range(16)]
    t0 = time.perf_counter()
    (tree,) = build_trajectory_trees([f"u_s_{i}" for i in range(16)], {"input_ids": rows})
    launch = lower_tree(tree)
    host_ms = (time.perf_counter() - t0) * 1e3
    meta = launch.meta
    tq = meta.total_q
    gd = torch.Generator(device=device).manual_seed(6)
    r = lambda *shape: torch.randn(*shape, device=device, generator=gd).bfloat16()  # noqa: E731
    q, k, v, dout = r(tq, hq, d), r(tq, hkv, d), r(tq, hkv, d), r(tq, hq, d)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    index = launch.prefix_index.to(device)

    def one_launch():
        out, _ = TPRPrefixAttention.apply(qa, ka, va, ka.index_select(0, index), va.index_select(0, index), meta,
                                          scale)
        out.backward(dout)

    spans = [(meta.cu_seqlens_q[i], meta.cu_seqlens_q[i + 1]) for i in range(meta.num_leaves)]
    paths = []
    for anc in meta.leaf_ancestors:
        rows_idx = [torch.arange(meta.cu_seqlens_q[launch.segments.index(launch.prefix_segments[n])],
                                 meta.cu_seqlens_q[launch.segments.index(launch.prefix_segments[n]) + 1])
                    for n in anc]
        paths.append(torch.cat(rows_idx).to(device) if rows_idx else None)
    seg_meta = [TPRPrefixMeta.shared_prefix(0 if p is None else p.numel(), [b - a]) for (a, b), p in zip(spans, paths)]

    def per_segment():
        for (a, b), p, m in zip(spans, paths, seg_meta):
            if p is None:
                pk = pv = ka.new_empty((0, hkv, d))
            else:
                pk, pv = ka.index_select(0, p), va.index_select(0, p)
            out, _ = TPRPrefixAttention.apply(qa[a:b], ka[a:b], va[a:b], pk, pv, m, scale)
            out.backward(dout[a:b])

    def timed(fn, n):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        times = []
        for _ in range(n):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
        return statistics.median(times)

    one_ms = timed(one_launch, args.steps)
    seg_ms = timed(per_segment, args.steps)
    flops = 14.0 * hq * d * meta.visible_pairs()
    print(json.dumps({
        "metric": "rollout tree fwd+bwd (one layer): one launch for every segment vs one visit per segment",
        "one_launch_ms": round(one_ms, 4),
        "per_segment_ms": round(seg_ms, 4),
        "one_launch_tflops": round(flops / (one_ms * 1e-3) / 1e12, 2),
        "per_segment_tflops": round(flops / (seg_ms * 1e-3) / 1e12, 2),
        "trie_build_and_lowering_host_ms": round(host_ms, 2),
        "config": {"rollouts": 16, "tokens_per_rollout": 4096, "segments": meta.num_leaves,
                   "prefix_nodes": meta.num_nodes, "packed_tokens": tq, "prefix_rows": meta.total_prefix,
                   "visible_pairs_per_head": meta.visible_pairs(), "q_heads": hq, "kv_heads": hkv, "head_dim": d,
                   "dtype": "bf16"},
        "steps": args.steps, "warmup": args.warmup,
    }), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="qwen3-4b",
                    choices=["qwen3-4b", "plumbing-fp32", "long-session", "ragged", "turn-tree", "qwen35-attn", "head64",
                             "qwen3-4b-1sibling", "qwen3-4b-noprefix"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--recompute-dq", action="store_true",
                    help="use the plan without a dS store (dQ recomputes S and dP; small workspace); "
                         "the same as --ds-store-budget 0")
    ap.add_argument("--ds-store-budget", type=int, default=None, metavar="BYTES",
                    help="bytes the backward's dS store may take (default: the library's, 8 GiB)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="before the timed steps, run one plain device copy of MIB MiB (read MIB, write MIB): "
                         "the calibration dispatch for rocprofv3 FETCH_SIZE / WRITE_SIZE")
    ap.add_argument("--relay", action="store_true",
                    help="instead of the step benchmark, time one leaf-batch visit with the reference's "
                         "concat/anchor/split relay and with PrefixKVStack's in-kernel fp32 relay")
    ap.add_argument("--tree-launch", action="store_true",
                    help="instead of the step benchmark, time a depth-3 rollout tree run as one launch "
                         "(lower_tree) and as one visit per segment")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the kernels would shard by KV-head group, with no exchange, or by sibling, with one "
              "fixed-order reduction of the prefix gradient)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs an MI355X GPU", file=sys.stderr)
        return 2

    if args.relay:
        return relay_bench(args)
    if args.tree_launch:
        return tree_launch_bench(args)

    from bridge_amd import _lib
    from bridge_amd.meta import DS_STORE_DEFAULT_BYTES
    from bridge_amd.prefix_attention import prefix_attention_backward, prefix_attention_forward

    device = torch.device("cuda", 0)
    desc, meta, hq, hkv, d, dtype = workload(args.workload)
    scale = 1.0 / math.sqrt(d)
    gen = torch.Generator(device=device).manual_seed(1234)
    tq, tp = meta.total_q, meta.total_prefix
    q = torch.randn(tq, hq, d, device=device, generator=gen).to(dtype)
    k = torch.randn(tq, hkv, d, device=device, generator=gen).to(dtype)
    v = torch.randn(tq, hkv, d, device=device, generator=gen).to(dtype)
    pk = torch.randn(tp, hkv, d, device=device, generator=gen).to(dtype)
    pv = torch.randn(tp, hkv, d, device=device, generator=gen).to(dtype)
    dout = torch.randn(tq, hq, d, device=device, generator=gen).to(dtype)
    budget = 0 if args.recompute_dq else args.ds_store_budget
    plan = meta.plan(hq, hkv, d, dtype, device, ds_store_budget=budget)

    buffers = {"dq": torch.empty_like(q), "dk": torch.empty_like(k), "dv": torch.empty_like(v),
               "dprefix_k": torch.empty_like(pk), "dprefix_v": torch.empty_like(pv),
               "delta": torch.empty((hq, tq), dtype=torch.float32, device=device),
               "workspace": (torch.empty(plan.workspace_bytes, dtype=torch.uint8, device=device)
                             if plan.workspace_bytes else None)}
    stream = torch.cuda.current_stream(device)

    # one fwd+bwd step, enqueued phase by phase so that each kernel can be
    # timed with events on the stream it runs on
    phases = [None, _lib.TPR_BWD_DELTA, _lib.TPR_BWD_DKDV_TILES, _lib.TPR_BWD_DKDV_REDUCE, _lib.TPR_BWD_DQ]

    def step(events=None):
        out = lse = None
        for i, ph in enumerate(phases):
            if events:
                events[i].record(stream)
            if ph is None:
                out, lse = prefix_attention_forward(q, k, v, pk, pv, meta, scale)
            else:
                prefix_attention_backward(q, k, v, pk, pv, out, lse, dout, meta, scale, phases=ph, buffers=buffers,
                                          ds_store_budget=budget)
        if events:
            events[len(phases)].record(stream)

    if args.copy_probe:
        src = torch.ones(args.copy_probe * (1 << 20) // 2, dtype=torch.bfloat16, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(len(phases) + 1)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(device)
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(events[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    peak_bytes = torch.cuda.max_memory_allocated(device)  # of the timed steps: inputs, outputs, workspace

    def avg(a, b):
        return statistics.mean(e[a].elapsed_time(e[b]) for e in events)

    fwd_ms, delta_ms, dkdv_ms, reduce_ms, dq_ms = avg(0, 1), avg(1, 2), avg(2, 3), avg(3, 4), avg(4, 5)
    pairs = meta.visible_pairs()
    unit = 2.0 * hq * d * pairs          # FLOP of one GEMM over the visible pairs
    total_flops = 7.0 * unit            # fwd (2 GEMMs) + bwd (5 GEMMs)
    value = total_flops / (ms_per_step * 1e-3) / 1e12
    # the SIMT kernels compute in fp32 on the vector ALUs, whatever the I/O dtype
    peak = BF16_PEAK_TFLOPS if plan.path == "mfma" else FP32_PEAK_TFLOPS
    prefix = {"32x32x16": "tpr::mfma_", "16x16x32": "tpr::m16_", None: "tpr::simt_"}[plan.mfma_shape]
    # executed MFMA work per kernel: the forward 2 GEMMs, dK/dV 4; dQ 1 from
    # the dS store, 3 when it recomputes S and dP
    kernels = {
        "fwd": (fwd_ms, 2.0 * unit, prefix + "fwd"),
        "dkdv": (dkdv_ms, 4.0 * unit, prefix + "dkdv"),
        "dq": (dq_ms, (1.0 if plan.dq_from_ds else 3.0) * unit, prefix + ("dqs" if plan.dq_from_ds else "dq")),
    }
    dom = max(kernels, key=lambda n: kernels[n][0])
    dom_ms, dom_flops, dom_name = kernels[dom]
    achieved = dom_flops / (dom_ms * 1e-3) / 1e12

    result = {
        "metric": ("prefix-attn fwd+bwd TFLOP/s & % bf16 MFMA peak, Qwen3-4B shape, 1 GPU"
                   if args.workload == "qwen3-4b" else
                   f"prefix-attn fwd+bwd TFLOP/s & % of peak, {args.workload} workload, 1 GPU"),
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16" if dtype == torch.bfloat16 else "fp32",
        "data": "synthetic N(0,1) inputs, seeded",
        "config": {
            "workload": desc,
            "prefix_tokens": tp,
            "suffix_tokens": tq,
            "siblings": meta.num_leaves,
            "q_heads": hq,
            "kv_heads": hkv,
            "head_dim": d,
            "visible_pairs_per_head": pairs,
            "fwd_bwd_flop": total_flops,
            "dq": "from the dS store" if plan.dq_from_ds else "recomputed",
            "workspace_bytes": plan.workspace_bytes,
            "ds_store_budget_bytes": DS_STORE_DEFAULT_BYTES if budget is None else budget,
            "peak_memory_bytes": peak_bytes,
        },
        "fraction_of_peak": round(value / peak, 4),
        "fwd_tflops": round(2.0 * unit / (fwd_ms * 1e-3) / 1e12, 2),
        "tokens_per_s": round(tq / (ms_per_step * 1e-3), 1),
        "kernel_ms": {"fwd": round(fwd_ms, 4), "delta": round(delta_ms, 4), "dkdv": round(dkdv_ms, 4),
                      "dkdv_reduce": round(reduce_ms, 4), "dq": round(dq_ms, 4)},
        "roofline": {
            "kernel": dom_name,
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic_bytes(args.workload, dom_name),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(meta, hq, hkv, d)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
