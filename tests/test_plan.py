"""CPU tests of the native planner (tpr_attn_plan): tree validation, work-list
coverage, XCD-aware ordering and the segment-tree lowering. Host code only."""

import math
from collections import Counter

import pytest
import torch

from bridge_amd import TPRPrefixMeta, _lib

CPU = torch.device("cpu")

# header word indices (bridge_amd/csrc/tpr_common.h)
PF = dict(MAGIC=0, NUM_LEAVES=2, NUM_NODES=3, MAX_DEPTH=4, TOTAL_Q=5, TOTAL_PREFIX=6, HQ=7, HKV=8, D=9,
          PATH=11, OFF_CU=12, OFF_NODE_OFF=13, OFF_ANC=14, OFF_NODE_LEAF=15, N_QBLK=16, OFF_QBLK=17,
          OFF_LEAF_QBLK=18, N_FWD=19, OFF_FWD=20, N_DKDV=21, OFF_DKDV=22, N_RED=23, TOTAL_WORDS=27,
          OFF_RUNS=28, MAX_RUNS=29, DS_SLOTS=30, OFF_DS=31, MASK_COLS=32, N_DQS=33, OFF_DQS=34)

FWD_WAVES = 8  # waves per forward / dQ workgroup (kFwdWaves)


def decode(plan):
    w = plan.host.tolist()
    assert w[PF["MAGIC"]] == 0x31525054 and w[PF["TOTAL_WORDS"]] == len(w)
    fwd = [tuple(w[w[PF["OFF_FWD"]] + 4 * i: w[PF["OFF_FWD"]] + 4 * i + 4]) for i in range(w[PF["N_FWD"]])]
    dkdv = [tuple(w[w[PF["OFF_DKDV"]] + 8 * i: w[PF["OFF_DKDV"]] + 8 * i + 8]) for i in range(w[PF["N_DKDV"]])]
    qblk = [tuple(w[w[PF["OFF_QBLK"]] + 2 * i: w[PF["OFF_QBLK"]] + 2 * i + 2]) for i in range(w[PF["N_QBLK"]])]
    return w, fwd, dkdv, qblk


def tiles_of(dkdv, block_rows=64):
    """The (src, seg, key0, kvh, lo, hi, slot) tiles of dK/dV items, a paired
    item (last word 1 + second key0) giving both of its suffix tiles; the
    second tile's query range starts (key0 - key0b) / block_rows blocks
    earlier and ends at the same block."""
    out = []
    for src, seg, key0, kvh, lo, hi, slot, pair in dkdv:
        if src < 0:
            continue
        out.append((src, seg, key0, kvh, lo, hi, slot))
        if pair > 0:
            k0b = pair - 1
            out.append((src, seg, k0b, kvh, lo - (key0 - k0b) // block_rows, hi, slot))
    return out


@pytest.mark.parametrize("hq,hkv", [(32, 8), (8, 2), (4, 4), (6, 2), (4, 2)])
def test_forward_items_cover_every_query_row_once(hq, hkv):
    meta = TPRPrefixMeta(cu_seqlens_q=(0, 100, 100, 357), node_offsets=(0, 64, 200),
                         leaf_ancestors=((0, 1), (0,), (0,)))
    plan = meta.plan(hq, hkv, 128, torch.bfloat16, CPU)
    assert plan.path == "mfma"
    _, fwd, _, _ = decode(plan)
    g = hq // hkv
    # a forward/dQ workgroup is FWD_WAVES waves of 32 tokens each: hpw query
    # heads (the largest divisor of the group size that divides FWD_WAVES),
    # FWD_WAVES / hpw waves per head
    hpw = math.gcd(g, FWD_WAVES)
    tpw = 32 * (FWD_WAVES // hpw)
    covered = Counter()
    for leaf, tok0, qh0, kvh in fwd:
        if leaf < 0:
            continue
        assert kvh == qh0 // g and qh0 % hpw == 0
        length = meta.cu_seqlens_q[leaf + 1] - meta.cu_seqlens_q[leaf]
        for h in range(qh0, qh0 + hpw):
            for t in range(tok0, min(tok0 + tpw, length)):
                covered[(leaf, t, h)] += 1
    expected = {(s, t, h) for s in range(3) for t in range(meta.cu_seqlens_q[s + 1] - meta.cu_seqlens_q[s])
                for h in range(hq)}
    assert set(covered) == expected and set(covered.values()) == {1}


def test_xcd_ordering_pins_kv_heads_and_is_lpt_per_xcd():
    meta = TPRPrefixMeta.shared_prefix(4096, [4096] * 4)
    plan = meta.plan(32, 8, 128, torch.bfloat16, CPU)
    _, fwd, dkdv, _ = decode(plan)
    # the prefix tiles' query range (4 siblings x 64 query blocks) is below one
    # CU's share of the launch (about 388 blocks), so no tile is split
    tpw = 32 * (FWD_WAVES // 4)  # tokens per forward workgroup (4 query heads of the group)
    # dK/dV: 32 prefix tiles, and each leaf's 32 suffix tiles as 16 mirror
    # pairs (tile j with tile 31 - j), per KV head
    assert len(fwd) == 4 * (4096 // tpw) * 8 and len(dkdv) == (32 + 4 * 16) * 8
    assert all(item[6] == -1 for item in dkdv) and plan.host[23].item() == 0   # no partial slots, no reductions
    assert len(tiles_of(dkdv)) == (32 + 4 * 32) * 8
    for i, (leaf, tok0, qh0, kvh) in enumerate(fwd):
        assert leaf >= 0 and kvh == i % 8
    for i, item in enumerate(dkdv):
        assert item[3] == i % 8
    # forward: leaf-major (equal leaves keep their order), decreasing causal
    # work (prefix + tokens seen) within a leaf, in each XCD queue
    for x in range(8):
        key = [(leaf, -(4096 + min(tok0 + tpw, 4096))) for (leaf, tok0, _, _) in fwd[x::8]]
        assert key == sorted(key)


def test_forward_items_of_ragged_leaves_run_longest_leaf_first():
    lens = [300, 900, 64, 900, 513]
    meta = TPRPrefixMeta.shared_prefix(256, lens)
    _, fwd, _, _ = decode(meta.plan(32, 8, 128, torch.bfloat16, CPU))
    rank = {s: r for r, s in enumerate(sorted(range(len(lens)), key=lambda s: -lens[s]))}  # stable: 1 before 3
    for x in range(8):
        leaves = [leaf for (leaf, _, _, _) in fwd[x::8] if leaf >= 0]
        assert [rank[s] for s in leaves] == sorted(rank[s] for s in leaves)


def test_dkdv_items_cover_every_key_tile_and_query_block():
    meta = TPRPrefixMeta(cu_seqlens_q=(0, 33, 98, 138, 155), node_offsets=(0, 130, 200, 270, 290),
                         leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2)))   # node 3 is unused
    plan = meta.plan(8, 2, 128, torch.bfloat16, CPU)
    w, _, dkdv, qblk = decode(plan)
    leaf_qblk = w[w[PF["OFF_LEAF_QBLK"]]: w[PF["OFF_LEAF_QBLK"]] + 5]
    seen = Counter()
    for src, seg, key0, kvh, lo, hi, slot in tiles_of(dkdv):
        assert slot == -1
        seen[(src, seg, key0, kvh)] += 1
        leaves = {qblk[i][0] for i in range(lo, hi)}
        if src == 0:
            expected = {s for s, a in enumerate(meta.leaf_ancestors) if seg in a}
            assert leaves == expected
            assert (lo, hi) == ((leaf_qblk[min(expected)], leaf_qblk[max(expected) + 1]) if expected else (lo, lo))
        else:
            assert leaves <= {seg} and hi == leaf_qblk[seg + 1]
            assert all(qblk[i][1] + 64 > key0 for i in range(lo, hi))
    for n in range(4):
        length = meta.node_offsets[n + 1] - meta.node_offsets[n]
        for k0 in range(0, length, 128):
            for h in range(2):
                assert seen[(0, n, k0, h)] == 1
    for s in range(4):
        length = meta.cu_seqlens_q[s + 1] - meta.cu_seqlens_q[s]
        for k0 in range(0, length, 128):
            for h in range(2):
                assert seen[(1, s, k0, h)] == 1


def test_split_prefix_tiles_have_ordered_partials_and_reductions():
    meta = TPRPrefixMeta.shared_prefix(300, [4096, 4096, 100, 4096])
    plan = meta.plan(8, 2, 128, torch.bfloat16, CPU)
    w, _, dkdv, qblk = decode(plan)
    reds = [tuple(w[w[24] + 8 * i: w[24] + 8 * i + 8]) for i in range(w[PF["N_RED"]])]
    n_slots = w[25]
    # workspace: stat area (2 constants padded to 64 floats, then lse*log2e and
    # -delta per (query head, token), each rounded up to 64 floats), then the
    # fp32 partial slots, then the dS store (16 KiB per slot and query head)
    total_q = 4096 * 3 + 100
    stat_floats = 64 + 2 * ((8 * total_q + 63) // 64 * 64)
    fp32_bytes = (stat_floats + n_slots * 2 * 128 * 128) * 4
    assert n_slots > 0 and plan.dq_from_ds and plan.workspace_bytes == fp32_bytes + w[PF["DS_SLOTS"]] * 8 * 16384
    compact = meta.plan(8, 2, 128, torch.bfloat16, CPU, recompute_dq=True)
    assert not compact.dq_from_ds and compact.workspace_bytes == fp32_bytes
    by_slot = {item[6]: item for item in dkdv if item[0] >= 0 and item[6] >= 0}
    assert sorted(by_slot) == list(range(n_slots))
    for src, seg, key0, kvh, slot0, nslots, _, _ in reds:
        parts = [by_slot[slot0 + j] for j in range(nslots)]
        assert all(p[:4] == (src, seg, key0, kvh) for p in parts)
        # chunks tile the query range contiguously, in order
        for a, b in zip(parts, parts[1:]):
            assert a[5] == b[4]
        assert all(p[5] - p[4] <= (64 if src == 0 else 256) for p in parts)
    # every direct tile streams at most 256 query blocks (its LDS table)
    assert all(t[5] - t[4] <= 256 for t in tiles_of(dkdv))
    # each (tile, head) is either direct or reduced, never both
    direct = {t[:4] for t in tiles_of(dkdv) if t[6] < 0}
    reduced = {r[:4] for r in reds}
    assert not direct & reduced


@pytest.mark.parametrize("d,kt", [(128, 128), (256, 64)])
def test_suffix_tiles_pair_with_their_mirror(d, kt):
    """bf16 MFMA at head_dim 128 and 256 (kt keys per dK/dV tile, 64-query
    blocks), where one dK/dV workgroup fills a CU: suffix tile j of a
    leaf with T tiles shares an item with tile T-1-j (the shorter one named
    first), so all pairs of a leaf stream the same number of query blocks; the
    middle tile of an odd count, and tiles whose query range is split (and
    their mirrors), stay alone; every (tile, KV head) is covered once."""
    lens = [4096, 4000, 333, 100, 20000]
    meta = TPRPrefixMeta.shared_prefix(256, lens)
    plan = meta.plan(8, 2, d, torch.bfloat16, CPU)
    w, _, dkdv, qblk = decode(plan)
    per = kt // 64  # query blocks per tile
    leaf_qblk = w[w[PF["OFF_LEAF_QBLK"]]: w[PF["OFF_LEAF_QBLK"]] + len(lens) + 1]
    items = [it for it in dkdv if it[0] >= 0]
    pair_blocks = {}
    paired = set()
    for src, seg, key0, kvh, lo, hi, slot, pair in items:
        if pair == 0:
            continue
        ntiles = -(-lens[seg] // kt)
        k0b = pair - 1
        assert src == 1 and slot == -1 and key0 > k0b and key0 // kt == ntiles - 1 - k0b // kt
        assert lo == leaf_qblk[seg] + key0 // 64 and hi == leaf_qblk[seg + 1]
        long_range = hi - (leaf_qblk[seg] + k0b // 64)
        assert long_range <= 256
        pair_blocks.setdefault(seg, set()).add((hi - lo) + long_range)
        paired |= {(seg, key0 // kt, kvh), (seg, k0b // kt, kvh)}
    # all pairs of a leaf stream the same number of blocks
    assert all(len(v) == 1 for v in pair_blocks.values())
    singles = {(it[1], it[2] // kt, it[3]) for it in items if it[0] == 1 and it[7] == 0}
    for seg, n in enumerate(lens):
        ntiles = -(-n // kt)
        blocks = leaf_qblk[seg + 1] - leaf_qblk[seg]
        for j in range(ntiles):
            mirror = ntiles - 1 - j
            long_j = min(j, mirror)
            pairable = mirror != j and blocks - per * long_j <= 256
            for h in range(2):
                assert ((seg, j, h) in paired) == pairable, (seg, j)
                assert ((seg, j, h) in singles) != pairable, (seg, j)
    if kt == 128:
        # the 20000-token leaf (313 blocks): tiles 0..28 stream more than 256
        # blocks (split), so they and their mirrors 128..156 stay alone, and
        # so does the middle tile 78
        assert {j for (seg, j, h) in singles if seg == 4 and h == 0} == set(range(29)) | set(range(128, 157)) | {78}
        assert {j for (seg, j, h) in singles if seg == 2 and h == 0} == {1} and (3, 0, 0) in singles
    else:
        # 313 tiles of 64 keys: tiles 0..56 split, their mirrors 256..312 alone,
        # middle 156; the 333- and 100-token leaves (6 and 2 tiles) pair fully
        assert {j for (seg, j, h) in singles if seg == 4 and h == 0} == set(range(57)) | set(range(256, 313)) | {156}
        assert not {j for (seg, j, h) in singles if seg in (2, 3)}
    # coverage of every (tile, head) once, prefix and suffix
    seen = Counter(t[:4] for t in tiles_of(dkdv) if t[6] < 0)
    reds = [tuple(w[w[24] + 8 * i: w[24] + 8 * i + 8]) for i in range(w[PF["N_RED"]])]
    seen.update(r[:4] for r in reds)
    expected = {(0, 0, k0, h) for k0 in range(0, 256, kt) for h in range(2)}
    expected |= {(1, s, k0, h) for s, n in enumerate(lens) for k0 in range(0, n, kt) for h in range(2)}
    assert set(seen) == expected and set(seen.values()) == {1}


def test_suffix_tiles_stay_single_where_dkdv_workgroups_share_a_cu():
    """head_dim 64 (several dK/dV workgroups per CU) and the SIMT kernels."""
    meta = TPRPrefixMeta.shared_prefix(64, [1000, 700])
    for d, dtype, path in ((64, torch.bfloat16, "mfma"), (128, torch.float32, "simt"),
                           (96, torch.bfloat16, "simt"), (256, torch.float32, "simt")):
        plan = meta.plan(8, 2, d, dtype, CPU)
        assert plan.path == path
        _, _, dkdv, _ = decode(plan)
        assert all(it[7] == 0 for it in dkdv)


def key_runs(plan):
    """(max_runs, per-leaf [(row, len)]) from the plan's key-run table."""
    w = plan.host.tolist()
    off, width = w[PF["OFF_RUNS"]], w[PF["MAX_RUNS"]]
    runs = []
    for s in range(w[PF["NUM_LEAVES"]]):
        e = w[off + 2 * width * s: off + 2 * width * (s + 1)]
        pairs = [(e[2 * i], e[2 * i + 1]) for i in range(width)]
        n = sum(1 for _, ln in pairs if ln > 0)
        assert all(ln > 0 for _, ln in pairs[:n]) and pairs[n:] == [(0, 0)] * (width - n)
        runs.append(pairs[:n])
    return width, runs


def test_deep_chain_laid_out_root_first_is_one_key_run():
    depth = 9
    meta = TPRPrefixMeta(cu_seqlens_q=(0, 5), node_offsets=tuple(range(0, 4 * depth + 1, 4)),
                         leaf_ancestors=(tuple(range(depth)),))
    plan = meta.plan(4, 2, 128, torch.bfloat16, CPU)
    assert plan.path == "mfma"
    assert key_runs(plan) == (1, [[(0, 36)]])


def test_deep_chain_laid_out_leaf_first_keeps_one_run_per_node():
    # root = node 8 at rows [32, 36), its child node 7 at [28, 32), ...: no
    # ancestor starts where the previous one (root first) ends
    depth = 12
    meta = TPRPrefixMeta(cu_seqlens_q=(0, 5), node_offsets=tuple(range(0, 4 * depth + 1, 4)),
                         leaf_ancestors=(tuple(reversed(range(depth))),))
    plan = meta.plan(4, 2, 128, torch.bfloat16, CPU)
    assert plan.path == "mfma"
    assert key_runs(plan) == (12, [[(4 * n, 4) for n in reversed(range(depth))]])


def test_key_runs_merge_adjacent_ancestors_and_drop_empty_nodes():
    # node 0 [0, 10), node 1 empty, node 2 [10, 30) under 1, node 3 [30, 45) under 0
    meta = TPRPrefixMeta(cu_seqlens_q=(0, 5, 9, 12), node_offsets=(0, 10, 10, 30, 45),
                         leaf_ancestors=((0, 1, 2), (0, 3), ()))
    width, runs = key_runs(meta.plan(8, 2, 128, torch.bfloat16, CPU))
    assert width == 2
    assert runs == [[(0, 30)], [(0, 10), (30, 15)], []]
    # the visible keys of each leaf are unchanged by the merging
    for leaf, leaf_runs in enumerate(runs):
        assert sum(ln for _, ln in leaf_runs) == meta.prefix_length(leaf)


def test_kernel_family_by_dtype_and_head_dim():
    meta = TPRPrefixMeta.shared_prefix(512, [512, 512])
    def kind(hq, hkv, d, dtype):
        plan = meta.plan(hq, hkv, d, dtype, CPU)
        return plan.path, plan.mfma_shape
    assert kind(4, 4, 64, torch.float32) == ("simt", None)
    assert kind(4, 4, 64, torch.bfloat16) == ("mfma", "16x16x32")
    assert kind(4, 4, 128, torch.float32) == ("simt", None)
    assert kind(4, 4, 128, torch.bfloat16) == ("mfma", "32x32x16")
    assert kind(8, 2, 256, torch.bfloat16) == ("mfma", "16x16x32")
    assert kind(8, 2, 256, torch.float32) == ("simt", None)
    assert kind(6, 2, 96, torch.bfloat16) == ("simt", None)


def test_mfma16_work_items():
    """head_dim 64 / 256: forward items of 32 tokens x 4 waves / gcd(G, 4) heads,
    dK/dV items of 64 keys, 64-query blocks."""
    meta = TPRPrefixMeta.shared_prefix(100, [130, 64])
    plan = meta.plan(8, 2, 256, torch.bfloat16, CPU)
    w, fwd, dkdv, qblk = decode(plan)
    items = [i for i in fwd if i[0] >= 0]
    # G = 4: 4 heads x 32 tokens per item
    assert sorted((i[0], i[1], i[2]) for i in items) == sorted(
        (leaf, tok, qh) for leaf, n in ((0, 130), (1, 64)) for tok in range(0, n, 32) for qh in (0, 4))
    tiles = [i for i in dkdv if i[0] >= 0]
    prefix_tiles = sorted((i[2], i[3]) for i in tiles if i[0] == 0)
    assert prefix_tiles == [(k0, h) for k0 in (0, 64) for h in (0, 1)]
    assert all(i[2] % 64 == 0 for i in tiles)
    assert qblk == [(0, 0), (0, 64), (0, 128), (1, 0)]


def test_plan_is_cached_per_configuration():
    meta = TPRPrefixMeta.shared_prefix(8, [4])
    a = meta.plan(4, 2, 128, torch.bfloat16, CPU)
    assert meta.plan(4, 2, 128, torch.bfloat16, CPU) is a
    assert meta.plan(4, 2, 64, torch.bfloat16, CPU) is not a


@pytest.mark.parametrize(
    ("kwargs", "exc", "match"),
    [
        (dict(cu_seqlens_q=(0, 4, 8), node_offsets=(0, 4, 8), leaf_ancestors=((0, 1), (1,))), ValueError,
         "inconsistent paths"),
        (dict(cu_seqlens_q=(0, 4, 8, 12), node_offsets=(0, 4, 8), leaf_ancestors=((0,), (1,), (0,))), ValueError,
         "not contiguous"),
        (dict(cu_seqlens_q=(0, 4), node_offsets=(0, 4), leaf_ancestors=((3,),)), ValueError, "out of range"),
        (dict(cu_seqlens_q=(0, 4), node_offsets=(0, 4, 6), leaf_ancestors=((-1, 0),)), ValueError, "padding"),
        (dict(cu_seqlens_q=(0, 4, 2), node_offsets=(0, 4), leaf_ancestors=((0,), (0,))), ValueError,
         "non-decreasing"),
        (dict(cu_seqlens_q=(1, 4), node_offsets=(0, 4), leaf_ancestors=((0,),)), ValueError, r"cu_seqlens_q\[0\]"),
        (dict(cu_seqlens_q=(0, 4), node_offsets=(0, 5, 3), leaf_ancestors=((0,),)), ValueError, "node_offsets"),
        (dict(cu_seqlens_q=(0, 4), node_offsets=(0, 4), leaf_ancestors=((0, 0),)), ValueError, "inconsistent"),
    ],
)
def test_planner_rejects_invalid_trees(kwargs, exc, match):
    meta = TPRPrefixMeta(**kwargs)
    with pytest.raises(exc, match=match):
        meta.plan(4, 2, 128, torch.bfloat16, CPU)


@pytest.mark.parametrize(("hq", "hkv", "d", "exc", "match"),
                         [(6, 4, 128, ValueError, "divisible"), (4, 2, 264, NotImplementedError, "at most 256"),
                          (4, 2, 60, NotImplementedError, "multiple of 8")])
def test_planner_rejects_unsupported_heads(hq, hkv, d, exc, match):
    with pytest.raises(exc, match=match):
        TPRPrefixMeta.shared_prefix(8, [4]).plan(hq, hkv, d, torch.bfloat16, CPU)


def test_planner_rejects_other_dtypes():
    with pytest.raises(ValueError, match="bfloat16 and torch.float32"):
        TPRPrefixMeta.shared_prefix(8, [4]).plan(4, 2, 128, torch.float16, CPU)


def test_planner_rejects_unknown_plan_flags():
    import ctypes

    from bridge_amd import _lib
    lib = _lib.load()
    cu = (ctypes.c_int32 * 2)(0, 4)
    no = (ctypes.c_int32 * 2)(0, 8)
    an = (ctypes.c_int32 * 1)(0)
    for flags, ok in ((0, True), (_lib.TPR_PLAN_RECOMPUTE_DQ, True), (_lib.TPR_PLAN_MASKED, True),
                      (_lib.TPR_PLAN_MASKED | _lib.TPR_PLAN_RECOMPUTE_DQ, True), (4, False), (-1, False)):
        desc = _lib.TprTreeDesc(1, 1, 1, 4, 2, 128, _lib.TPR_DTYPE_BF16, flags, ctypes.cast(cu, ctypes.c_void_p),
                                ctypes.cast(no, ctypes.c_void_p), ctypes.cast(an, ctypes.c_void_p))
        words = ctypes.c_int64(0)
        rc = lib.tpr_attn_plan(ctypes.byref(desc), None, 0, ctypes.byref(words))
        assert (rc == _lib.TPR_OK) == ok, (flags, rc)
        if not ok:
            assert rc == _lib.TPR_ERR_INVALID_ARGUMENT and b"plan flags" in lib.tpr_attn_last_error()


@pytest.mark.parametrize("dtype, d", [(torch.bfloat16, 128), (torch.bfloat16, 64), (torch.float32, 96)])
def test_masked_plan_runs_simt_items_over_every_suffix_key(dtype, d):
    """A masked plan (the mask the only visibility rule) runs the SIMT
    kernels whatever the dtype and head size, records the longest key
    sequence as the least mask row length, gives every suffix tile's dK/dV
    item all of its leaf's query blocks (a mask may show later keys), and
    still covers every key tile once."""
    meta = TPRPrefixMeta(cu_seqlens_q=(0, 33, 98, 138, 155), node_offsets=(0, 130, 200, 270, 290),
                         leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2)))
    plan = meta.plan(8, 2, d, dtype, CPU, masked=True)
    assert plan.path == "simt" and plan.masked and not plan.dq_from_ds and plan.workspace_bytes == 0
    w, fwd, dkdv, qblk = decode(plan)
    assert w[PF["MASK_COLS"]] == meta.max_keys() == 200 + 65
    leaf_qblk = w[w[PF["OFF_LEAF_QBLK"]]: w[PF["OFF_LEAF_QBLK"]] + 5]
    seen = Counter()
    for src, seg, key0, kvh, lo, hi, slot in tiles_of(dkdv):
        seen[(src, seg, key0, kvh)] += 1
        if src == 1:
            assert (lo, hi) == (leaf_qblk[seg], leaf_qblk[seg + 1])
    for s in range(4):
        length = meta.cu_seqlens_q[s + 1] - meta.cu_seqlens_q[s]
        assert all(seen[(1, s, k0, h)] == 1 for k0 in range(0, length, 64) for h in range(2))
    assert not meta.plan(8, 2, d, dtype, CPU).masked


def test_segment_tree_lowering_turn_tree():
    # root 2048 -> 4 branches x 1024 -> 4 leaves x 1024 each (turn-boundary tree, depth 3)
    parents = {0: None}
    lengths = {0: 2048}
    for b in range(4):
        parents[1 + b] = 0
        lengths[1 + b] = 1024
    for i in range(16):
        parents[100 + i] = 1 + i // 4
        lengths[100 + i] = 1024
    meta, nodes, leaves = TPRPrefixMeta.from_segment_tree(parents, lengths)
    assert nodes == (0, 1, 2, 3, 4) and leaves == tuple(range(100, 116))
    assert meta.node_offsets == (0, 2048, 3072, 4096, 5120, 6144)
    assert meta.leaf_ancestors == tuple((0, 1 + i // 4) for i in range(16))
    assert meta.visible_pairs() == 58728448
    meta.plan(32, 8, 128, torch.bfloat16, CPU)  # valid for the planner


def test_segment_tree_lowering_of_a_long_chain_is_iterative():
    """A chain of 2500 segments (deeper than Python's recursion limit) lowers to
    2499 nested nodes and one leaf; a side branch keeps insertion order."""
    n = 2500
    parents = {0: None, **{s: s - 1 for s in range(1, n)}}
    lengths = {s: 1 + s % 3 for s in range(n)}
    parents[n] = 0                      # second child of the root, inserted last
    lengths[n] = 7
    meta, nodes, leaves = TPRPrefixMeta.from_segment_tree(parents, lengths)
    assert nodes == tuple(range(n - 1)) and leaves == (n - 1, n)
    assert meta.leaf_ancestors[0] == tuple(range(n - 1)) and meta.leaf_ancestors[1] == (0,)
    assert meta.cu_seqlens_q == (0, lengths[n - 1], lengths[n - 1] + 7)
    assert meta.node_offsets[-1] == sum(lengths[s] for s in range(n - 1))


def test_segment_tree_lowering_rejects_two_roots():
    with pytest.raises(ValueError, match="exactly one root"):
        TPRPrefixMeta.from_segment_tree({0: None, 1: None}, {0: 1, 1: 1})


def test_empty_leaves_and_prefixless_trees_plan():
    meta = TPRPrefixMeta.shared_prefix(0, [0, 5, 0])
    plan = meta.plan(4, 1, 128, torch.bfloat16, CPU)
    _, fwd, dkdv, _ = decode(plan)
    assert {item[0] for item in fwd if item[0] >= 0} == {1}
    assert all(item[0] == 1 for item in dkdv if item[0] >= 0)


def _ds_tables(w):
    """(base, first): tiles ahead of each segment (nodes, then leaf suffixes)
    in a query block's dQ walk, and each query block's first slot."""
    m, n, nq = w[PF["NUM_NODES"]], w[PF["NUM_LEAVES"]], w[PF["N_QBLK"]]
    off = w[PF["OFF_DS"]]
    return w[off:off + m + n], w[off + m + n: off + m + n + nq + 1]


def _ds_reads_and_writes(meta, hq, hkv, d=128):
    """Emulate the slot arithmetic of the bf16 backward with a dS store: the
    (slot, query head, wave block) triples every dK/dV stage writes (slot =
    first[block] + base[segment] + tile), and those every dQ wave reads (slot =
    first[block] + position of the tile in the wave's key walk: ancestor nodes
    root first, then the suffix; a block wholly past its segment's end is
    masked, not read). Both take the plan's own dQ items (8 waves). head_dim
    128: 128-key tiles of four 32-key wave blocks, dQ waves of 64 tokens
    streaming 64-key halves; head_dim 256: 64-key tiles of four 16-key wave
    blocks, dQ waves of 32 tokens streaming whole tiles. Also returns, per dQ
    wave, the byte offsets of its reads in the [KV head][slot][query head of
    the group] store."""
    plan = meta.plan(hq, hkv, d, torch.bfloat16, CPU)
    assert plan.dq_from_ds
    kt, wk, wt, step = (128, 32, 64, 64) if d == 128 else (64, 16, 32, 64)
    waves = 8
    head_bytes = kt * 64 * 2
    w, fwd, dkdv, qblk = decode(plan)
    # the dQ kernel's own items
    fwd = [tuple(w[w[PF["OFF_DQS"]] + 4 * i: w[PF["OFF_DQS"]] + 4 * i + 4]) for i in range(w[PF["N_DQS"]])]
    assert fwd
    g = hq // hkv
    n_slots = w[PF["DS_SLOTS"]]
    base, first = _ds_tables(w)
    m = meta.num_nodes
    cu, no = meta.cu_seqlens_q, meta.node_offsets
    leaf_qblk = w[w[PF["OFF_LEAF_QBLK"]]: w[PF["OFF_LEAF_QBLK"]] + meta.num_leaves + 1]

    def seg_len(src, seg):
        return no[seg + 1] - no[seg] if src == 0 else cu[seg + 1] - cu[seg]

    writes = Counter()
    for src, seg, key0, kvh, lo, hi, _ in tiles_of(dkdv):
        for qb in range(lo, hi):
            slot = first[qb] + base[seg if src == 0 else m + seg] + key0 // kt
            assert first[qb] <= slot < first[qb + 1] <= n_slots
            for wv in range(4):
                if key0 + wk * wv < seg_len(src, seg):  # active waves only
                    for head in range(kvh * g, kvh * g + g):
                        writes[(slot, head, wv)] += 1
    reads = set()
    wave_offsets = []
    hpw = math.gcd(g, waves)
    tpw = wt * (waves // hpw)
    for leaf, tok0, qh0, kvh in fwd:
        if leaf < 0:
            continue
        length = cu[leaf + 1] - cu[leaf]
        segs = [(0, nd, no[nd + 1] - no[nd], no[nd + 1] - no[nd]) for nd in meta.leaf_ancestors[leaf]
                if no[nd + 1] > no[nd]]
        segs.append((1, leaf, length, min(length, tok0 + tpw)))
        for wave in range(waves):
            head, tw0 = qh0 + wave % hpw, tok0 + wt * (wave // hpw)
            if tw0 >= length:
                continue
            qb = leaf_qblk[leaf] + tw0 // 64
            pos, offs = 0, []
            for src, seg, slen, lim in segs:
                for key0 in range(0, lim, kt):
                    for k0 in range(key0, min(key0 + kt, lim), step):  # the dQ kernel's tiles (halves at 128)
                        if src == 1 and k0 > tw0 + wt - 1:
                            continue
                        slot = first[qb] + pos
                        assert slot == first[qb] + base[seg if src == 0 else m + seg] + key0 // kt
                        assert first[qb] <= slot < first[qb + 1]
                        offs.append(((kvh * n_slots + slot) * g + head - kvh * g) * head_bytes + (k0 - key0) * 128)
                        for wv in range((k0 - key0) // wk, (k0 - key0 + step) // wk):
                            if key0 + wk * wv < slen:
                                reads.add((slot, head, wv))
                    pos += 1
            wave_offsets.append(offs)
    return n_slots, writes, reads, wave_offsets


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (16, 2), (32, 8), (6, 2), (4, 4), (16, 1)])
def test_dq_from_store_items_cover_every_query_row_once(hq, hkv, d):
    """The dS-store dQ kernels take the plan's own work items (PF_N_DQS /
    PF_OFF_DQS): 8 waves of one query head each, 64 tokens (one query block)
    at head_dim 128 and 32 at head_dim 256, hpw = gcd(group, 8) heads per
    item, so 8 / hpw times a wave's tokens per item. Every (leaf, token,
    query head) is in exactly one item, items of one KV head only, and an
    item's tokens start a query block; the list exists only with a dS store."""
    meta = TPRPrefixMeta(cu_seqlens_q=(0, 100, 163, 163, 420), node_offsets=(0, 64, 200),
                         leaf_ancestors=((0, 1), (0, 1), (0,), (0,)))
    plan = meta.plan(hq, hkv, d, torch.bfloat16, CPU)
    assert plan.path == "mfma" and plan.dq_from_ds
    w = plan.host.tolist()
    n, off = w[PF["N_DQS"]], w[PF["OFF_DQS"]]
    assert n > 0 and off > 0
    items = [tuple(w[off + 4 * i: off + 4 * i + 4]) for i in range(n)]
    g = hq // hkv
    hpw = math.gcd(g, 8)
    tpw = (64 if d == 128 else 32) * (8 // hpw)
    covered = Counter()
    for leaf, tok0, qh0, kvh in items:
        if leaf < 0:
            continue
        assert kvh == qh0 // g and qh0 % hpw == 0 and tok0 % tpw == 0
        length = meta.cu_seqlens_q[leaf + 1] - meta.cu_seqlens_q[leaf]
        assert 0 <= tok0 < length
        for h in range(qh0, qh0 + hpw):
            for t in range(tok0, min(tok0 + tpw, length)):
                covered[(leaf, t, h)] += 1
    expected = {(s, t, h) for s in range(4) for t in range(meta.cu_seqlens_q[s + 1] - meta.cu_seqlens_q[s])
                for h in range(hq)}
    assert set(covered) == expected and set(covered.values()) == {1}
    # no list where dQ recomputes and takes the forward's items
    for dd, kw in ((d, dict(recompute_dq=True)), (64, {})):
        other = meta.plan(hq, hkv, dd, torch.bfloat16, CPU, **kw).host.tolist()
        assert other[PF["N_DQS"]] == 0 and other[PF["OFF_DQS"]] == 0


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("case", ["split_prefix", "depth3_ragged", "empty_leaves", "gqa8", "gqa3", "mha"])
def test_ds_store_is_written_once_before_every_dq_read(case, d):
    trees = {
        "split_prefix": (TPRPrefixMeta.shared_prefix(300, [4096, 4096, 100, 4096]), 8, 2),
        "depth3_ragged": (TPRPrefixMeta(cu_seqlens_q=(0, 33, 98, 138, 155, 420), node_offsets=(0, 130, 200, 270),
                                        leaf_ancestors=((0, 1), (0, 1), (0, 2), (0, 2), (0,))), 8, 2),
        "empty_leaves": (TPRPrefixMeta.shared_prefix(50, [0, 260, 0, 64]), 4, 1),
        "gqa8": (TPRPrefixMeta.shared_prefix(130, [70, 300]), 16, 2),
        "gqa3": (TPRPrefixMeta.shared_prefix(200, [129, 20, 257]), 6, 2),
        "mha": (TPRPrefixMeta.shared_prefix(0, [200, 65]), 4, 4),
    }
    meta, hq, hkv = trees[case]
    n_slots, writes, reads, wave_offsets = _ds_reads_and_writes(meta, hq, hkv, d)
    assert set(writes.values()) == {1}  # no block is written twice
    assert reads <= set(writes)         # every read block was written
    # the store holds exactly the visible (tile, query block) pairs: each slot is read
    assert {r[0] for r in reads} == set(range(n_slots))
    # a dQ wave's reads move forward through the store, one slot of its group per tile
    head_bytes = (128 if d == 128 else 64) * 64 * 2
    for offs in wave_offsets:
        assert offs == sorted(offs)
        assert all(0 <= o < n_slots * hq * head_bytes for o in offs)


def test_ds_store_size_at_the_qwen3_layer_shape():
    """Prefix 4096 + 4 x 4096, GQA 32/8: 32 prefix tiles x 256 query blocks
    plus, per leaf, sum over its 32 suffix tiles of (64 - 2 j) blocks."""
    meta = TPRPrefixMeta.shared_prefix(4096, [4096] * 4)
    plan = meta.plan(32, 8, 128, torch.bfloat16, CPU)
    w = plan.host.tolist()
    slots = 32 * 256 + 4 * sum(64 - 2 * j for j in range(32))
    assert w[PF["DS_SLOTS"]] == slots == 12416
    fp32 = meta.plan(32, 8, 128, torch.bfloat16, CPU, recompute_dq=True).workspace_bytes
    assert plan.workspace_bytes == fp32 + slots * 32 * 16384  # 6.5 GB
    # head_dim 256 (64-key tiles, 8 KiB per head and slot) stores dS too; other paths never do
    q35 = meta.plan(8, 2, 256, torch.bfloat16, CPU)
    slots256 = 64 * 256 + 4 * sum(64 - j for j in range(64))
    assert q35.dq_from_ds and q35.host.tolist()[PF["DS_SLOTS"]] == slots256
    assert q35.workspace_bytes == meta.plan(8, 2, 256, torch.bfloat16, CPU, recompute_dq=True).workspace_bytes + \
        slots256 * 8 * 8192  # 1.6 GB
    assert not meta.plan(32, 8, 64, torch.bfloat16, CPU).dq_from_ds
    assert not meta.plan(32, 8, 128, torch.float32, CPU).dq_from_ds


def test_ds_store_follows_the_byte_budget():
    """The plan has a dS store only when it fits the budget: at the Qwen3-4B
    layer shape the store is 12,416 slots x 32 heads x 16 KiB = 6.51 GB, so a
    budget of one byte less recomputes dQ (small workspace) and one of exactly
    that size stores; the default budget (8 GiB) stores; prefix 32768 + 8 x
    2048 (67,712 slots, 35.5 GB) recomputes under the default and stores
    under a 40 GB budget; budget 0 and recompute_dq=True never store."""
    from bridge_amd.meta import DS_STORE_DEFAULT_BYTES
    assert DS_STORE_DEFAULT_BYTES == _lib.TPR_DS_STORE_DEFAULT_BYTES == 8 << 30
    meta = TPRPrefixMeta.shared_prefix(4096, [4096] * 4)
    store = 12416 * 32 * 16384
    small = meta.plan(32, 8, 128, torch.bfloat16, CPU, ds_store_budget=0)
    assert not small.dq_from_ds and small.host.tolist()[PF["DS_SLOTS"]] == 0
    assert small.workspace_bytes < 8 << 20  # lse*log2e and -delta rows: 2 x 32 x 16384 floats
    for budget, stores in ((store - 1, False), (store, True), (None, True), (1 << 40, True)):
        plan = meta.plan(32, 8, 128, torch.bfloat16, CPU, ds_store_budget=budget)
        assert plan.dq_from_ds == stores, budget
        assert plan.workspace_bytes == small.workspace_bytes + (store if stores else 0)
    assert not meta.plan(32, 8, 128, torch.bfloat16, CPU, recompute_dq=True, ds_store_budget=1 << 40).dq_from_ds

    big = TPRPrefixMeta.shared_prefix(32768, [2048] * 8)
    slots = 256 * 256 + 8 * sum(32 - 2 * j for j in range(16))
    assert slots == 67712 and slots * 32 * 16384 > DS_STORE_DEFAULT_BYTES
    plan = big.plan(32, 8, 128, torch.bfloat16, CPU)
    assert not plan.dq_from_ds and plan.host.tolist()[PF["DS_SLOTS"]] == 0
    assert plan.workspace_bytes == big.plan(32, 8, 128, torch.bfloat16, CPU, ds_store_budget=0).workspace_bytes
    large = big.plan(32, 8, 128, torch.bfloat16, CPU, ds_store_budget=40 * 10**9)
    assert large.dq_from_ds and large.host.tolist()[PF["DS_SLOTS"]] == slots
    # head_dim 256 (8 KiB per head and slot) under the same rule
    q35 = meta.plan(8, 2, 256, torch.bfloat16, CPU)
    assert q35.dq_from_ds
    need = q35.workspace_bytes - meta.plan(8, 2, 256, torch.bfloat16, CPU, ds_store_budget=0).workspace_bytes
    assert not meta.plan(8, 2, 256, torch.bfloat16, CPU, ds_store_budget=need - 1).dq_from_ds
    assert meta.plan(8, 2, 256, torch.bfloat16, CPU, ds_store_budget=need).dq_from_ds


@pytest.mark.parametrize("budget", [-1, -5, 1.5, True, "8G"])
def test_ds_store_budget_rejects_invalid_values(budget):
    meta = TPRPrefixMeta.shared_prefix(64, [64])
    with pytest.raises(ValueError, match="ds_store_budget"):
        meta.plan(4, 1, 128, torch.bfloat16, CPU, ds_store_budget=budget)


def test_planner_rejects_negative_store_budgets_other_than_the_default():
    """Through the C ABI: TPR_DS_STORE_DEFAULT (-1) is the default budget,
    any other negative value is an invalid argument."""
    import ctypes
    lib = _lib.load()
    cu = (ctypes.c_int32 * 2)(0, 64)
    no = (ctypes.c_int32 * 2)(0, 64)
    an = (ctypes.c_int32 * 1)(0)
    words = ctypes.c_int64(0)
    for budget, ok in ((_lib.TPR_DS_STORE_DEFAULT, True), (0, True), (1, True), (-2, False)):
        desc = _lib.TprTreeDesc(1, 1, 1, 4, 1, 128, _lib.TPR_DTYPE_BF16, 0, ctypes.cast(cu, ctypes.c_void_p),
                                ctypes.cast(no, ctypes.c_void_p), ctypes.cast(an, ctypes.c_void_p), budget)
        rc = lib.tpr_attn_plan(ctypes.byref(desc), None, 0, ctypes.byref(words))
        assert (rc == _lib.TPR_OK) == ok, budget
        if not ok:
            assert rc == _lib.TPR_ERR_INVALID_ARGUMENT and b"ds_store_max_bytes" in lib.tpr_attn_last_error()
