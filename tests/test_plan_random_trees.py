"""CPU tests of the native planner on seeded random prefix trees: the work-list
invariants the kernels rely on, checked on the plans themselves (host code
only). The trees are those of the GPU random-tree parity tests: random
segment trees with empty nodes and leaves, relabelled node ids (so a leaf's
ancestors form anywhere from one key run to one run per node), and deep
chains with side branches.

- Forward items (head_dim 64, 128, 256), and the dQ items of a dS-store
  plan: every (leaf, token, query head) in exactly one item.
- dK/dV items: every (segment, key tile, KV head) present, its query blocks
  exactly those that see it (every query block of the leaves under a prefix
  node; a suffix tile's blocks from its diagonal to the leaf's end), split
  tiles as disjoint chunks whose union is that range, each fp32 partial slot
  used once.
- Key runs (the forward's and dQ's key stream over the prefix): each leaf's
  runs, expanded, are its ancestors' prefix_k/v rows root first, with no two
  runs adjacent in prefix_k/v and no empty run.
- dS store (bf16 head_dim 128 and 256): every block dQ reads was written
  exactly once by dK/dV, every slot is read, each dQ wave's reads move
  forward through the store.
"""

import math
from collections import Counter, defaultdict

import pytest
import torch

from test_gpu_random_trees import random_meta
from test_plan import PF, _ds_reads_and_writes, decode, key_runs, tiles_of

CPU = torch.device("cpu")
HEADS = [(32, 8), (8, 2), (6, 2), (4, 4), (16, 2)]
SEEDS = range(16)


def _case(seed):
    meta = random_meta(700 + seed, deep=seed % 4 == 3)
    hq, hkv = HEADS[seed % len(HEADS)]
    return meta, hq, hkv


def _leaf_len(meta, s):
    return meta.cu_seqlens_q[s + 1] - meta.cu_seqlens_q[s]


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("seed", SEEDS)
def test_forward_items_cover_every_query_row_once(seed, d):
    meta, hq, hkv = _case(seed)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, CPU)
    assert plan.path == "mfma"
    _, fwd, _, _ = decode(plan)
    g = hq // hkv
    # head_dim 128: 8 waves of 32 tokens; head_dim 64 and 256: 128-row items
    # of 32 tokens x 4 / hpw heads
    waves = 8 if d == 128 else 4
    hpw = math.gcd(g, waves)
    tpw = 32 * (waves // hpw)
    covered = Counter()
    for leaf, tok0, qh0, kvh in fwd:
        if leaf < 0:
            continue
        assert kvh == qh0 // g and qh0 % hpw == 0 and 0 <= tok0 < _leaf_len(meta, leaf)
        for h in range(qh0, qh0 + hpw):
            for t in range(tok0, min(tok0 + tpw, _leaf_len(meta, leaf))):
                covered[(leaf, t, h)] += 1
    expected = {(s, t, h) for s in range(meta.num_leaves) for t in range(_leaf_len(meta, s)) for h in range(hq)}
    assert set(covered) == expected and set(covered.values()) <= {1}


@pytest.mark.parametrize("d,kt", [(64, 64), (128, 128), (256, 64)])
@pytest.mark.parametrize("seed", SEEDS)
def test_dkdv_tiles_stream_exactly_the_query_blocks_that_see_them(seed, d, kt):
    meta, hq, hkv = _case(seed)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, CPU)
    w, _, dkdv, qblk = decode(plan)
    n_leaves = meta.num_leaves
    leaf_qblk = w[w[PF["OFF_LEAF_QBLK"]]: w[PF["OFF_LEAF_QBLK"]] + n_leaves + 1]
    assert leaf_qblk[-1] == len(qblk)
    chunks = defaultdict(list)
    slots = Counter()
    for src, seg, key0, kvh, lo, hi, slot in tiles_of(dkdv):
        assert key0 % kt == 0 and 0 <= kvh < hkv and lo <= hi
        chunks[(src, seg, key0, kvh)].append((lo, hi))
        if slot >= 0:
            slots[slot] += 1
    assert set(slots.values()) <= {1} and sorted(slots) == list(range(len(slots)))

    def expected_blocks(src, seg, key0):
        if src == 0:
            leaves = [s for s, a in enumerate(meta.leaf_ancestors) if seg in a]
            return set(range(leaf_qblk[min(leaves)], leaf_qblk[max(leaves) + 1])) if leaves else set()
        # a suffix tile is seen by the leaf's blocks whose last row reaches key0
        return {b for b in range(leaf_qblk[seg], leaf_qblk[seg + 1]) if qblk[b][1] + 64 > key0}

    want = set()
    for n in range(meta.num_nodes):
        for key0 in range(0, meta.node_offsets[n + 1] - meta.node_offsets[n], kt):
            want |= {(0, n, key0, h) for h in range(hkv)}
    for s in range(n_leaves):
        for key0 in range(0, _leaf_len(meta, s), kt):
            want |= {(1, s, key0, h) for h in range(hkv)}
    # every tile with a query block that sees it is planned; none that is not a tile
    assert set(chunks) <= want
    for tile in want:
        blocks = expected_blocks(*tile[:3])
        got = Counter(b for lo, hi in chunks.get(tile, []) for b in range(lo, hi))
        assert set(got) == blocks, tile
        assert set(got.values()) <= {1}, tile
        if blocks:
            assert all(qblk[b][0] in ([tile[1]] if tile[0] == 1 else range(n_leaves)) for b in blocks)


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("seed", SEEDS)
def test_dq_from_store_items_cover_every_query_row_once(seed, d):
    """The dS-store dQ kernels' own items: 8 waves of one query head, 64
    tokens each at head_dim 128 and 32 at 256, gcd(group, 8) heads per item."""
    meta, hq, hkv = _case(seed)
    plan = meta.plan(hq, hkv, d, torch.bfloat16, CPU)
    w = plan.host.tolist()
    n, off = w[PF["N_DQS"]], w[PF["OFF_DQS"]]
    if meta.total_q == 0:
        assert not plan.dq_from_ds
        return
    assert plan.dq_from_ds and n > 0
    g = hq // hkv
    hpw = math.gcd(g, 8)
    tpw = (64 if d == 128 else 32) * (8 // hpw)
    covered = Counter()
    for i in range(n):
        leaf, tok0, qh0, kvh = w[off + 4 * i: off + 4 * i + 4]
        if leaf < 0:
            continue
        assert kvh == qh0 // g and qh0 % hpw == 0 and tok0 % tpw == 0 and 0 <= tok0 < _leaf_len(meta, leaf)
        for h in range(qh0, qh0 + hpw):
            for t in range(tok0, min(tok0 + tpw, _leaf_len(meta, leaf))):
                covered[(leaf, t, h)] += 1
    expected = {(s, t, h) for s in range(meta.num_leaves) for t in range(_leaf_len(meta, s)) for h in range(hq)}
    assert set(covered) == expected and set(covered.values()) <= {1}


@pytest.mark.parametrize("d", [128, 256])
@pytest.mark.parametrize("seed", SEEDS)
def test_ds_store_is_written_once_before_every_dq_read(seed, d):
    meta, hq, hkv = _case(seed)
    if meta.total_q == 0:
        pytest.skip("a tree without query rows has no backward")
    n_slots, writes, reads, wave_offsets = _ds_reads_and_writes(meta, hq, hkv, d)
    assert set(writes.values()) <= {1}
    assert reads <= set(writes)
    assert {r[0] for r in reads} == set(range(n_slots))
    head_bytes = (128 if d == 128 else 64) * 64 * 2
    for offs in wave_offsets:
        assert offs == sorted(offs)
        assert all(0 <= o < n_slots * hq * head_bytes for o in offs)


@pytest.mark.parametrize("seed", SEEDS)
def test_key_runs_list_each_leafs_ancestor_rows_root_first(seed):
    meta, hq, hkv = _case(seed)
    width, runs = key_runs(meta.plan(hq, hkv, 128, torch.bfloat16, CPU))
    no = meta.node_offsets
    assert width == max([len(r) for r in runs] + [0])
    for leaf, leaf_runs in enumerate(runs):
        rows = [r for a in meta.leaf_ancestors[leaf] for r in range(no[a], no[a + 1])]
        assert [r for row, ln in leaf_runs for r in range(row, row + ln)] == rows
        # maximal: a run never starts where the previous one ends
        assert all(r0 + l0 != r1 for (r0, l0), (r1, _) in zip(leaf_runs, leaf_runs[1:]))
