// tpr_plan.cpp -- host planner: validates the prefix tree and lowers it to the
// flat int32 plan blob the kernels consume (tree metadata + work lists).
//
// The tree contract follows the reference's SegmentPlan
// (verl/models/mcore/tpr/segment_plan.py:153-313: one parent per segment,
// children start at the parent's end) after lowering to packed offsets, and
// the prefix path order of KVStack.build_past_key_values (kv_stack.py:139-154).
//
// Work lists are ordered for the MI355X dispatcher: workgroup i runs on XCD
// i % 8, so items are dealt into 8 per-XCD queues (all items of one KV head
// on the same XCD when the head count allows it, so that head's prefix K/V
// tiles are fetched into one L2), each queue in decreasing-work order, and
// interleaved back into one array.

#include <algorithm>
#include <cstring>
#include <numeric>
#include <vector>

#include "../../include/tpr_attn.h"
#include "tpr_common.h"
#include "tpr_host.h"

namespace tpr {
namespace {

constexpr int kXcds = 8;

struct Item {
  std::vector<int32_t> words;
  int64_t work;
  int32_t kvh;
};

int gcd_int(int a, int b) { return b == 0 ? a : gcd_int(b, a % b); }

// Deal items into per-XCD queues and interleave; pads with empty items
// (first word -1) so every queue has the same length.
std::vector<int32_t> order_for_xcds(std::vector<Item>& items, int hkv, int words_per_item, int32_t* count) {
  std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) { return a.work > b.work; });
  std::vector<std::vector<const Item*>> queue(kXcds);
  std::vector<int64_t> load(kXcds, 0);
  for (const Item& it : items) {
    int best = -1;
    if (hkv % kXcds == 0) {
      best = it.kvh % kXcds;
    } else if (kXcds % hkv == 0) {
      // head h owns XCDs {h, h + hkv, h + 2*hkv, ...}
      for (int x = it.kvh; x < kXcds; x += hkv)
        if (best < 0 || load[x] < load[best]) best = x;
    } else {
      for (int x = 0; x < kXcds; x++)
        if (best < 0 || load[x] < load[best]) best = x;
    }
    queue[best].push_back(&it);
    load[best] += it.work;
  }
  size_t depth = 0;
  for (auto& q : queue) depth = std::max(depth, q.size());
  std::vector<int32_t> out;
  out.reserve(depth * kXcds * words_per_item);
  for (size_t i = 0; i < depth; i++) {
    for (int x = 0; x < kXcds; x++) {
      if (i < queue[x].size()) {
        out.insert(out.end(), queue[x][i]->words.begin(), queue[x][i]->words.end());
      } else {
        std::vector<int32_t> empty(words_per_item, 0);
        empty[0] = -1;
        out.insert(out.end(), empty.begin(), empty.end());
      }
    }
  }
  // drop trailing all-empty rows (cannot happen: the first row is full when any item exists)
  *count = static_cast<int32_t>(depth * kXcds);
  if (items.empty()) {
    out.clear();
    *count = 0;
  }
  return out;
}

}  // namespace

static int build_plan(const TprTreeDesc* t, std::vector<int32_t>& plan) {
  if (!t) return fail(TPR_ERR_INVALID_ARGUMENT, "tree descriptor is NULL");
  const int N = t->num_leaves, M = t->num_nodes, depth = t->max_depth;
  const int Hq = t->num_q_heads, Hkv = t->num_kv_heads, D = t->head_dim;
  if (N <= 0) return fail(TPR_ERR_INVALID_ARGUMENT, "num_leaves must be positive, got %d", N);
  if (M < 0) return fail(TPR_ERR_INVALID_ARGUMENT, "num_nodes must be non-negative, got %d", M);
  if (depth < 0) return fail(TPR_ERR_INVALID_ARGUMENT, "max_depth must be non-negative, got %d", depth);
  if (M > 0 && depth == 0) return fail(TPR_ERR_INVALID_ARGUMENT, "max_depth must be positive when nodes exist");
  if (Hq <= 0 || Hkv <= 0 || D <= 0)
    return fail(TPR_ERR_INVALID_ARGUMENT, "head counts and head_dim must be positive, got Hq=%d Hkv=%d D=%d", Hq, Hkv, D);
  if (Hq % Hkv != 0)
    return fail(TPR_ERR_INVALID_ARGUMENT, "query head count must be divisible by KV head count, got Q=%d, KV=%d", Hq, Hkv);
  if (D > 256 || D % 8 != 0)
    return fail(TPR_ERR_UNSUPPORTED, "head_dim must be a multiple of 8 and at most 256, got %d", D);
  if (t->dtype != TPR_DTYPE_BF16 && t->dtype != TPR_DTYPE_FP32)
    return fail(TPR_ERR_INVALID_ARGUMENT, "unknown dtype %d", t->dtype);
  if (t->flags & ~(TPR_PLAN_RECOMPUTE_DQ | TPR_PLAN_MASKED))
    return fail(TPR_ERR_INVALID_ARGUMENT, "unknown plan flags 0x%x", static_cast<unsigned>(t->flags));
  if (t->ds_store_max_bytes < 0 && t->ds_store_max_bytes != TPR_DS_STORE_DEFAULT)
    return fail(TPR_ERR_INVALID_ARGUMENT, "ds_store_max_bytes must be 0, TPR_DS_STORE_DEFAULT or positive, got %lld",
                static_cast<long long>(t->ds_store_max_bytes));
  if (!t->cu_seqlens_q || !t->node_offsets || (N * depth > 0 && !t->leaf_ancestors))
    return fail(TPR_ERR_INVALID_ARGUMENT, "tree metadata pointers must not be NULL");

  const int32_t* cu = t->cu_seqlens_q;
  const int32_t* no = t->node_offsets;
  const int32_t* anc = t->leaf_ancestors;
  if (cu[0] != 0) return fail(TPR_ERR_INVALID_ARGUMENT, "cu_seqlens_q[0] must be 0, got %d", cu[0]);
  for (int s = 0; s < N; s++)
    if (cu[s + 1] < cu[s]) return fail(TPR_ERR_INVALID_ARGUMENT, "cu_seqlens_q must be non-decreasing (leaf %d)", s);
  if (no[0] != 0) return fail(TPR_ERR_INVALID_ARGUMENT, "node_offsets[0] must be 0, got %d", no[0]);
  for (int n = 0; n < M; n++)
    if (no[n + 1] < no[n]) return fail(TPR_ERR_INVALID_ARGUMENT, "node_offsets must be non-decreasing (node %d)", n);

  // ancestor paths: ids in [0, M), -1 padding only at the end, no repeats,
  // each node at one depth with one identical path above it.
  std::vector<int> node_depth(M, -1), leaf_lo(M, -1), leaf_hi(M, -1), leaf_count(M, 0);
  std::vector<int> node_parent(M, -2);
  for (int s = 0; s < N; s++) {
    bool ended = false;
    for (int d = 0; d < depth; d++) {
      int n = anc[s * depth + d];
      if (n == -1) { ended = true; continue; }
      if (ended) return fail(TPR_ERR_INVALID_ARGUMENT, "leaf %d ancestor list has a node after -1 padding", s);
      if (n < 0 || n >= M) return fail(TPR_ERR_INVALID_ARGUMENT, "leaf %d ancestor %d out of range [0, %d)", s, n, M);
      int parent = d == 0 ? -1 : anc[s * depth + d - 1];
      if (node_depth[n] == -1) {
        node_depth[n] = d;
        node_parent[n] = parent;
        leaf_lo[n] = s;
      } else if (node_depth[n] != d || node_parent[n] != parent) {
        return fail(TPR_ERR_INVALID_ARGUMENT, "node %d has inconsistent paths (leaf %d): not a tree", n, s);
      }
      leaf_hi[n] = s + 1;
      leaf_count[n]++;
    }
  }
  for (int n = 0; n < M; n++) {
    if (leaf_count[n] == 0) { leaf_lo[n] = 0; leaf_hi[n] = 0; continue; }
    if (leaf_hi[n] - leaf_lo[n] != leaf_count[n])
      return fail(TPR_ERR_INVALID_ARGUMENT,
                  "descendant leaves of node %d are not contiguous; number leaves in DFS order", n);
  }

  // a masked plan runs the SIMT kernels, the ones that read a key mask
  const bool masked = (t->flags & TPR_PLAN_MASKED) != 0;
  const int path = t->dtype != TPR_DTYPE_BF16 || masked ? PATH_SIMT
                   : D == kMfmaD             ? PATH_MFMA
                   : (D == 64 || D == 256)   ? PATH_MFMA16
                                             : PATH_SIMT;
  const bool mfma_family = path != PATH_SIMT;
  const int G = Hq / Hkv;
  std::vector<int64_t> prefix_len(N, 0);
  for (int s = 0; s < N; s++)
    for (int d = 0; d < depth; d++) {
      int n = anc[s * depth + d];
      if (n >= 0) prefix_len[s] += no[n + 1] - no[n];
    }
  // a masked plan's least mask row length: the longest key sequence of any leaf
  int64_t mask_cols = 0;
  if (masked) {
    mask_cols = 1;
    for (int s = 0; s < N; s++) mask_cols = std::max<int64_t>(mask_cols, prefix_len[s] + cu[s + 1] - cu[s]);
    if (mask_cols > INT32_MAX)
      return fail(TPR_ERR_UNSUPPORTED, "a masked plan needs key sequences of at most 2^31 - 1 keys, got %lld",
                  static_cast<long long>(mask_cols));
  }

  // ---- key runs (the MFMA forward / dQ key streams) --------------------------
  // A leaf's ancestors, root first, as runs of rows of prefix_k/v: an ancestor
  // that starts where the previous one ends extends its run (in DFS layout a
  // chain of first children is one run), and empty nodes add nothing. Every
  // ancestor key is visible to every query of the leaf, so only the rows
  // matter, not the node boundaries.
  std::vector<int32_t> runs_flat;
  int max_runs = 0;
  std::vector<std::vector<int32_t>> leaf_runs(N);
  for (int s = 0; s < N; s++) {
    std::vector<int32_t>& r = leaf_runs[s];
    for (int d = 0; d < depth; d++) {
      const int n = anc[s * depth + d];
      if (n < 0) break;
      const int32_t row = no[n], len = no[n + 1] - no[n];
      if (len == 0) continue;
      if (!r.empty() && r[r.size() - 2] + r.back() == row)
        r.back() += len;
      else
        r.insert(r.end(), {row, len});
    }
    max_runs = std::max(max_runs, static_cast<int>(r.size() / 2));
  }
  const int run_words = 2 * std::max(max_runs, 1);
  runs_flat.assign(static_cast<size_t>(N) * run_words, 0);
  for (int s = 0; s < N; s++)
    std::copy(leaf_runs[s].begin(), leaf_runs[s].end(), runs_flat.begin() + static_cast<size_t>(s) * run_words);

  // ---- query-block list (dK/dV granularity) --------------------------------
  const int BQ = mfma_family ? kDkdvQ : kSimtTile;
  std::vector<int32_t> qblk, leaf_qblk(N + 1, 0);
  for (int s = 0; s < N; s++) {
    leaf_qblk[s] = static_cast<int32_t>(qblk.size() / 2);
    for (int tok = 0; tok < cu[s + 1] - cu[s]; tok += BQ) {
      qblk.push_back(s);
      qblk.push_back(tok);
    }
  }
  leaf_qblk[N] = static_cast<int32_t>(qblk.size() / 2);
  const int32_t n_qblk = leaf_qblk[N];

  // ---- forward / dQ items -----------------------------------------------------
  int heads_per_wg, tokens_per_wg;
  if (path == PATH_MFMA) {
    heads_per_wg = gcd_int(G, kFwdWaves);
    tokens_per_wg = kFwdTokens * (kFwdWaves / heads_per_wg);
  } else if (path == PATH_MFMA16) {
    heads_per_wg = gcd_int(G, kM16Waves);
    tokens_per_wg = kM16Tokens * (kM16Waves / heads_per_wg);
  } else {
    heads_per_wg = 1;
    tokens_per_wg = kSimtQ;
  }
  // Leaf-major order (longest leaf first, largest token blocks first within a
  // leaf): the workgroups that run together on an XCD then share one leaf's
  // suffix K/V besides the prefix, which keeps both in its L2.
  std::vector<int> leaf_rank(N);
  {
    std::vector<int> by_len(N);
    for (int s = 0; s < N; s++) by_len[s] = s;
    std::stable_sort(by_len.begin(), by_len.end(),
                     [&](int x, int y) { return cu[x + 1] - cu[x] > cu[y + 1] - cu[y]; });
    for (int r = 0; r < N; r++) leaf_rank[by_len[r]] = r;
  }
  // items of `heads` query heads x `tokens` tokens of one leaf, dealt to the XCDs
  auto query_items = [&](int heads, int tokens, int32_t* count) {
    std::vector<Item> items;
    for (int s = 0; s < N; s++) {
      const int len = cu[s + 1] - cu[s];
      for (int tok = 0; tok < len; tok += tokens) {
        // keys the item streams: under a mask every suffix key may be visible
        const int64_t keys = prefix_len[s] + (masked ? len : std::min(tok + tokens, len));
        for (int qh = 0; qh < Hq; qh += heads) {
          Item it;
          it.words = {s, tok, qh, qh / G};
          it.work = keys + static_cast<int64_t>(N - leaf_rank[s]) * (int64_t{1} << 40);
          it.kvh = qh / G;
          items.push_back(std::move(it));
        }
      }
    }
    return order_for_xcds(items, Hkv, 4, count);
  };
  int32_t n_fwd = 0;
  std::vector<int32_t> fwd_words = query_items(heads_per_wg, tokens_per_wg, &n_fwd);

  // ---- dK/dV items ---------------------------------------------------------
  // One item per (KV segment tile, KV head). On the MFMA path an item streams
  // at most kDkdvMaxBlocks query blocks (its block table lives in LDS). A
  // prefix tile -- the tile every sibling reads -- carries N siblings' work;
  // when its query range exceeds about one CU's share of the whole launch
  // (clamped to [kDkdvPrefixChunk, kDkdvMaxBlocks] blocks) it is split into
  // chunks that each write an fp32 partial, summed afterwards in chunk (=
  // leaf) order by a reduction item. Ranges that fit stay whole: no partials
  // and no reduction.
  const int KT = path == PATH_MFMA ? kDkdvKeys : path == PATH_MFMA16 ? m16_keys(D) : kSimtKeys;
  int prefix_cap = kDkdvPrefixChunk;
  if (mfma_family) {
    int64_t total = 0;  // query blocks streamed over all (tile, KV head) items
    for (int n = 0; n < M; n++)
      total += static_cast<int64_t>((no[n + 1] - no[n] + KT - 1) / KT) * Hkv *
               (leaf_qblk[leaf_hi[n]] - leaf_qblk[leaf_lo[n]]);
    for (int s = 0; s < N; s++)
      for (int k0 = 0; k0 < cu[s + 1] - cu[s]; k0 += KT)
        total += static_cast<int64_t>(Hkv) * (leaf_qblk[s + 1] - leaf_qblk[s] - k0 / BQ);
    prefix_cap = static_cast<int>(std::min<int64_t>(kDkdvMaxBlocks,
                                                    std::max<int64_t>(kDkdvPrefixChunk, total / kPlanCus)));
  }
  std::vector<Item> dkdv;
  std::vector<int32_t> red;
  int32_t n_slots = 0, max_split = 1;
  auto add_tile = [&](int src, int seg, int k0, int h, int32_t lo, int32_t hi) {
    const int32_t range = hi - lo;
    int chunk = range;
    if (mfma_family) {
      const int cap = src == 0 ? prefix_cap : kDkdvMaxBlocks;
      if (range > cap) {
        const int pieces = (range + cap - 1) / cap;
        chunk = (range + pieces - 1) / pieces;
      }
    }
    if (chunk >= range || range == 0) {
      Item it;
      it.words = {src, seg, k0, h, lo, hi, -1, 0};
      it.work = static_cast<int64_t>(range) * G + 1;
      it.kvh = h;
      dkdv.push_back(std::move(it));
      return;
    }
    const int32_t slot0 = n_slots;
    int pieces = 0;
    for (int32_t b = lo; b < hi; b += chunk, pieces++) {
      Item it;
      it.words = {src, seg, k0, h, b, std::min(hi, b + chunk), n_slots++, 0};
      it.work = static_cast<int64_t>(std::min(hi, b + chunk) - b) * G + 1;
      it.kvh = h;
      dkdv.push_back(std::move(it));
    }
    red.insert(red.end(), {src, seg, k0, h, slot0, pieces, 0, 0});
    max_split = std::max(max_split, pieces);
  };
  for (int n = 0; n < M; n++) {
    const int len = no[n + 1] - no[n];
    // a node no leaf descends from gets an empty query range: its items write zeros
    const int32_t lo = leaf_qblk[leaf_lo[n]], hi = leaf_qblk[leaf_hi[n]];
    for (int k0 = 0; k0 < len; k0 += KT)
      for (int h = 0; h < Hkv; h++) add_tile(0, n, k0, h, lo, hi);
  }
  // Suffix tiles: where one dK/dV workgroup fills a CU (the MFMA kernels at
  // head_dim 128 and 256), tile j of a leaf with T tiles is paired with its
  // mirror T-1-j in one item (DK_PAIR) when neither is split: the pair
  // streams the mirror's blocks last-first, then tile j's first-last, so all
  // pairs of a leaf take about the same time and read the same query block
  // at the same time (the copies are shared in L2). At head_dim 64 three
  // dK/dV workgroups share a CU and hide each other's start; pairs measured
  // slower there (2.29 -> 2.38 ms at prefix 4096 + 4 x 4096, GQA 32/8).
  const bool pair_tiles = path == PATH_MFMA || (path == PATH_MFMA16 && D == 256);
  for (int s = 0; s < N; s++) {
    const int len = cu[s + 1] - cu[s];
    const int tiles = (len + KT - 1) / KT;
    auto first_block = [&](int j) { return leaf_qblk[s] + j * KT / BQ; };
    for (int j = 0; j < tiles; j++) {
      const int mirror = tiles - 1 - j;
      const int lo_tile = std::min(j, mirror);   // the longer query range
      if (pair_tiles && mirror != j && leaf_qblk[s + 1] - first_block(lo_tile) <= kDkdvMaxBlocks) {
        if (j == lo_tile) {
          const int32_t blocks = (leaf_qblk[s + 1] - first_block(j)) + (leaf_qblk[s + 1] - first_block(mirror));
          for (int h = 0; h < Hkv; h++) {
            Item it;
            it.words = {1, s, mirror * KT, h, first_block(mirror), leaf_qblk[s + 1], -1, j * KT + 1};
            it.work = static_cast<int64_t>(blocks) * G + 2;
            it.kvh = h;
            dkdv.push_back(std::move(it));
          }
        }
        continue;
      }
      // causal: the blocks from the tile's own on; under a mask every block of the leaf
      const int32_t lo = masked ? leaf_qblk[s] : first_block(j);
      for (int h = 0; h < Hkv; h++) add_tile(1, s, j * KT, h, lo, leaf_qblk[s + 1]);
    }
  }
  int32_t n_dkdv = 0;
  std::vector<int32_t> dkdv_words = order_for_xcds(dkdv, Hkv, DK_WORDS, &n_dkdv);

  // ---- dS store (bf16 head_dim 128 and 256) -------------------------------------
  // Every (key tile, query block) pair the dK/dV items stream gets one slot.
  // Slots are numbered query-block-major, in the order the dQ kernel walks a
  // block's keys: the leaf's ancestor nodes root first (each node's tiles in
  // key order), then the leaf's suffix tiles up to the one holding the
  // block's last token. So slot(segment, tile t, block b) = first[b] +
  // base[segment] + t, where base[] counts the tiles ahead of a segment in
  // that walk -- the same for every block below a node, since they share the
  // path above it. The store is laid out [KV head][slot][query head of the
  // group][tile x 64 block] (ds_head_bytes each), so a dQ work item -- one
  // block of one KV head's group -- reads one contiguous stretch.
  std::vector<int32_t> ds_table;
  int64_t ds_slots = 0;
  const bool ds_path = path == PATH_MFMA || (path == PATH_MFMA16 && D == 256);
  const int64_t ds_budget = t->ds_store_max_bytes == TPR_DS_STORE_DEFAULT ? TPR_DS_STORE_DEFAULT_BYTES
                                                                          : t->ds_store_max_bytes;
  if (ds_path && ds_budget > 0 && !(t->flags & TPR_PLAN_RECOMPUTE_DQ)) {
    auto ntiles = [&](int64_t len) { return static_cast<int32_t>((len + KT - 1) / KT); };
    std::vector<int32_t> base(static_cast<size_t>(M) + N, 0), first(static_cast<size_t>(n_qblk) + 1, 0);
    for (int s = 0; s < N; s++) {
      int32_t ahead = 0;
      for (int d = 0; d < depth; d++) {
        const int n = anc[s * depth + d];
        if (n < 0) break;
        base[n] = ahead;  // the same from every leaf below n
        ahead += ntiles(no[n + 1] - no[n]);
      }
      base[M + s] = ahead;
      const int len = cu[s + 1] - cu[s];
      for (int b = leaf_qblk[s]; b < leaf_qblk[s + 1]; b++) {
        const int last = std::min(len, (b - leaf_qblk[s] + 1) * BQ) - 1;  // the block's last token
        ds_slots += ahead + last / KT + 1;
        first[b + 1] = static_cast<int32_t>(std::min<int64_t>(ds_slots, INT32_MAX));
      }
    }
    if (ds_slots > 0 && ds_slots < INT32_MAX && ds_slots * Hq * ds_head_bytes(path, D) <= ds_budget) {
      ds_table = std::move(base);
      ds_table.insert(ds_table.end(), first.begin(), first.end());
    } else {
      ds_slots = 0;
    }
  }

  // ---- dQ items of the dS store -------------------------------------------------
  // The dQ-from-store kernels run 8 waves (two per SIMD) of kDqsTokens tokens
  // at head_dim 128 (a whole query block per wave) and kM16Tokens at head_dim
  // 256, twice the forward's tokens per workgroup, so every K tile they copy
  // serves twice the queries.
  int32_t n_dqs = 0;
  std::vector<int32_t> dqs_words;
  if (ds_slots > 0) {
    const int heads = gcd_int(G, kM16DqsWaves);
    const int tokens = (path == PATH_MFMA ? kDqsTokens : kM16Tokens) * (kM16DqsWaves / heads);
    dqs_words = query_items(heads, tokens, &n_dqs);
  }

  // ---- assemble ----------------------------------------------------------------
  plan.assign(PF_HEADER_WORDS, 0);
  auto append = [&](const int32_t* src, size_t count) {
    int32_t off = static_cast<int32_t>(plan.size());
    plan.insert(plan.end(), src, src + count);
    return off;
  };
  plan[PF_MAGIC] = kPlanMagic;
  plan[PF_VERSION] = kPlanVersion;
  plan[PF_NUM_LEAVES] = N;
  plan[PF_NUM_NODES] = M;
  plan[PF_MAX_DEPTH] = depth;
  plan[PF_TOTAL_Q] = cu[N];
  plan[PF_TOTAL_PREFIX] = no[M];
  plan[PF_HQ] = Hq;
  plan[PF_HKV] = Hkv;
  plan[PF_D] = D;
  plan[PF_DTYPE] = t->dtype;
  plan[PF_PATH] = path;
  plan[PF_OFF_CU] = append(cu, N + 1);
  plan[PF_OFF_NODE_OFF] = append(no, M + 1);
  plan[PF_OFF_ANC] = append(anc ? anc : cu, static_cast<size_t>(N) * depth);
  std::vector<int32_t> nl(2 * M);
  for (int n = 0; n < M; n++) { nl[2 * n] = leaf_lo[n]; nl[2 * n + 1] = leaf_hi[n]; }
  plan[PF_OFF_NODE_LEAF] = append(nl.data(), nl.size());
  plan[PF_N_QBLK] = n_qblk;
  plan[PF_OFF_QBLK] = append(qblk.data(), qblk.size());
  plan[PF_OFF_LEAF_QBLK] = append(leaf_qblk.data(), leaf_qblk.size());
  plan[PF_N_FWD] = n_fwd;
  plan[PF_OFF_FWD] = append(fwd_words.data(), fwd_words.size());
  plan[PF_N_DKDV] = n_dkdv;
  plan[PF_OFF_DKDV] = append(dkdv_words.data(), dkdv_words.size());
  plan[PF_N_RED] = static_cast<int32_t>(red.size() / RD_WORDS);
  plan[PF_OFF_RED] = append(red.data(), red.size());
  plan[PF_N_SLOTS] = n_slots;
  plan[PF_MAX_SPLIT] = max_split;
  plan[PF_OFF_RUNS] = append(runs_flat.data(), runs_flat.size());
  plan[PF_MAX_RUNS] = std::max(max_runs, 1);
  plan[PF_DS_SLOTS] = static_cast<int32_t>(ds_slots);
  plan[PF_OFF_DS] = ds_table.empty() ? 0 : append(ds_table.data(), ds_table.size());
  plan[PF_MASK_COLS] = static_cast<int32_t>(mask_cols);
  plan[PF_N_DQS] = n_dqs;
  plan[PF_OFF_DQS] = dqs_words.empty() ? 0 : append(dqs_words.data(), dqs_words.size());
  plan[PF_TOTAL_WORDS] = static_cast<int32_t>(plan.size());
  return TPR_OK;
}

}  // namespace tpr

extern "C" int tpr_attn_plan(const TprTreeDesc* tree, int32_t* plan, int64_t capacity_words,
                             int64_t* words_needed) {
  tpr::clear_error();
  std::vector<int32_t> blob;
  int rc = tpr::build_plan(tree, blob);
  if (rc != TPR_OK) return rc;
  if (words_needed) *words_needed = static_cast<int64_t>(blob.size());
  if (!plan) return TPR_OK;
  if (capacity_words < static_cast<int64_t>(blob.size()))
    return tpr::fail(TPR_ERR_BUFFER_TOO_SMALL, "plan needs %zu words, capacity is %lld", blob.size(),
                     static_cast<long long>(capacity_words));
  std::memcpy(plan, blob.data(), blob.size() * sizeof(int32_t));
  return TPR_OK;
}
