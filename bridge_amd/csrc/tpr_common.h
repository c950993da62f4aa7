// tpr_common.h -- layout of the launch-plan blob shared by the host planner
// (tpr_plan.cpp) and the kernels, plus the tile shapes each kernel family
// uses. The plan is a flat int32 array: a fixed header of offsets/counts,
// the tree metadata and the per-kernel work lists.
#pragma once

#include <stdint.h>

namespace tpr {

constexpr int32_t kPlanMagic = 0x31525054;  // "TPR1"
constexpr int32_t kPlanVersion = 7;

// Header word indices.
enum PlanField : int {
  PF_MAGIC = 0,
  PF_VERSION,
  PF_NUM_LEAVES,
  PF_NUM_NODES,
  PF_MAX_DEPTH,
  PF_TOTAL_Q,
  PF_TOTAL_PREFIX,
  PF_HQ,
  PF_HKV,
  PF_D,
  PF_DTYPE,
  PF_PATH,           // KernelPath
  PF_OFF_CU,         // cu_seqlens_q [N+1]
  PF_OFF_NODE_OFF,   // node_offsets [M+1]
  PF_OFF_ANC,        // leaf_ancestors [N*max_depth]
  PF_OFF_NODE_LEAF,  // node leaf range [M][2] = {first leaf, last leaf + 1}
  PF_N_QBLK,         // number of query blocks (dK/dV kernel granularity)
  PF_OFF_QBLK,       // query blocks [n][2] = {leaf, token start within leaf}
  PF_OFF_LEAF_QBLK,  // first query block of each leaf [N+1]
  PF_N_FWD,          // forward / dQ work items
  PF_OFF_FWD,        // [n][4] = {leaf, token start, first q head, kv head}; leaf < 0 = empty
  PF_N_DKDV,         // dK/dV work items
  PF_OFF_DKDV,       // [n][8] = DkdvItem
  PF_N_RED,          // split-reduction items
  PF_OFF_RED,        // [n][RED_WORDS] = RedItem
  PF_N_SLOTS,        // fp32 partial slots (each kDkdvKeys x D x 2 floats)
  PF_MAX_SPLIT,      // most partial slots reduced into one tile
  PF_TOTAL_WORDS,
  PF_OFF_RUNS,       // key runs [N][max_runs][2] = {first row in prefix_k/v, rows}: the leaf's
                     // ancestor nodes root first, nodes adjacent in prefix_k/v merged, empty
                     // nodes dropped; {0, 0} pads a leaf with fewer runs
  PF_MAX_RUNS,       // most key runs of any leaf
  PF_DS_SLOTS,       // dS slots of the head_dim-128 / 256 backward (0: dQ recomputes the scores)
  PF_OFF_DS,         // dS slot table: [M + N] tiles ahead of each segment (nodes, then leaf
                     // suffixes) in the dQ walk of a query block below it, then
                     // [n_qblk + 1] first slot of each query block; slot of (segment, tile t,
                     // block b) = first[b] + base[segment] + t
  PF_MASK_COLS,      // plan built for a key mask (TPR_PLAN_MASKED): the longest key sequence
                     // of any leaf (the least mask row length); 0 = not a masked plan
  PF_N_DQS,          // dQ work items of a dS-store plan (0: dQ takes the forward items)
  PF_OFF_DQS,        // [n][4] like the forward items: 8 waves of kDqsTokens (head_dim 128) or
                     // kM16Tokens (head_dim 256) tokens each
  PF_HEADER_WORDS = 40
};

enum KernelPath : int32_t {
  PATH_SIMT = 0,    // fp32-accumulate SIMT kernels (fp32, or bf16 with another head_dim)
  PATH_MFMA = 1,    // bf16 MFMA kernels, head_dim 128 (32x32x16 MFMA)
  PATH_MFMA16 = 2   // bf16 MFMA kernels, head_dim 64 or 256 (16x16x32 MFMA)
};

// dK/dV work item: one (KV segment tile, KV head) and the query blocks that see it.
enum DkdvField : int {
  DK_SRC = 0,   // 0 = prefix node (fully visible), 1 = leaf suffix (causal)
  DK_SEG,       // node id or leaf id
  DK_KEY0,      // first key of the tile, relative to the segment
  DK_KVH,       // KV head
  DK_QB_LO,     // query-block range [lo, hi) in the global query-block list
  DK_QB_HI,
  DK_SLOT,      // -1: write dK/dV directly; else fp32 partial slot
  DK_PAIR,      // 0, or 1 + first key of a second suffix tile of the same leaf
                // and KV head, streamed after this one (pairs are never split)
  DK_WORDS = 8
};

// Split-reduction item: sum fp32 partial slots [slot0, slot0 + nslots) of one
// (KV segment tile, KV head) in slot order and write dK/dV in the I/O dtype.
enum RedField : int {
  RD_SRC = 0,   // 0 = prefix node, 1 = leaf suffix
  RD_SEG,
  RD_KEY0,
  RD_KVH,
  RD_SLOT0,
  RD_NSLOTS,
  RD_PAD0,
  RD_PAD1,
  RD_WORDS = 8
};

// ---- tile shapes -----------------------------------------------------------
// SIMT family (fp32, or bf16 with head_dim != 128; head_dim a multiple of 8, at most 256)
constexpr int kSimtQ = 64;      // queries per forward / dQ block (one head)
constexpr int kSimtKeys = 64;   // keys per dK/dV block
constexpr int kSimtTile = 32;   // keys (fwd/dQ) or queries (dK/dV) staged per LDS tile

// MFMA family (bf16, head_dim 128)
constexpr int kMfmaD = 128;
constexpr int kFwdWaves = 8;          // waves per forward / dQ workgroup
constexpr int kFwdTokens = 32;        // tokens per wave (one query head per wave)
constexpr int kDqsTokens = 64;        // tokens per wave of the dQ-from-store kernel (one query block)
constexpr int kFwdKeys = 64;          // keys per LDS tile
constexpr int kDkdvWaves = 4;         // waves per dK/dV workgroup
constexpr int kDkdvKeys = 32 * kDkdvWaves;  // keys per dK/dV workgroup (32 per wave)
constexpr int kDkdvQ = 64;            // queries per staged query block
constexpr int kDkdvMaxBlocks = 256;   // query blocks one dK/dV item may stream (LDS table size)
constexpr int kDkdvPrefixChunk = 64;  // smallest chunk a prefix tile is split into
constexpr int kPlanCus = 256;         // compute units the dK/dV work is balanced over (MI355X)
// dS store (bf16 head_dim 128 and 256): the dK/dV kernel writes each dS block
// it computes, bf16, and dQ = scale dS K reads them instead of recomputing S
// and dP. One slot per (dK/dV key tile, query block it is visible to) holds,
// per query head, the tile x 64 block as four wave blocks in the dK/dV
// kernel's register order: at head_dim 128 a 128-key tile of 4 KiB wave
// blocks (32 keys each), at head_dim 256 a 64-key tile of 2 KiB wave blocks
// (16 keys each). The store is [KV head][slot][query head of the group]
// blocks (ds_offset), slots numbered query-block-major in the dQ kernel's key
// order (PF_OFF_DS), so each dQ work item reads one contiguous stretch. A plan has a store only when it fits the caller's budget
// (TprTreeDesc.ds_store_max_bytes).
constexpr int kDsHeadBytes = kDkdvKeys * kDkdvQ * 2;          // 16 KiB per query head per slot (head_dim 128)
// MFMA backward workspace, ahead of the partial slots: two constants (+inf,
// 0) that rows past a query block's end are copied from, then lse * log2e per
// (query head, token) in the lse layout, then -delta in the same layout.
constexpr int kStatRowsOffset = 64;   // floats before the lse*log2e rows
// MFMA16 family (bf16, head_dim 64 and 256)
constexpr int kM16Waves = 4;          // waves per workgroup (all kernels)
constexpr int kM16Tokens = 32;        // forward / dQ tokens per wave (two 16-query sub-blocks)
constexpr int kM16DqsWaves = 8;       // waves of the head_dim-256 dQ-from-store workgroup (two per SIMD)
// dK/dV keys per wave: one 16-key block (at head_dim 256 the accumulators of
// two would not fit the register file; at 64 two measured no faster)
constexpr int m16_wave_keys(int /*head_dim*/) { return 16; }
constexpr int m16_keys(int d) { return m16_wave_keys(d) * kM16Waves; }  // keys per dK/dV workgroup
// bytes per query head per slot of a plan's dS store
constexpr int ds_head_bytes(int path, int d) {
  return (path == PATH_MFMA ? kDkdvKeys : m16_keys(d)) * kDkdvQ * 2;
}
constexpr int kMfmaRegRuns = 8;       // key runs a forward / dQ workgroup holds in registers; a
                                      // launch with longer run lists reads them from the plan

}  // namespace tpr
