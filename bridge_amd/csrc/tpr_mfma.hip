// tpr_mfma.hip -- gfx950 bf16 MFMA prefix-reuse attention kernels (head_dim 128).
//
// Forward and dQ: one workgroup = 4 waves sharing one KV head; wave w owns 32
// tokens of one query head of the GQA group, so every K/V tile staged in LDS
// feeds all query heads of the group. The key loop runs over the ancestor
// prefix nodes (fully visible, root first) and then the leaf's own suffix
// (right-down causal), keeping one online-softmax state (max, sum, O) in
// registers across both phases: the fp32 (out, max, sum) merge of the
// reference's prefix FULL and suffix CAUSAL blocks
// (verl/models/mcore/tpr/parallel/ring_attention.py:588-636) happens in the
// loop instead of between kernel calls.
//
// dK/dV: one workgroup = 4 waves x 32 keys of one KV segment tile and KV head;
// it streams every query block that sees those keys (for a prefix node: all
// descendant leaves, every query head of the group) in the plan's fixed
// order, so a prefix node's gradient is summed over siblings in registers,
// without atomics (the deterministic counterpart of
// verl/models/mcore/tpr/prefix_state.py:565-573).
//
// MFMA layout (v_mfma_f32_32x32x16_bf16): A lane l holds row l%32, k-slots
// 8*(l/32)+i; B lane l holds column l%32, same k-slots; accumulator register r
// of lane l holds (row 8*(r/4) + 4*(l/32) + r%4, column l%32). Scores are
// computed transposed (S^T = K Q^T) with the key rows permuted by sigma32, so
// a lane holds one query and 8-key runs; P^T then feeds the P.V MFMA as its B
// operand straight from registers, and V is read column-wise from its
// row-major LDS tile with ds_read_tr16_b64.

#include <type_traits>

#include "tpr_kernel_util.h"

namespace tpr {
namespace {

constexpr int kTileBytes = kTileRows * 256;   // 64 rows x 128 bf16
typedef int i32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufferRsrcWord3 = 0x00020000;  // raw (untyped) buffer resource, gfx9 data format field
constexpr int kCachePolicyNt = 2;             // buffer access cache policy: non-temporal (streaming)

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ f32x16 mfma(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Per-lane byte offsets, within a swizzled tile (plus `bias`), of the
// operand reads. The swizzle of row r depends only on r mod 16, so rows 16m further
// down are the same offsets plus 4096m: only the first 16 or 32 rows' offsets
// are kept, and row blocks, buffers and tiles are immediate offsets.
struct FwdLdsOffsets {
  uint32_t k[8];     // K row sigma32(n), columns 16c + 8h .. +7 (c = 0..7)
  uint32_t v[4][2];  // V rows 8h + (l%16)/4 (+4), column 32db + 16((l/16)&1) + 4(l%4)
};

__device__ __forceinline__ FwdLdsOffsets make_fwd_lds_offsets(int lane, uint32_t bias = 0) {
  FwdLdsOffsets o;
  const int n = lane & 31, h = lane >> 5, g = lane >> 4, i = lane & 15;
#pragma unroll
  for (int c = 0; c < 8; c++) o.k[c] = bias + static_cast<uint32_t>(swz_off(sigma32(n), 16 * c + 8 * h));
#pragma unroll
  for (int db = 0; db < 4; db++) {
    const int row = 8 * h + (i >> 2), col = 32 * db + ((g & 1) << 4) + ((i & 3) << 2);
    o.v[db][0] = bias + static_cast<uint32_t>(swz_off(row, col));
    o.v[db][1] = bias + static_cast<uint32_t>(swz_off(row + 4, col));
  }
  return o;
}

// Transposed operand read at precomputed offsets (two ds_read_tr16_b64; lo:
// rows +0..3, hi: rows +4..7): lane l gets 8 consecutive rows of column
// c0 + (l % 32) of a row-major swizzled tile -- the B operand layout of a
// 32x32x16 MFMA whose k index runs down the tile.
__device__ __forceinline__ bf16x8 lds_col8_at(const char* base, uint32_t lo, uint32_t hi) {
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + lo));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + hi));
  bf16x8 r;
  const bf16x4 l4 = __builtin_bit_cast(bf16x4, a);
  const bf16x4 h4 = __builtin_bit_cast(bf16x4, b);
  r[0] = l4[0]; r[1] = l4[1]; r[2] = l4[2]; r[3] = l4[3];
  r[4] = h4[0]; r[5] = h4[1]; r[6] = h4[2]; r[7] = h4[3];
  return r;
}

// Per-lane part of a 64-row tile copy: which row / chunk this lane moves in
// each of its 16 / kWaves DMA blocks, and the resulting byte offset for a
// full tile (row stride `row_bytes`).
template <int kWaves>
struct DmaLanes {
  static constexpr int kBlocks = 16 / kWaves;
  uint32_t voff[kBlocks];
  int row[kBlocks];
  uint32_t cbytes[kBlocks];
};

template <int kWaves>
__device__ __forceinline__ DmaLanes<kWaves> make_dma_lanes(uint32_t row_bytes, int wave, int lane) {
  static_assert(kWaves == 4, "the tile4 lane map (tpr_lanes.h) is for 4 waves of 4 blocks");
  DmaLanes<kWaves> p;
#pragma unroll
  for (int j = 0; j < DmaLanes<kWaves>::kBlocks; j++) {
    p.row[j] = tile4_row(wave, lane, j);
    p.cbytes[j] = tile4_chunk_bytes_swz(wave, lane, j);
    p.voff[j] = tile4_lane_bytes_swz(wave, lane, row_bytes, j);
  }
  return p;
}

// Copy rows [0, 64) of the tile starting at `src` (uniform; rows at or beyond
// `len` re-read row len - 1) into the swizzled LDS tile at `lds_tile`.
template <int kWaves>
__device__ __forceinline__ void dma_tile_s(const char* src, uint32_t row_bytes, int len, uint32_t lds_tile,
                                           const DmaLanes<kWaves>& p, int wave) {
  constexpr int kBlocks = DmaLanes<kWaves>::kBlocks;
  if (len >= kTileRows) {
#pragma unroll
    for (int j = 0; j < kBlocks; j++) dma16sb(src, p.voff[j], lds_tile + (wave * kBlocks + j) * 1024);
  } else {
#pragma unroll
    for (int j = 0; j < kBlocks; j++)
      dma16sb(src, static_cast<uint32_t>(min(p.row[j], len - 1)) * row_bytes + p.cbytes[j],
             lds_tile + (wave * kBlocks + j) * 1024);
  }
}

// Per-lane part of a 64-row tile copy by 4 waves: lane l of wave w moves, in
// block j = 0..3, row 16w + 4j + l/16 and the 16-byte source chunk
// swz_chunk(row, l%16) = (l%16) ^ ((l/16) << 2) ^ j, i.e. chunk bytes
// cb0 ^ 16j; full[j] is that block's byte offset in a full tile.
struct TileLanes4 {
  uint32_t row0;     // 16w + l/16
  uint32_t cb0;      // 16 * ((l%16) ^ ((l/16) << 2))
  uint32_t full[4];  // (row0 + 4j) * row_bytes + (cb0 ^ 16j)
};

__device__ __forceinline__ TileLanes4 make_tile_lanes4(int wave, int lane, uint32_t row_bytes) {
  TileLanes4 p;
  p.row0 = static_cast<uint32_t>(tile4_row(wave, lane, 0));
  p.cb0 = tile4_chunk_bytes(lane, 0);
#pragma unroll
  for (int j = 0; j < 4; j++) p.full[j] = tile4_lane_bytes(wave, lane, row_bytes, j);
  return p;
}

// Copy rows [0, 64) of the tile starting at `src` (uniform; rows at or beyond
// `len` re-read row len - 1) into the swizzled LDS tile at `lds_tile`; this
// wave moves its four 1 KiB blocks (one asm group). A full tile whose row
// stride is the one p.full was made for (`full_ok`) uses those offsets;
// other tiles compute them.
__device__ __forceinline__ void dma_tile4(const char* src, uint32_t row_bytes, int len, uint32_t lds_tile,
                                          const TileLanes4& p, int wave, bool full_ok) {
  const uint32_t dst = lds_tile + wave * 4096;
  if (len >= kTileRows && full_ok) {
    dma_blocks4(src, p.full[0], p.full[1], p.full[2], p.full[3], dst);
  } else {
    const uint32_t last = static_cast<uint32_t>(len - 1);
    uint32_t v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = min(p.row0 + 4u * j, last) * row_bytes + (p.cb0 ^ (16u * j));
    dma_blocks4_m0(src, v[0], v[1], v[2], v[3], dst);
  }
}

// The forward's tile copy: the same lanes as TileLanes4, the offsets computed
// per copy (the forward runs slower holding four more offset registers
// through its tile loop). Per-lane part of a 64-row tile copy by 4 waves, in two registers: lane l of
// wave w moves, in block j = 0..3, row 16w + 4j + l/16 and the 16-byte source
// chunk swz_chunk(row, l%16) = (l%16) ^ ((l/16) << 2) ^ j, i.e. chunk bytes
// cb0 ^ 16j.
struct FwdTileLanes {
  uint32_t row0;  // 16w + l/16
  uint32_t cb0;   // 16 * ((l%16) ^ ((l/16) << 2))
};

__device__ __forceinline__ FwdTileLanes make_fwd_tile_lanes(int wave, int lane) {
  return FwdTileLanes{static_cast<uint32_t>(16 * wave + (lane >> 4)),
                    static_cast<uint32_t>(16 * ((lane & 15) ^ ((lane >> 4) << 2)))};
}

// Copy rows [0, 64) of the tile starting at `src` (uniform; rows at or beyond
// `len` re-read row len - 1) into the swizzled LDS tile at `lds_tile`; this
// wave moves its four 1 KiB blocks.
__device__ __forceinline__ void dma_tile4_fwd(const char* src, uint32_t row_bytes, int len, uint32_t lds_tile,
                                              FwdTileLanes p, int wave) {
  const uint32_t last = static_cast<uint32_t>(len - 1);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint32_t row = min(p.row0 + 4u * j, last);
    dma16s(src, row * row_bytes + (p.cb0 ^ (16u * j)), lds_tile + (wave * 4 + j) * 1024);
  }
}

// Store a wave's 32-query x 128-d output tile (accumulator layout: lane n + 32h
// holds query n, d = 32db + 8g + 4h + b in acc[db][4g + b]) scaled by `mul`
// (per lane) as bf16, through the wave's private 8 KiB of LDS `stage`, so that
// every global store is 16 lanes x 16 B = one whole 256-byte row. The stores
// are non-temporal (the rows are written once and would otherwise evict the
// shared prefix from L2) and cover full lines, which a non-temporal store of a
// partial line would not: the direct 8-byte stores cost ~4.5x their bytes in
// HBM writes. Rows r >= nrows are not stored. LDS layout: row r, 16-byte chunk
// c at r * 256 + ((c ^ (r % 16)) << 4), so both the 8-byte writes and the
// row-linear 16-byte reads spread over all banks.
__device__ __forceinline__ void store_tile_rows(char* stage, const f32x16 (&acc)[4], float mul, bf16* dst,
                                                int64_t row_stride, int nrows, int lane) {
  // The lane index is laundered so that the per-lane LDS offsets are formed
  // here: hoisted above the caller's tile loop they stay live through it and
  // take the registers its pipelined operand reads need.
  asm volatile("" : "+v"(lane));
  const int n = lane & 31, h = lane >> 5;
#pragma unroll
  for (int db = 0; db < 4; db++)
#pragma unroll
    for (int g = 0; g < 4; g++) {
      bf16x4 v4;
#pragma unroll
      for (int b = 0; b < 4; b++) v4[b] = static_cast<bf16>(acc[db][4 * g + b] * mul);
      *reinterpret_cast<bf16x4*>(stage + n * 256 + (((4 * db + g) ^ (n & 15)) << 4) + 8 * h) = v4;
    }
  // the wave's LDS writes are done before its reads (no other wave touches `stage`)
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int row = 4 * i + (lane >> 4), c = lane & 15;
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(stage + row * 256 + ((c ^ (row & 15)) << 4));
    if (row < nrows) __builtin_nontemporal_store(v, reinterpret_cast<bf16x8*>(dst + row * row_stride + 8 * c));
  }
}

// ---------------------------------------------------------------------------
// Forward
//
// The 8 waves form two groups of 4, one wave of each group per SIMD, that
// alternate between two phases at every workgroup barrier:
//   M(j): S[j+1] = K[j+1] Q^T and O += P[j] V[j]   (MFMA, LDS reads)
//   V(j): P[j+1] = softmax(S[j+1]), rescaling O     (VALU only)
// Group B runs one phase behind group A, so on every SIMD one wave's MFMAs
// overlap the other wave's softmax. The K/V tile copies are split between the
// groups: group A issues K[j+2] at the end of its M(j) phase, group B V[j+1]
// at the start of its V(j-1) phase; each group waits for its own copies before
// the barrier ahead of their first reader. K runs one tile ahead of V; two K
// and two V buffers (64 KiB) suffice.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void qk_tile(const char* kt, const bf16x8 (&qv)[8], const FwdLdsOffsets& lo,
                                        f32x16 (&s)[2]) {
#pragma unroll
  for (int kb = 0; kb < 2; kb++) {
    s[kb] = f32x16{};
#pragma unroll
    for (int c = 0; c < 8; c++)
      s[kb] = mfma(*reinterpret_cast<const bf16x8*>(kt + kb * 32 * 256 + lo.k[c]), qv[c], s[kb]);
  }
}

// Running-max slack of the lazy rescale, in log2 units: O, l are rescaled only
// when a row's max exceeds the max they are referenced to by more than this,
// so unscaled probabilities stay <= 2^8 (exact arithmetic, fp32/bf16 safe).
constexpr float kRescaleSlack = 8.f;

// dK/dV: S and dP MFMAs written as asm with their accumulators in VGPRs
#ifndef TPR_DKDV_VGPR_SP
#define TPR_DKDV_VGPR_SP 1
#endif
#ifndef TPR_MPHASE_AHEAD
#define TPR_MPHASE_AHEAD 4
#endif
constexpr int kMphaseAhead = TPR_MPHASE_AHEAD;  // LDS reads issued ahead in a forward M phase (even)

// kRunList: key runs read from the plan (more than kMfmaRegRuns); kStrided:
// q, k or v rows wider than packed (the packed instance folds every row
// stride to a constant)
template <bool kRunList, bool kStrided>
__global__ __launch_bounds__(512) void mfma_fwd(KernelArgs a) {
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh0 = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  static_assert(kFwdWaves == 8, "two groups of one wave per SIMD");
  const int grp = wave >> 2;                         // 0: group A, 1: group B (copies the tiles)
  const int hpw = a.hpw;                             // query heads per workgroup
  const int head = qh0 + wave % hpw;
  const int tw0 = tok0 + kFwdTokens * (wave / hpw);  // first token of this wave
  const int tpw = kFwdTokens * (kFwdWaves / hpw);    // tokens per workgroup
  const int suffix_keys = min(len, tok0 + tpw);
  const int n = lane & 31, h = lane >> 5;
  const int t = tw0 + n;                             // this lane's query token

  const int64_t qstride = static_cast<int64_t>(a.hq) * kMfmaD;  // output rows (packed)
  // row bytes of the suffix K and V (views of a wider buffer allowed) and of
  // the packed prefix K/V
  const uint32_t p_rb = static_cast<uint32_t>(a.hkv) * kMfmaD * 2;
  const uint32_t k_rb = kStrided ? static_cast<uint32_t>(a.k_rs) * 2 : p_rb;
  const uint32_t v_rb = kStrided ? static_cast<uint32_t>(a.v_rs) * 2 : p_rb;
  const int64_t q_rs = kStrided ? a.q_rs : qstride;
  // Q as the B operand of S^T = K Q^T: lane holds Q[t][16c + 8h .. +7]. Issued
  // first, so that its latency runs under the key-table loads and the first
  // tile's copy.
  bf16x8 qv[8];
  {
    const bf16* qp = static_cast<const bf16*>(a.q) + static_cast<int64_t>(row0 + min(t, len - 1)) * q_rs +
                     head * kMfmaD + 8 * h;
#pragma unroll
    for (int c = 0; c < 8; c++) qv[c] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(qp + 16 * c));
  }

  __shared__ __attribute__((aligned(1024))) char smem[4 * kTileBytes];  // K0 K1 V0 V1
  static_assert(sizeof(smem) >= kFwdWaves * 8192, "the output rows are staged in the tile buffers");
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));

  const char* kbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.k) + kvh * kMfmaD);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.v) + kvh * kMfmaD);
  const char* pkbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pk) + kvh * kMfmaD);
  const char* pvbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pv) + kvh * kMfmaD);
  const FwdTileLanes dl = make_fwd_tile_lanes(wave & 3, lane);
  const FwdLdsOffsets lo = make_fwd_lds_offsets(lane);

  const auto seg = load_keys<kRunList>(a, leaf, suffix_keys);
  const int ntiles = seg.ntiles;
  const KvSources src{kbase, vbase, pkbase, pvbase, k_rb, v_rb, p_rb};
  // Copy cursors. Group B copies K[0], K[1] and V[0] before the tile loop,
  // then V[j+1] at the start of its softmax phase V(j-1); group A copies
  // K[j+2] at the end of its MFMA phase M(j), which the other group's
  // softmax phase outlasts. Both wait for their copies one phase later,
  // before the barrier ahead of the first M phase that reads them.
  KvCursor dv = kv_begin(seg, src);  // B: the next V tile
  if (grp) dma_tile4_fwd(dv.k, dv.krb, kv_len(dv), lds0, dl, wave & 3);  // K[0]
  KvCursor ka = dv;                  // A: the next K tile (tile 2 when the loop starts); B: tile 1 first
  if (ntiles > 1) kv_next(seg, src, ka);
  // every wave's mask cursor: the tile whose scores the next V phase masks
  KvCursor mc = kv_begin(seg, src);


  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; i++) o[i] = f32x16{};
  float m = -1e30f, l = 0.f;  // running max (raw score units) the O/l are referenced to
  float s_max = -1e30f;       // the lane's max over the scores of the tile in s (unmasked)
  const float c2 = a.scale * kLog2e;
  const float slack = kRescaleSlack / c2;
  f32x16 s[2];
  bf16x8 pb[2][2];

  // group B before the loop: K[1] into K buffer 1 and V[0] into V buffer 0
  auto issue_prologue = [&]() {
    if (ntiles > 1) dma_tile4_fwd(ka.k, ka.krb, kv_len(ka), lds0 + kTileBytes, dl, wave & 3);
    dma_tile4_fwd(dv.v, dv.vrb, kv_len(dv), lds0 + 2 * kTileBytes, dl, wave & 3);
    if (ntiles > 1) kv_next(seg, src, dv);
  };
  // group B, start of iteration j: V[j+1] into V buffer (j+1)&1
  auto issue_v = [&](int j) {
    if (j + 1 < ntiles) dma_tile4_fwd(dv.v, dv.vrb, kv_len(dv), lds0 + (2 + ((j + 1) & 1)) * kTileBytes, dl, wave & 3);
    if (j + 2 < ntiles) kv_next(seg, src, dv);
  };
  // group A, end of M(j): K[j+2] into K buffer j&1 (free: K[j] was last read
  // in group B's M(j-1), before the barrier that opened M(j))
  auto issue_k = [&](int j) {
    if (j + 2 < ntiles) dma_tile4_fwd(ka.k, ka.krb, kv_len(ka), lds0 + ((j + 2) & 1) * kTileBytes, dl, wave & 3);
    if (j + 3 < ntiles) kv_next(seg, src, ka);
  };
  // M(j): scores of tile j+1 (if with_s) and P[j] V[j] (if with_pv); par = j & 1
  auto mphase = [&](auto with_s, auto with_pv, auto par) {
    constexpr int P = decltype(par)::value;
    const char* kt = smem + (1 - P) * kTileBytes;
    const char* vt = smem + (2 + P) * kTileBytes;
    if constexpr (decltype(with_s)::value) qk_tile(kt, qv, lo, s);
    if constexpr (decltype(with_pv)::value) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
          const char* vr = vt + (kb * 32 + 16 * cc) * 256;
#pragma unroll
          for (int db = 0; db < 4; db++) o[db] = mfma(lds_col8_at(vr, lo.v[db][0], lo.v[db][1]), pb[kb][cc], o[db]);
        }
    }
    if constexpr (decltype(with_s)::value) {
      // the lane's max over the new scores, taken while the P V MFMAs run
      // (the softmax phase uses it unless the tile is masked)
      s_max = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) s_max = fmaxf(s_max, s[kb][r]);
      asm volatile("" : "+v"(s_max));  // formed in this phase, not sunk past its barrier
    }
    if constexpr (decltype(with_s)::value && decltype(with_pv)::value) {
      // 48 LDS reads (16 K rows, 32 transposed V halves) for 32 MFMAs: keep
      // kMphaseAhead reads in flight ahead of the MFMA that consumes them
      __builtin_amdgcn_sched_group_barrier(0x100, kMphaseAhead, 0);
      static_for<(48 - kMphaseAhead) / 2>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      });
      __builtin_amdgcn_sched_group_barrier(0x008, 32 - (48 - kMphaseAhead) / 2, 0);
    }
  };
  // V(j): softmax of the scores of tile j+1 into pb, rescaling O and l
  auto vphase = [&](int j) {
    // visibility: key kb*32 + 16*(r/8) + 8*h + r%8 <= lim. A tile entirely in
    // this wave's future gets lim < 0 (nothing visible).
    float mt = s_max;
    const bool m_suffix = mc.d == 0;
    if (mc.rem < kTileRows || (m_suffix && mc.pos0 + kTileRows - 1 > tw0)) {
      int lim = kv_len(mc) - 1 - 8 * h;
      if (m_suffix) lim = min(lim, t - mc.pos0 - 8 * h);
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) s[kb][r] = (kb * 32 + 16 * (r >> 3) + (r & 7) <= lim) ? s[kb][r] : -INFINITY;
      mt = s[0][0];
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) mt = fmaxf(mt, s[kb][r]);
    }
    if (j + 2 < ntiles) kv_next(seg, src, mc);
    // Lanes n and n + 32 hold the same query row (different keys) and share
    // its reference max m. A row outgrew m iff one of its two halves did, so
    // the test needs no exchange; the row max over both halves is formed only
    // on the (rare) rescale path, which keeps the cross-lane round trip off
    // the common path.
    if (__any(mt > m + slack)) {  // some row outgrew its reference max: rescale
      mt = wave_max32(mt);
      const float m_new = fmaxf(m, mt);
      const float alpha = fast_exp2((m - m_new) * c2);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int db = 0; db < 4; db++) o[db] *= alpha;
    }
    const float mc2 = m * c2;
    float ls = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int cc = 0; cc < 2; cc++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float p = fast_exp2(fmaf(s[kb][8 * cc + i], c2, -mc2));
          ls += p;  // fp32 row sum of the unrounded probabilities
          pb[kb][cc][i] = static_cast<bf16>(p);
        }
        pin(pb[kb][cc]);
      }
    l += ls;
  };

#pragma unroll
  for (int c = 0; c < 8; c++) settle(qv[c]);
  wait_dma();
  __syncthreads();  // K[0] landed

  // A workgroup barrier that also fences the instruction scheduler: the
  // phases' register-only work (MFMAs, exps) must not migrate across it.
  auto phase_barrier = [] {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr std::true_type yes{};
  constexpr std::false_type no{};
  constexpr std::integral_constant<int, 0> even{};
  constexpr std::integral_constant<int, 1> odd{};
  // Both groups pass 2 * ntiles + 2 barriers; B's phase k runs between
  // barriers k and k + 1, A's between barriers k - 1 and k. The tile loop is
  // unrolled by two so that the buffer parity, and with it every LDS address
  // offset, is a compile-time constant.
  if (grp == 0) {
    if (ntiles > 2) kv_next(seg, src, ka);  // A's K cursor starts at tile 2
    auto body = [&](auto par, int j) {
      mphase(yes, yes, par);
      __builtin_amdgcn_sched_barrier(0);
      issue_k(j);
      phase_barrier();
      vphase(j);
      __builtin_amdgcn_sched_barrier(0);
      wait_dma();
      phase_barrier();
    };
    mphase(yes, no, odd);
    phase_barrier();
    vphase(-1);
    phase_barrier();
    int j = 0;
    for (; j + 2 < ntiles; j += 2) {
      body(even, j);
      body(odd, j + 1);
    }
    if (j + 1 < ntiles) body(even, j++);
    if (j & 1) mphase(no, yes, odd);
    else mphase(no, yes, even);
    phase_barrier();
    phase_barrier();
  } else {
    auto body = [&](auto par, int j) {
      issue_v(j);
      vphase(j - 1);
      phase_barrier();
      mphase(yes, yes, par);
      __builtin_amdgcn_sched_barrier(0);
      wait_dma();
      phase_barrier();
    };
    issue_prologue();
    phase_barrier();
    mphase(yes, no, odd);
    wait_dma();
    phase_barrier();
    int j = 0;
    for (; j + 2 < ntiles; j += 2) {
      body(even, j);
      body(odd, j + 1);
    }
    if (j + 1 < ntiles) body(even, j++);
    vphase(j - 1);
    phase_barrier();
    if (j & 1) mphase(no, yes, odd);
    else mphase(no, yes, even);
    phase_barrier();
  }

  const float lt = wave_sum32(l);  // all 64 lanes take part in the exchange
  if (tw0 >= len) return;
  const float inv = 1.f / lt;
  if (h == 0 && t < len) a.lse[static_cast<int64_t>(head) * a.total_q + row0 + t] = m * a.scale + logf(lt);
  // O as whole non-temporal rows: cacheable stores would park the output in
  // L2 and evict the shared prefix K/V the other workgroups of the XCD still
  // read. Every tile read finished before the last barrier, so the tile
  // buffers are free for the row staging.
  store_tile_rows(smem + wave * 8192, o, inv,
                  static_cast<bf16*>(a.out) + static_cast<int64_t>(row0 + tw0) * qstride + head * kMfmaD, qstride,
                  len - tw0, lane);
}

// ---------------------------------------------------------------------------
// delta[h][t] = sum_d dout[t][h][d] * out[t][h][d] (head_dim 128). A workgroup
// takes 64 tokens of one head: 16 lanes per (t, h) row, one 16-byte load of
// each tensor per lane and row, four rows per 16-lane group (eight loads in
// flight per lane). The row sums meet in LDS so that the per-head outputs --
// delta, and the stat rows the dK/dV kernel copies per query block
// (-lse*log2e, -delta) -- are written 64 consecutive floats at a time. Also
// the two constants for rows past a block's end.
// ---------------------------------------------------------------------------
constexpr int kDeltaTokens = 64;

__global__ __launch_bounds__(256) void mfma_delta(KernelArgs a) {
  const int head = blockIdx.y;
  const int t0 = blockIdx.x * kDeltaTokens;
  const int c = threadIdx.x & 15, r = threadIdx.x >> 4;
  __shared__ float sums[kDeltaTokens];
  bf16x8 o[4], g[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int t = t0 + 16 * k + r;
    if (t < a.total_q) {
      const int64_t at = (static_cast<int64_t>(t) * a.hq + head) * kMfmaD + 8 * c;
      o[k] = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(a.out_in) + at);
      g[k] = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(a.dout) + at);
    } else {
      o[k] = bf16x8{};
      g[k] = bf16x8{};
    }
  }
#pragma unroll
  for (int k = 0; k < 4; k++) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) s = fmaf(static_cast<float>(o[k][i]), static_cast<float>(g[k][i]), s);
    s += __shfl_xor(s, 8);
    s += __shfl_xor(s, 4);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 1);
    if (c == 0) sums[16 * k + r] = s;
  }
  __syncthreads();
  const int i = threadIdx.x;
  if (i < kDeltaTokens && t0 + i < a.total_q) {
    const int64_t at = static_cast<int64_t>(head) * a.total_q + t0 + i;
    const float s = sums[i];
    a.delta[at] = s;
    a.stat_ws[kStatRowsOffset + at] = -(a.lse_in[at] * kLog2e);  // the dK/dV kernel copies these rows
    a.ndelta_ws[at] = -s;
  }
  if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    a.stat_ws[0] = -INFINITY;  // -lse*log2e of a query past a block's end: P = 0
    a.stat_ws[1] = 0.f;       // its -delta
  }
}

// ---------------------------------------------------------------------------
// dQ: same workgroup shape, key stream and two-group ping-pong as the forward.
//   M(j): dQ^T += K[j]^T dS^T[j], S^T[j+1] = K[j+1] Q^T, dP^T[j+1] = V[j+1] dO^T
//   V(j): dS^T[j+1] = P^T (dP^T - delta), P^T = exp(scale S^T - lse)
// dQ = scale * dQ at the end. The A operand of dQ^T is K^T: instead of every
// wave reading K column-wise (ds_read_tr16_b64, several times slower than row
// reads), group A's V(j) phase transposes K[j+1] once into a K^T tile
// (rows = head dims, 64 keys each) that all waves then read row-wise. Group B
// copies K[j+2] and V[j+2] at the start of its V(j-1) phase and waits for them
// at the end of its M(j). Two buffers each of K, V and K^T (96 KiB).
// ---------------------------------------------------------------------------
constexpr int kKtRowBytes = 128;  // K^T tile: 128 rows (head dims) x 64 keys

// Byte offset of 16-byte chunk `chunk` (keys 8*chunk..+7) of row d of a K^T
// tile. The chunk is XOR-ed with ((d >> 1) & 7) ^ ((d & 1) << 2): measured
// on gfx950 (LDS bank-conflict counter, one wave writing / reading this
// pattern), this leaves both the transposing b128 writes (lane l: row l % 32,
// chunk l / 32) and the row-wise b128 reads of the dQ MFMA free of bank
// conflicts, where (d >> 1) & 7 alone costs 8 conflict cycles per write and
// d & 7 alone 4 per read.
__device__ __forceinline__ uint32_t kt_off(int d, int chunk) {
  return static_cast<uint32_t>(d * kKtRowBytes + ((chunk ^ ((d >> 1) & 7) ^ ((d & 1) << 2)) << 4));
}

#ifndef TPR_DQ_AHEAD
#define TPR_DQ_AHEAD 4
#endif
constexpr int kDqAhead = TPR_DQ_AHEAD;  // LDS reads issued ahead in a dQ M phase

template <bool kRunList, bool kStrided>  // as mfma_fwd
__global__ __launch_bounds__(512) void mfma_dq(KernelArgs a) {
  static_assert(kFwdWaves == 8, "two groups of one wave per SIMD");
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh0 = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = wave >> 2;                         // 0: group A (transposes K), 1: group B (copies)
  const int hpw = a.hpw;
  const int head = qh0 + wave % hpw;
  const int tw0 = tok0 + kFwdTokens * (wave / hpw);
  const int tpw = kFwdTokens * (kFwdWaves / hpw);
  const int suffix_keys = min(len, tok0 + tpw);
  const int n = lane & 31, h = lane >> 5;
  const int t = tw0 + n;
  const int tc = min(t, len - 1);

  const int64_t qstride = static_cast<int64_t>(a.hq) * kMfmaD;  // dO and dQ rows (packed)
  // row bytes of the suffix K and V (views of a wider buffer allowed) and of
  // the packed prefix K/V; the full-tile copy offsets are made for the latter
  const uint32_t p_rb = static_cast<uint32_t>(a.hkv) * kMfmaD * 2;
  const uint32_t k_rb = kStrided ? static_cast<uint32_t>(a.k_rs) * 2 : p_rb;
  const uint32_t v_rb = kStrided ? static_cast<uint32_t>(a.v_rs) * 2 : p_rb;
  const int64_t q_rs = kStrided ? a.q_rs : qstride;

  // K0 K1 V0 V1 (row-major, swizzled) | T0 T1 (K^T)
  __shared__ __attribute__((aligned(1024))) char smem[6 * kTileBytes];
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  constexpr int kT = 4 * kTileBytes;  // K^T buffers

  const char* kbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.k) + kvh * kMfmaD);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.v) + kvh * kMfmaD);
  const char* pkbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pk) + kvh * kMfmaD);
  const char* pvbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pv) + kvh * kMfmaD);
  const TileLanes4 dl = make_tile_lanes4(wave & 3, lane, p_rb);
  // K/V row reads (A operands of S, dP) and, for group A, the transposing reads
  const FwdLdsOffsets lo = make_fwd_lds_offsets(lane);
  // K^T reads (A operand of dQ^T): row 32db + n, keys 32kb + 16cc + 8h: the
  // offset is ktb ^ (64kb + 32cc) + 4096db (+ buffer), as the swizzle of row
  // 32db + n is that of row n
  uint32_t ktb = static_cast<uint32_t>(kT) + kt_off(n, h);
  // group A's transposing column reads: columns 32w.. (w = wave & 3), the
  // offsets of lo.v[w] computed directly (a wave-indexed register array would
  // be moved to memory by the compiler)
  uint32_t tro[2];
  {
    const int g = lane >> 4, i = lane & 15;
    const int row = 8 * h + (i >> 2), col = 32 * (wave & 3) + ((g & 1) << 4) + ((i & 3) << 2);
    tro[0] = static_cast<uint32_t>(swz_off(row, col));
    tro[1] = static_cast<uint32_t>(swz_off(row + 4, col));
  }

  const auto seg = load_keys<kRunList>(a, leaf, suffix_keys);
  const int ntiles = seg.ntiles;
  auto kv_rb = [&](const TileLoc& x, bool is_k) __attribute__((always_inline)) {
    return x.suffix ? (is_k ? k_rb : v_rb) : p_rb;
  };
  auto kv_src = [&](const TileLoc& x, bool is_k) __attribute__((always_inline)) {
    const char* b = x.suffix ? (is_k ? kbase : vbase) : (is_k ? pkbase : pvbase);
    return b + x.row * static_cast<int64_t>(kv_rb(x, is_k));
  };
  // group B's copy cursor: the next tile whose K and V it copies
  Cursor dc = cursor_begin(seg);
  TileLoc tl_c = cursor_tile(dc);
  if (grp) {
    dma_tile4(kv_src(tl_c, true), kv_rb(tl_c, true), tl_c.len, lds0, dl, wave & 3, kv_rb(tl_c, true) == p_rb);
    dma_tile4(kv_src(tl_c, false), kv_rb(tl_c, false), tl_c.len, lds0 + 2 * kTileBytes, dl, wave & 3,
              kv_rb(tl_c, false) == p_rb);
  }
  if (ntiles > 1) {
    cursor_next(seg, dc);
    tl_c = cursor_tile(dc);
  }
  Cursor mc = cursor_begin(seg);
  TileLoc tl_m = cursor_tile(mc);

  bf16x8 qv[8], gv[8];
  {
    const int64_t off = static_cast<int64_t>(row0 + tc) * qstride + head * kMfmaD + 8 * h;
    const int64_t qoff = kStrided ? static_cast<int64_t>(row0 + tc) * q_rs + head * kMfmaD + 8 * h : off;
    const bf16* qp = static_cast<const bf16*>(a.q) + qoff;
    const bf16* gp = static_cast<const bf16*>(a.dout) + off;
#pragma unroll
    for (int c = 0; c < 8; c++) {
      qv[c] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(qp + 16 * c));
      gv[c] = __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(gp + 16 * c));
    }
  }
  const int64_t stat = static_cast<int64_t>(head) * a.total_q + row0 + tc;
  const float c2 = a.scale * kLog2e;
  const float lse2 = a.lse_in[stat] * kLog2e;
  const float delta = a.delta[stat];

  f32x16 dq[4];
#pragma unroll
  for (int i = 0; i < 4; i++) dq[i] = f32x16{};
  f32x16 s[2], dp[2];
  bf16x8 dsb[2][2];

  // group B, start of iteration j: copy K[j+2] and V[j+2] into buffers j & 1
  auto issue = [&](int j) __attribute__((always_inline)) {
    if (j + 2 < ntiles) {
      const int b = j & 1;
      dma_tile4(kv_src(tl_c, true), kv_rb(tl_c, true), tl_c.len, lds0 + b * kTileBytes, dl, wave & 3,
                kv_rb(tl_c, true) == p_rb);
      dma_tile4(kv_src(tl_c, false), kv_rb(tl_c, false), tl_c.len, lds0 + (2 + b) * kTileBytes, dl, wave & 3,
                kv_rb(tl_c, false) == p_rb);
    }
    if (j + 3 < ntiles) {
      cursor_next(seg, dc);
      tl_c = cursor_tile(dc);
    }
  };
  // group A wave w: rows 32w..32w+31 of K^T[x] from K[x] (buffer parity P):
  // four column reads of 16 keys x 32 dims, one 16-byte chunk per lane each
  auto transpose_k = [&](auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    const char* src = smem + P * kTileBytes;
    char* dst = smem + kT + P * kTileBytes;
    const int d = 32 * (wave & 3) + n;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const bf16x8 x = lds_col8_at(src + 16 * g * 256, tro[0], tro[1]);
      *reinterpret_cast<bf16x8*>(dst + kt_off(d, 2 * g + h)) = x;
    }
  };
  // M(j), P = j & 1: S, dP of tile j+1 (if with_sd) and dQ += dS[j] K[j] (if with_dq)
  auto mphase = [&](auto with_sd, auto with_dq, auto par) __attribute__((always_inline)) {
    constexpr int P = decltype(par)::value;
    const char* kn = smem + (1 - P) * kTileBytes;        // K[j+1]
    const char* vn = smem + (3 - P) * kTileBytes;        // V[j+1]
    const char* kt = smem + P * kTileBytes;              // K^T[j] (+ kT in ktb)
    if constexpr (decltype(with_dq)::value) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int cc = 0; cc < 2; cc++) {
          const uint32_t o = ktb ^ static_cast<uint32_t>(64 * kb + 32 * cc);
#pragma unroll
          for (int db = 0; db < 4; db++)
            dq[db] = mfma(*reinterpret_cast<const bf16x8*>(kt + 4096 * db + o), dsb[kb][cc], dq[db]);
        }
    }
    if constexpr (decltype(with_sd)::value) {
#pragma unroll
      for (int kb = 0; kb < 2; kb++) {
        s[kb] = f32x16{};
        dp[kb] = f32x16{};
#pragma unroll
        for (int c = 0; c < 8; c++) {
          s[kb] = mfma(*reinterpret_cast<const bf16x8*>(kn + kb * 32 * 256 + lo.k[c]), qv[c], s[kb]);
          dp[kb] = mfma(*reinterpret_cast<const bf16x8*>(vn + kb * 32 * 256 + lo.k[c]), gv[c], dp[kb]);
        }
      }
    }
    if constexpr (kDqAhead > 0 && decltype(with_sd)::value && decltype(with_dq)::value) {
      // 48 row reads for 48 MFMAs: keep kDqAhead reads in flight
      __builtin_amdgcn_sched_group_barrier(0x100, kDqAhead, 0);
      static_for<48 - kDqAhead>([&](auto) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      });
      __builtin_amdgcn_sched_group_barrier(0x008, kDqAhead, 0);
    }
  };
  // V(j): dS of tile j+1 into dsb
  auto vphase = [&](int j) __attribute__((always_inline)) {
    if (tl_m.len < kTileRows || (tl_m.suffix && tl_m.pos0 + kTileRows - 1 > tw0)) {
      int lim = tl_m.len - 1 - 8 * h;
      if (tl_m.suffix) lim = min(lim, t - tl_m.pos0 - 8 * h);
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) s[kb][r] = (kb * 32 + 16 * (r >> 3) + (r & 7) <= lim) ? s[kb][r] : -INFINITY;
    }
    if (j + 2 < ntiles) {
      cursor_next(seg, mc);
      tl_m = cursor_tile(mc);
    }
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
#pragma unroll
      for (int cc = 0; cc < 2; cc++) {
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const float p = fast_exp2(fmaf(s[kb][8 * cc + i], c2, -lse2));
          dsb[kb][cc][i] = static_cast<bf16>(p * (dp[kb][8 * cc + i] - delta));
        }
        pin(dsb[kb][cc]);
      }
  };
  auto phase_barrier = [] {
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
  };
  constexpr std::true_type yes{};
  constexpr std::false_type no{};
  constexpr std::integral_constant<int, 0> even{};
  constexpr std::integral_constant<int, 1> odd{};
  // Every wave runs every phase: a tile it does not see is masked to P = 0
  // (dS = 0). One M-phase body per buffer parity keeps the live registers
  // within the two-waves-per-SIMD budget.
  auto last_m = [&]() __attribute__((always_inline)) {
    if ((ntiles - 1) & 1) mphase(no, yes, odd);
    else mphase(no, yes, even);
  };
  auto run = [&](auto body) __attribute__((always_inline)) {
    int j = 0;
    for (; j + 2 < ntiles; j += 2) {
      body(even, j);
      body(odd, j + 1);
    }
    if (j + 1 < ntiles) body(even, j);
  };

#pragma unroll
  for (int c = 0; c < 8; c++) {
    settle(qv[c]);
    settle(gv[c]);
  }
  settle(lse2);
  settle(delta);
  wait_dma();
  __syncthreads();  // K[0], V[0] landed

  // Both groups pass 2 * ntiles + 2 barriers, B one phase behind A. A's V(j)
  // also transposes K[j+1] (buffer parity of j + 1).
  if (grp == 0) {
    mphase(yes, no, odd);
    phase_barrier();
    transpose_k(even);
    vphase(-1);
    phase_barrier();
    run([&](auto par, int j) __attribute__((always_inline)) {
      constexpr int P = decltype(par)::value;
      mphase(yes, yes, par);
      phase_barrier();
      if (j + 1 < ntiles) transpose_k(std::integral_constant<int, 1 - P>{});
      vphase(j);
      phase_barrier();
    });
    last_m();
    phase_barrier();
    phase_barrier();
  } else {
    issue(-1);
    phase_barrier();
    mphase(yes, no, odd);
    __builtin_amdgcn_sched_barrier(0);
    wait_dma();
    phase_barrier();
    run([&](auto par, int j) __attribute__((always_inline)) {
      issue(j);
      vphase(j - 1);
      phase_barrier();
      mphase(yes, yes, par);
      __builtin_amdgcn_sched_barrier(0);
      wait_dma();
      phase_barrier();
    });
    vphase(ntiles - 2);
    phase_barrier();
    last_m();
    phase_barrier();
  }

  if (tw0 >= len) return;
  // every tile read finished before the last barrier: the tile buffers are free
  store_tile_rows(smem + wave * 8192, dq, a.scale,
                  static_cast<bf16*>(a.dq) + static_cast<int64_t>(row0 + tw0) * qstride + head * kMfmaD, qstride,
                  len - tw0, lane);
}

// ---------------------------------------------------------------------------
// dQ from the dS store: dQ^T = K^T dS^T, times scale -- the forward's P V
// product with V -> K and P -> dS, the dS blocks read from what the dK/dV
// kernel stored instead of recomputed from Q, K, dO and V. Work items are the
// plan's own (PF_OFF_DQS): 8 waves, two per SIMD, each one whole 64-query
// block of one query head, so every K^T operand a wave reads from LDS feeds
// two MFMAs (its two 32-query sub-blocks) and every K row copied serves 512
// query rows. The key stream follows the dK/dV kernel's tiling: the leaf's
// ancestor nodes root first, then its suffix, each in 128-key tiles of two
// 64-key halves, so every half lies in one dS slot. Per half: every wave
// copies two 1 KiB blocks of the K rows (swizzled like the forward's V tile,
// read column-wise as the A operand) and its own 64 x 64 dS block (8 KiB),
// then runs 32 MFMAs.
// A slot holds a head's 128 x 64 block as four 4 KiB wave blocks of 32 keys,
// each [32-query half j][16-query quarter qc][lane L] x 8 queries, lane L
// holding key L % 32 and queries 32 j + 16 qc + 8 (L / 32) .. +7 (the dK/dV
// kernel's register order). The copy puts chunk L of each 1 KiB block at
// L ^ (8 (L / 32) + 4 qc), which spreads every 32-lane pass of the
// transposed operand reads over all 64 banks. K and dS are double-buffered
// (two halves of K and of every wave's dS: 160 KiB of LDS). The next half's
// K rows are copied right after the barrier that frees their buffer; a
// wave's dS buffer is its own, so the dS two halves ahead is copied into it
// as soon as the wave's reads of the current half's dS have returned.
// ---------------------------------------------------------------------------
template <bool kStrided>
__global__ __launch_bounds__(512) void mfma_dqs(KernelArgs a) {
  const int32_t* item = a.plan + a.off_dqs + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh0 = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int32_t* no = a.plan + a.off_node_off;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hpw = a.hpw_dqs;
  const int head = qh0 + wave % hpw;
  const int tw0 = tok0 + kDqsTokens * (wave / hpw);  // first token of this wave (a query block's first)
  const int tpw = kDqsTokens * (kFwdWaves / hpw);
  const int suffix_keys = min(len, tok0 + tpw);
  const bool wave_ok = tw0 < len;
  const int qb = a.plan[a.off_leaf_qblk + leaf] + tw0 / kDkdvQ;  // the wave's query block
  static_assert(kDqsTokens == kDkdvQ, "a dQ wave is one query block of the dS slots");

  const int64_t qstride = static_cast<int64_t>(a.hq) * kMfmaD;
  const uint32_t p_rb = static_cast<uint32_t>(a.hkv) * kMfmaD * 2;
  const uint32_t k_rb = kStrided ? static_cast<uint32_t>(a.k_rs) * 2 : p_rb;

  constexpr int kBufs = 2;
  constexpr int kDsWave = 8192;                   // one wave's dS block per half
  constexpr int kDsOff = kBufs * kTileBytes;      // K [buffer] | dS [buffer][wave]
  __shared__ __attribute__((aligned(1024))) char smem[kBufs * (kTileBytes + kFwdWaves * kDsWave)];
  static_assert(sizeof(smem) >= kFwdWaves * 2 * 8192, "the output rows are staged in the tile buffers");
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));

  const char* kbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.k) + kvh * kMfmaD);
  const char* pkbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pk) + kvh * kMfmaD);
  // K copy: wave w moves blocks 2w, 2w + 1 of the tile (rows 8w + 4j + l / 16)
  const uint32_t krow0 = static_cast<uint32_t>(8 * wave + (lane >> 4));
  const uint32_t kcb0 = static_cast<uint32_t>(16 * ((lane & 15) ^ ((lane >> 4) << 2)));
  const FwdLdsOffsets lo = make_fwd_lds_offsets(lane);
  // dS copy of one 32-query half, block (kb, qc) = 2 kb + qc: lane l fetches
  // the chunk that lands at l (the swizzle is its own inverse)
  uint32_t dsv[4];
#pragma unroll
  for (int j = 0; j < 4; j++) dsv[j] = dqs_ds_lane_bytes(lane, j);
  // dS^T operand reads (B: lane l gets query l % 32, keys 8 (l / 32) + 0..7
  // of a 16-key step). As a source row of ds_read_tr16_b64, lane l (group
  // g = l / 16, e = (l % 16) / 4, m = l % 4) addresses key 8 (g / 2) + 4 t + e,
  // queries 16 (g % 2) + 4 m .. +3; t = 0 / 1 gives keys +0..3 / +4..7.
  uint32_t dso[2];
  {
    const int g = lane >> 4, e = (lane & 15) >> 2, m = lane & 3, qc = g & 1;
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int L = 8 * (g >> 1) + 4 * t + e + 32 * (m >> 1);
      dso[t] = qc * 1024 + 16 * (L ^ (8 * (L >> 5) + 4 * qc)) + 8 * (m & 1);
    }
  }

  // Key stream cursor (uniform): ancestor index cd (max_depth = the suffix,
  // past it = the end), first row, length, key limit, tile key, half, and the
  // tile's position in the stream. Plan words inside the stream are scalar
  // loads. The dS slots of the wave's query block are numbered in this same
  // order from the block's first slot, so slot = first + cpos; at
  // [KV head][slot][query head of the group] the wave's blocks follow each
  // other tile by tile.
  const int depth = a.max_depth;
  const int32_t* anc = a.plan + a.off_anc + static_cast<int64_t>(leaf) * depth;
  int cd = -1, crow = 0, clen = 0, clim = 0, ckey = 0, chalf = 0, cpos = 0;
  auto next_segment = [&]() {
    for (;;) {
      cd++;
      if (cd < depth) {
        const int nd = plan_word(anc + cd);
        if (nd >= 0) {
          crow = plan_word(no + nd);
          const int l = plan_word(no + nd + 1) - crow;
          if (l == 0) continue;
          clen = clim = l;
          break;
        }
        cd = depth;  // -1 pads the list: the suffix is next
      }
      if (cd == depth) {
        crow = row0;
        clen = len;
        clim = suffix_keys;
      } else {
        clen = clim = 0;  // past the end
      }
      break;
    }
    ckey = 0;
    chalf = 0;
  };
  auto advance = [&]() {
    chalf++;
    if (chalf == 2 || ckey + kTileRows * chalf >= clim) {
      chalf = 0;
      ckey += kDkdvKeys;
      cpos++;
      if (ckey >= clim) next_segment();
    }
  };
  // this wave's dS blocks: its query block's first slot, its head
  const char* ds_wave = nullptr;
  if (wave_ok) {
    const int first = plan_word(a.plan + a.off_ds_first + qb);
    ds_wave = static_cast<const char*>(a.ds) +
              ((static_cast<int64_t>(kvh) * a.ds_slots + first) * a.group + (head - kvh * a.group)) * kDsHeadBytes;
  }
  const int64_t ds_tile_bytes = static_cast<int64_t>(a.group) * kDsHeadBytes;  // one slot of the group

  // A half of the stream (uniform): its K rows, their count, whether this
  // wave reads it (prefix halves: every wave; suffix halves: those not
  // entirely in the wave's future) and its dS source. `more` is false past
  // the end.
  struct Half {
    const char* k;
    const char* ds;
    uint32_t rb;
    int rows;
    bool vis, more;
  };
  auto half_here = [&]() __attribute__((always_inline)) {
    const int k0 = ckey + kTileRows * chalf;
    const bool suffix = cd == depth;
    Half t;
    t.more = clim > 0;
    t.rb = suffix ? k_rb : p_rb;
    t.k = (suffix ? kbase : pkbase) + static_cast<int64_t>(crow + k0) * t.rb;
    t.ds = ds_wave + cpos * ds_tile_bytes + 2 * chalf * 4096;
    t.rows = min(kTileRows, clen - k0);
    t.vis = t.more && wave_ok && (!suffix || k0 <= tw0 + kDqsTokens - 1);
    return t;
  };
  // copy a half's K rows into K buffer b (2 blocks per wave), and the wave's
  // 8 KiB of its dS (two 32-query halves of 4 blocks each) into dS buffer b
  // if it reads the half
  auto issue_k = [&](const Half& t, int b) __attribute__((always_inline)) {
    const uint32_t last = static_cast<uint32_t>(t.rows - 1);
#pragma unroll
    for (int j = 0; j < 2; j++)  // block 2w + j: rows 8w + 4j + l / 16; the swizzle's row term is (2w + j) % 4
      dma16s(t.k, min(krow0 + 4u * j, last) * t.rb + (kcb0 ^ (16u * ((2 * wave + j) & 3))),
             lds0 + b * kTileBytes + (2 * wave + j) * 1024);
  };
  auto issue_ds = [&](const Half& t, int b) __attribute__((always_inline)) {
    if (t.vis) {
      const uint32_t dst = lds0 + kDsOff + (b * kFwdWaves + wave) * kDsWave;
      dma_blocks4_nt(t.ds, dsv[0], dsv[1], dsv[2], dsv[3], dst);
      dma_blocks4_nt(t.ds + 2048, dsv[0], dsv[1], dsv[2], dsv[3], dst + 4096);
    }
  };

  f32x16 dq[2][4];
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) dq[j][i] = f32x16{};
  // 32 MFMAs on buffer b: key step st = (kb, kc) covers keys 32 kb + 16 kc ..
  // +15. The dS operands of key step st are read with the K^T operands, four
  // slots ahead of their first MFMA, so the MFMAs start after three reads.
  // LDS reads return in issue order: once slot 12's MFMAs (the first to use
  // key step 3) have issued, every read of the wave's dS buffer has returned
  // and the dS of half `next` may be copied into it.
  auto compute = [&](int b, int rows, const Half& next) __attribute__((always_inline)) {
    const char* kt = smem + b * kTileBytes;
    const char* dt = smem + kDsOff + (b * kFwdWaves + wave) * kDsWave;
    if (rows < kTileRows) {
      // a segment's last half: zero the dS of keys at or past `rows` in the
      // wave's buffer (its copy has landed), lane l the chunk it copied for
      // key 32 kb + l % 32 of each 1 KiB block
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
        if (32 * kb + (lane & 31) >= rows) {
#pragma unroll
          for (int j = 0; j < 2; j++)
#pragma unroll
            for (int qc = 0; qc < 2; qc++)
              *reinterpret_cast<bf16x8*>(const_cast<char*>(dt) + j * 4096 + kb * 2048 + qc * 1024 +
                                         16 * (lane ^ (8 * (lane >> 5) + 4 * qc))) = bf16x8{};
        }
    }
    bf16x8 f[2][4];  // dS^T operands of the two 32-query halves and four key steps
    auto read_f = [&](auto sc) __attribute__((always_inline)) {
      constexpr int st = decltype(sc)::value;
#pragma unroll
      for (int j = 0; j < 2; j++)
        f[j][st] = lds_col8_at(dt + j * 4096 + (st >> 1) * 2048 + (st & 1) * 256, dso[0], dso[1]);
    };
    // one fenced slot per (key step st, head-dim block db): the K^T operand,
    // read kRead slots ahead, and its two MFMAs
    constexpr int kRead = 4, kRing = kRead + 1;
    bf16x8 ra[kRing];
    auto read_slot = [&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value, st = i / 4, db = i % 4;
      ra[i % kRing] = lds_col8_at(kt + (32 * (st >> 1) + 16 * (st & 1)) * 256, lo.v[db][0], lo.v[db][1]);
    };
    read_f(std::integral_constant<int, 0>{});
    static_for<kRead>([&](auto ic) { read_slot(ic); });
    static_for<16>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i == 13) issue_ds(next, b);
      if constexpr (i + kRead < 16) {
        if constexpr ((i + kRead) % 4 == 0) read_f(std::integral_constant<int, (i + kRead) / 4>{});
        read_slot(std::integral_constant<int, i + kRead>{});
      }
#pragma unroll
      for (int j = 0; j < 2; j++) dq[j][i % 4] = mfma(ra[i % kRing], f[j][i / 4], dq[j][i % 4]);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Half j sits in K buffer and dS buffer j % 2. At step i the K rows of
  // half i + 1 are copied after the barrier (every wave is then done with
  // half i - 1's K buffer), and the dS of half i + 2 as soon as the wave holds
  // half i's dS operands in registers, so the dS stream runs two halves
  // ahead. Copies complete in issue order: at the top of step i the last
  // ones issued are half i + 1's dS (8 blocks), and waiting until at most
  // those are outstanding means half i's K rows and dS have landed.
  next_segment();
  Half t0 = half_here();
  issue_k(t0, 0);
  issue_ds(t0, 0);
  advance();
  Half t1 = half_here();
  if (t1.more) issue_ds(t1, 1);
  int b = 0;
  for (;;) {
    if (t1.vis) asm volatile("s_waitcnt vmcnt(8)");
    else wait_dma();
    __syncthreads();  // half i has landed; every wave is done with the other K buffer (half i - 1)
    Half t2{};
    if (t1.more) {
      issue_k(t1, b ^ 1);
      advance();
      t2 = half_here();
    }
    if (t0.vis) compute(b, t0.rows, t2);
    else issue_ds(t2, b);  // the wave did not copy half i's dS: its buffer is free
    if (!t1.more) break;
    t0 = t1;
    t1 = t2;
    b ^= 1;
  }
  __syncthreads();  // every LDS read is done: the buffers are free for the row staging
  if (!wave_ok) return;
#pragma unroll
  for (int j = 0; j < 2; j++)
    if (tw0 + 32 * j < len)
      store_tile_rows(smem + (2 * wave + j) * 8192, dq[j], a.scale,
                      static_cast<bf16*>(a.dq) + static_cast<int64_t>(row0 + tw0 + 32 * j) * qstride + head * kMfmaD,
                      qstride, len - tw0 - 32 * j, lane);
}

// ---------------------------------------------------------------------------
// dK/dV
//   S = Q K^T (query rows permuted by sigma32), P = exp(scale S - lse),
//   dP = dO V^T, dS = P (dP - delta), dV += P^T dO, dK += dS^T Q, dK *= scale.
// K/V of the wave's 32 keys are B operands held in registers; Q/dO blocks of
// 64 queries are copied to LDS and read row-wise (A operands) and
// column-wise (B operands of dV/dK, ds_read_tr16_b64). A stage is one query
// block of kHeads query heads of the GQA group (2 when the group size is even:
// half the stages, and with them half the per-stage barriers and copy waits).
// ---------------------------------------------------------------------------
// MFMA slots (position k within a head's sub-block sequence) at which the
// dK/dV stage stores the two 16-query halves of a dS block: the first half
// is complete at k = 22, the second at k = 27
#ifndef TPR_DS_STORE_K1
#define TPR_DS_STORE_K1 23
#endif
#ifndef TPR_DS_STORE_K2
#define TPR_DS_STORE_K2 28
#endif
#ifndef TPR_DKDV_INTERLEAVE
#define TPR_DKDV_INTERLEAVE 1
#endif
// S / dP MFMAs of the dK/dV stage with the accumulator in VGPRs (the softmax
// VALU reads it there) and the K / V operand in AGPRs. The compiler gives every
// MFMA of a kernel one accumulator class; the dK/dV accumulators need AGPRs, so
// these two chains are written as asm. Hazards the compiler no longer tracks
// for them: a VALU read of the result needs ~19 wait states after the chain's
// last MFMA (the stage schedule puts it at least 4 MFMA slots later), and a
// chained MFMA reads its predecessor's result as srcC with the other
// sub-block's MFMA between them, the spacing the builtin form also uses.
__device__ __forceinline__ f32x16 mfma_vsp_init(bf16x8 a, bf16x8 b_agpr, f32x16 c) {
  f32x16 d;
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %3" : "=&v"(d) : "v"(a), "a"(b_agpr), "v"(c));
  return d;
}
__device__ __forceinline__ void mfma_vsp_acc(f32x16& d, bf16x8 a, bf16x8 b_agpr) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "a"(b_agpr));
}

// dK/dV stage slots: with kInterleave the two 32-query sub-blocks of a head
// alternate slot by slot (slot m: sub-block m % 2, position m / 2), so each
// sub-block's dependent steps (S -> P -> dV, dP -> dS -> dK) are two slots
// apart and the other sub-block's work fills the gap; otherwise they run
// one after the other (slot m: sub-block m / 32, position m % 32).
constexpr bool kInterleave = TPR_DKDV_INTERLEAVE;
constexpr int slot_sub(int m) { return kInterleave ? (m & 1) : (m >> 5); }
constexpr int slot_pos(int m) { return kInterleave ? (m >> 1) : (m & 31); }

// kStrided as in mfma_fwd; kStoreDs: also store every dS block to the dS
// store (a.ds) for the dQ kernel
template <int kHeads, bool kStrided, bool kStoreDs>
__global__ __launch_bounds__(256) void mfma_dkdv(KernelArgs a) {
  const int32_t* item = a.plan + a.off_dkdv + DK_WORDS * blockIdx.x;
  if (item[DK_SRC] < 0) return;
  const bool prefix = item[DK_SRC] == 0;
  const int seg = item[DK_SEG], kvh = item[DK_KVH];
  const int32_t* cu = a.plan + a.off_cu;
  const int32_t* no = a.plan + a.off_node_off;
  const int32_t* qblk = a.plan + a.off_qblk;
  const int seg_row0 = prefix ? no[seg] : cu[seg];
  const int seg_len = prefix ? no[seg + 1] - no[seg] : cu[seg + 1] - cu[seg];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 31, h = lane >> 5;

  const int64_t kstride = static_cast<int64_t>(a.hkv) * kMfmaD;  // packed K/V rows: prefix inputs, every output

  // two stage buffers of kHeads (Q, dO) tile pairs: the copies of stage s + 1
  // run during stage s
  __shared__ __attribute__((aligned(1024))) char smem[2 * kHeads * 2 * kTileBytes];
  __shared__ __attribute__((aligned(256))) float stats[2][kHeads][2][kTileRows];  // [buf][head][-lse*log2e | -delta][row]
  // query-block table of the current tile: {first packed row, token start
  // within the leaf, valid rows, dS slot}
  __shared__ int4 qtab[kDkdvMaxBlocks];

  const int spb = a.group / kHeads;  // stages per query block
  const bf16* qbase = static_cast<const bf16*>(a.q);
  const bf16* gbase = static_cast<const bf16*>(a.dout);

  // An item is one key tile, or two suffix tiles of one leaf and KV head
  // (DK_PAIR): a tile and its mirror, so that all pairs of a leaf stream about
  // the same number of query blocks. A suffix tile alone, or the first of a
  // pair, streams its blocks last-first; the second of a pair streams
  // first-last. The pairs of a leaf that run together on one XCD then read
  // the same query block at the same time -- the first tiles count down from
  // the leaf's last block, the second ones up from their diagonal at the
  // same pace -- and share its copies in L2. Prefix tiles stream first-last:
  // they all start together and see the same blocks.
  const int ntiles = item[DK_PAIR] > 0 ? 2 : 1;
  for (int tile = 0; tile < ntiles; tile++) {
    const int key0 = tile == 0 ? item[DK_KEY0] : item[DK_PAIR] - 1;
    const int qb_hi = item[DK_QB_HI];
    const int qb_lo = tile == 0 ? item[DK_QB_LO] : item[DK_QB_LO] - (item[DK_KEY0] - key0) / kTileRows;
    const bool first_last = prefix || tile == 1;
    const int kw0 = key0 + 32 * wave;          // first key position of this wave
    const int kp = kw0 + n;                     // this lane's key position (B-operand column)
    const bool wave_active = kw0 < seg_len;
    const int nstage = (qb_hi - qb_lo) * spb;

    // block table of this tile (planner guarantees <= kDkdvMaxBlocks), read
    // from the plan once, so the stage loop touches no plan memory
    if (tile > 0) __syncthreads();  // every wave is done with the previous tile's table
    const int nblk = qb_hi - qb_lo;
    // the tile's dS slot in the numbering of query block qb: first[qb] + the
    // tiles ahead of it in the dQ walk of any block below its segment
    const int ds_ahead = kStoreDs ? a.plan[a.off_ds + (prefix ? seg : a.num_nodes + seg)] + key0 / kDkdvKeys : 0;
    for (int i = threadIdx.x; i < nblk; i += blockDim.x) {
      const int qb = first_last ? qb_lo + i : qb_hi - 1 - i;
      const int lf = qblk[2 * qb], tok = qblk[2 * qb + 1];
      const int r0 = cu[lf];
      qtab[i] = int4{r0 + tok, tok, min(kTileRows, cu[lf + 1] - r0 - tok),
                     kStoreDs ? a.plan[a.off_ds_first + qb] + ds_ahead : 0};
    }
    __syncthreads();

    // Stage s is (query block s / spb, head pair s % spb), tracked by counters
    // (no division in the loop): `cur` is the stage being computed, `nxt` the
    // one being copied.
    struct StageCursor {
      int blk, sub;
    };
    auto advance = [&](StageCursor c) __attribute__((always_inline)) {
      return c.sub + 1 == spb ? StageCursor{c.blk + 1, 0} : StageCursor{c.blk, c.sub + 1};
    };
    // row bytes of dO (packed; the full-block lane offsets are made for it)
    // and of Q (a view of a wider buffer allowed)
    const uint32_t g_rb = static_cast<uint32_t>(a.hq) * kMfmaD * 2;
    const uint32_t q_rb = kStrided ? static_cast<uint32_t>(a.q_rs) * 2 : g_rb;
    const bool q_packed = !kStrided || q_rb == g_rb;
    const DmaLanes<kDkdvWaves> dl = make_dma_lanes<kDkdvWaves>(g_rb, wave, lane);
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
    // copy the Q and dO rows [row, row + 64) of query head qh into the stage buffer at byte `tile`
    auto issue_stage = [&](int row, int nq, int qh, uint32_t tile) __attribute__((always_inline)) {
      const int64_t col = static_cast<int64_t>(qh) * kMfmaD * 2;
      const int64_t goff = col + static_cast<int64_t>(row) * g_rb;
      const int64_t qoff = kStrided ? col + static_cast<int64_t>(row) * q_rb : goff;
      const uint32_t dst = lds0 + tile + wave * 4096;
      const char* qs = reinterpret_cast<const char*>(qbase) + qoff;
      const char* gs = reinterpret_cast<const char*>(gbase) + goff;
      if (nq >= kTileRows && q_packed) {
        dma_blocks4(qs, dl.voff[0], dl.voff[1], dl.voff[2], dl.voff[3], dst);
        dma_blocks4(gs, dl.voff[0], dl.voff[1], dl.voff[2], dl.voff[3], dst + kTileBytes);
      } else {  // rows at or beyond nq re-read row nq - 1
        uint32_t vq[4], vg[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          vg[j] = static_cast<uint32_t>(min(dl.row[j], nq - 1)) * g_rb + dl.cbytes[j];
          vq[j] = kStrided ? static_cast<uint32_t>(min(dl.row[j], nq - 1)) * q_rb + dl.cbytes[j] : vg[j];
        }
        dma_blocks4_m0(qs, vq[0], vq[1], vq[2], vq[3], dst);
        dma_blocks4_m0(gs, vg[0], vg[1], vg[2], vg[3], dst + kTileBytes);
      }
    };

    // -lse*log2e (which 0) and -delta (which 1) of the stage's 64 query rows of
    // each of its heads, copied into its stat buffer like the tiles -- wave w
    // copies (head w / 2, which w % 2); rows past the block end copy the
    // constants -inf / 0 of the workspace, so their P and dS are exactly 0.
    const uint32_t stats0 = __builtin_amdgcn_readfirstlane(lds_address(stats));
    auto issue_stats = [&](int row, int nq, int qh, int buf) __attribute__((always_inline)) {
      const int hh = wave >> 1, which = wave & 1;
      if (hh < kHeads) {
        const int64_t at = static_cast<int64_t>(qh + hh) * a.total_q + row + lane;
        const float* rows = which == 0 ? a.stat_ws + kStatRowsOffset : a.ndelta_ws;
        dma4_lane(lane < nq ? rows + at : a.stat_ws + which,
                  stats0 + ((buf * kHeads + hh) * 2 + which) * kTileRows * 4);
      }
    };
    auto issue = [&](StageCursor c, int buf) __attribute__((always_inline)) {
      const int4 e = qtab[c.blk];
      const int row = __builtin_amdgcn_readfirstlane(e.x), nq = __builtin_amdgcn_readfirstlane(e.z);
      const int qh = kvh * a.group + c.sub * kHeads;
      issue_stats(row, nq, qh, buf);
#pragma unroll
      for (int hh = 0; hh < kHeads; hh++)
        issue_stage(row, nq, qh + hh, static_cast<uint32_t>((buf * kHeads + hh) * 2 * kTileBytes));
    };
    StageCursor cur{0, 0};
    if (nstage > 0) issue(cur, 0);
    char* ds_stage = nullptr;  // this stage's dS blocks (dS store only)

    bf16x8 kv[8], vv[8];
    {
      const bf16* kb = static_cast<const bf16*>(prefix ? a.pk : a.k);
      const bf16* vb = static_cast<const bf16*>(prefix ? a.pv : a.v);
      const int key = seg_row0 + min(kp, seg_len - 1);
      const int64_t off = static_cast<int64_t>(key) * kstride + kvh * kMfmaD + 8 * h;
      const int64_t koff = prefix || !kStrided ? off : static_cast<int64_t>(key) * a.k_rs + kvh * kMfmaD + 8 * h;
      const int64_t voff = prefix || !kStrided ? off : static_cast<int64_t>(key) * a.v_rs + kvh * kMfmaD + 8 * h;
#pragma unroll
      for (int c = 0; c < 8; c++) {
        kv[c] = *reinterpret_cast<const bf16x8*>(kb + koff + 16 * c);
        vv[c] = *reinterpret_cast<const bf16x8*>(vb + voff + 16 * c);
      }
    }
    f32x16 dk[4], dv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      dk[i] = f32x16{};
      dv[i] = f32x16{};
    }
    // K as the S operand, pre-scaled by scale*log2e (rounded to bf16): the S
    // chain then produces the exponent of P directly
    {
      const float c2 = a.scale * kLog2e;
#pragma unroll
      for (int c = 0; c < 8; c++)
#pragma unroll
        for (int i = 0; i < 8; i++) kv[c][i] = static_cast<bf16>(static_cast<float>(kv[c][i]) * c2);
    }

    // K/V live in AGPRs from here on: the S / dP MFMAs that read them are
    // inline asm, before which the compiler inserts no wait states, so the
    // accvgpr writes must not land next to their first use inside the loop.
#pragma unroll
    for (int c = 0; c < 8; c++) {
      settle_acc(kv[c]);
      settle_acc(vv[c]);
    }
    wait_dma();
    __syncthreads();

    // One stage: 64 queries of each of its kHeads heads against the wave's 32
    // keys, each head as two 32-query sub-blocks j of 32 MFMAs -- S (8), dP (8),
    // dV (8), dK (8). The stage is laid out as one fixed sequence of 64 kHeads
    // slots, one MFMA per slot (head m / 64), fenced so the compiler keeps the
    // order:
    //  * the LDS operands of an MFMA are read kAhead MFMAs of the same
    //    sub-block earlier -- across the boundary between heads too, so the
    //    second head's first MFMAs do not wait for a fresh pipeline;
    //  * the S chain starts from -lse*log2e and the K operand is pre-scaled by
    //    scale*log2e, so the chain ends at the exponent: P = exp2(acc). P of
    //    sub-block j is computed under its dP and first dV MFMAs, dS = P * acc
    //    (the dP chain started from -delta) under its dV and first dK MFMAs, so
    //    the VALU work runs while the matrix core is busy.
    // On a diagonal stage (diag), key kp is visible from query index qi of
    // sub-block j iff qi >= lim - 32j; other stages skip the mask. Queries past
    // the block end carry -lse*log2e = -inf, so their P and dS are exactly 0.
    constexpr int kAhead = 4;  // MFMAs of the same sub-block between a read and its use
    constexpr int kSlotAhead = kInterleave ? 2 * kAhead : kAhead;
    constexpr int kSlots = 64 * kHeads;
    // Lane offsets of the operand reads; the second set carries a 64 KiB bias so
    // that the reads of stage buffer 1 (at 64 KiB when kHeads is 2) keep their
    // constant part within the 16-bit LDS instruction offset.
    constexpr uint32_t kBuf1Bias = kHeads * 2 * kTileBytes >= 65536 ? 65536u : 0u;
    const FwdLdsOffsets lo0 = make_fwd_lds_offsets(lane);
    const FwdLdsOffsets lo1 = make_fwd_lds_offsets(lane, kBuf1Bias);
    auto stage = [&](auto diag, auto bufc, int lim) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      const FwdLdsOffsets& lo = buf ? lo1 : lo0;
      bf16x8 rq[kHeads][2][8], rg[kHeads][2][8], cg[kHeads][2][2][4], cq[kHeads][2][2][4];
      f32x4 l2v[kHeads][2][4], dlv[kHeads][2][4];
      f32x16 sc[kHeads][2], dpv[kHeads][2];
      float p[kHeads][2][16], dsv[kHeads][2][16];
      bf16x8 pb[kHeads][2][2], d8[kHeads][2][2];
      // Q tile of head hh (minus the bias of the offset set used for this
      // buffer); its dO tile follows it
      auto qtile = [&](int hh) __attribute__((always_inline)) {
        return smem + (buf * kHeads + hh) * 2 * kTileBytes - (buf ? kBuf1Bias : 0u);
      };
      // operands of slot M (head M / 64; sub-block and position of M % 64)
      auto read_for = [&](auto mc) __attribute__((always_inline)) {
        constexpr int M = decltype(mc)::value, hh = M / 64, m = M % 64, j = slot_sub(m), k = slot_pos(m);
        const char* qt = qtile(hh);
        const char* gt = qt + kTileBytes;
        // rows 32j + sigma32(n) and the 16-row groups of the column reads are
        // the lane offsets of lo plus 8192j / 4096(2j + cc) (immediates)
        if constexpr (k < 8) {
          rq[hh][j][k] = *reinterpret_cast<const bf16x8*>(qt + 8192 * j + lo.k[k]);
        } else if constexpr (k < 16) {
          rg[hh][j][k - 8] = *reinterpret_cast<const bf16x8*>(gt + 8192 * j + lo.k[k - 8]);
        } else if constexpr (k < 24) {
          constexpr int cc = (k - 16) >> 2, db = (k - 16) & 3;
          cg[hh][j][cc][db] = lds_col8_at(gt + 4096 * (2 * j + cc), lo.v[db][0], lo.v[db][1]);
        } else {
          constexpr int cc = (k - 24) >> 2, db = (k - 24) & 3;
          cq[hh][j][cc][db] = lds_col8_at(qt + 4096 * (2 * j + cc), lo.v[db][0], lo.v[db][1]);
        }
      };
      // -lse*log2e (which 0) or -delta (which 1) of the lane's 16 queries of
      // sub-block j of head hh, in the accumulator layout: register 4i + e holds
      // query 16 (i / 2) + 4 (i % 2) + e of the lane's 8-row group
      auto read_stats = [&](auto hc, auto jc, auto wc) __attribute__((always_inline)) {
        constexpr int hh = decltype(hc)::value, j = decltype(jc)::value, which = decltype(wc)::value;
        const float* src = &stats[buf][hh][which][0] + 32 * j + 8 * h;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(src + 16 * (i >> 1) + 4 * (i & 1));
          if constexpr (which) dlv[hh][j][i] = v;
          else l2v[hh][j][i] = v;
        }
      };
      auto acc_of = [&](const f32x4 (&x)[4]) __attribute__((always_inline)) {
        f32x16 c;
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int e = 0; e < 4; e++) c[4 * i + e] = x[i][e];
        return c;
      };
      auto mfma_at = [&](auto mc) __attribute__((always_inline)) {
        constexpr int M = decltype(mc)::value, hh = M / 64, m = M % 64, j = slot_sub(m), k = slot_pos(m);
        if constexpr (k < 8) {
          if constexpr (!TPR_DKDV_VGPR_SP) sc[hh][j] = mfma(rq[hh][j][k], kv[k], k == 0 ? acc_of(l2v[hh][j]) : sc[hh][j]);
          else if constexpr (k == 0) sc[hh][j] = mfma_vsp_init(rq[hh][j][k], kv[k], acc_of(l2v[hh][j]));
          else mfma_vsp_acc(sc[hh][j], rq[hh][j][k], kv[k]);
        } else if constexpr (k < 16) {
          if constexpr (!TPR_DKDV_VGPR_SP)
            dpv[hh][j] = mfma(rg[hh][j][k - 8], vv[k - 8], k == 8 ? acc_of(dlv[hh][j]) : dpv[hh][j]);
          else if constexpr (k == 8) dpv[hh][j] = mfma_vsp_init(rg[hh][j][k - 8], vv[k - 8], acc_of(dlv[hh][j]));
          else mfma_vsp_acc(dpv[hh][j], rg[hh][j][k - 8], vv[k - 8]);
        } else if constexpr (k < 24) {
          constexpr int cc = (k - 16) >> 2, db = (k - 16) & 3;
          dv[db] = mfma(pb[hh][j][cc], cg[hh][j][cc][db], dv[db]);
        } else {
          constexpr int cc = (k - 24) >> 2, db = (k - 24) & 3;
          dk[db] = mfma(d8[hh][j][cc], cq[hh][j][cc][db], dk[db]);
        }
      };
      // register r of a sub-block holds query 16*(r/8) + r%8 of the lane's 8-row group
      auto p_elem = [&](auto hc, auto jc, auto rc) __attribute__((always_inline)) {
        constexpr int hh = decltype(hc)::value, j = decltype(jc)::value, r = decltype(rc)::value;
        constexpr int qi = 16 * (r >> 3) + (r & 7);
        float x = sc[hh][j][r];  // scale*log2e*S - lse*log2e
        if constexpr (decltype(diag)::value) x = qi >= lim - 32 * j ? x : -INFINITY;
        p[hh][j][r] = fast_exp2(x);
        if constexpr ((r & 7) == 7) {
#pragma unroll
          for (int i = 0; i < 8; i++) pb[hh][j][r >> 3][i] = static_cast<bf16>(p[hh][j][(r & 8) + i]);
        }
      };
      auto ds_elem = [&](auto hc, auto jc, auto rc) __attribute__((always_inline)) {
        constexpr int hh = decltype(hc)::value, j = decltype(jc)::value, r = decltype(rc)::value;
        dsv[hh][j][r] = p[hh][j][r] * dpv[hh][j][r];  // the dP chain started from -delta
        if constexpr ((r & 7) == 7) {
#pragma unroll
          for (int i = 0; i < 8; i++) d8[hh][j][r >> 3][i] = static_cast<bf16>(dsv[hh][j][(r & 8) + i]);
        }
      };
      using I0 = std::integral_constant<int, 0>;
      using I1 = std::integral_constant<int, 1>;
      // Reads are issued in pairs, the later slot's first: LDS reads complete in
      // order, so the wait before the earlier slot's MFMA covers both and the
      // later slot's MFMA needs none.
      static_for<kSlotAhead / 2>([&](auto pc) __attribute__((always_inline)) {
        constexpr int q = 2 * decltype(pc)::value;
        read_for(std::integral_constant<int, q + 1>{});
        read_for(std::integral_constant<int, q>{});
      });
      read_stats(I0{}, I0{}, I0{});
      read_stats(I0{}, I1{}, I0{});
      static_for<kSlots>([&](auto mc) __attribute__((always_inline)) {
        constexpr int M = decltype(mc)::value, hh = M / 64, m = M % 64, j = slot_sub(m), k = slot_pos(m);
        using H = std::integral_constant<int, hh>;
        using J = std::integral_constant<int, j>;
        if constexpr (m % 2 == 0 && M + kSlotAhead + 1 < kSlots) {
          read_for(std::integral_constant<int, M + kSlotAhead + 1>{});
          read_for(std::integral_constant<int, M + kSlotAhead>{});
        }
        if constexpr (m == 56 && hh + 1 < kHeads) {  // the next head's -lse rows, ahead of its S chains
          read_stats(std::integral_constant<int, hh + 1>{}, I0{}, I0{});
          read_stats(std::integral_constant<int, hh + 1>{}, I1{}, I0{});
        }
        if constexpr (k == 4) read_stats(H{}, J{}, I1{});  // -delta: the dP chain starts from it at k = 8
        mfma_at(mc);
        // dS of head hh, sub-block j, 16-query half cc: whole 1 KiB lines,
        // streaming (nt) buffer stores from the stage's uniform base (a
        // 32-bit lane offset, not a 64-bit address per lane)
        auto store_ds = [&](int cc) __attribute__((always_inline)) {
          __builtin_amdgcn_raw_buffer_store_b128(
              __builtin_bit_cast(i32x4, d8[hh][j][cc]),
              __builtin_amdgcn_make_buffer_rsrc(ds_stage, 0, kHeads * kDsHeadBytes, kBufferRsrcWord3),
              hh * kDsHeadBytes + (2 * j + cc) * 1024 + 16 * lane, 0, kCachePolicyNt);
        };
        if constexpr (kStoreDs && k == TPR_DS_STORE_K1) store_ds(0);
        if constexpr (kStoreDs && k == TPR_DS_STORE_K2) store_ds(1);
        static_for<16>([&](auto rc) __attribute__((always_inline)) {
          constexpr int r = decltype(rc)::value;
          if constexpr (k == 9 + (r * 10) / 16) p_elem(H{}, J{}, rc);   // P: slots 9..18 (pb[0] by 13, pb[1] by 18)
          if constexpr (k == 19 + (r * 9) / 16) ds_elem(H{}, J{}, rc);  // dS: slots 19..27 (d8[0] by 22, d8[1] by 27)
        });
        __builtin_amdgcn_sched_barrier(0);
      });
    };

    // Stages [sidx, end) of the stage loop, with (diag) or without the causal
    // mask in the body.
    // one stage; the buffer parity is a compile-time constant so that every
    // LDS address in the stage is a precomputed lane offset plus an immediate
    auto one_stage = [&](auto diag, auto bufc, int sidx) __attribute__((always_inline)) {
      constexpr int buf = decltype(bufc)::value;
      const int tok0 = __builtin_amdgcn_readfirstlane(qtab[cur.blk].y);
      if constexpr (kStoreDs) {
        // this stage's dS blocks: slot, heads kvh G + sub kHeads + hh, this wave's 32 keys
        const int slot = __builtin_amdgcn_readfirstlane(qtab[cur.blk].w);
        ds_stage = static_cast<char*>(a.ds) +
                   ((static_cast<int64_t>(kvh) * a.ds_slots + slot) * a.group + cur.sub * kHeads) * kDsHeadBytes +
                   wave * 4096;
      }
      const StageCursor nxt = advance(cur);
      if (sidx + 1 < nstage) issue(nxt, buf ^ 1);
      if (wave_active) {
        // key kp is visible from query index qi (of the stage) iff qi >= lim;
        // off this wave's diagonal lim <= -64 (all visible)
        const int lim = tok0 < kw0 + 31 ? kp - tok0 - 8 * h : -64;
        stage(diag, bufc, lim);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {  // accumulators stay in AGPRs across the stage loop
        settle_acc(dk[i]);
        settle_acc(dv[i]);
      }
#pragma unroll
      for (int c = 0; c < 8; c++) {  // so do the K/V operands (MFMAs read them there)
        settle_acc(kv[c]);
        settle_acc(vv[c]);
      }
      cur = nxt;
      wait_dma();  // stage sidx + 1 has landed
      __syncthreads();
    };
    auto run_stages = [&](auto diag, int sidx, int end) __attribute__((always_inline)) {
      constexpr std::integral_constant<int, 0> b0{};
      constexpr std::integral_constant<int, 1> b1{};
      if (sidx < end && (sidx & 1)) one_stage(diag, b1, sidx++);
      for (; sidx + 1 < end; sidx += 2) {
        one_stage(diag, b0, sidx);
        one_stage(diag, b1, sidx + 1);
      }
      if (sidx < end) one_stage(diag, b0, sidx);
    };
    // (suffix) the stages whose query block crosses some wave's causal diagonal
    // run with the mask -- the leading ones in first-last order, the trailing
    // ones in last-first order -- all others without it
    int ndiag = 0;
    if (!prefix) {
      int nb = 0;
      while (nb < nblk && qtab[first_last ? nb : nblk - 1 - nb].y < key0 + kDkdvKeys - 1) nb++;
      ndiag = nb * spb;
    }
    const int lead = first_last ? ndiag : 0, trail = first_last ? nstage : nstage - ndiag;
    run_stages(std::true_type{}, 0, lead);
    run_stages(std::false_type{}, lead, trail);
    run_stages(std::true_type{}, trail, nstage);

    if (wave_active) {
      // accumulator register r of lane l: key 8*(r/4) + 4*h + r%4 of the wave,
      // d = 32*db + n. The lane index is laundered so the store addresses are
      // formed here, not hoisted out of the tile loop (where they would stay
      // live across the stage loop).
      int el = lane;
      asm volatile("" : "+v"(el));
      const int n = el & 31, h = el >> 5;
      const int slot = item[DK_SLOT];  // -1 for a pair: its tiles are never split
      if (slot >= 0) {
        // split tile: fp32 partial [kDkdvKeys][128] for dK (already scaled) then dV
        float* pk = a.ws + static_cast<int64_t>(slot) * 2 * kDkdvKeys * kMfmaD;
        float* pv = pk + kDkdvKeys * kMfmaD;
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = 32 * wave + 8 * (r >> 2) + 4 * h + (r & 3);
#pragma unroll
          for (int db = 0; db < 4; db++) {
            pk[key * kMfmaD + 32 * db + n] = dk[db][r] * a.scale;
            pv[key * kMfmaD + 32 * db + n] = dv[db][r];
          }
        }
      } else if (prefix && a.acc_prefix) {
        // fp32 relay accumulators: add this (unsplit) tile's gradient, the scaled
        // product rounded as the ordinary path rounds it, then one add (no fma)
#pragma clang fp contract(off)
        float* dkf = static_cast<float*>(a.dpk);
        float* dvf = static_cast<float*>(a.dpv);
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = kw0 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (key >= seg_len) continue;
          const int64_t off = static_cast<int64_t>(seg_row0 + key) * kstride + kvh * kMfmaD + n;
#pragma unroll
          for (int db = 0; db < 4; db++) {
            dkf[off + 32 * db] += dk[db][r] * a.scale;
            dvf[off + 32 * db] += dv[db][r];
          }
        }
      } else {
        bf16* dkd = static_cast<bf16*>(prefix ? a.dpk : a.dk);
        bf16* dvd = static_cast<bf16*>(prefix ? a.dpv : a.dv);
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int key = kw0 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (key >= seg_len) continue;
          const int64_t off = static_cast<int64_t>(seg_row0 + key) * kstride + kvh * kMfmaD + n;
#pragma unroll
          for (int db = 0; db < 4; db++) {
            dkd[off + 32 * db] = static_cast<bf16>(dk[db][r] * a.scale);
            dvd[off + 32 * db] = static_cast<bf16>(dv[db][r]);
          }
        }
      }
    }
  }  // tiles
}

// ---------------------------------------------------------------------------
// Second pass of split dK/dV tiles: sum the fp32 partial slots of one
// (segment tile, KV head) in slot order -- slot order is query-block order,
// i.e. leaf order -- and write dK/dV. Deterministic: fixed summation order,
// one writer per element.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void mfma_reduce(KernelArgs a) {
  const int32_t* item = a.plan + a.off_red + RD_WORDS * blockIdx.x;
  const bool prefix = item[RD_SRC] == 0;
  const int seg = item[RD_SEG], key0 = item[RD_KEY0], kvh = item[RD_KVH];
  const int slot0 = item[RD_SLOT0], nslots = item[RD_NSLOTS];
  const int32_t* cu = a.plan + a.off_cu;
  const int32_t* no = a.plan + a.off_node_off;
  const int seg_row0 = prefix ? no[seg] : cu[seg];
  const int keys = min(kDkdvKeys, (prefix ? no[seg + 1] - no[seg] : cu[seg + 1] - cu[seg]) - key0);
  const int64_t kstride = static_cast<int64_t>(a.hkv) * kMfmaD;
  bf16* dkd = static_cast<bf16*>(prefix ? a.dpk : a.dk);
  bf16* dvd = static_cast<bf16*>(prefix ? a.dpv : a.dv);
  const int64_t slot_floats = 2 * kDkdvKeys * kMfmaD;
  // 4 consecutive d per thread: 32 threads per key row, 8 key rows per pass
  for (int e = threadIdx.x; e < 2 * keys * (kMfmaD / 4); e += blockDim.x) {
    const int which = e / (keys * (kMfmaD / 4));   // 0 = dK, 1 = dV
    const int rem = e % (keys * (kMfmaD / 4));
    const int key = rem / (kMfmaD / 4), d4 = rem % (kMfmaD / 4);
    const float* src = a.ws + static_cast<int64_t>(slot0) * slot_floats + which * kDkdvKeys * kMfmaD +
                       key * kMfmaD + 4 * d4;
    f32x4 acc = *reinterpret_cast<const f32x4*>(src);
    for (int j = 1; j < nslots; j++) acc += *reinterpret_cast<const f32x4*>(src + j * slot_floats);
    const int64_t at = static_cast<int64_t>(seg_row0 + key0 + key) * kstride + kvh * kMfmaD + 4 * d4;
    if (prefix && a.acc_prefix) {  // fp32 relay accumulators
      f32x4* dst = reinterpret_cast<f32x4*>(static_cast<float*>(which ? a.dpv : a.dpk) + at);
      *dst = *dst + acc;
      continue;
    }
    bf16x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = static_cast<bf16>(acc[i]);
    *reinterpret_cast<bf16x4*>((which ? dvd : dkd) + at) = o;
  }
}

// Whether any of q, k, v has rows wider than packed.
bool strided_rows(const KernelArgs& a) {
  return a.q_rs != static_cast<int64_t>(a.hq) * kMfmaD || a.k_rs != static_cast<int64_t>(a.hkv) * kMfmaD ||
         a.v_rs != static_cast<int64_t>(a.hkv) * kMfmaD;
}

template <bool kRunList>
void launch_fwd_tile(const KernelArgs& a, hipStream_t s) {
  if (strided_rows(a))
    hipLaunchKernelGGL((mfma_fwd<kRunList, true>), dim3(a.n_items), dim3(64 * kFwdWaves), 0, s, a);
  else
    hipLaunchKernelGGL((mfma_fwd<kRunList, false>), dim3(a.n_items), dim3(64 * kFwdWaves), 0, s, a);
}

template <int kHeads>
void launch_dkdv_heads(const KernelArgs& a, int n_dkdv, hipStream_t s) {
  const bool st = strided_rows(a), ds = a.ds != nullptr;
  if (st && ds)
    hipLaunchKernelGGL((mfma_dkdv<kHeads, true, true>), dim3(n_dkdv), dim3(256), 0, s, a);
  else if (st)
    hipLaunchKernelGGL((mfma_dkdv<kHeads, true, false>), dim3(n_dkdv), dim3(256), 0, s, a);
  else if (ds)
    hipLaunchKernelGGL((mfma_dkdv<kHeads, false, true>), dim3(n_dkdv), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((mfma_dkdv<kHeads, false, false>), dim3(n_dkdv), dim3(256), 0, s, a);
}

template <bool kRunList>
void launch_dq_tile(const KernelArgs& a, int n_fwd, hipStream_t s) {
  if (strided_rows(a))
    hipLaunchKernelGGL((mfma_dq<kRunList, true>), dim3(n_fwd), dim3(64 * kFwdWaves), 0, s, a);
  else
    hipLaunchKernelGGL((mfma_dq<kRunList, false>), dim3(n_fwd), dim3(64 * kFwdWaves), 0, s, a);
}

}  // namespace

int launch_mfma_fwd(const KernelArgs& a, hipStream_t s) {
  if (a.n_items > 0) {
    if (a.max_runs > kMfmaRegRuns)
      launch_fwd_tile<true>(a, s);
    else
      launch_fwd_tile<false>(a, s);
  }
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

int launch_mfma_delta(const KernelArgs& a, hipStream_t s) {
  const int blocks = (a.total_q + kDeltaTokens - 1) / kDeltaTokens;
  if (blocks > 0 && a.hq > 0) hipLaunchKernelGGL(mfma_delta, dim3(blocks, a.hq), dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

int launch_mfma_bwd(const KernelArgs& a, int n_fwd, int n_dkdv, int n_red, hipStream_t s) {
  if (n_dkdv > 0) {
    if (a.group % 2 == 0)
      launch_dkdv_heads<2>(a, n_dkdv, s);
    else
      launch_dkdv_heads<1>(a, n_dkdv, s);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  if (n_red > 0) {
    hipLaunchKernelGGL(mfma_reduce, dim3(n_red), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  if (n_fwd > 0) {
    if (a.ds && strided_rows(a))
      hipLaunchKernelGGL((mfma_dqs<true>), dim3(n_fwd), dim3(64 * kFwdWaves), 0, s, a);
    else if (a.ds)
      hipLaunchKernelGGL((mfma_dqs<false>), dim3(n_fwd), dim3(64 * kFwdWaves), 0, s, a);
    else if (a.max_runs > kMfmaRegRuns)
      launch_dq_tile<true>(a, n_fwd, s);
    else
      launch_dq_tile<false>(a, n_fwd, s);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  return 0;
}

}  // namespace tpr
