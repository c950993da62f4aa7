// tpr_mfma16.hip -- gfx950 bf16 MFMA prefix-reuse attention kernels for head_dim
// 64 and 256 (v_mfma_f32_16x16x32_bf16).
//
// Same math, key streams, work lists and fixed-order sibling sum as the
// head_dim-128 family (tpr_mfma.hip); the tiling is built on the 16-wide MFMA
// so that head_dim 256 fits the register file: a forward / dQ wave owns 32
// query tokens of one head as two 16-query sub-blocks, a dK/dV wave owns one
// 16-key block. One wave per SIMD, 4 waves per workgroup; K/V (forward, dQ) and Q/dO
// (dK/dV) tiles of 64 rows are staged in LDS by the gfx950 DMA, double
// buffered, one workgroup barrier per tile.
//
// MFMA layout (measured on gfx950): A lane l holds row l%16, k-slots
// 8*(l/16)+i; B lane l holds column l%16, the same k-slots; result register r
// of lane l holds (row 4*(l/16) + r, column l%16).
//
// Score tiles are computed with the 64 rows of a tile (keys in the forward
// and dQ, queries in dK/dV) permuted inside each 32-row half: accumulator block
// b (16 rows) row m = 4g + r holds tile row 32(b/2) + 8g + 4(b%2) + r. Lane l
// (g = l/16) then holds, over blocks 2t and 2t+1, the 8 consecutive tile rows
// 32t + 8g + 0..7 of its column -- exactly the k-slots the next MFMA (P.V,
// dS.K, P^T.dO, dS^T.Q) reads as an operand from registers.
//
// LDS tiles are row-major, 2*D bytes per row, with the 16-byte chunk index
// XOR-swizzled by bits of the row (Geo::swz) so that the row reads of 16
// permuted rows and the transposed reads (ds_read_tr16_b64) are free of bank
// conflicts.

#include "tpr_kernel_util.h"

namespace tpr {
namespace {

typedef __attribute__((address_space(3))) s16x4 lds_s16x4_m16;
typedef int i32x4_m16 __attribute__((ext_vector_type(4)));
// bytes per query head per dS slot: the 64-key dK/dV tile x 64 queries
constexpr int m16_ds_head_bytes(int d) { return m16_keys(d) * kDkdvQ * 2; }
// forward waves per workgroup. head_dim 256 runs 8 waves of 16 queries: about
// 200 registers, so two waves share a SIMD, and LDS returns operands to each
// wave at its own rate (one wave of 32 queries needed 342 registers and ran
// alone). head_dim 64 runs 4 waves of 32 queries (162 registers).
constexpr int m16_fwd_waves(int d) { return d == 256 ? 8 : kM16Waves; }

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int kD>
struct Geo {
  static_assert(kD == 64 || kD == 256, "the 16-wide family serves head_dim 64 and 256");
  static constexpr int RB = 2 * kD;              // bytes per tile row
  static constexpr int NC = kD / 8;              // 16-byte chunks per row
  static constexpr int TB = kTileRows * RB;      // bytes per 64-row tile
  static constexpr int NS = kD / 32;             // 32-wide k-steps over head_dim
  static constexpr int ND = kD / 16;             // 16-wide head_dim blocks
  static constexpr int RPB = 1024 / RB;          // tile rows per 1 KiB DMA block
  static constexpr int BPW = TB / 1024 / kM16Waves;  // DMA blocks per wave per tile
  // Physical 16-byte chunk = logical chunk ^ swz(row), chosen so that no tile
  // read has a bank conflict (bank = byte address / 4 mod 64). One pass of a
  // 16-byte row read (row_operand) serves lanes 0-7 and 32-39 (and the like):
  // 8 permuted rows, varying in row bits 0, 1 and 3, at logical chunks c and
  // c + 2. One pass of a transposed read (col_operand) serves 32 lanes: 8 rows
  // varying in the same bits, at chunks c and c + 1 (c even). Both passes
  // cover all 64 banks when the XOR is a bijection of row bits (0, 1, 3) onto
  // the bank-group bits other than chunk bit 1, and onto those other than
  // chunk bit 0. At 512-byte rows (head_dim 256, bank group = chunk mod 16)
  // swz = 3 r0 + 4 r1 + 8 r3; at 128-byte rows (head_dim 64) row bit 0 already
  // picks the bank half, and swz = 3 r3 + 4 r1.
  __device__ static __forceinline__ int swz(int row) {
    if constexpr (kD == 256) return ((row & 1) * 3) | ((row & 2) << 1) | (row & 8);
    else return (((row >> 3) & 1) * 3) | ((row & 2) << 1);
  }
  // byte offset of element (row, col) of a swizzled tile
  __device__ static __forceinline__ uint32_t off(int row, int col) {
    return static_cast<uint32_t>(row * RB + (((col >> 3) ^ swz(row)) << 4) + ((col & 7) << 1));
  }
};

// tile row of accumulator block b, row m (see the file comment)
__device__ __forceinline__ int perm_row(int b, int m) { return 32 * (b >> 1) + 8 * (m >> 2) + 4 * (b & 1) + (m & 3); }

// Row read: the A operand rows 16..31 of a 32-wide k-step s of block b: lane
// l reads tile row perm_row(b, l % 16), columns 32 s + 8 (l / 16) .. +7.
template <int kD>
__device__ __forceinline__ bf16x8 row_operand(const char* tile, int b, int s, int lane) {
  const int row = perm_row(b, lane & 15);
  return *reinterpret_cast<const bf16x8*>(tile + Geo<kD>::off(row, 32 * s + 8 * (lane >> 4)));
}

// Transposed read: the operand whose lane l holds column c0 + l % 16 and the 8
// consecutive tile rows r0 + 8 (l / 16) .. +7 (two ds_read_tr16_b64: lane i of
// each 16-lane group addresses row r0 + 8 g + i / 4 (+ 4), columns
// c0 + 4 (i % 4) .. +3, and receives column c0 + i of the group's 4 rows).
template <int kD>
__device__ __forceinline__ bf16x8 col_operand(const char* tile, int r0, int c0, int lane) {
  const int i = lane & 15, g = lane >> 4;
  const int row = r0 + 8 * g + (i >> 2), col = c0 + 4 * (i & 3);
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_m16*)(tile + Geo<kD>::off(row, col)));
  const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_m16*)(tile + Geo<kD>::off(row + 4, col)));
  const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo), h4 = __builtin_bit_cast(bf16x4, hi);
  bf16x8 r;
  r[0] = l4[0]; r[1] = l4[1]; r[2] = l4[2]; r[3] = l4[3];
  r[4] = h4[0]; r[5] = h4[1]; r[6] = h4[2]; r[7] = h4[3];
  return r;
}

// Copy rows [0, 64) of the tile whose row 0 is at `src` (uniform; rows at or
// beyond `len` re-read row len - 1; row stride `stride` bytes) into the
// swizzled LDS tile at `lds_tile`: this wave's BPW 1 KiB blocks. Lane l of
// block b lands at physical chunk l % NC of tile row b*RPB + l/NC, so it
// fetches the logical chunk that swizzles there.
template <int kD, int kWaves = kM16Waves>
__device__ __forceinline__ void copy_tile(const char* src, uint32_t stride, int len, uint32_t lds_tile, int wave,
                                          int lane) {
  using T = Geo<kD>;
  constexpr int kBPW = T::TB / 1024 / kWaves;  // DMA blocks per wave
#pragma unroll
  for (int j = 0; j < kBPW; j++) {
    const int b = wave * kBPW + j;
    const int row = b * T::RPB + lane / T::NC;
    const int chunk = (lane % T::NC) ^ T::swz(row);
    const uint32_t voff = static_cast<uint32_t>(min(row, len - 1)) * stride + 16u * chunk;
    dma16s(src, voff, lds_tile + b * 1024);
  }
}

// bf16x8 operand from two accumulator blocks: [x[0..3], y[0..3]]
__device__ __forceinline__ bf16x8 pack8(const float (&x)[4], const float (&y)[4]) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    r[i] = static_cast<bf16>(x[i]);
    r[4 + i] = static_cast<bf16>(y[i]);
  }
  return r;
}

__device__ __forceinline__ float xmax16(float x) {  // max over lanes l, l^16, l^32, l^48
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float xsum16(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

constexpr float kSlack16 = 8.f;  // lazy-rescale slack in log2 units (as the head_dim-128 forward)

// ---------------------------------------------------------------------------
// Forward. Wave w: query head qh0 + w % hpw, tokens tw0 .. tw0 + 16 kQS - 1
// as kQS 16-query sub-blocks qs (two at head_dim 64, one at 256). Per 64-key
// tile: S^T (4 blocks of 16 keys x 16 queries per sub-block) = K Q^T with K
// rows from LDS (A) and Q in registers
// (B); online softmax in registers (lane l holds 16 keys of query l % 16; the
// other 48 keys of the tile sit in lanes l ^ 16, l ^ 32, l ^ 48); then
// O^T += V^T P^T with V^T read transposed from LDS (A) and P^T from registers.
// kRunList: key runs read from the plan; kStrided: q, k or v rows wider than
// packed (the packed instance folds every row stride to a constant).
// ---------------------------------------------------------------------------
template <int kD, bool kRunList, bool kStrided>
__global__ __launch_bounds__(64 * m16_fwd_waves(kD)) void m16_fwd(KernelArgs a) {
  using T = Geo<kD>;
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh0 = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // kFW waves of kQS 16-query sub-blocks each (the planner's work item is
  // kM16Waves x kM16Tokens query rows either way)
  constexpr int kFW = m16_fwd_waves(kD), kQS = kFW * 16 == kM16Waves * kM16Tokens ? 1 : 2, kTokW = 16 * kQS;
  static_assert(kFW * kTokW == kM16Waves * kM16Tokens, "a workgroup covers the planner's work item");
  const int hpw = a.hpw;
  const int head = qh0 + wave % hpw;
  const int tw0 = tok0 + kTokW * (wave / hpw);
  const int tpw = kTokW * (kFW / hpw);
  const int suffix_keys = min(len, tok0 + tpw);
  const int i16 = lane & 15, g = lane >> 4;

  const int64_t qstride = static_cast<int64_t>(a.hq) * kD;
  const uint32_t row_bytes = static_cast<uint32_t>(a.hkv) * kD * 2;
  __shared__ __attribute__((aligned(1024))) char smem[4 * T::TB];  // K0 K1 V0 V1
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  const char* kbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.k) + kvh * kD);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.v) + kvh * kD);
  const char* pkbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pk) + kvh * kD);
  const char* pvbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pv) + kvh * kD);
  // row bytes of a tile's source: prefix K/V packed, suffix K/V as the caller's views
  const uint32_t k_rb = kStrided ? static_cast<uint32_t>(a.k_rs) * 2 : row_bytes;
  const uint32_t v_rb = kStrided ? static_cast<uint32_t>(a.v_rs) * 2 : row_bytes;
  const int64_t q_rs = kStrided ? a.q_rs : qstride;
  auto kv_rb = [&](const TileLoc& x, bool is_k) { return x.suffix ? (is_k ? k_rb : v_rb) : row_bytes; };
  auto kv_src = [&](const TileLoc& x, bool is_k) {
    const char* b = x.suffix ? (is_k ? kbase : vbase) : (is_k ? pkbase : pvbase);
    return b + x.row * static_cast<int64_t>(kv_rb(x, is_k));
  };

  const auto seg = load_keys<kRunList>(a, leaf, suffix_keys);
  const int ntiles = seg.ntiles;
  Cursor cc = cursor_begin(seg);  // the tile being copied
  TileLoc tl_c = cursor_tile(cc);
  Cursor mc = cursor_begin(seg);  // the tile being computed
  TileLoc tl = cursor_tile(mc);
  copy_tile<kD, kFW>(kv_src(tl_c, true), kv_rb(tl_c, true), tl_c.len, lds0, wave, lane);
  copy_tile<kD, kFW>(kv_src(tl_c, false), kv_rb(tl_c, false), tl_c.len, lds0 + 2 * T::TB, wave, lane);

  // Q of the lane's query l % 16 of each sub-block: the B operand of S^T
  bf16x8 qv[kQS][T::NS];
#pragma unroll
  for (int qs = 0; qs < kQS; qs++) {
    const int t = min(tw0 + 16 * qs + i16, len - 1);
    const bf16* qp = static_cast<const bf16*>(a.q) + static_cast<int64_t>(row0 + t) * q_rs + head * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < T::NS; s++) qv[qs][s] = *reinterpret_cast<const bf16x8*>(qp + 32 * s);
  }
  f32x4 o[kQS][T::ND];
#pragma unroll
  for (int qs = 0; qs < kQS; qs++)
#pragma unroll
    for (int db = 0; db < T::ND; db++) o[qs][db] = f32x4{};
  float m[kQS], l[kQS];  // running max (raw score units), lane-partial sum
#pragma unroll
  for (int qs = 0; qs < kQS; qs++) {
    m[qs] = -1e30f;
    l[qs] = 0.f;
  }
  const float c2 = a.scale * kLog2e;
  const float slack = kSlack16 / c2;

#pragma unroll
  for (int qs = 0; qs < kQS; qs++)
#pragma unroll
    for (int s = 0; s < T::NS; s++) settle(qv[qs][s]);
  wait_dma();
  __syncthreads();

  // With two waves per SIMD (8 waves: w and w + 4 share one), the upper four
  // issue their share of the next tile's copies after the S slots instead of
  // before them, so that each wave's copy issue runs beside its SIMD
  // partner's MFMAs.
  const bool copy_late = kFW == 8 && wave >= 4;
  for (int j = 0; j < ntiles; j++) {
    const int buf = j & 1;
    if (j + 1 < ntiles) {
      cursor_next(seg, cc);
      tl_c = cursor_tile(cc);
    }
    // copy tile j+1 into the other buffer (read by tile j-1, released by the last barrier)
    auto issue_next = [&]() __attribute__((always_inline)) {
      if (j + 1 < ntiles) {
        copy_tile<kD, kFW>(kv_src(tl_c, true), kv_rb(tl_c, true), tl_c.len, lds0 + (1 - buf) * T::TB, wave, lane);
        copy_tile<kD, kFW>(kv_src(tl_c, false), kv_rb(tl_c, false), tl_c.len, lds0 + (3 - buf) * T::TB, wave, lane);
      }
    };
    if (!copy_late) issue_next();
    const char* kt = smem + buf * T::TB;
    const char* vt = smem + (2 + buf) * T::TB;

    // mask (register r of key block b holds key 32 (b/2) + 8 g + 4 (b%2) + r of
    // the tile), online softmax against the running max, P packed for P V
    auto softmax = [&](f32x4 (&sv)[kQS][4], bf16x8 (&pb)[kQS][2]) __attribute__((always_inline)) {
      const bool partial = tl.len < kTileRows || (tl.suffix && tl.pos0 + kTileRows - 1 > tw0);
      if (partial) {
#pragma unroll
        for (int qs = 0; qs < kQS; qs++) {
          const int t = tw0 + 16 * qs + i16;
          int lim = tl.len - 1;
          if (tl.suffix) lim = min(lim, t - tl.pos0);
#pragma unroll
          for (int b = 0; b < 4; b++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
              const int key = 32 * (b >> 1) + 8 * g + 4 * (b & 1) + r;
              sv[qs][b][r] = key <= lim ? sv[qs][b][r] : -INFINITY;
            }
        }
      }
#pragma unroll
      for (int qs = 0; qs < kQS; qs++) {
        float mt = sv[qs][0][0];
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
          for (int r = 0; r < 4; r++) mt = fmaxf(mt, sv[qs][b][r]);
        // The four lanes of a query share its reference max: one of them
        // outgrew it iff the query did, so at head_dim 64 the exchange waits
        // for the rescale (forward 1.25 -> 1.16 ms at prefix 4096 + 4 x 4096,
        // GQA 32/8). At head_dim 256 that form measured slower (1.30 -> 1.33
        // ms, GQA 8/2), and the exchange stays in front of the test.
        if constexpr (kD == 256) mt = xmax16(mt);
        if (__any(mt > m[qs] + slack)) {  // some query outgrew its reference max: rescale
          if constexpr (kD != 256) mt = xmax16(mt);
          const float m_new = fmaxf(m[qs], mt);
          const float alpha = fast_exp2((m[qs] - m_new) * c2);
          m[qs] = m_new;
          l[qs] *= alpha;
#pragma unroll
          for (int db = 0; db < T::ND; db++) o[qs][db] *= alpha;
        }
        const float mc2 = m[qs] * c2;
        float pf[4][4];
        float ls = 0.f;
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            pf[b][r] = fast_exp2(fmaf(sv[qs][b][r], c2, -mc2));
            ls += pf[b][r];
          }
        l[qs] += ls;
        pb[qs][0] = pack8(pf[0], pf[1]);
        pb[qs][1] = pack8(pf[2], pf[3]);
      }
    };
    // The tile is one fixed sequence of fenced slots: the S slots (k-step s,
    // key block b), then the P V slots (head-dim block db, key step t). Each
    // slot reads one operand from LDS (a K row block, or V read transposed)
    // for two MFMAs (the wave's two query sub-blocks), and each read is
    // issued kRead slots ahead of its use, so the MFMAs do not wait on LDS
    // latency. The softmax runs after the last S slot, while the first P V
    // operands are already in flight.
    constexpr int kS = 4 * T::NS;             // S slots
    constexpr int kSlots = kS + 2 * T::ND;    // + P V slots
    constexpr int kRead = 4, kRing = kRead + 1;
    bf16x8 ring[kRing];                       // slot i's operand sits at i % kRing
    auto read_slot = [&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i < kS) {
        ring[i % kRing] = row_operand<kD>(kt, i % 4, i / 4, lane);
      } else {
        constexpr int k = i - kS;
        ring[i % kRing] = col_operand<kD>(vt, 32 * (k % 2), 16 * (k / 2), lane);
      }
    };
    static_for<kRead>([&](auto ic) { read_slot(ic); });
    f32x4 sa[kQS][4];
#pragma unroll
    for (int qs = 0; qs < kQS; qs++)
#pragma unroll
      for (int b = 0; b < 4; b++) sa[qs][b] = f32x4{};
    bf16x8 pb[kQS][2];
    static_for<kSlots>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i + kRead < kSlots) read_slot(std::integral_constant<int, i + kRead>{});
      if constexpr (i == kS) {
        if (copy_late) issue_next();
      }
      if constexpr (i < kS) {
        constexpr int b = i % 4, s = i / 4;
#pragma unroll
        for (int qs = 0; qs < kQS; qs++) sa[qs][b] = mfma16(ring[i % kRing], qv[qs][s], sa[qs][b]);
        if constexpr (i == kS - 1) softmax(sa, pb);
      } else {
        constexpr int k = i - kS, db = k / 2, t = k % 2;
#pragma unroll
        for (int qs = 0; qs < kQS; qs++) o[qs][db] = mfma16(ring[i % kRing], pb[qs][t], o[qs][db]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    if (j + 1 < ntiles) {
      cursor_next(seg, mc);
      tl = cursor_tile(mc);
    }
    wait_dma();
    __syncthreads();
  }

  // O^T register r of block db: head dim 16 db + 4 g + r of query l % 16
#pragma unroll
  for (int qs = 0; qs < kQS; qs++) {
    const float lt = xsum16(l[qs]);
    const int t = tw0 + 16 * qs + i16;
    if (tw0 + 16 * qs >= len || t >= len) continue;
    const float inv = 1.f / lt;
    bf16* op = static_cast<bf16*>(a.out) + static_cast<int64_t>(row0 + t) * qstride + head * kD + 4 * g;
#pragma unroll
    for (int db = 0; db < T::ND; db++) {
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; r++) v4[r] = static_cast<bf16>(o[qs][db][r] * inv);
      *reinterpret_cast<bf16x4*>(op + 16 * db) = v4;
    }
    if (g == 0) a.lse[static_cast<int64_t>(head) * a.total_q + row0 + t] = m[qs] * a.scale + logf(lt);
  }
}

// ---------------------------------------------------------------------------
// delta = rowsum(dO * O) per (token, head); also the stat rows the dK/dV kernel
// copies: -lse*log2e, -delta, and the constants (-inf, 0) of rows past a
// query block's end. 16 lanes per row.
// ---------------------------------------------------------------------------
template <int kD>
__global__ __launch_bounds__(256) void m16_delta(KernelArgs a) {
  const int64_t rows = static_cast<int64_t>(a.total_q) * a.hq;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  float s = 0.f;
  if (row < rows) {
#pragma unroll
    for (int k = 0; k < kD / 128 + (kD < 128 ? 1 : 0); k++) {
      const int col = kD >= 128 ? 128 * k + 8 * c : 4 * c;
      if (kD >= 128) {
        const bf16x8 o = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(a.out_in) + row * kD + col);
        const bf16x8 d = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(a.dout) + row * kD + col);
#pragma unroll
        for (int i = 0; i < 8; i++) s = fmaf(static_cast<float>(o[i]), static_cast<float>(d[i]), s);
      } else {
        const bf16x4 o = *reinterpret_cast<const bf16x4*>(static_cast<const bf16*>(a.out_in) + row * kD + col);
        const bf16x4 d = *reinterpret_cast<const bf16x4*>(static_cast<const bf16*>(a.dout) + row * kD + col);
#pragma unroll
        for (int i = 0; i < 4; i++) s = fmaf(static_cast<float>(o[i]), static_cast<float>(d[i]), s);
      }
    }
  }
  s += __shfl_xor(s, 8);
  s += __shfl_xor(s, 4);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 1);
  if (c == 0 && row < rows) {
    const int64_t at = (row % a.hq) * a.total_q + row / a.hq;
    a.delta[at] = s;
    a.stat_ws[kStatRowsOffset + at] = -(a.lse_in[at] * kLog2e);
    a.ndelta_ws[at] = -s;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    a.stat_ws[0] = -INFINITY;
    a.stat_ws[1] = 0.f;
  }
}

// ---------------------------------------------------------------------------
// dQ. Same workgroup shape and key stream as the forward. Per 64-key tile:
// S^T = K Q^T and dP^T = V dO^T (K, V rows from LDS; Q, dO in registers),
// P = exp2(scale*log2e S - lse*log2e), dS = P (dP - delta), then
// dQ^T += K^T dS^T with K^T read transposed from the K tile.
// ---------------------------------------------------------------------------
template <int kD, bool kRunList, bool kStrided>
__global__ __launch_bounds__(256) void m16_dq(KernelArgs a) {
  using T = Geo<kD>;
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh0 = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];

  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hpw = a.hpw;
  const int head = qh0 + wave % hpw;
  const int tw0 = tok0 + kM16Tokens * (wave / hpw);
  const int tpw = kM16Tokens * (kM16Waves / hpw);
  const int suffix_keys = min(len, tok0 + tpw);
  const int i16 = lane & 15, g = lane >> 4;

  const int64_t qstride = static_cast<int64_t>(a.hq) * kD;
  const uint32_t row_bytes = static_cast<uint32_t>(a.hkv) * kD * 2;
  __shared__ __attribute__((aligned(1024))) char smem[4 * T::TB];  // K0 K1 V0 V1
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  const char* kbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.k) + kvh * kD);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.v) + kvh * kD);
  const char* pkbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pk) + kvh * kD);
  const char* pvbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pv) + kvh * kD);
  // row bytes of a tile's source: prefix K/V packed, suffix K/V as the caller's views
  const uint32_t k_rb = kStrided ? static_cast<uint32_t>(a.k_rs) * 2 : row_bytes;
  const uint32_t v_rb = kStrided ? static_cast<uint32_t>(a.v_rs) * 2 : row_bytes;
  const int64_t q_rs = kStrided ? a.q_rs : qstride;
  auto kv_rb = [&](const TileLoc& x, bool is_k) { return x.suffix ? (is_k ? k_rb : v_rb) : row_bytes; };
  auto kv_src = [&](const TileLoc& x, bool is_k) {
    const char* b = x.suffix ? (is_k ? kbase : vbase) : (is_k ? pkbase : pvbase);
    return b + x.row * static_cast<int64_t>(kv_rb(x, is_k));
  };

  const auto seg = load_keys<kRunList>(a, leaf, suffix_keys);
  const int ntiles = seg.ntiles;
  Cursor cc = cursor_begin(seg);
  TileLoc tl_c = cursor_tile(cc);
  Cursor mc = cursor_begin(seg);
  TileLoc tl = cursor_tile(mc);
  copy_tile<kD>(kv_src(tl_c, true), kv_rb(tl_c, true), tl_c.len, lds0, wave, lane);
  copy_tile<kD>(kv_src(tl_c, false), kv_rb(tl_c, false), tl_c.len, lds0 + 2 * T::TB, wave, lane);

  bf16x8 qv[2][T::NS], gv[2][T::NS];
  float lse2[2], delta[2];
#pragma unroll
  for (int qs = 0; qs < 2; qs++) {
    const int t = min(tw0 + 16 * qs + i16, len - 1);
    const int64_t off = static_cast<int64_t>(row0 + t) * qstride + head * kD + 8 * g;
    const int64_t qoff = static_cast<int64_t>(row0 + t) * q_rs + head * kD + 8 * g;
#pragma unroll
    for (int s = 0; s < T::NS; s++) {
      qv[qs][s] = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(a.q) + qoff + 32 * s);
      gv[qs][s] = *reinterpret_cast<const bf16x8*>(static_cast<const bf16*>(a.dout) + off + 32 * s);
    }
    const int64_t at = static_cast<int64_t>(head) * a.total_q + row0 + t;
    lse2[qs] = a.lse_in[at] * kLog2e;
    delta[qs] = a.delta[at];
  }
  f32x4 dq[2][T::ND];
#pragma unroll
  for (int qs = 0; qs < 2; qs++)
#pragma unroll
    for (int db = 0; db < T::ND; db++) dq[qs][db] = f32x4{};
  const float c2 = a.scale * kLog2e;

#pragma unroll
  for (int qs = 0; qs < 2; qs++) {
#pragma unroll
    for (int s = 0; s < T::NS; s++) {
      settle(qv[qs][s]);
      settle(gv[qs][s]);
    }
    settle(lse2[qs]);
    settle(delta[qs]);
  }
  wait_dma();
  __syncthreads();

  for (int j = 0; j < ntiles; j++) {
    const int buf = j & 1;
    if (j + 1 < ntiles) {
      cursor_next(seg, cc);
      tl_c = cursor_tile(cc);
      copy_tile<kD>(kv_src(tl_c, true), kv_rb(tl_c, true), tl_c.len, lds0 + (1 - buf) * T::TB, wave, lane);
      copy_tile<kD>(kv_src(tl_c, false), kv_rb(tl_c, false), tl_c.len, lds0 + (3 - buf) * T::TB, wave, lane);
    }
    const char* kt = smem + buf * T::TB;
    const char* vt = smem + (2 + buf) * T::TB;

    // One fixed sequence of fenced slots, as in the forward: the S / dP slots
    // (k-step s, key block b: a K and a V row block, four MFMAs), dS after the
    // last of them, then the dQ slots (head-dim block db, key step t: K read
    // transposed, two MFMAs). Operand reads run kRead slots ahead of use.
    constexpr int kS = 4 * T::NS;
    constexpr int kSlots = kS + 2 * T::ND;
    constexpr int kRead = 4, kRing = kRead + 1;
    bf16x8 ra[kRing], rb[kRing];
    auto read_slot = [&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i < kS) {
        ra[i % kRing] = row_operand<kD>(kt, i % 4, i / 4, lane);
        rb[i % kRing] = row_operand<kD>(vt, i % 4, i / 4, lane);
      } else {
        constexpr int k = i - kS;
        ra[i % kRing] = col_operand<kD>(kt, 32 * (k % 2), 16 * (k / 2), lane);
      }
    };
    static_for<kRead>([&](auto ic) { read_slot(ic); });
    f32x4 sa[2][4], pa[2][4];
#pragma unroll
    for (int qs = 0; qs < 2; qs++)
#pragma unroll
      for (int b = 0; b < 4; b++) {
        sa[qs][b] = f32x4{};
        pa[qs][b] = f32x4{};
      }
    bf16x8 dsb[2][2];
    // dS = P (dP - delta), P = exp2(S scale log2e - lse log2e), masked
    auto grad_scores = [&]() __attribute__((always_inline)) {
      const bool partial = tl.len < kTileRows || (tl.suffix && tl.pos0 + kTileRows - 1 > tw0);
#pragma unroll
      for (int qs = 0; qs < 2; qs++) {
        const int t = tw0 + 16 * qs + i16;
        int lim = tl.len - 1;
        if (tl.suffix) lim = min(lim, t - tl.pos0);
        float df[4][4];
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int key = 32 * (b >> 1) + 8 * g + 4 * (b & 1) + r;
            float x = fmaf(sa[qs][b][r], c2, -lse2[qs]);
            if (partial) x = key <= lim ? x : -INFINITY;
            df[b][r] = fast_exp2(x) * (pa[qs][b][r] - delta[qs]);
          }
        dsb[qs][0] = pack8(df[0], df[1]);
        dsb[qs][1] = pack8(df[2], df[3]);
      }
    };
    static_for<kSlots>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i + kRead < kSlots) read_slot(std::integral_constant<int, i + kRead>{});
      if constexpr (i < kS) {
        constexpr int b = i % 4, s = i / 4;
#pragma unroll
        for (int qs = 0; qs < 2; qs++) {
          sa[qs][b] = mfma16(ra[i % kRing], qv[qs][s], sa[qs][b]);
          pa[qs][b] = mfma16(rb[i % kRing], gv[qs][s], pa[qs][b]);
        }
        if constexpr (i == kS - 1) grad_scores();
      } else {
        constexpr int k = i - kS, db = k / 2, t = k % 2;
        // dQ^T += K^T dS^T: A = K^T (16 head dims x 32 keys of step t), B = dS^T
#pragma unroll
        for (int qs = 0; qs < 2; qs++) dq[qs][db] = mfma16(ra[i % kRing], dsb[qs][t], dq[qs][db]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    if (j + 1 < ntiles) {
      cursor_next(seg, mc);
      tl = cursor_tile(mc);
    }
    wait_dma();
    __syncthreads();
  }

#pragma unroll
  for (int qs = 0; qs < 2; qs++) {
    const int t = tw0 + 16 * qs + i16;
    if (tw0 + 16 * qs >= len || t >= len) continue;
    bf16* dp = static_cast<bf16*>(a.dq) + static_cast<int64_t>(row0 + t) * qstride + head * kD + 4 * g;
#pragma unroll
    for (int db = 0; db < T::ND; db++) {
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; r++) v4[r] = static_cast<bf16>(dq[qs][db][r] * a.scale);
      *reinterpret_cast<bf16x4*>(dp + 16 * db) = v4;
    }
  }
}

// ---------------------------------------------------------------------------
// dQ from the dS store (head_dim 256): dQ^T += K^T dS^T over the dS blocks
// the dK/dV kernel stored, instead of recomputing S and dP. A workgroup is
// kM16DqsWaves = 8 waves of 32 tokens of one query head each (the plan's own
// dQ items, PF_OFF_DQS: twice the forward's tokens), two waves per SIMD, so
// that every K tile copied to LDS serves twice the queries of a 4-wave
// workgroup and one wave's copies issue while its partner computes. The key
// stream follows the dK/dV tiling: the leaf's ancestor nodes root first, then
// its suffix, in 64-key tiles, one dS slot each. A slot holds a head's 64 x 64
// block as four 2 KiB wave blocks (16 keys each) of [32-query half][lane L] x
// 8 queries, lane L holding key L % 16 and queries 32 t + 8 (L / 16) .. +7.
// Per tile every wave copies its share of the K rows (4 of the tile's 32
// blocks; read transposed as the A operand) and its own 4 KiB of dS (the four
// wave blocks' halves of its 32 queries), then runs 64 MFMAs. The copy puts
// chunk L of each 1 KiB block at L ^ (4 ((L >> 4) & 1)), which spreads every
// 32-lane pass of the transposed dS reads over all 64 banks. The dS blocks
// (the HBM stream) are copied two tiles ahead of the one being computed into
// three buffers, the K rows (mostly L2 hits) one tile ahead into two: 160 KiB.
// ---------------------------------------------------------------------------
template <int kD, bool kStrided>
__global__ __launch_bounds__(64 * kM16DqsWaves) void m16_dqs(KernelArgs a) {
  using T = Geo<kD>;
  static_assert(kD == 256, "the dS store serves head_dim 256 on this family");
  constexpr int kW = kM16DqsWaves;
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
  const int tw0 = tok0 + kM16Tokens * (wave / hpw);
  const int tpw = kM16Tokens * (kW / hpw);
  const int suffix_keys = min(len, tok0 + tpw);
  const int i16 = lane & 15, g = lane >> 4;
  const bool wave_ok = tw0 < len;
  const int qb = a.plan[a.off_leaf_qblk + leaf] + tw0 / kDkdvQ;  // the wave's query block
  const int jq = (tw0 / kM16Tokens) & 1;                          // and its 32-query half of it

  const int64_t qstride = static_cast<int64_t>(a.hq) * kD;
  const uint32_t p_rb = static_cast<uint32_t>(a.hkv) * kD * 2;
  const uint32_t k_rb = kStrided ? static_cast<uint32_t>(a.k_rs) * 2 : p_rb;
  constexpr int kKeys = m16_keys(kD);                 // keys per tile (= per dS slot)
  constexpr int kSlotHead = m16_ds_head_bytes(kD);    // 8 KiB per head per slot
  constexpr int kKBufs = 2, kDsBufs = 3, kDsWave = 4096;
  constexpr int kDsOff = kKBufs * T::TB;              // K [buffer] | dS [buffer][wave]
  __shared__ __attribute__((aligned(1024))) char smem[kKBufs * T::TB + kDsBufs * kW * kDsWave];
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
  const char* kbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.k) + kvh * kD);
  const char* pkbase = reinterpret_cast<const char*>(static_cast<const bf16*>(a.pk) + kvh * kD);

  // dS copy: block w (wave block w of the slot, this wave's query half) lands
  // at 1024 w; lane l fetches the chunk that lands at l (the swizzle is its own inverse)
  uint32_t dsl[4];
#pragma unroll
  for (int j = 0; j < 4; j++) dsl[j] = m16_dqs_ds_lane_bytes(lane, j);
  // dS^T operand reads (B: lane l gets query 16 qs + l % 16, keys 32 t + 8 (l / 16) + 0..7).
  // As a source row of ds_read_tr16_b64, lane l (group g, e = (l % 16) / 4,
  // m = l % 4) addresses key 8 g + 4 h + e of the 32-key step (wave block
  // 2 t + g / 2, its key 8 (g % 2) + 4 h + e), queries 16 qs + 4 m .. +3;
  // h = 0 / 1 gives keys +0..3 / +4..7, qs adds 512 bytes, t 2048.
  uint32_t dso[2];
  {
    const int e = (lane & 15) >> 2, m = lane & 3;
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const int L = 8 * (g & 1) + 4 * hh + e + 16 * (m >> 1);
      dso[hh] = 1024u * (g >> 1) + 16u * (L ^ (4 * ((L >> 4) & 1))) + 8u * (m & 1);
    }
  }

  // key stream cursor (uniform; plan words through the scalar cache), with
  // the tile's position in the stream: the dS slots of the wave's query block
  // are numbered in this order from the block's first slot (slot = first +
  // cpos), so at [KV head][slot][query head of the group] the wave's blocks
  // follow each other tile by tile
  const int depth = a.max_depth;
  const int32_t* anc = a.plan + a.off_anc + static_cast<int64_t>(leaf) * depth;
  int cd = -1, crow = 0, clen = 0, clim = 0, ckey = 0, cpos = 0;
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
  };
  auto advance = [&]() {
    ckey += kKeys;
    cpos++;
    if (ckey >= clim) next_segment();
  };
  const char* ds_wave = nullptr;  // this wave's dS blocks: first slot of its query block, its head and half
  if (wave_ok) {
    const int first = plan_word(a.plan + a.off_ds_first + qb);
    ds_wave = static_cast<const char*>(a.ds) +
              ((static_cast<int64_t>(kvh) * a.ds_slots + first) * a.group + (head - kvh * a.group)) * kSlotHead +
              jq * 1024;
  }
  const int64_t ds_tile_bytes = static_cast<int64_t>(a.group) * kSlotHead;  // one slot of the group

  // A tile of the stream (uniform): its K rows, their count, whether this
  // wave reads it (prefix tiles: every wave; suffix tiles: those not entirely
  // in the wave's future) and its dS position. `more` is false past the end.
  struct Tile {
    const char* k;
    uint32_t rb;
    int rows, pos;
    bool vis, more;
  };
  auto tile_here = [&]() __attribute__((always_inline)) {
    const bool suffix = cd == depth;
    Tile t;
    t.more = clim > 0;
    t.rb = suffix ? k_rb : p_rb;
    t.k = (suffix ? kbase : pkbase) + static_cast<int64_t>(crow + ckey) * t.rb;
    t.rows = min(kKeys, clen - ckey);
    t.pos = cpos;
    t.vis = t.more && wave_ok && (!suffix || ckey <= tw0 + kM16Tokens - 1);
    return t;
  };
  auto issue_k = [&](const Tile& t, int kb) __attribute__((always_inline)) {
    copy_tile<kD, kW>(t.k, t.rb, t.rows, lds0 + kb * T::TB, wave, lane);
  };
  auto issue_ds = [&](const Tile& t, int sb) __attribute__((always_inline)) {
    if (t.vis)
      dma_blocks4_nt(ds_wave + t.pos * ds_tile_bytes, dsl[0], dsl[1], dsl[2], dsl[3],
                     lds0 + kDsOff + (sb * kW + wave) * kDsWave);
  };

  f32x4 dq[2][T::ND];
#pragma unroll
  for (int qs = 0; qs < 2; qs++)
#pragma unroll
    for (int db = 0; db < T::ND; db++) dq[qs][db] = f32x4{};
  // 64 MFMAs on K buffer kb and dS buffer sb; keys at or past `rows` (the
  // segment's end) read as zero dS
  auto compute = [&](int kb, int sb, int rows) __attribute__((always_inline)) {
    const char* kt = smem + kb * T::TB;
    const char* dt = smem + kDsOff + (sb * kW + wave) * kDsWave;
    bf16x8 f[2][2];  // [qs][t]
#pragma unroll
    for (int qs = 0; qs < 2; qs++)
#pragma unroll
      for (int t = 0; t < 2; t++) {
        const char* base = dt + 2048 * t + 512 * qs;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_m16*)(base + dso[0]));
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_m16*)(base + dso[1]));
        const bf16x4 l4 = __builtin_bit_cast(bf16x4, lo), h4 = __builtin_bit_cast(bf16x4, hi);
        bf16x8 r;
        r[0] = l4[0]; r[1] = l4[1]; r[2] = l4[2]; r[3] = l4[3];
        r[4] = h4[0]; r[5] = h4[1]; r[6] = h4[2]; r[7] = h4[3];
        f[qs][t] = r;
      }
    if (rows < kKeys) {  // a segment's last tile only
#pragma unroll
      for (int qs = 0; qs < 2; qs++)
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
          for (int i = 0; i < 8; i++)
            if (32 * t + 8 * g + i >= rows) f[qs][t][i] = static_cast<bf16>(0.f);
    }
    // one fenced slot per (key step t, head-dim block db): the K^T operand
    // (head dims 16 db.., keys 32 t..), read kRead slots ahead, and two MFMAs
    constexpr int kSlots = 2 * T::ND;
    constexpr int kRead = 4, kRing = kRead + 1;
    bf16x8 ra[kRing];
    auto read_slot = [&](auto ic) __attribute__((always_inline)) {
      constexpr int i = decltype(ic)::value;
      ra[i % kRing] = col_operand<kD>(kt, 32 * (i / T::ND), 16 * (i % T::ND), lane);
    };
    static_for<kRead>([&](auto ic) { read_slot(ic); });
    static_for<kSlots>([&](auto ic) {
      constexpr int i = decltype(ic)::value, t = i / T::ND, db = i % T::ND;
      if constexpr (i + kRead < kSlots) read_slot(std::integral_constant<int, i + kRead>{});
#pragma unroll
      for (int qs = 0; qs < 2; qs++) dq[qs][db] = mfma16(ra[i % kRing], f[qs][t], dq[qs][db]);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Tiles i (computed), i + 1 (K and dS in flight) and i + 2 (dS in flight):
  // K of tile j in K buffer j % 2, dS in dS buffer j % 3. At step i the K rows
  // of tile i + 1 and the dS of tile i + 2 are issued, in that order; copies
  // complete in issue order, so waiting until at most the last dS copies are
  // outstanding means both K and dS of the next tile have landed.
  static_assert(T::TB / 1024 / kW == 4, "4 K copies per wave per tile");
  next_segment();
  Tile t0 = tile_here();
  issue_k(t0, 0);
  issue_ds(t0, 0);
  advance();
  Tile t1 = tile_here();
  if (t1.more) issue_ds(t1, 1);
  int kb = 0, sb = 0;
  for (;;) {
    if (t1.vis) asm volatile("s_waitcnt vmcnt(4)");  // the last issued copies are t1's dS (4 blocks)
    else asm volatile("s_waitcnt vmcnt(0)");
    __syncthreads();  // tile i has landed; every wave is done with tile i - 1's buffers
    Tile t2{};
    if (t1.more) {
      advance();
      t2 = tile_here();
      issue_k(t1, kb ^ 1);
      if (t2.more) issue_ds(t2, sb == 0 ? kDsBufs - 1 : sb - 1);  // buffer (i + 2) % 3
    }
    if (t0.vis) compute(kb, sb, t0.rows);
    if (!t1.more) break;
    t0 = t1;
    t1 = t2;
    kb ^= 1;
    sb = sb == kDsBufs - 1 ? 0 : sb + 1;
  }

  if (!wave_ok) return;
#pragma unroll
  for (int qs = 0; qs < 2; qs++) {
    const int t = tw0 + 16 * qs + i16;
    if (tw0 + 16 * qs >= len || t >= len) continue;
    bf16* dp = static_cast<bf16*>(a.dq) + static_cast<int64_t>(row0 + t) * qstride + head * kD + 4 * g;
#pragma unroll
    for (int db = 0; db < T::ND; db++) {
      bf16x4 v4;
#pragma unroll
      for (int r = 0; r < 4; r++) v4[r] = static_cast<bf16>(dq[qs][db][r] * a.scale);
      *reinterpret_cast<bf16x4*>(dp + 16 * db) = v4;
    }
  }
}

// ---------------------------------------------------------------------------
// dK/dV. One workgroup = 4 waves x 16 keys (KB 16-key blocks kb per wave) of
// one KV segment tile and KV head; it streams every 64-query block that
// sees the tile -- for a prefix node every descendant leaf and every query
// head of the group -- in the plan's fixed order, so a prefix node's gradient
// is the sum over its leaves in registers, without atomics. Per stage (one
// block, one head), for each pair of 16-query blocks t:
//   S = Q K^T, dP = dO V^T (Q, dO rows from LDS, permuted; K, V of the key
//   blocks in registers, so every row read feeds KB MFMAs),
//   P = exp2(scale*log2e S - lse*log2e), dS = P (dP - delta),
//   dV += P^T dO, dK += dS^T Q (dO, Q read transposed from LDS, again shared
//   by the key blocks).
// ---------------------------------------------------------------------------
// kStrided as in m16_fwd; kStoreDs: also store every dS block to the dS store
// (a.ds, head_dim 256) for the dQ kernel
template <int kD, bool kStrided, bool kStoreDs>
__global__ __launch_bounds__(256) void m16_dkdv(KernelArgs a) {
  using T = Geo<kD>;
  constexpr int kWaveKeys = m16_wave_keys(kD);
  constexpr int kKeys = m16_keys(kD);
  constexpr int KB = kWaveKeys / 16;  // 16-key blocks per wave
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
  const int i16 = lane & 15, g = lane >> 4;

  const int64_t kstride = static_cast<int64_t>(a.hkv) * kD;  // packed K/V rows: prefix inputs, every output
  const uint32_t g_rb = static_cast<uint32_t>(a.hq) * kD * 2;  // dO row bytes (packed)
  const uint32_t q_rb = kStrided ? static_cast<uint32_t>(a.q_rs) * 2 : g_rb;  // Q row bytes

  __shared__ __attribute__((aligned(1024))) char smem[2 * 2 * T::TB];           // [buf][Q | dO]
  __shared__ __attribute__((aligned(256))) float stats[2][2][kTileRows];       // [buf][-lse*log2e | -delta][row]
  __shared__ int4 qtab[kDkdvMaxBlocks];

  // An item is one key tile, or two suffix tiles of one leaf (DK_PAIR), a
  // tile and its mirror: the first streams its query blocks last-first, the
  // second first-last, so the pairs of a leaf that run together read the
  // same block at the same time and share its copies in L2. A lone suffix
  // tile streams last-first (all tiles of a leaf end at its last block);
  // prefix tiles first-last.
  const int ntiles = item[DK_PAIR] > 0 ? 2 : 1;
  for (int tile = 0; tile < ntiles; tile++) {
    const int key0 = tile == 0 ? item[DK_KEY0] : item[DK_PAIR] - 1;
    const int qb_hi = item[DK_QB_HI];
    const int qb_lo = tile == 0 ? item[DK_QB_LO] : item[DK_QB_LO] - (item[DK_KEY0] - key0) / kTileRows;
    const bool first_last = prefix || tile == 1;
    const int kw0 = key0 + kWaveKeys * wave;  // first key position of this wave
    const bool wave_active = kw0 < seg_len;

    if (tile > 0) __syncthreads();  // every wave is done with the previous tile's table
    // the tile's dS slot in the numbering of query block qb: first[qb] + the
    // tiles ahead of it in the dQ walk of any block below its segment
    const int ds_ahead = kStoreDs ? a.plan[a.off_ds + (prefix ? seg : a.num_nodes + seg)] + key0 / kKeys : 0;
    for (int i = threadIdx.x; i < qb_hi - qb_lo; i += blockDim.x) {
      const int qb = first_last ? qb_lo + i : qb_hi - 1 - i;
      const int lf = qblk[2 * qb], tok = qblk[2 * qb + 1];
      const int r0 = cu[lf];
      qtab[i] = int4{r0 + tok, tok, min(kTileRows, cu[lf + 1] - r0 - tok),
                     kStoreDs ? a.plan[a.off_ds_first + qb] + ds_ahead : 0};
    }
    __syncthreads();

    const int group = a.group;
    const int nstage = (qb_hi - qb_lo) * group;  // stage s: query block s / group, head s % group
    const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_address(smem));
    const uint32_t stats0 = __builtin_amdgcn_readfirstlane(lds_address(stats));
    auto issue = [&](int blk, int hh, int buf) {
      const int4 e = qtab[blk];
      const int row = __builtin_amdgcn_readfirstlane(e.x), nq = __builtin_amdgcn_readfirstlane(e.z);
      const int qh = kvh * group + hh;
      const int64_t col = static_cast<int64_t>(qh) * kD * 2;
      const int64_t goff = col + static_cast<int64_t>(row) * g_rb;
      const int64_t qoff = kStrided ? col + static_cast<int64_t>(row) * q_rb : goff;
      const uint32_t tile = lds0 + buf * 2 * T::TB;
      copy_tile<kD>(reinterpret_cast<const char*>(a.q) + qoff, q_rb, nq, tile, wave, lane);
      copy_tile<kD>(reinterpret_cast<const char*>(a.dout) + goff, g_rb, nq, tile + T::TB, wave, lane);
      if (wave < 2) {  // wave 0: -lse*log2e, wave 1: -delta; rows past the block end copy -inf / 0
        const int64_t at = static_cast<int64_t>(qh) * a.total_q + row + lane;
        const float* rows = wave == 0 ? a.stat_ws + kStatRowsOffset : a.ndelta_ws;
        dma4_lane(lane < nq ? rows + at : a.stat_ws + wave, stats0 + (buf * 2 + wave) * kTileRows * 4);
      }
    };
    if (nstage > 0) issue(0, 0, 0);

    // K / V of the lane's key kw0 + 16 kb + l % 16: the B operands of
    // S = Q K^T and dP = dO V^T
    bf16x8 kv[KB][T::NS], vv[KB][T::NS];
#pragma unroll
    for (int kb = 0; kb < KB; kb++) {
      const bf16* kbase = static_cast<const bf16*>(prefix ? a.pk : a.k);
      const bf16* vbase = static_cast<const bf16*>(prefix ? a.pv : a.v);
      const int key = min(kw0 + 16 * kb + i16, seg_len - 1);
      const int64_t off = static_cast<int64_t>(seg_row0 + key) * kstride + kvh * kD + 8 * g;
      const int64_t koff = prefix || !kStrided ? off : static_cast<int64_t>(seg_row0 + key) * a.k_rs + kvh * kD + 8 * g;
      const int64_t voff = prefix || !kStrided ? off : static_cast<int64_t>(seg_row0 + key) * a.v_rs + kvh * kD + 8 * g;
#pragma unroll
      for (int s = 0; s < T::NS; s++) {
        kv[kb][s] = *reinterpret_cast<const bf16x8*>(kbase + koff + 32 * s);
        vv[kb][s] = *reinterpret_cast<const bf16x8*>(vbase + voff + 32 * s);
      }
    }
    // register r of block [kb][db]: key 16 kb + 4 g + r of the wave, head dim 16 db + l % 16
    f32x4 dk[KB][T::ND], dv[KB][T::ND];
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
      for (int db = 0; db < T::ND; db++) {
        dk[kb][db] = f32x4{};
        dv[kb][db] = f32x4{};
      }
    const float c2 = a.scale * kLog2e;
#pragma unroll
    for (int kb = 0; kb < KB; kb++)
#pragma unroll
      for (int s = 0; s < T::NS; s++) {
        settle(kv[kb][s]);
        settle(vv[kb][s]);
      }
    wait_dma();
    __syncthreads();

    for (int sidx = 0; sidx < nstage; sidx++) {
      const int buf = sidx & 1;
      const int blk = sidx / group;
      if (sidx + 1 < nstage) issue((sidx + 1) / group, (sidx + 1) % group, buf ^ 1);
      if (wave_active) {
        const int tok0 = __builtin_amdgcn_readfirstlane(qtab[blk].y);
        // dS store: this stage's block (slot, head kvh G + sidx % G, this wave's 16 keys)
        char* ds_stage = nullptr;
        if constexpr (kStoreDs) {
          const int slot = __builtin_amdgcn_readfirstlane(qtab[blk].w);
          ds_stage = static_cast<char*>(a.ds) +
                     ((static_cast<int64_t>(kvh) * a.ds_slots + slot) * group + sidx % group) * m16_ds_head_bytes(kD) +
                     wave * (m16_ds_head_bytes(kD) / kM16Waves);
        }
        const char* qt = smem + buf * 2 * T::TB;
        const char* gt = qt + T::TB;
        const float* nlse = &stats[buf][0][0];
        const float* ndel = &stats[buf][1][0];
        // query q of the block visible from key kp iff kp <= tok0 + q (suffix tiles)
        const bool diag = !prefix && tok0 < kw0 + kWaveKeys - 1;
        // The stage is one fixed sequence of slots, each fenced: per query-block
        // pair t, the S / dP slots (e = 0, 1; k-steps s) and then the dV / dK
        // slots (head-dim blocks db). Every slot takes two operands from LDS
        // (Q and dO rows, or dO and Q read transposed), and those reads are
        // issued kRead slots ahead of the slot that uses them, so the MFMAs do
        // not wait on LDS latency; the softmax of block (t, e) runs after its
        // last S / dP slot, and its statistics are read at the block's first.
        constexpr int kSD = 2 * T::NS;       // S / dP slots per t
        constexpr int kPT = kSD + T::ND;     // slots per t
        constexpr int kSlots = 2 * kPT;
        constexpr int kRead = 4, kRing = kRead + 1;
        bf16x8 ra[kRing], rb[kRing];         // slot i's operands sit at i % kRing
        auto read_slot = [&](auto ic) __attribute__((always_inline)) {
          constexpr int i = decltype(ic)::value;
          constexpr int t = i / kPT, j = i % kPT;
          if constexpr (j < kSD) {
            constexpr int b = 2 * t + j / T::NS, s = j % T::NS;
            ra[i % kRing] = row_operand<kD>(qt, b, s, lane);
            rb[i % kRing] = row_operand<kD>(gt, b, s, lane);
          } else {
            constexpr int db = j - kSD;
            ra[i % kRing] = col_operand<kD>(gt, 32 * t, 16 * db, lane);
            rb[i % kRing] = col_operand<kD>(qt, 32 * t, 16 * db, lane);
          }
        };
        static_for<kRead>([&](auto ic) { read_slot(ic); });
        f32x4 sa[KB], pa[KB];
        f32x4 ls, dl;                                  // -lse*log2e, -delta of the block's queries
        float pf[KB][2][4], df[KB][2][4];              // [key block][query block 2t + e][register]
        bf16x8 pT[KB], dT[KB];                         // queries 32 t + 8 g + 0..7 of key 16 kb + l % 16
        static_for<kSlots>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          constexpr int t = i / kPT, j = i % kPT;
          if constexpr (i + kRead < kSlots) read_slot(std::integral_constant<int, i + kRead>{});
          if constexpr (j < kSD) {
            constexpr int e = j / T::NS, s = j % T::NS;
            if constexpr (s == 0) {
#pragma unroll
              for (int kb = 0; kb < KB; kb++) {
                sa[kb] = f32x4{};
                pa[kb] = f32x4{};
              }
              // register r: query 32 t + 8 g + 4 e + r of the block
              ls = *reinterpret_cast<const f32x4*>(nlse + 32 * t + 8 * g + 4 * e);
              dl = *reinterpret_cast<const f32x4*>(ndel + 32 * t + 8 * g + 4 * e);
            }
#pragma unroll
            for (int kb = 0; kb < KB; kb++) {
              sa[kb] = mfma16(ra[i % kRing], kv[kb][s], sa[kb]);
              pa[kb] = mfma16(rb[i % kRing], vv[kb][s], pa[kb]);
            }
            if constexpr (s == T::NS - 1) {
              const int q0 = 32 * t + 8 * g + 4 * e;
#pragma unroll
              for (int kb = 0; kb < KB; kb++) {
                const int kp = kw0 + 16 * kb + i16;
#pragma unroll
                for (int r = 0; r < 4; r++) {
                  float x = fmaf(sa[kb][r], c2, ls[r]);
                  if (diag) x = kp <= tok0 + q0 + r ? x : -INFINITY;
                  pf[kb][e][r] = fast_exp2(x);
                  df[kb][e][r] = pf[kb][e][r] * (pa[kb][r] + dl[r]);
                }
              }
              if constexpr (e == 1) {
#pragma unroll
                for (int kb = 0; kb < KB; kb++) {
                  pT[kb] = pack8(pf[kb][0], pf[kb][1]);
                  dT[kb] = pack8(df[kb][0], df[kb][1]);
                }
                if constexpr (kStoreDs) {
                  // dS of the 32-query half t, lane l: key l % 16, queries 32 t + 8 (l / 16) .. +7:
                  // one whole 1 KiB line, streaming buffer store from the stage's uniform base
                  static_assert(KB == 1, "one 16-key block per wave");
                  __builtin_amdgcn_raw_buffer_store_b128(
                      __builtin_bit_cast(i32x4_m16, dT[0]),
                      __builtin_amdgcn_make_buffer_rsrc(ds_stage, 0, m16_ds_head_bytes(kD) / kM16Waves, 0x00020000),
                      t * 1024 + 16 * lane, 0, 2 /* non-temporal */);
                }
              }
            }
          } else {
            constexpr int db = j - kSD;
#pragma unroll
            for (int kb = 0; kb < KB; kb++) {
              dv[kb][db] = mfma16(pT[kb], ra[i % kRing], dv[kb][db]);
              dk[kb][db] = mfma16(dT[kb], rb[i % kRing], dk[kb][db]);
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        });
      }
      wait_dma();  // stage sidx + 1 has landed
      __syncthreads();
    }

    if (wave_active) {
      // lane index laundered so the store addresses are formed here, not
      // hoisted out of the tile loop
      int el = lane;
      asm volatile("" : "+v"(el));
      const int i16 = el & 15, g = el >> 4;
      const int slot = item[DK_SLOT];  // -1 for a pair: its tiles are never split
      if (slot >= 0) {  // split tile: fp32 partial [kKeys][kD] for dK (already scaled) then dV
        float* pk = a.ws + static_cast<int64_t>(slot) * 2 * kKeys * kD;
        float* pv = pk + kKeys * kD;
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int key = kWaveKeys * wave + 16 * kb + 4 * g + r;
#pragma unroll
            for (int db = 0; db < T::ND; db++) {
              pk[key * kD + 16 * db + i16] = dk[kb][db][r] * a.scale;
              pv[key * kD + 16 * db + i16] = dv[kb][db][r];
            }
          }
      } else if (prefix && a.acc_prefix) {
#pragma clang fp contract(off)
        float* dkf = static_cast<float*>(a.dpk);
        float* dvf = static_cast<float*>(a.dpv);
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int key = kw0 + 16 * kb + 4 * g + r;
            if (key >= seg_len) continue;
            const int64_t off = static_cast<int64_t>(seg_row0 + key) * kstride + kvh * kD + i16;
#pragma unroll
            for (int db = 0; db < T::ND; db++) {
              dkf[off + 16 * db] += dk[kb][db][r] * a.scale;
              dvf[off + 16 * db] += dv[kb][db][r];
            }
          }
      } else {
        bf16* dkd = static_cast<bf16*>(prefix ? a.dpk : a.dk);
        bf16* dvd = static_cast<bf16*>(prefix ? a.dpv : a.dv);
#pragma unroll
        for (int kb = 0; kb < KB; kb++)
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const int key = kw0 + 16 * kb + 4 * g + r;
            if (key >= seg_len) continue;
            const int64_t off = static_cast<int64_t>(seg_row0 + key) * kstride + kvh * kD + i16;
#pragma unroll
            for (int db = 0; db < T::ND; db++) {
              dkd[off + 16 * db] = static_cast<bf16>(dk[kb][db][r] * a.scale);
              dvd[off + 16 * db] = static_cast<bf16>(dv[kb][db][r]);
            }
          }
      }
    }
  }  // tiles
}

// Second pass of split dK/dV tiles: the fp32 partial slots of one (segment
// tile, KV head) summed in slot (= leaf) order, written once.
template <int kD>
__global__ __launch_bounds__(256) void m16_reduce(KernelArgs a) {
  constexpr int kKeys = m16_keys(kD);
  const int32_t* item = a.plan + a.off_red + RD_WORDS * blockIdx.x;
  const bool prefix = item[RD_SRC] == 0;
  const int seg = item[RD_SEG], key0 = item[RD_KEY0], kvh = item[RD_KVH];
  const int slot0 = item[RD_SLOT0], nslots = item[RD_NSLOTS];
  const int32_t* cu = a.plan + a.off_cu;
  const int32_t* no = a.plan + a.off_node_off;
  const int seg_row0 = prefix ? no[seg] : cu[seg];
  const int keys = min(kKeys, (prefix ? no[seg + 1] - no[seg] : cu[seg + 1] - cu[seg]) - key0);
  const int64_t kstride = static_cast<int64_t>(a.hkv) * kD;
  bf16* dkd = static_cast<bf16*>(prefix ? a.dpk : a.dk);
  bf16* dvd = static_cast<bf16*>(prefix ? a.dpv : a.dv);
  const int64_t slot_floats = 2 * kKeys * kD;
  for (int e = threadIdx.x; e < 2 * keys * (kD / 4); e += blockDim.x) {
    const int which = e / (keys * (kD / 4));  // 0 = dK, 1 = dV
    const int rem = e % (keys * (kD / 4));
    const int key = rem / (kD / 4), d4 = rem % (kD / 4);
    const float* src = a.ws + static_cast<int64_t>(slot0) * slot_floats + which * kKeys * kD + key * kD + 4 * d4;
    f32x4 acc = *reinterpret_cast<const f32x4*>(src);
    for (int j = 1; j < nslots; j++) acc += *reinterpret_cast<const f32x4*>(src + j * slot_floats);
    const int64_t at = static_cast<int64_t>(seg_row0 + key0 + key) * kstride + kvh * kD + 4 * d4;
    if (prefix && a.acc_prefix) {
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
template <int kD>
bool strided_rows(const KernelArgs& a) {
  return a.q_rs != static_cast<int64_t>(a.hq) * kD || a.k_rs != static_cast<int64_t>(a.hkv) * kD ||
         a.v_rs != static_cast<int64_t>(a.hkv) * kD;
}

template <int kD, bool kRunList>
void launch_fwd_runs(const KernelArgs& a, hipStream_t s) {
  if (strided_rows<kD>(a))
    hipLaunchKernelGGL((m16_fwd<kD, kRunList, true>), dim3(a.n_items), dim3(64 * m16_fwd_waves(kD)), 0, s, a);
  else
    hipLaunchKernelGGL((m16_fwd<kD, kRunList, false>), dim3(a.n_items), dim3(64 * m16_fwd_waves(kD)), 0, s, a);
}

template <int kD>
int launch_fwd_d(const KernelArgs& a, hipStream_t s) {
  if (a.n_items > 0) {
    if (a.max_runs > kMfmaRegRuns)
      launch_fwd_runs<kD, true>(a, s);
    else
      launch_fwd_runs<kD, false>(a, s);
  }
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

template <int kD>
int launch_dkdv_d(const KernelArgs& a, int n_dkdv, int n_red, hipStream_t s) {
  if (n_dkdv > 0) {
    const bool st = strided_rows<kD>(a), ds = kD == 256 && a.ds != nullptr;
    if (st && ds)
      hipLaunchKernelGGL((m16_dkdv<kD, true, kD == 256>), dim3(n_dkdv), dim3(64 * kM16Waves), 0, s, a);
    else if (st)
      hipLaunchKernelGGL((m16_dkdv<kD, true, false>), dim3(n_dkdv), dim3(64 * kM16Waves), 0, s, a);
    else if (ds)
      hipLaunchKernelGGL((m16_dkdv<kD, false, kD == 256>), dim3(n_dkdv), dim3(64 * kM16Waves), 0, s, a);
    else
      hipLaunchKernelGGL((m16_dkdv<kD, false, false>), dim3(n_dkdv), dim3(64 * kM16Waves), 0, s, a);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  if (n_red > 0) {
    hipLaunchKernelGGL((m16_reduce<kD>), dim3(n_red), dim3(256), 0, s, a);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  return 0;
}

template <int kD, bool kRunList>
void launch_dq_runs(const KernelArgs& a, int n_fwd, hipStream_t s) {
  if (strided_rows<kD>(a))
    hipLaunchKernelGGL((m16_dq<kD, kRunList, true>), dim3(n_fwd), dim3(64 * kM16Waves), 0, s, a);
  else
    hipLaunchKernelGGL((m16_dq<kD, kRunList, false>), dim3(n_fwd), dim3(64 * kM16Waves), 0, s, a);
}

template <int kD>
int launch_dq_d(const KernelArgs& a, int n_fwd, hipStream_t s) {
  if constexpr (kD == 256) {
    if (n_fwd > 0 && a.ds) {  // dQ from the dS store
      if (strided_rows<kD>(a))
        hipLaunchKernelGGL((m16_dqs<kD, true>), dim3(n_fwd), dim3(64 * kM16DqsWaves), 0, s, a);
      else
        hipLaunchKernelGGL((m16_dqs<kD, false>), dim3(n_fwd), dim3(64 * kM16DqsWaves), 0, s, a);
      return hipGetLastError() != hipSuccess ? 4 : 0;
    }
  }
  if (n_fwd > 0) {
    if (a.max_runs > kMfmaRegRuns)
      launch_dq_runs<kD, true>(a, n_fwd, s);
    else
      launch_dq_runs<kD, false>(a, n_fwd, s);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  return 0;
}

}  // namespace

// The file is compiled once per head size (TPR_M16_HEAD_DIM = 64 or 256) and
// kernel group (TPR_M16_GROUP, bits: 1 = forward and delta, 2 = dK/dV and its
// reduction, 4 = dQ), so that each gets its own code-generation flags. Each
// object exports the launchers of its head size and groups
// (launch_m16_<kernel>_d64 or _d256).
#ifndef TPR_M16_HEAD_DIM
#error "compile tpr_mfma16.hip with -DTPR_M16_HEAD_DIM=64 or -DTPR_M16_HEAD_DIM=256"
#endif
#ifndef TPR_M16_GROUP
#define TPR_M16_GROUP 7
#endif
constexpr int kM16HeadDim = TPR_M16_HEAD_DIM;
static_assert(kM16HeadDim == 64 || kM16HeadDim == 256, "the 16-wide family serves head_dim 64 and 256");
#define TPR_M16_CAT2(a, b) a##b
#define TPR_M16_CAT(a, b) TPR_M16_CAT2(a, b)
#define TPR_M16_NAME(name) TPR_M16_CAT(name, TPR_M16_HEAD_DIM)

#if TPR_M16_GROUP & 1
int TPR_M16_NAME(launch_m16_fwd_d)(const KernelArgs& a, hipStream_t s) { return launch_fwd_d<kM16HeadDim>(a, s); }

int TPR_M16_NAME(launch_m16_delta_d)(const KernelArgs& a, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.total_q) * a.hq;
  const int blocks = static_cast<int>((rows + 15) / 16);
  if (blocks > 0) hipLaunchKernelGGL(m16_delta<kM16HeadDim>, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

#endif

#if TPR_M16_GROUP & 4
int TPR_M16_NAME(launch_m16_dq_d)(const KernelArgs& a, int n_fwd, hipStream_t s) {
  return launch_dq_d<kM16HeadDim>(a, n_fwd, s);
}
#endif

#if TPR_M16_GROUP & 2
int TPR_M16_NAME(launch_m16_dkdv_d)(const KernelArgs& a, int n_dkdv, int n_red, hipStream_t s) {
  return launch_dkdv_d<kM16HeadDim>(a, n_dkdv, n_red, s);
}
#endif

}  // namespace tpr
