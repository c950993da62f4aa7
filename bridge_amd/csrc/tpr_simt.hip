// tpr_simt.hip -- SIMT (non-MFMA) prefix-reuse attention kernels.
//
// The path for fp32 inputs (fp32 accumulate, tolerance 1e-4 against the fp64
// oracle) and for the head dims the MFMA family does not cover (any multiple
// of 8 up to 256). A row -- a query row in the forward and dQ, a key row in
// dK/dV -- is spread over kL = DMAX / 32 adjacent lanes, each holding 32 of
// its elements in registers: lane c of a group holds the 8 chunks of 4
// elements starting at 4*kL*j + 4*c (j < 8), so the kL lanes reading chunk j
// of an LDS row read 16*kL contiguous bytes. Dot products are summed over the
// group with DPP lane swaps, in an order that gives every lane of the group
// the same bits, so the softmax state stays identical across the group.
// K/V (or Q/dO) tiles are staged in LDS as fp32 and read by every row group
// at once (broadcast reads).
//
// Math (per leaf, per query head; reference: _fa_fp32_reference.py:12-28):
//   s_j = scale * q . k_j over keys j = cat(ancestor nodes, suffix keys <= i)
//   out = sum_j softmax(s)_j v_j,  lse = log sum_j exp(s_j)
// Backward (standard softmax-attention gradients, recomputing P from lse):
//   p_j = exp(s_j - lse), dv_j += p_j dout, dp_j = dout . v_j,
//   ds_j = p_j (dp_j - delta), delta = dout . out,
//   dq = scale sum_j ds_j k_j, dk_j += scale ds_j q.
// Key streams: the leaf's own suffix, then its ancestors' key runs (the
// plan's run table: ancestors root first, rows adjacent in prefix_k/v merged).
//
// Masked plans (kMask): a physical key mask replaces the causal rule, as in
// the reference's custom-mask mode (rectangular_attention.py:112-122): key
// c of a leaf's sequence cat(ancestors, suffix) is visible to query row r iff
// mask[r][c] == 0, so every suffix key is streamed, and the dK/dV items of a
// suffix tile cover every query block of the leaf. The mask bytes of each
// (query tile, key tile) pair are staged in LDS with the tiles. A row with no
// visible key ends with l = 0: its output is 0, its lse -inf, and every p of
// it is 0 in the backward (p is selected by visibility, never computed from
// that lse).

#include "tpr_device.h"

namespace tpr {
namespace {

// Rows staged per LDS tile: 16 KiB of fp32 per tile at most.
template <int DMAX>
constexpr int simt_tile() { return DMAX >= 256 ? 16 : 32; }

__device__ __forceinline__ f32x4 load4(const float* p) { return f32x4{p[0], p[1], p[2], p[3]}; }
__device__ __forceinline__ f32x4 load4(const bf16* p) {
  return f32x4{static_cast<float>(p[0]), static_cast<float>(p[1]), static_cast<float>(p[2]),
               static_cast<float>(p[3])};
}
__device__ __forceinline__ void store4(float* p, f32x4 v) {
  p[0] = v.x;
  p[1] = v.y;
  p[2] = v.z;
  p[3] = v.w;
}
__device__ __forceinline__ void store4(bf16* p, f32x4 v) {
  p[0] = static_cast<bf16>(v.x);
  p[1] = static_cast<bf16>(v.y);
  p[2] = static_cast<bf16>(v.z);
  p[3] = static_cast<bf16>(v.w);
}

// The lane's 32 elements of one row of a global [*, heads, d] tensor, times
// `mul`; elements at or beyond d are 0.
template <int kL, typename T>
__device__ __forceinline__ void load_slice(const T* row, int d, int c, float mul, f32x4 (&x)[8]) {
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int e = 4 * kL * j + 4 * c;
    x[j] = e < d ? load4(row + e) * mul : f32x4{0.f, 0.f, 0.f, 0.f};
  }
}

template <int kL, typename T>
__device__ __forceinline__ void store_slice(T* row, int d, int c, float mul, const f32x4 (&x)[8]) {
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const int e = 4 * kL * j + 4 * c;
    if (e < d) store4(row + e, x[j] * mul);
  }
}

// The lane's 32 elements of one row of an fp32 LDS tile with DMAX columns.
template <int kL>
__device__ __forceinline__ void read_slice(const float* lds_row, int c, f32x4 (&x)[8]) {
#pragma unroll
  for (int j = 0; j < 8; j++) x[j] = *reinterpret_cast<const f32x4*>(lds_row + 4 * kL * j + 4 * c);
}

template <int kL>
__device__ __forceinline__ float dot_lds(const f32x4 (&x)[8], const float* lds_row, int c) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const f32x4 y = *reinterpret_cast<const f32x4*>(lds_row + 4 * kL * j + 4 * c);
    s += x[j].x * y.x;
    s += x[j].y * y.y;
    s += x[j].z * y.z;
    s += x[j].w * y.w;
  }
  return s;
}

__device__ __forceinline__ float dot_regs(const f32x4 (&x)[8], const f32x4 (&y)[8]) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    s += x[j].x * y[j].x;
    s += x[j].y * y[j].y;
    s += x[j].z * y[j].z;
    s += x[j].w * y[j].w;
  }
  return s;
}

// acc += p * lds row (the lane's 32 elements)
template <int kL>
__device__ __forceinline__ void axpy_lds(f32x4 (&acc)[8], float p, const float* lds_row, int c) {
#pragma unroll
  for (int j = 0; j < 8; j++) acc[j] += p * *reinterpret_cast<const f32x4*>(lds_row + 4 * kL * j + 4 * c);
}

// x from the lane the DPP control selects (quad_perm / row_half_mirror stay
// within the lane's aligned group of 8, so every source lane is active).
template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, 0xF, 0xF, false));
}

// Sum over the kL (2, 4 or 8) adjacent lanes of an aligned group. Each step
// adds the partner's partial sum of the same size, and addition commutes, so
// all lanes of the group end with the same bits.
template <int kL>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(kL == 2 || kL == 4 || kL == 8, "2, 4 or 8 lanes per row");
  x += dpp<0xB1>(x);                          // quad_perm(1, 0, 3, 2): lane ^ 1
  if constexpr (kL >= 4) x += dpp<0x4E>(x);   // quad_perm(2, 3, 0, 1): lane ^ 2
  if constexpr (kL >= 8) x += dpp<0x141>(x);  // row_half_mirror: lane i <-> 7 - i of 8
  return x;
}

// bf16 dot-product operands. With bf16 inputs the dot products (q . k,
// dout . v) take their operands as bf16 -- the inputs' own values, so the
// products are exact -- two per v_dot2c_f32_bf16 into an fp32 sum: half the
// instructions of the fp32 FMA chain. Lane c of a row group holds the 4
// chunks of 8 elements at 8*kL*j + 8*c (16-byte LDS reads); the fp32 axpy
// operands keep the 4-element chunks above, a different partition of the
// same row, which the group sum does not care about.
struct Bf16Pairs {
  bf16x2 p[4];
};

template <int kL>
__device__ __forceinline__ void load_slice_bf(const bf16* row, int d, int c, bf16x8 (&x)[4]) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int e = 8 * kL * j + 8 * c;
    bf16x8 v;
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = e < d ? row[e + i] : static_cast<bf16>(0.f);
    x[j] = v;
  }
}

__device__ __forceinline__ float dot_bf(const bf16x8 (&x)[4], const bf16x8 (&y)[4]) {
  float s0 = 0.f, s1 = 0.f;  // two chains: half the dependent latency
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const Bf16Pairs a = __builtin_bit_cast(Bf16Pairs, x[j]);
    const Bf16Pairs b = __builtin_bit_cast(Bf16Pairs, y[j]);
    s0 = __builtin_amdgcn_fdot2_f32_bf16(a.p[0], b.p[0], s0, false);
    s1 = __builtin_amdgcn_fdot2_f32_bf16(a.p[1], b.p[1], s1, false);
    s0 = __builtin_amdgcn_fdot2_f32_bf16(a.p[2], b.p[2], s0, false);
    s1 = __builtin_amdgcn_fdot2_f32_bf16(a.p[3], b.p[3], s1, false);
  }
  return s0 + s1;
}

template <int kL>
__device__ __forceinline__ float dot_lds_bf(const bf16x8 (&x)[4], const bf16* lds_row, int c) {
  bf16x8 y[4];
#pragma unroll
  for (int j = 0; j < 4; j++) y[j] = *reinterpret_cast<const bf16x8*>(lds_row + 8 * kL * j + 8 * c);
  return dot_bf(x, y);
}

// Stage rows of a bf16 tensor into a bf16 LDS tile of DMAX columns (as
// stage_tile, without the conversion).
template <int DMAX>
__device__ __forceinline__ void stage_tile_bf(bf16* tile, const bf16* base, int64_t stride, int64_t row0, int rows,
                                              int valid, int d) {
  for (int idx = threadIdx.x; idx < rows * (DMAX / 8); idx += blockDim.x) {
    const int r = idx / (DMAX / 8), e = 8 * (idx % (DMAX / 8));
    bf16x8 x;
#pragma unroll
    for (int i = 0; i < 8; i++) x[i] = static_cast<bf16>(0.f);
    if (r < valid && e < d) {
      const bf16* src = base + (row0 + r) * stride + e;
#pragma unroll
      for (int i = 0; i < 8; i++) x[i] = src[i];
    }
    *reinterpret_cast<bf16x8*>(tile + r * DMAX + e) = x;
  }
}

// Stage rows [row0, row0 + rows) of a [*, heads, d] tensor (row stride
// `stride` elements, head offset applied to `base`) into an fp32 LDS tile of
// DMAX columns; rows at or beyond `valid` and columns at or beyond d are 0.
template <int DMAX, typename T>
__device__ __forceinline__ void stage_tile(float* tile, const T* base, int64_t stride, int64_t row0, int rows,
                                           int valid, int d) {
  for (int idx = threadIdx.x; idx < rows * (DMAX / 4); idx += blockDim.x) {
    const int r = idx / (DMAX / 4), e = 4 * (idx % (DMAX / 4));
    f32x4 x = {0.f, 0.f, 0.f, 0.f};
    if (r < valid && e < d) x = load4(base + (row0 + r) * stride + e);
    *reinterpret_cast<f32x4*>(tile + r * DMAX + e) = x;
  }
}

// Segment sg of a forward / dQ workgroup's key stream: 0 = the leaf's suffix
// (the first `suffix_keys` keys, causal), 1 + r = key run r of the leaf.
// Sets the segment's K and V row strides (elements): the caller's for the
// suffix, packed for the prefix. Returns false past the last run.
template <typename T>
__device__ __forceinline__ bool key_segment(const KernelArgs& a, int leaf, int sg, int suffix_keys, int kvh,
                                            const T*& kb, const T*& vb, int64_t& kst, int64_t& vst, int& seg_len) {
  const int64_t ks = static_cast<int64_t>(a.hkv) * a.d;
  if (sg == 0) {
    const int row0 = a.plan[a.off_cu + leaf];
    kb = static_cast<const T*>(a.k) + static_cast<int64_t>(row0) * a.k_rs + kvh * a.d;
    vb = static_cast<const T*>(a.v) + static_cast<int64_t>(row0) * a.v_rs + kvh * a.d;
    kst = a.k_rs;
    vst = a.v_rs;
    seg_len = suffix_keys;
    return true;
  }
  if (sg > a.max_runs) return false;
  const int32_t* run = a.plan + a.off_runs + 2 * (leaf * a.max_runs + sg - 1);
  seg_len = run[1];
  if (seg_len == 0) return false;  // {0, 0} pads the run list
  kb = static_cast<const T*>(a.pk) + static_cast<int64_t>(run[0]) * ks + kvh * a.d;
  vb = static_cast<const T*>(a.pv) + static_cast<int64_t>(run[0]) * ks + kvh * a.d;
  kst = vst = ks;
  return true;
}

// Stage mask bytes of query rows [row0, row0 + rows) and key columns
// [col0, col0 + cols) into LDS (rows x cols, row-major); entries of rows at or
// beyond valid_rows and columns at or beyond valid_cols read as hidden (1).
__device__ __forceinline__ void stage_mask(uint8_t* ms, const KernelArgs& a, int64_t row0, int rows, int valid_rows,
                                           int64_t col0, int cols, int valid_cols) {
  for (int idx = threadIdx.x; idx < rows * cols; idx += blockDim.x) {
    const int r = idx / cols, c = idx % cols;
    ms[idx] = r < valid_rows && c < valid_cols ? a.mask[(row0 + r) * a.mask_rs + col0 + c] : uint8_t{1};
  }
}

// Mask column of the first key of a segment in a leaf's key sequence: the
// lengths of the leaf's ancestors ahead of node `node` (all of them for
// node < 0, i.e. the leaf's own suffix).
__device__ __forceinline__ int leaf_key_column(const KernelArgs& a, int leaf, int node) {
  const int32_t* anc = a.plan + a.off_anc + static_cast<int64_t>(leaf) * a.max_depth;
  const int32_t* no = a.plan + a.off_node_off;
  int col = 0;
  for (int i = 0; i < a.max_depth; i++) {
    const int n = anc[i];
    if (n < 0 || n == node) break;
    col += no[n + 1] - no[n];
  }
  return col;
}

// ---------------------------------------------------------------------------
// Forward: block = kSimtQ queries of one head of one leaf, kL lanes per query.
template <typename T, int DMAX, bool kMask>
__global__ __launch_bounds__(kSimtQ * DMAX / 32) void simt_fwd(KernelArgs a) {
  constexpr int kL = DMAX / 32, kTile = simt_tile<DMAX>();
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];
  const int d = a.d;
  const int c = threadIdx.x % kL;
  const int t = tok0 + static_cast<int>(threadIdx.x) / kL;
  const bool valid = t < len;
  const int64_t qs = static_cast<int64_t>(a.hq) * d;

  constexpr bool kBf = __is_same(T, bf16);  // bf16 dot operands (K tile in bf16)
  __shared__ __attribute__((aligned(16))) float Ks[kBf ? 4 : kTile * DMAX];
  __shared__ __attribute__((aligned(16))) bf16 Kb[kBf ? kTile * DMAX : 8];
  __shared__ __attribute__((aligned(16))) float Vs[kTile * DMAX];
  __shared__ uint8_t Ms[kMask ? kSimtQ * kTile : 4];

  const float cs = a.scale * kLog2e;
  f32x4 q[8], o[8];
  bf16x8 qb[4];
  const T* qrow = static_cast<const T*>(a.q) + static_cast<int64_t>(row0 + (valid ? t : 0)) * a.q_rs + qh * d;
  if constexpr (kBf) load_slice_bf<kL>(qrow, d, c, qb);
  else load_slice<kL>(qrow, d, c, cs, q);
#pragma unroll
  for (int j = 0; j < 8; j++) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  // causal: the suffix keys up to the block's last query; masked: all of them
  const int suffix_keys = kMask ? len : min(len, tok0 + kSimtQ);
  const int suffix_col = kMask ? leaf_key_column(a, leaf, -1) : 0;  // mask column of suffix key 0
  int run_col = 0;                                                  // ... of the current run's key 0
  const T *kb, *vb;
  int64_t ks, vs;
  int seg_len;
  for (int sg = 0; key_segment<T>(a, leaf, sg, suffix_keys, kvh, kb, vb, ks, vs, seg_len); sg++) {
    const bool causal = sg == 0;
    const int seg_col = sg == 0 ? suffix_col : run_col;
    for (int j0 = 0; j0 < seg_len; j0 += kTile) {
      const int nk = min(kTile, seg_len - j0);
      __syncthreads();
      if constexpr (kBf) stage_tile_bf<DMAX>(Kb, kb, ks, j0, kTile, nk, d);
      else stage_tile<DMAX>(Ks, kb, ks, j0, kTile, nk, d);
      stage_tile<DMAX>(Vs, vb, vs, j0, kTile, nk, d);
      if constexpr (kMask) stage_mask(Ms, a, row0 + tok0, kSimtQ, len - tok0, seg_col + j0, kTile, nk);
      __syncthreads();
      float s[kTile];
      float mt = m;
#pragma unroll
      for (int j = 0; j < kTile; j++) {
        float x;
        if constexpr (kBf) x = group_sum<kL>(dot_lds_bf<kL>(qb, Kb + j * DMAX, c)) * cs;
        else x = group_sum<kL>(dot_lds<kL>(q, Ks + j * DMAX, c));
        bool vis;
        if constexpr (kMask) vis = j < nk && !Ms[(t - tok0) * kTile + j];
        else vis = j < nk && (!causal || j0 + j <= t);
        s[j] = vis ? x : -INFINITY;
        mt = fmaxf(mt, s[j]);
      }
      // nothing visible yet for this row: keep the (empty) state as it is
      const float mref = mt == -INFINITY ? 0.f : mt;
      const float alpha = exp2f(m - mref);
      l *= alpha;
#pragma unroll
      for (int j = 0; j < 8; j++) o[j] *= alpha;
#pragma unroll
      for (int j = 0; j < kTile; j++) {
        const float p = exp2f(s[j] - mref);
        l += p;
        axpy_lds<kL>(o, p, Vs + j * DMAX, c);
      }
      m = mt;
    }
    if (sg > 0) run_col += seg_len;
  }
  if (!valid) return;
  // l == 0 only for a row a mask hides every key of: out 0, lse -inf
  store_slice<kL>(static_cast<T*>(a.out) + static_cast<int64_t>(row0 + t) * qs + qh * d, d, c,
                  l > 0.f ? 1.f / l : 0.f, o);
  if (c == 0)
    a.lse[static_cast<int64_t>(qh) * a.total_q + row0 + t] = l > 0.f ? (m + log2f(l)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// delta[h][t] = sum_d dout[t][h][d] * out[t][h][d]; one thread per (t, h) row.
template <typename T>
__global__ __launch_bounds__(256) void simt_delta(KernelArgs a) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t rows = static_cast<int64_t>(a.total_q) * a.hq;
  if (row >= rows) return;
  const int64_t t = row / a.hq, h = row % a.hq;
  const T* o = static_cast<const T*>(a.out_in) + row * a.d;
  const T* g = static_cast<const T*>(a.dout) + row * a.d;
  float s = 0.f;
  for (int i = 0; i < a.d; i++) s += to_f32(o[i]) * to_f32(g[i]);
  a.delta[h * a.total_q + t] = s;
}

// ---------------------------------------------------------------------------
// dQ: block = kSimtQ queries of one head of one leaf (the forward's items).
template <typename T, int DMAX, bool kMask>
__global__ __launch_bounds__(kSimtQ * DMAX / 32) void simt_dq(KernelArgs a) {
  constexpr int kL = DMAX / 32, kTile = simt_tile<DMAX>();
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];
  const int d = a.d;
  const int c = threadIdx.x % kL;
  const int t = tok0 + static_cast<int>(threadIdx.x) / kL;
  const bool valid = t < len;
  const int tr = valid ? t : 0;
  const int64_t qs = static_cast<int64_t>(a.hq) * d;

  constexpr bool kBf = __is_same(T, bf16);  // bf16 dot operands (K, V tiles also in bf16)
  __shared__ __attribute__((aligned(16))) float Ks[kTile * DMAX];
  __shared__ __attribute__((aligned(16))) float Vs[kBf ? 4 : kTile * DMAX];
  __shared__ __attribute__((aligned(16))) bf16 Kb[kBf ? kTile * DMAX : 8];
  __shared__ __attribute__((aligned(16))) bf16 Vb[kBf ? kTile * DMAX : 8];
  __shared__ uint8_t Ms[kMask ? kSimtQ * kTile : 4];

  const float cs = a.scale * kLog2e;
  f32x4 q[8], g[8], dq[8];
  bf16x8 qb[4], gb[4];
  const T* qrow = static_cast<const T*>(a.q) + static_cast<int64_t>(row0 + tr) * a.q_rs + qh * d;
  const T* grow = static_cast<const T*>(a.dout) + static_cast<int64_t>(row0 + tr) * qs + qh * d;
  if constexpr (kBf) {
    load_slice_bf<kL>(qrow, d, c, qb);
    load_slice_bf<kL>(grow, d, c, gb);
  } else {
    load_slice<kL>(qrow, d, c, cs, q);
    load_slice<kL>(grow, d, c, 1.f, g);
  }
#pragma unroll
  for (int j = 0; j < 8; j++) dq[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int64_t stat = static_cast<int64_t>(qh) * a.total_q + row0 + tr;
  const float lse2 = a.lse_in[stat] * kLog2e;
  const float delta = a.delta[stat];

  const int suffix_keys = kMask ? len : min(len, tok0 + kSimtQ);
  const int suffix_col = kMask ? leaf_key_column(a, leaf, -1) : 0;
  int run_col = 0;
  const T *kb, *vb;
  int64_t ks, vs;
  int seg_len;
  for (int sg = 0; key_segment<T>(a, leaf, sg, suffix_keys, kvh, kb, vb, ks, vs, seg_len); sg++) {
    const bool causal = sg == 0;
    const int seg_col = sg == 0 ? suffix_col : run_col;
    for (int j0 = 0; j0 < seg_len; j0 += kTile) {
      const int nk = min(kTile, seg_len - j0);
      __syncthreads();
      stage_tile<DMAX>(Ks, kb, ks, j0, kTile, nk, d);
      if constexpr (kBf) {
        stage_tile_bf<DMAX>(Kb, kb, ks, j0, kTile, nk, d);
        stage_tile_bf<DMAX>(Vb, vb, vs, j0, kTile, nk, d);
      } else {
        stage_tile<DMAX>(Vs, vb, vs, j0, kTile, nk, d);
      }
      if constexpr (kMask) stage_mask(Ms, a, row0 + tok0, kSimtQ, len - tok0, seg_col + j0, kTile, nk);
      __syncthreads();
      for (int j = 0; j < nk; j++) {
        float s, dp;
        if constexpr (kBf) {
          s = group_sum<kL>(dot_lds_bf<kL>(qb, Kb + j * DMAX, c)) * cs;
          dp = group_sum<kL>(dot_lds_bf<kL>(gb, Vb + j * DMAX, c));
        } else {
          s = group_sum<kL>(dot_lds<kL>(q, Ks + j * DMAX, c));
          dp = group_sum<kL>(dot_lds<kL>(g, Vs + j * DMAX, c));
        }
        bool vis;
        if constexpr (kMask) vis = !Ms[(t - tok0) * kTile + j];
        else vis = !causal || j0 + j <= t;
        const float ds = vis ? exp2f(s - lse2) * (dp - delta) : 0.f;
        axpy_lds<kL>(dq, ds, Ks + j * DMAX, c);
      }
    }
    if (sg > 0) run_col += seg_len;
  }
  if (!valid) return;
  store_slice<kL>(static_cast<T*>(a.dq) + static_cast<int64_t>(row0 + t) * qs + qh * d, d, c, a.scale, dq);
}

// ---------------------------------------------------------------------------
// dK/dV: block = kSimtKeys keys of one KV head of one segment (prefix node or
// leaf suffix), kL lanes per key; loops over every query block (and every
// query head of the group) that sees the keys, in the plan's fixed order, so
// a prefix node's gradient is summed over its descendant leaves in leaf order
// without atomics.
template <typename T, int DMAX, bool kMask>
__global__ __launch_bounds__(kSimtKeys * DMAX / 32) void simt_dkdv(KernelArgs a) {
  constexpr int kL = DMAX / 32, kTile = simt_tile<DMAX>();
  const int32_t* item = a.plan + a.off_dkdv + DK_WORDS * blockIdx.x;
  if (item[DK_SRC] < 0) return;
  const bool prefix = item[DK_SRC] == 0;
  const int seg = item[DK_SEG], key0 = item[DK_KEY0], kvh = item[DK_KVH];
  const int qb_lo = item[DK_QB_LO], qb_hi = item[DK_QB_HI];
  const int32_t* cu = a.plan + a.off_cu;
  const int32_t* no = a.plan + a.off_node_off;
  const int32_t* qblk = a.plan + a.off_qblk;
  const int d = a.d;
  const int64_t qs = static_cast<int64_t>(a.hq) * d, ks = static_cast<int64_t>(a.hkv) * d;
  const int seg_row0 = prefix ? no[seg] : cu[seg];
  const int seg_len = prefix ? no[seg + 1] - no[seg] : cu[seg + 1] - cu[seg];
  const int c = threadIdx.x % kL;
  const int kp = key0 + static_cast<int>(threadIdx.x) / kL;  // key position within its segment
  const bool valid = kp < seg_len;
  const int64_t krow = static_cast<int64_t>(seg_row0 + (valid ? kp : 0));
  const T* kbase = static_cast<const T*>(prefix ? a.pk : a.k);
  const T* vbase = static_cast<const T*>(prefix ? a.pv : a.v);

  // The dot operands stay fp32 here: q_i and dout_i are needed in fp32 for
  // the dK/dV updates anyway, and bf16 copies of the Q/dO tiles as well cost
  // more in LDS traffic than the bf16 dot products save (measured).
  __shared__ __attribute__((aligned(16))) float Qs[kTile * DMAX];
  __shared__ __attribute__((aligned(16))) float Gs[kTile * DMAX];
  __shared__ float Ls[kTile], Ds[kTile];  // lse * log2e, delta
  __shared__ uint8_t Ms[kMask ? kTile * kSimtKeys : 4];

  f32x4 kr[8], vr[8], dk[8], dv[8];
  load_slice<kL>(kbase + krow * (prefix ? ks : a.k_rs) + kvh * d, d, c, a.scale * kLog2e, kr);
  load_slice<kL>(vbase + krow * (prefix ? ks : a.v_rs) + kvh * d, d, c, 1.f, vr);
#pragma unroll
  for (int j = 0; j < 8; j++) {
    dk[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  for (int qb = qb_lo; qb < qb_hi; qb++) {
    const int leaf = qblk[2 * qb], tok0 = qblk[2 * qb + 1];
    const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];
    const int nblk = min(kSimtTile, len - tok0);
    // mask column of the item's first key in this leaf's key sequence
    const int col0 = kMask ? leaf_key_column(a, leaf, prefix ? seg : -1) + key0 : 0;
    for (int gh = 0; gh < a.group; gh++) {
      const int qh = kvh * a.group + gh;
      for (int sub = 0; sub < nblk; sub += kTile) {
        const int nq = min(kTile, nblk - sub);
        const int64_t r0 = static_cast<int64_t>(row0) + tok0 + sub;
        __syncthreads();
        stage_tile<DMAX>(Qs, static_cast<const T*>(a.q) + qh * d, a.q_rs, r0, kTile, nq, d);
        stage_tile<DMAX>(Gs, static_cast<const T*>(a.dout) + qh * d, qs, r0, kTile, nq, d);
        for (int i = threadIdx.x; i < kTile; i += blockDim.x) {
          const int64_t at = static_cast<int64_t>(qh) * a.total_q + r0 + (i < nq ? i : 0);
          Ls[i] = a.lse_in[at] * kLog2e;
          Ds[i] = a.delta[at];
        }
        if constexpr (kMask) stage_mask(Ms, a, r0, kTile, nq, col0, kSimtKeys, seg_len - key0);
        __syncthreads();
        for (int i = 0; i < nq; i++) {
          f32x4 qi[8], gi[8];
          read_slice<kL>(Qs + i * DMAX, c, qi);
          read_slice<kL>(Gs + i * DMAX, c, gi);
          const float s = group_sum<kL>(dot_regs(kr, qi));
          const float dp = group_sum<kL>(dot_regs(vr, gi));
          // causal: key kp is visible to query tok0 + sub + i iff kp <= tok0 + sub + i
          bool vis;
          if constexpr (kMask) vis = !Ms[i * kSimtKeys + (kp - key0)];
          else vis = prefix || kp <= tok0 + sub + i;
          const float p = vis ? exp2f(s - Ls[i]) : 0.f;
          const float ds = p * (dp - Ds[i]);
#pragma unroll
          for (int j = 0; j < 8; j++) {
            dv[j] += p * gi[j];
            dk[j] += ds * qi[j];
          }
        }
      }
    }
  }
  if (!valid) return;
  const int64_t at = krow * ks + kvh * d;
  if (prefix && a.acc_prefix) {
#pragma clang fp contract(off)  // rounded product, then one add
    float* dkf = static_cast<float*>(a.dpk) + at;
    float* dvf = static_cast<float*>(a.dpv) + at;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int e = 4 * kL * j + 4 * c;
      if (e < d) {
        store4(dkf + e, load4(dkf + e) + dk[j] * a.scale);
        store4(dvf + e, load4(dvf + e) + dv[j]);
      }
    }
    return;
  }
  store_slice<kL>(static_cast<T*>(prefix ? a.dpk : a.dk) + at, d, c, a.scale, dk);
  store_slice<kL>(static_cast<T*>(prefix ? a.dpv : a.dv) + at, d, c, 1.f, dv);
}

template <typename T, bool kMask>
int launch_fwd_t(const KernelArgs& a, hipStream_t s) {
  if (a.n_items <= 0) return 0;
  if (a.d <= 64) hipLaunchKernelGGL((simt_fwd<T, 64, kMask>), dim3(a.n_items), dim3(kSimtQ * 2), 0, s, a);
  else if (a.d <= 128) hipLaunchKernelGGL((simt_fwd<T, 128, kMask>), dim3(a.n_items), dim3(kSimtQ * 4), 0, s, a);
  else hipLaunchKernelGGL((simt_fwd<T, 256, kMask>), dim3(a.n_items), dim3(kSimtQ * 8), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

template <typename T, bool kMask>
int launch_bwd_t(const KernelArgs& a, int n_fwd, int n_dkdv, hipStream_t s) {
  if (n_dkdv > 0) {
    if (a.d <= 64) hipLaunchKernelGGL((simt_dkdv<T, 64, kMask>), dim3(n_dkdv), dim3(kSimtKeys * 2), 0, s, a);
    else if (a.d <= 128) hipLaunchKernelGGL((simt_dkdv<T, 128, kMask>), dim3(n_dkdv), dim3(kSimtKeys * 4), 0, s, a);
    else hipLaunchKernelGGL((simt_dkdv<T, 256, kMask>), dim3(n_dkdv), dim3(kSimtKeys * 8), 0, s, a);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  if (n_fwd > 0) {
    if (a.d <= 64) hipLaunchKernelGGL((simt_dq<T, 64, kMask>), dim3(n_fwd), dim3(kSimtQ * 2), 0, s, a);
    else if (a.d <= 128) hipLaunchKernelGGL((simt_dq<T, 128, kMask>), dim3(n_fwd), dim3(kSimtQ * 4), 0, s, a);
    else hipLaunchKernelGGL((simt_dq<T, 256, kMask>), dim3(n_fwd), dim3(kSimtQ * 8), 0, s, a);
    if (hipGetLastError() != hipSuccess) return 4;
  }
  return 0;
}

}  // namespace

int launch_simt_fwd(const KernelArgs& a, bool fp32, hipStream_t s) {
  if (a.mask) return fp32 ? launch_fwd_t<float, true>(a, s) : launch_fwd_t<bf16, true>(a, s);
  return fp32 ? launch_fwd_t<float, false>(a, s) : launch_fwd_t<bf16, false>(a, s);
}

int launch_delta(const KernelArgs& a, bool fp32, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.total_q) * a.hq;
  const int blocks = static_cast<int>((rows + 255) / 256);
  if (blocks == 0) return 0;
  if (fp32)
    hipLaunchKernelGGL(simt_delta<float>, dim3(blocks), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(simt_delta<bf16>, dim3(blocks), dim3(256), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

int launch_simt_bwd(const KernelArgs& a, int n_fwd, int n_dkdv, bool fp32, hipStream_t s) {
  if (a.mask)
    return fp32 ? launch_bwd_t<float, true>(a, n_fwd, n_dkdv, s) : launch_bwd_t<bf16, true>(a, n_fwd, n_dkdv, s);
  return fp32 ? launch_bwd_t<float, false>(a, n_fwd, n_dkdv, s) : launch_bwd_t<bf16, false>(a, n_fwd, n_dkdv, s);
}

}  // namespace tpr
