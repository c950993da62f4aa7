// tpr_simt.hip -- SIMT (non-MFMA) prefix-reuse attention kernels.
//
// The path for fp32 inputs (fp32 accumulate, tolerance 1e-4 against the fp64
// oracle) and for any head_dim <= 128 the MFMA family does not cover. One
// thread owns one query row (forward, dQ) or one key row (dK/dV); K/V (or
// Q/dO) tiles are staged through LDS and shared by the 64 threads of a block.
//
// Math (per leaf, per query head; reference: _fa_fp32_reference.py:12-28):
//   s_j = scale * q . k_j over keys j = cat(ancestor nodes, suffix keys <= i)
//   out = sum_j softmax(s)_j v_j,  lse = log sum_j exp(s_j)
// Backward (standard softmax-attention gradients, recomputing P from lse):
//   p_j = exp(s_j - lse), dv_j += p_j dout, dp_j = dout . v_j,
//   ds_j = p_j (dp_j - delta), delta = dout . out,
//   dq = scale sum_j ds_j k_j, dk_j += scale ds_j q.

#include "tpr_device.h"

namespace tpr {
namespace {

template <typename T>
__device__ __forceinline__ void load_row(const T* src, int d, float* dst) {
  for (int i = 0; i < d; i++) dst[i] = to_f32(src[i]);
}

// Stage `rows` rows of a [*, heads, d] tensor into an fp32 LDS tile; rows at
// or beyond `valid` and columns at or beyond `d` are zero-filled.
template <typename T, int DMAX>
__device__ __forceinline__ void stage_rows(float (*tile)[DMAX + 1], const T* base, int64_t row_stride,
                                           int row0, int rows, int valid, int d) {
  for (int idx = threadIdx.x; idx < rows * DMAX; idx += blockDim.x) {
    const int r = idx / DMAX, c = idx % DMAX;
    tile[r][c] = (r < valid && c < d) ? to_f32(base[static_cast<int64_t>(row0 + r) * row_stride + c]) : 0.f;
  }
}

// ---------------------------------------------------------------------------
// Forward: block = 64 queries of one head of one leaf.
template <typename T, int DMAX>
__global__ __launch_bounds__(kSimtQ) void simt_fwd(KernelArgs a) {
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int32_t* no = a.plan + a.off_node_off;
  const int32_t* anc = a.plan + a.off_anc;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];
  const int d = a.d;
  const int t = tok0 + threadIdx.x;
  const bool valid = t < len;
  const int64_t qs = static_cast<int64_t>(a.hq) * d, ks = static_cast<int64_t>(a.hkv) * d;

  __shared__ float Ks[kSimtTile][DMAX + 1];
  __shared__ float Vs[kSimtTile][DMAX + 1];

  float q[DMAX], acc[DMAX];
  const float c = a.scale * kLog2e;
  {
    const T* src = static_cast<const T*>(a.q) + static_cast<int64_t>(row0 + (valid ? t : 0)) * qs + qh * d;
    for (int i = 0; i < DMAX; i++) q[i] = i < d ? to_f32(src[i]) * c : 0.f;
  }
  for (int i = 0; i < DMAX; i++) acc[i] = 0.f;
  float m = -INFINITY, l = 0.f;

  const int tok_last = min(len, tok0 + kSimtQ);  // suffix keys needed by the block
  const int nseg = a.max_depth + 1;
  for (int sg = 0; sg < nseg; sg++) {
    const T *kb, *vb;
    int seg_len;
    bool causal;
    if (sg < a.max_depth) {
      const int n = anc[leaf * a.max_depth + sg];
      if (n < 0) continue;
      kb = static_cast<const T*>(a.pk) + static_cast<int64_t>(no[n]) * ks + kvh * d;
      vb = static_cast<const T*>(a.pv) + static_cast<int64_t>(no[n]) * ks + kvh * d;
      seg_len = no[n + 1] - no[n];
      causal = false;
    } else {
      kb = static_cast<const T*>(a.k) + static_cast<int64_t>(row0) * ks + kvh * d;
      vb = static_cast<const T*>(a.v) + static_cast<int64_t>(row0) * ks + kvh * d;
      seg_len = tok_last;
      causal = true;
    }
    for (int j0 = 0; j0 < seg_len; j0 += kSimtTile) {
      const int nk = min(kSimtTile, seg_len - j0);
      __syncthreads();
      stage_rows<T, DMAX>(Ks, kb, ks, j0, kSimtTile, nk, d);
      stage_rows<T, DMAX>(Vs, vb, ks, j0, kSimtTile, nk, d);
      __syncthreads();
      float s[kSimtTile];
      float mt = m;
      for (int j = 0; j < kSimtTile; j++) {
        float x = 0.f;
        for (int i = 0; i < DMAX; i++) x += q[i] * Ks[j][i];
        const bool vis = j < nk && (!causal || j0 + j <= t);
        s[j] = vis ? x : -INFINITY;
        mt = fmaxf(mt, s[j]);
      }
      if (mt == -INFINITY) continue;  // nothing visible yet for this row
      const float alpha = exp2f(m - mt);
      l *= alpha;
      for (int i = 0; i < DMAX; i++) acc[i] *= alpha;
      for (int j = 0; j < kSimtTile; j++) {
        const float p = exp2f(s[j] - mt);
        l += p;
        for (int i = 0; i < DMAX; i++) acc[i] += p * Vs[j][i];
      }
      m = mt;
    }
  }
  if (!valid) return;
  const float inv = 1.f / l;
  T* dst = static_cast<T*>(a.out) + static_cast<int64_t>(row0 + t) * qs + qh * d;
  for (int i = 0; i < d; i++) dst[i] = from_f32<T>(acc[i] * inv);
  a.lse[static_cast<int64_t>(qh) * a.total_q + row0 + t] = (m + log2f(l)) * kLn2;
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
// dQ: block = 64 queries of one head of one leaf (same items as the forward).
template <typename T, int DMAX>
__global__ __launch_bounds__(kSimtQ) void simt_dq(KernelArgs a) {
  const int32_t* item = a.plan + a.off_fwd + 4 * blockIdx.x;
  const int leaf = item[0];
  if (leaf < 0) return;
  const int tok0 = item[1], qh = item[2], kvh = item[3];
  const int32_t* cu = a.plan + a.off_cu;
  const int32_t* no = a.plan + a.off_node_off;
  const int32_t* anc = a.plan + a.off_anc;
  const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];
  const int d = a.d;
  const int t = tok0 + threadIdx.x;
  const bool valid = t < len;
  const int tr = valid ? t : 0;
  const int64_t qs = static_cast<int64_t>(a.hq) * d, ks = static_cast<int64_t>(a.hkv) * d;

  __shared__ float Ks[kSimtTile][DMAX + 1];
  __shared__ float Vs[kSimtTile][DMAX + 1];

  float q[DMAX], g[DMAX], dq[DMAX];
  {
    const T* qsrc = static_cast<const T*>(a.q) + static_cast<int64_t>(row0 + tr) * qs + qh * d;
    const T* gsrc = static_cast<const T*>(a.dout) + static_cast<int64_t>(row0 + tr) * qs + qh * d;
    for (int i = 0; i < DMAX; i++) {
      q[i] = i < d ? to_f32(qsrc[i]) : 0.f;
      g[i] = i < d ? to_f32(gsrc[i]) : 0.f;
      dq[i] = 0.f;
    }
  }
  const float lse = a.lse_in[static_cast<int64_t>(qh) * a.total_q + row0 + tr];
  const float delta = a.delta[static_cast<int64_t>(qh) * a.total_q + row0 + tr];

  const int tok_last = min(len, tok0 + kSimtQ);
  const int nseg = a.max_depth + 1;
  for (int sg = 0; sg < nseg; sg++) {
    const T *kb, *vb;
    int seg_len;
    bool causal;
    if (sg < a.max_depth) {
      const int n = anc[leaf * a.max_depth + sg];
      if (n < 0) continue;
      kb = static_cast<const T*>(a.pk) + static_cast<int64_t>(no[n]) * ks + kvh * d;
      vb = static_cast<const T*>(a.pv) + static_cast<int64_t>(no[n]) * ks + kvh * d;
      seg_len = no[n + 1] - no[n];
      causal = false;
    } else {
      kb = static_cast<const T*>(a.k) + static_cast<int64_t>(row0) * ks + kvh * d;
      vb = static_cast<const T*>(a.v) + static_cast<int64_t>(row0) * ks + kvh * d;
      seg_len = tok_last;
      causal = true;
    }
    for (int j0 = 0; j0 < seg_len; j0 += kSimtTile) {
      const int nk = min(kSimtTile, seg_len - j0);
      __syncthreads();
      stage_rows<T, DMAX>(Ks, kb, ks, j0, kSimtTile, nk, d);
      stage_rows<T, DMAX>(Vs, vb, ks, j0, kSimtTile, nk, d);
      __syncthreads();
      for (int j = 0; j < nk; j++) {
        if (causal && j0 + j > t) break;
        float s = 0.f, dp = 0.f;
        for (int i = 0; i < DMAX; i++) {
          s += q[i] * Ks[j][i];
          dp += g[i] * Vs[j][i];
        }
        const float p = expf(s * a.scale - lse);
        const float ds = p * (dp - delta);
        for (int i = 0; i < DMAX; i++) dq[i] += ds * Ks[j][i];
      }
    }
  }
  if (!valid) return;
  T* dst = static_cast<T*>(a.dq) + static_cast<int64_t>(row0 + t) * qs + qh * d;
  for (int i = 0; i < d; i++) dst[i] = from_f32<T>(dq[i] * a.scale);
}

// ---------------------------------------------------------------------------
// dK/dV: block = 64 keys of one KV head of one segment (prefix node or leaf
// suffix); loops over every query block (and every query head of the group)
// that sees the keys, in the plan's fixed order, so a prefix node's gradient
// is summed over its descendant leaves in leaf order without atomics.
template <typename T, int DMAX>
__global__ __launch_bounds__(kSimtKeys) void simt_dkdv(KernelArgs a) {
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
  const int kp = key0 + threadIdx.x;  // key position within its segment
  const bool valid = kp < seg_len;
  const int64_t krow = static_cast<int64_t>(seg_row0 + (valid ? kp : 0));
  const T* kbase = static_cast<const T*>(prefix ? a.pk : a.k);
  const T* vbase = static_cast<const T*>(prefix ? a.pv : a.v);

  __shared__ float Qs[kSimtTile][DMAX + 1];
  __shared__ float Gs[kSimtTile][DMAX + 1];
  __shared__ float Ls[kSimtTile], Ds[kSimtTile];

  float kr[DMAX], vr[DMAX], dk[DMAX], dv[DMAX];
  for (int i = 0; i < DMAX; i++) {
    kr[i] = i < d ? to_f32(kbase[krow * ks + kvh * d + i]) : 0.f;
    vr[i] = i < d ? to_f32(vbase[krow * ks + kvh * d + i]) : 0.f;
    dk[i] = 0.f;
    dv[i] = 0.f;
  }
  for (int qb = qb_lo; qb < qb_hi; qb++) {
    const int leaf = qblk[2 * qb], tok0 = qblk[2 * qb + 1];
    const int row0 = cu[leaf], len = cu[leaf + 1] - cu[leaf];
    const int nq = min(kSimtTile, len - tok0);
    for (int g = 0; g < a.group; g++) {
      const int qh = kvh * a.group + g;
      __syncthreads();
      stage_rows<T, DMAX>(Qs, static_cast<const T*>(a.q) + qh * d, qs, row0 + tok0, kSimtTile, nq, d);
      stage_rows<T, DMAX>(Gs, static_cast<const T*>(a.dout) + qh * d, qs, row0 + tok0, kSimtTile, nq, d);
      for (int i = threadIdx.x; i < kSimtTile; i += blockDim.x) {
        const int64_t at = static_cast<int64_t>(qh) * a.total_q + row0 + tok0 + (i < nq ? i : 0);
        Ls[i] = a.lse_in[at];
        Ds[i] = a.delta[at];
      }
      __syncthreads();
      if (!valid) continue;
      for (int i = 0; i < nq; i++) {
        if (!prefix && kp > tok0 + i) continue;  // causal: key kp visible to query tok0+i iff kp <= tok0+i
        float s = 0.f, dp = 0.f;
        for (int x = 0; x < DMAX; x++) {
          s += kr[x] * Qs[i][x];
          dp += vr[x] * Gs[i][x];
        }
        const float p = expf(s * a.scale - Ls[i]);
        const float ds = p * (dp - Ds[i]);
        for (int x = 0; x < DMAX; x++) {
          dv[x] += p * Gs[i][x];
          dk[x] += ds * Qs[i][x];
        }
      }
    }
  }
  if (!valid) return;
  if (prefix && a.acc_prefix) {
#pragma clang fp contract(off)  // rounded product, then one add
    float* dkf = static_cast<float*>(a.dpk) + krow * ks + kvh * d;
    float* dvf = static_cast<float*>(a.dpv) + krow * ks + kvh * d;
    for (int i = 0; i < d; i++) {
      dkf[i] += dk[i] * a.scale;
      dvf[i] += dv[i];
    }
    return;
  }
  T* dkd = static_cast<T*>(prefix ? a.dpk : a.dk) + krow * ks + kvh * d;
  T* dvd = static_cast<T*>(prefix ? a.dpv : a.dv) + krow * ks + kvh * d;
  for (int i = 0; i < d; i++) {
    dkd[i] = from_f32<T>(dk[i] * a.scale);
    dvd[i] = from_f32<T>(dv[i]);
  }
}

template <typename T, int DMAX>
int launch_simt_fwd_t(const KernelArgs& a, hipStream_t s) {
  if (a.n_items > 0) hipLaunchKernelGGL((simt_fwd<T, DMAX>), dim3(a.n_items), dim3(kSimtQ), 0, s, a);
  return hipGetLastError() == hipSuccess ? 0 : 4;
}

}  // namespace

int launch_simt_fwd(const KernelArgs& a, bool fp32, hipStream_t s) {
  if (fp32) return a.d <= 64 ? launch_simt_fwd_t<float, 64>(a, s) : launch_simt_fwd_t<float, 128>(a, s);
  return a.d <= 64 ? launch_simt_fwd_t<bf16, 64>(a, s) : launch_simt_fwd_t<bf16, 128>(a, s);
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
  KernelArgs b = a;
  if (n_dkdv > 0) {
    if (fp32) {
      if (a.d <= 64) hipLaunchKernelGGL((simt_dkdv<float, 64>), dim3(n_dkdv), dim3(kSimtKeys), 0, s, b);
      else hipLaunchKernelGGL((simt_dkdv<float, 128>), dim3(n_dkdv), dim3(kSimtKeys), 0, s, b);
    } else {
      if (a.d <= 64) hipLaunchKernelGGL((simt_dkdv<bf16, 64>), dim3(n_dkdv), dim3(kSimtKeys), 0, s, b);
      else hipLaunchKernelGGL((simt_dkdv<bf16, 128>), dim3(n_dkdv), dim3(kSimtKeys), 0, s, b);
    }
    if (hipGetLastError() != hipSuccess) return 4;
  }
  if (n_fwd > 0) {
    if (fp32) {
      if (a.d <= 64) hipLaunchKernelGGL((simt_dq<float, 64>), dim3(n_fwd), dim3(kSimtQ), 0, s, b);
      else hipLaunchKernelGGL((simt_dq<float, 128>), dim3(n_fwd), dim3(kSimtQ), 0, s, b);
    } else {
      if (a.d <= 64) hipLaunchKernelGGL((simt_dq<bf16, 64>), dim3(n_fwd), dim3(kSimtQ), 0, s, b);
      else hipLaunchKernelGGL((simt_dq<bf16, 128>), dim3(n_fwd), dim3(kSimtQ), 0, s, b);
    }
    if (hipGetLastError() != hipSuccess) return 4;
  }
  return 0;
}

}  // namespace tpr
