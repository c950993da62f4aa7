// tpr_device.h -- device helpers shared by the HIP kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tpr_common.h"
#include "tpr_lanes.h"

namespace tpr {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Arguments every kernel receives by value. Plan offsets are copied from the
// host header so kernels do not chase them through memory.
struct KernelArgs {
  const int32_t* plan;
  const void* q;
  const void* k;
  const void* v;
  const void* pk;
  const void* pv;
  const void* out_in;   // forward output (backward input)
  const void* dout;
  void* out;            // forward output
  float* lse;           // [Hq, Tq]
  float* delta;         // [Hq, Tq]
  const float* lse_in;  // backward input
  void* dq;
  void* dk;
  void* dv;
  void* dpk;
  void* dpv;
  int32_t acc_prefix;  // dpk/dpv are fp32 accumulators: add the prefix gradient instead of writing it
  float scale;
  int32_t hq, hkv, d, group;
  int32_t hpw;  // query heads per forward/dQ workgroup (MFMA path)
  int32_t total_q, total_prefix, max_depth;
  int32_t off_cu, off_node_off, off_anc, off_node_leaf;
  int32_t off_qblk, off_leaf_qblk, off_fwd, off_dkdv, off_red;
  int32_t off_runs, max_runs;  // key-run table [N][max_runs][2]
  int32_t n_items;
  float* ws;       // fp32 partial dK/dV slots of split tiles
  float* stat_ws;  // MFMA backward: [0] = -inf, [1] = 0, then -lse*log2e rows from kStatRowsOffset
  float* ndelta_ws;  // MFMA backward: -delta rows [Hq, Tq] (the dK/dV kernel's dP accumulator start)
  // token (row) strides of q, k and v in elements (the packed Hq*D / Hkv*D
  // unless the caller reads them out of a wider buffer); every other tensor
  // is packed
  int64_t q_rs, k_rs, v_rs;
  // dS store of the head_dim-128 / 256 backward (null: dQ recomputes the
  // scores): slot s of KV head g, query head g * group + e at block
  // (g * ds_slots + s) * group + e (ds_head_bytes each); the plan's slot
  // table: tiles ahead of each segment at off_ds (nodes first, then
  // num_nodes + leaf), first slot of each query block at off_ds_first
  void* ds;
  int32_t off_ds, off_ds_first, num_nodes;
  int64_t ds_slots;
  // the head_dim-256 dQ-from-store work items (PF_OFF_DQS) and their query
  // heads per workgroup
  int32_t off_dqs, hpw_dqs;
  // physical key mask of a masked plan (SIMT kernels): nonzero = hidden; row
  // = query row of q, column = key position in the row's leaf key sequence
  // (ancestor nodes root first, then the suffix)
  const uint8_t* mask;
  int64_t mask_rs;  // bytes
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return static_cast<bf16>(x); }

// byte offset of element (row, col) in a swizzled 256-byte-row tile (swz_chunk: tpr_lanes.h)
__device__ __forceinline__ int swz_off(int row, int col) {
  return row * 256 + (swz_chunk(row, col >> 3) << 4) + ((col & 7) << 1);
}

// Key permutation sigma applied to the A-operand rows of a 32x32x16 MFMA so
// that accumulator register r of lane-half h holds key 16*(r/8) + 8*h + r%8:
// the 8 registers of one 16-key chunk are then 8 consecutive keys, which is
// the k-slot order of the next MFMA's operand.
__device__ __forceinline__ int sigma32(int m) {
  const int a = m >> 3, h = (m >> 2) & 1, b = m & 3;
  return ((a >> 1) << 4) + (h << 3) + ((a & 1) << 2) + b;
}

__device__ __forceinline__ float wave_max32(float x) {  // max over lanes l and l^32
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float wave_sum32(float x) { return x + __shfl_xor(x, 32); }

}  // namespace tpr
