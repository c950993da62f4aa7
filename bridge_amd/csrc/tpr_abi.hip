// tpr_abi.hip -- extern "C" entry points of libtpr_attn.so: argument checks,
// plan-header decoding and kernel dispatch. Host code only.

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "../../include/tpr_attn.h"
#include "tpr_device.h"
#include "tpr_host.h"

namespace tpr {

int launch_simt_fwd(const KernelArgs& a, bool fp32, hipStream_t s);
int launch_delta(const KernelArgs& a, bool fp32, hipStream_t s);
int launch_simt_bwd(const KernelArgs& a, int n_fwd, int n_dkdv, bool fp32, hipStream_t s);
int launch_mfma_fwd(const KernelArgs& a, hipStream_t s);
int launch_mfma_bwd(const KernelArgs& a, int n_fwd, int n_dkdv, int n_red, hipStream_t s);
int launch_mfma_delta(const KernelArgs& a, hipStream_t s);
// the 16x16x32 family (tpr_mfma16.hip), one object per head size and kernel group
int launch_m16_fwd_d64(const KernelArgs& a, hipStream_t s);
int launch_m16_fwd_d256(const KernelArgs& a, hipStream_t s);
int launch_m16_delta_d64(const KernelArgs& a, hipStream_t s);
int launch_m16_delta_d256(const KernelArgs& a, hipStream_t s);
int launch_m16_dkdv_d64(const KernelArgs& a, int n_dkdv, int n_red, hipStream_t s);
int launch_m16_dkdv_d256(const KernelArgs& a, int n_dkdv, int n_red, hipStream_t s);
int launch_m16_dq_d64(const KernelArgs& a, int n_fwd, hipStream_t s);
int launch_m16_dq_d256(const KernelArgs& a, int n_fwd, hipStream_t s);
inline int launch_m16_fwd(const KernelArgs& a, hipStream_t s) {
  return a.d == 64 ? launch_m16_fwd_d64(a, s) : launch_m16_fwd_d256(a, s);
}
inline int launch_m16_delta(const KernelArgs& a, hipStream_t s) {
  return a.d == 64 ? launch_m16_delta_d64(a, s) : launch_m16_delta_d256(a, s);
}
// dK/dV tiles, their reduction, then dQ
inline int launch_m16_bwd(const KernelArgs& a, int n_fwd, int n_dkdv, int n_red, hipStream_t s) {
  const int rc = a.d == 64 ? launch_m16_dkdv_d64(a, n_dkdv, n_red, s) : launch_m16_dkdv_d256(a, n_dkdv, n_red, s);
  if (rc != 0) return rc;
  return a.d == 64 ? launch_m16_dq_d64(a, n_fwd, s) : launch_m16_dq_d256(a, n_fwd, s);
}

namespace {
thread_local char g_error[512] = "";

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_plan(const int32_t* plan_host, const int32_t* plan_device) {
  if (!plan_host || !plan_device) return fail(TPR_ERR_INVALID_ARGUMENT, "plan_host and plan_device must not be NULL");
  if (plan_host[PF_MAGIC] != kPlanMagic || plan_host[PF_VERSION] != kPlanVersion)
    return fail(TPR_ERR_INVALID_ARGUMENT, "plan_host is not a plan blob written by tpr_attn_plan (version %d)",
                kPlanVersion);
  return TPR_OK;
}

int check_scale(float scale) {
  if (!std::isfinite(scale) || scale <= 0.f)
    return fail(TPR_ERR_INVALID_ARGUMENT, "softmax_scale must be finite and positive, got %g", scale);
  return TPR_OK;
}

KernelArgs args_from_plan(const int32_t* ph, const int32_t* pd, float scale) {
  KernelArgs a;
  std::memset(&a, 0, sizeof(a));
  a.plan = pd;
  a.scale = scale;
  a.hq = ph[PF_HQ];
  a.hkv = ph[PF_HKV];
  a.d = ph[PF_D];
  a.group = a.hq / a.hkv;
  // query heads per forward / dQ workgroup: gcd(group, waves per workgroup)
  const int waves = ph[PF_PATH] == PATH_MFMA16 ? kM16Waves : kFwdWaves;
  a.hpw = 1;
  for (int g = waves; g >= 1; g--)
    if (a.group % g == 0 && waves % g == 0) { a.hpw = g; break; }
  a.total_q = ph[PF_TOTAL_Q];
  a.total_prefix = ph[PF_TOTAL_PREFIX];
  a.max_depth = ph[PF_MAX_DEPTH];
  a.off_cu = ph[PF_OFF_CU];
  a.off_node_off = ph[PF_OFF_NODE_OFF];
  a.off_anc = ph[PF_OFF_ANC];
  a.off_node_leaf = ph[PF_OFF_NODE_LEAF];
  a.off_qblk = ph[PF_OFF_QBLK];
  a.off_leaf_qblk = ph[PF_OFF_LEAF_QBLK];
  a.off_fwd = ph[PF_OFF_FWD];
  a.off_dkdv = ph[PF_OFF_DKDV];
  a.off_red = ph[PF_OFF_RED];
  a.off_runs = ph[PF_OFF_RUNS];
  a.max_runs = ph[PF_MAX_RUNS];
  a.off_dqs = ph[PF_OFF_DQS];
  // query heads per dQ-from-store workgroup (8 waves in both families)
  static_assert(kFwdWaves == kM16DqsWaves, "one dQ-from-store item layout");
  a.hpw_dqs = 1;
  for (int g = kM16DqsWaves; g >= 1; g--)
    if (a.group % g == 0 && kM16DqsWaves % g == 0) { a.hpw_dqs = g; break; }
  return a;
}

// Row strides of q, k and v (0 = packed), validated into the kernel arguments.
int set_row_strides(KernelArgs& a, const int32_t* ph, int64_t q_rs, int64_t k_rs, int64_t v_rs) {
  const int64_t elem = ph[PF_DTYPE] == TPR_DTYPE_FP32 ? 4 : 2;
  const int64_t packed_q = static_cast<int64_t>(a.hq) * a.d, packed_kv = static_cast<int64_t>(a.hkv) * a.d;
  const struct {
    int64_t given, packed;
    const char* name;
    int64_t* out;
  } rows[3] = {{q_rs, packed_q, "q", &a.q_rs}, {k_rs, packed_kv, "k", &a.k_rs}, {v_rs, packed_kv, "v", &a.v_rs}};
  for (const auto& r : rows) {
    const int64_t stride = r.given == 0 ? r.packed : r.given;
    if (stride < r.packed)
      return fail(TPR_ERR_INVALID_ARGUMENT, "%s_row_stride must be 0 or at least %lld elements, got %lld", r.name,
                  static_cast<long long>(r.packed), static_cast<long long>(r.given));
    if ((stride * elem) % 16 != 0)
      return fail(TPR_ERR_INVALID_ARGUMENT, "%s_row_stride must give rows of a multiple of 16 bytes, got %lld",
                  r.name, static_cast<long long>(stride));
    if (stride * elem > (int64_t{1} << 25))
      return fail(TPR_ERR_UNSUPPORTED, "%s_row_stride must give rows of at most 32 MiB, got %lld elements", r.name,
                  static_cast<long long>(stride));
    *r.out = stride;
  }
  return TPR_OK;
}

// The key mask: required by a masked plan, refused by any other.
int set_mask(KernelArgs& a, const int32_t* ph, const uint8_t* mask, int64_t row_stride) {
  const int64_t cols = ph[PF_MASK_COLS];
  if (cols == 0) {
    if (mask) return fail(TPR_ERR_INVALID_ARGUMENT, "a key mask needs a plan built with TPR_PLAN_MASKED");
    return TPR_OK;
  }
  if (!mask && ph[PF_TOTAL_Q] > 0)
    return fail(TPR_ERR_INVALID_ARGUMENT, "the plan was built with TPR_PLAN_MASKED: mask must not be NULL");
  const int64_t stride = row_stride == 0 ? cols : row_stride;
  if (stride < cols)
    return fail(TPR_ERR_INVALID_ARGUMENT, "mask_row_stride must be 0 or at least %lld bytes (the longest key "
                "sequence), got %lld", static_cast<long long>(cols), static_cast<long long>(row_stride));
  a.mask = mask;
  a.mask_rs = stride;
  return TPR_OK;
}

int check_tensor(const void* p, const char* name, bool needed, bool mfma) {
  if (!needed) return TPR_OK;
  if (!p) return fail(TPR_ERR_INVALID_ARGUMENT, "%s must not be NULL", name);
  if (mfma && !aligned16(p)) return fail(TPR_ERR_INVALID_ARGUMENT, "%s must be 16-byte aligned", name);
  return TPR_OK;
}
}  // namespace

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return status;
}

void clear_error() { g_error[0] = '\0'; }

}  // namespace tpr

using namespace tpr;

extern "C" int tpr_attn_abi_version(void) { return TPR_ATTN_ABI_VERSION; }

extern "C" const char* tpr_attn_last_error(void) { return g_error; }

namespace tpr {
namespace {
// floats of one stat row set of the MFMA backward ([Hq, Tq] padded to a
// multiple of 64, so every area after it stays 256-byte aligned)
size_t stat_row_floats(const int32_t* ph) {
  if (ph[PF_PATH] == PATH_SIMT || ph[PF_TOTAL_Q] <= 0) return 0;
  const size_t rows = static_cast<size_t>(ph[PF_HQ]) * static_cast<size_t>(ph[PF_TOTAL_Q]);
  return (rows + 63) / 64 * 64;
}
// floats of the stat area: the constants, the lse*log2e rows, the -delta rows
size_t stat_floats(const int32_t* ph) {
  const size_t rows = stat_row_floats(ph);
  return rows ? kStatRowsOffset + 2 * rows : 0;
}
}  // namespace
}  // namespace tpr

namespace tpr {
namespace {
// bytes before the dS store: the stat area and the fp32 partial slots
// (a multiple of 256: the stat rows are padded to 64 floats, a slot is
// keys x D x 2 floats)
size_t ws_fp32_bytes(const int32_t* ph) {
  const size_t slots = static_cast<size_t>(ph[PF_N_SLOTS]);
  const size_t keys = ph[PF_PATH] == PATH_MFMA16 ? m16_keys(ph[PF_D]) : kDkdvKeys;  // per partial slot
  return (stat_floats(ph) + slots * keys * static_cast<size_t>(ph[PF_D]) * 2) * sizeof(float);
}
size_t ds_bytes(const int32_t* ph) {
  return static_cast<size_t>(ph[PF_DS_SLOTS]) * static_cast<size_t>(ph[PF_HQ]) * ds_head_bytes(ph[PF_PATH], ph[PF_D]);
}
}  // namespace
}  // namespace tpr

extern "C" size_t tpr_attn_bwd_workspace_bytes(const int32_t* plan_host) {
  if (!plan_host || plan_host[PF_MAGIC] != kPlanMagic) return 0;
  return ws_fp32_bytes(plan_host) + ds_bytes(plan_host);
}

extern "C" int tpr_attn_fwd(const TprFwdParams* p, void* stream) {
  clear_error();
  if (!p) return fail(TPR_ERR_INVALID_ARGUMENT, "params must not be NULL");
  if (p->abi_version != TPR_ATTN_ABI_VERSION)
    return fail(TPR_ERR_INVALID_ARGUMENT, "abi_version %d does not match library version %d", p->abi_version,
                TPR_ATTN_ABI_VERSION);
  int rc = check_plan(p->plan_host, p->plan_device);
  if (rc) return rc;
  if ((rc = check_scale(p->softmax_scale))) return rc;
  const int32_t* ph = p->plan_host;
  const bool mfma = ph[PF_PATH] != PATH_SIMT;  // either MFMA family: 16-byte aligned rows
  const bool any_q = ph[PF_TOTAL_Q] > 0, any_p = ph[PF_TOTAL_PREFIX] > 0;
  if ((rc = check_tensor(p->q, "q", any_q, mfma)) || (rc = check_tensor(p->k, "k", any_q, mfma)) ||
      (rc = check_tensor(p->v, "v", any_q, mfma)) || (rc = check_tensor(p->out, "out", any_q, mfma)) ||
      (rc = check_tensor(p->lse, "lse", any_q, false)) ||
      (rc = check_tensor(p->prefix_k, "prefix_k", any_p, mfma)) ||
      (rc = check_tensor(p->prefix_v, "prefix_v", any_p, mfma)))
    return rc;
  KernelArgs a = args_from_plan(ph, p->plan_device, p->softmax_scale);
  if ((rc = set_row_strides(a, ph, p->q_row_stride, p->k_row_stride, p->v_row_stride))) return rc;
  if ((rc = set_mask(a, ph, p->mask, p->mask_row_stride))) return rc;
  a.q = p->q;
  a.k = p->k;
  a.v = p->v;
  a.pk = p->prefix_k;
  a.pv = p->prefix_v;
  a.out = p->out;
  a.lse = p->lse;
  a.n_items = ph[PF_N_FWD];
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = ph[PF_PATH] == PATH_MFMA     ? launch_mfma_fwd(a, s)
       : ph[PF_PATH] == PATH_MFMA16 ? launch_m16_fwd(a, s)
                                    : launch_simt_fwd(a, ph[PF_DTYPE] == TPR_DTYPE_FP32, s);
  if (rc) return fail(TPR_ERR_LAUNCH, "forward launch failed: %s", hipGetErrorString(hipGetLastError()));
  return TPR_OK;
}

extern "C" int tpr_attn_bwd(const TprBwdParams* p, void* stream) {
  return tpr_attn_bwd_phases(p, TPR_BWD_DELTA | TPR_BWD_DKDV | TPR_BWD_DQ, stream);
}

namespace tpr {
namespace {
// tpr_attn_bwd_phases with the workspace given separately (the caller's, or
// the library's static scratch for tpr_attn_bwd_noalloc).
int bwd_phases(const TprBwdParams* p, int phases, void* stream, void* workspace, size_t workspace_bytes) {
  constexpr int kAllPhases = TPR_BWD_DELTA | TPR_BWD_DKDV | TPR_BWD_DQ | TPR_BWD_DKDV_TILES | TPR_BWD_DKDV_REDUCE;
  if (phases <= 0 || (phases & ~kAllPhases))
    return fail(TPR_ERR_INVALID_ARGUMENT, "phases must be a non-empty mask of TPR_BWD_* bits, got %d", phases);
  if (!p) return fail(TPR_ERR_INVALID_ARGUMENT, "params must not be NULL");
  if (p->abi_version != TPR_ATTN_ABI_VERSION)
    return fail(TPR_ERR_INVALID_ARGUMENT, "abi_version %d does not match library version %d", p->abi_version,
                TPR_ATTN_ABI_VERSION);
  int rc = check_plan(p->plan_host, p->plan_device);
  if (rc) return rc;
  if ((rc = check_scale(p->softmax_scale))) return rc;
  if (p->flags & ~TPR_BWD_ACCUMULATE_PREFIX_F32)
    return fail(TPR_ERR_INVALID_ARGUMENT, "flags must be 0 or TPR_BWD_ACCUMULATE_PREFIX_F32, got %d", p->flags);
  const int32_t* ph = p->plan_host;
  const int path = ph[PF_PATH];
  const bool mfma = path != PATH_SIMT;  // either MFMA family: 16-byte aligned rows
  const bool any_q = ph[PF_TOTAL_Q] > 0, any_p = ph[PF_TOTAL_PREFIX] > 0;
  if ((rc = check_tensor(p->q, "q", any_q, mfma)) || (rc = check_tensor(p->k, "k", any_q, mfma)) ||
      (rc = check_tensor(p->v, "v", any_q, mfma)) || (rc = check_tensor(p->out, "out", any_q, mfma)) ||
      (rc = check_tensor(p->dout, "dout", any_q, mfma)) || (rc = check_tensor(p->lse, "lse", any_q, false)) ||
      (rc = check_tensor(p->delta, "delta", any_q, false)) || (rc = check_tensor(p->dq, "dq", any_q, mfma)) ||
      (rc = check_tensor(p->dk, "dk", any_q, mfma)) || (rc = check_tensor(p->dv, "dv", any_q, mfma)) ||
      (rc = check_tensor(p->prefix_k, "prefix_k", any_p, mfma)) ||
      (rc = check_tensor(p->prefix_v, "prefix_v", any_p, mfma)) ||
      (rc = check_tensor(p->dprefix_k, "dprefix_k", any_p, mfma)) ||
      (rc = check_tensor(p->dprefix_v, "dprefix_v", any_p, mfma)))
    return rc;
  const size_t need = tpr_attn_bwd_workspace_bytes(ph);
  if (need > 0 && (!workspace || workspace_bytes < need))
    return fail(TPR_ERR_BUFFER_TOO_SMALL, "backward workspace needs %zu bytes, got %zu", need, workspace_bytes);
  // the MFMA backward reads the partial slots as 16-byte vectors and DMA-copies
  // the stat rows; the layout keeps every slot 256-byte aligned from the base
  if (need > 0 && (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return fail(TPR_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
  KernelArgs a = args_from_plan(ph, p->plan_device, p->softmax_scale);
  if ((rc = set_row_strides(a, ph, p->q_row_stride, p->k_row_stride, p->v_row_stride))) return rc;
  if ((rc = set_mask(a, ph, p->mask, p->mask_row_stride))) return rc;
  a.q = p->q;
  a.k = p->k;
  a.v = p->v;
  a.pk = p->prefix_k;
  a.pv = p->prefix_v;
  a.out_in = p->out;
  a.dout = p->dout;
  a.lse_in = p->lse;
  a.delta = p->delta;
  a.dq = p->dq;
  a.dk = p->dk;
  a.dv = p->dv;
  a.dpk = p->dprefix_k;
  a.dpv = p->dprefix_v;
  a.acc_prefix = (p->flags & TPR_BWD_ACCUMULATE_PREFIX_F32) ? 1 : 0;
  a.stat_ws = static_cast<float*>(workspace);
  a.ndelta_ws = a.stat_ws ? a.stat_ws + kStatRowsOffset + stat_row_floats(ph) : nullptr;
  a.ws = a.stat_ws + stat_floats(ph);
  a.ds = ds_bytes(ph) ? static_cast<char*>(workspace) + ws_fp32_bytes(ph) : nullptr;
  a.off_ds = ph[PF_OFF_DS];
  a.off_ds_first = ph[PF_OFF_DS] + ph[PF_NUM_NODES] + ph[PF_NUM_LEAVES];
  a.ds_slots = ph[PF_DS_SLOTS];
  a.num_nodes = ph[PF_NUM_NODES];
  const bool fp32 = ph[PF_DTYPE] == TPR_DTYPE_FP32;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int n_dkdv = (phases & (TPR_BWD_DKDV | TPR_BWD_DKDV_TILES)) ? ph[PF_N_DKDV] : 0;
  const int n_red = (phases & (TPR_BWD_DKDV | TPR_BWD_DKDV_REDUCE)) ? ph[PF_N_RED] : 0;  // 0 on the SIMT path
  // dQ work items: the forward's, or a dS-store plan's own list
  const int n_dq = (phases & TPR_BWD_DQ) ? (ph[PF_N_DQS] > 0 ? ph[PF_N_DQS] : ph[PF_N_FWD]) : 0;
  if (phases & TPR_BWD_DELTA)
    rc = path == PATH_MFMA ? launch_mfma_delta(a, s) : path == PATH_MFMA16 ? launch_m16_delta(a, s)
                                                                          : launch_delta(a, fp32, s);
  if (!rc && (n_dkdv || n_red || n_dq))
    rc = path == PATH_MFMA     ? launch_mfma_bwd(a, n_dq, n_dkdv, n_red, s)
         : path == PATH_MFMA16 ? launch_m16_bwd(a, n_dq, n_dkdv, n_red, s)
                               : launch_simt_bwd(a, n_dq, n_dkdv, fp32, s);
  if (rc) return fail(TPR_ERR_LAUNCH, "backward launch failed: %s", hipGetErrorString(hipGetLastError()));
  return TPR_OK;
}
}  // namespace
}  // namespace tpr

extern "C" int tpr_attn_bwd_phases(const TprBwdParams* p, int phases, void* stream) {
  clear_error();
  if (!p) return fail(TPR_ERR_INVALID_ARGUMENT, "params must not be NULL");
  return bwd_phases(p, phases, stream, p->workspace, p->workspace_bytes);
}

// ---------------------------------------------------------------------------
// Allocation-free backward. The workspace is a file-scope device array, one
// copy per GPU, sized for kScratchBytes; its device address is looked up once
// per device (hipGetSymbolAddress, with that device current) and kept. Host
// code never passes the array's own name to a kernel: on the host it is only
// a stand-in for the symbol.
// ---------------------------------------------------------------------------
namespace tpr {
namespace {
constexpr size_t kScratchBytes = size_t{64} << 20;  // 64 MiB per GPU
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The lookup may load the library's code object on the device, which a
// stream capture must not see: the first call on a device has to be made
// outside capture, and a capturing stream that finds no address yet is
// refused with a message saying so.
int scratch_for_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0)
    return fail(TPR_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(hipGetLastError()));
  if (dev >= kMaxDevices) return fail(TPR_ERR_UNSUPPORTED, "device %d is beyond the %d this library tracks", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &capture) != hipSuccess)
      return fail(TPR_ERR_LAUNCH, "hipStreamIsCapturing failed: %s", hipGetErrorString(hipGetLastError()));
    if (capture != hipStreamCaptureStatusNone)
      return fail(TPR_ERR_INVALID_ARGUMENT,
                  "the first tpr_attn_bwd_noalloc call on device %d is being captured; make one call on that device "
                  "outside stream capture first (it looks up the static scratch's address)", dev);
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(TPR_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TPR_OK;
}
}  // namespace
}  // namespace tpr

extern "C" size_t tpr_attn_bwd_noalloc_max_workspace_bytes(void) { return kScratchBytes; }

extern "C" int tpr_attn_bwd_noalloc(const TprBwdParams* p, void* stream) {
  clear_error();
  if (!p) return fail(TPR_ERR_INVALID_ARGUMENT, "params must not be NULL");
  if (p->abi_version == TPR_ATTN_ABI_VERSION && p->plan_host && p->plan_host[PF_MAGIC] == kPlanMagic) {
    const size_t need = tpr_attn_bwd_workspace_bytes(p->plan_host);
    if (need > kScratchBytes)
      return fail(TPR_ERR_UNSUPPORTED,
                  "backward workspace needs %zu bytes, more than the %zu bytes of the library's static scratch; "
                  "build the plan with TPR_PLAN_RECOMPUTE_DQ (no dS store), or use tpr_attn_bwd with a "
                  "caller-allocated workspace", need, kScratchBytes);
  }
  void* ws = nullptr;
  int rc = scratch_for_current_device(static_cast<hipStream_t>(stream), &ws);
  if (rc) return rc;
  return bwd_phases(p, TPR_BWD_DELTA | TPR_BWD_DKDV | TPR_BWD_DQ, stream, ws, kScratchBytes);
}
