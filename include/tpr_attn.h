/*
 * tpr_attn.h -- C ABI of libtpr_attn.so, the gfx950 (MI355X) prefix-reuse
 * attention library.
 *
 * One call attends N sibling suffixes ("leaves") to the shared K/V of their
 * ancestor prefix segments ("nodes") plus their own causal suffix K/V:
 *
 *   query token i of leaf s sees every token of every ancestor node of s
 *   (root -> parent order) and suffix tokens j <= i of leaf s.
 *
 * With one leaf and one node this is exactly the reference's single-sequence
 * operator rectangular_causal_attention(q, cat(pk, k), cat(pv, v))
 * (verl/models/mcore/tpr/rectangular_attention.py:125-209, right-down causal
 * mask "key j visible to query i iff j <= P + i", sparse mode 3 at :30,118;
 * the same mask is stated by tests/models/mcore/tpr/parallel/_fa_fp32_reference.py:24-25).
 * The sibling-summed prefix gradient replaces the per-sibling anchor relay of
 * verl/models/mcore/tpr/kv_stack.py:175-203 and prefix_state.py:546-573.
 *
 * Layouts (all row-major, head_dim contiguous, "TND" as in
 * rectangular_attention.py:179-181):
 *   q, out, dq, dout : [total_q, num_q_heads, head_dim]       (leaves packed by cu_seqlens_q)
 *   k, v, dk, dv     : [total_q, num_kv_heads, head_dim]
 *   prefix_k/v, dprefix_k/v : [total_prefix, num_kv_heads, head_dim] (nodes packed by node_offsets)
 *   lse, delta       : float32 [num_q_heads, total_q]  (natural-log LSE of the scaled scores)
 * GQA: query head h reads KV head h / (num_q_heads / num_kv_heads)
 * (_fa_fp32_reference.py:20-21, contiguous query-head groups).
 *
 * Ownership: the caller allocates every buffer, including the plan blob and
 * the backward workspace. The library never allocates or frees device memory,
 * keeps no pointer after a call returns, holds no mutable global state except
 * the thread-local error string, and never synchronises the stream.
 * Launches are enqueued on the stream given; results are deterministic
 * (no floating-point atomics; every output element has one writer or a
 * fixed-order reduction).
 *
 * Errors: every entry point returns TPR_OK (0) or a TprStatus; the message of
 * the last failure on the calling thread is returned by tpr_attn_last_error().
 */
#ifndef TPR_ATTN_H
#define TPR_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TPR_ATTN_ABI_VERSION 6

typedef enum TprStatus {
  TPR_OK = 0,
  TPR_ERR_INVALID_ARGUMENT = 1, /* bad shape / metadata / pointer */
  TPR_ERR_UNSUPPORTED = 2,      /* valid request this build has no kernel for */
  TPR_ERR_BUFFER_TOO_SMALL = 3, /* plan or workspace capacity too small */
  TPR_ERR_LAUNCH = 4            /* the HIP runtime rejected a launch */
} TprStatus;

/* head_dim: a multiple of 8, at most 256. bf16 with head_dim 128 runs on the
 * 32x32x16 MFMA kernels, bf16 with head_dim 64 or 256 on the 16x16x32 MFMA
 * kernels (any tree depth); fp32 and the other head sizes on the SIMT
 * kernels. All accumulate in fp32. */
typedef enum TprDtype {
  TPR_DTYPE_BF16 = 0, /* bf16 in/out, fp32 accumulation */
  TPR_DTYPE_FP32 = 1  /* fp32 in/out, fp32 accumulation */
} TprDtype;

/* Host-side description of the prefix tree, input of the planner.
 * Mirrors the reference's tree metadata: SegmentSpec/SegmentPlan
 * (verl/models/mcore/tpr/segment_plan.py:67-313) lowered to packed offsets.
 *   cu_seqlens_q[num_leaves+1]   leaf suffix offsets into q/k/v rows
 *   node_offsets[num_nodes+1]    node offsets into prefix_k/prefix_v rows
 *   leaf_ancestors[num_leaves*max_depth]  node ids of each leaf's path,
 *       root first, padded with -1 at the end (kv_stack.py:139-154 order).
 * Every node must be the ancestor of a contiguous range of leaves (true when
 * leaves are numbered in DFS order, segment_plan.py:266-275), and a node that
 * appears in a path must appear at the same depth in every path.
 *
 * dS store. A bf16 head_dim-128 or 256 plan may have the dK/dV kernel store
 * every dS block it computes (bf16, 2 bytes per visible (query, key) pair and
 * query head) in the backward workspace, and the dQ kernel read them: dQ =
 * scale dS K then costs one matrix product instead of three (the scores S and
 * dP recomputed). ds_store_max_bytes is the caller's budget for that store:
 * the plan has one only when it fits, otherwise dQ recomputes and the
 * workspace stays small (a few MB: statistics and split-tile partials).
 *   ds_store_max_bytes = 0                      no store (the zeroed default)
 *   ds_store_max_bytes = TPR_DS_STORE_DEFAULT   the library's default budget,
 *                        TPR_DS_STORE_DEFAULT_BYTES (8 GiB): the Qwen3-4B
 *                        layer shape (prefix 4096 + 4 x 4096, GQA 32/8) needs
 *                        6.5 GB, prefix 32768 + 8 x 2048 needs 35.5 GB
 *   ds_store_max_bytes > 0                      at most that many bytes
 * TPR_PLAN_RECOMPUTE_DQ forces no store whatever the budget (needed by
 * tpr_attn_bwd_noalloc for shapes whose store would not fit its scratch).
 * Other paths ignore both. The store's size is tpr_attn_bwd_workspace_bytes()
 * of the plan minus that of the same tree planned with budget 0.
 *
 * Key mask. TPR_PLAN_MASKED builds a plan for calls that pass a physical key
 * mask (TprFwdParams.mask): the mask is then the only visibility rule, as in
 * the reference's custom-mask mode (sparse mode 0, rectangular_attention.py:
 * 112-122) -- the causal rule is not applied on top of it, so a mask may also
 * show a leaf's later suffix keys. Such a plan always runs the SIMT kernels
 * (any dtype and head size), with no dS store; every call with it must pass a
 * mask, and a call with a mask must use such a plan.
 * flags: 0 or an OR of TPR_PLAN_RECOMPUTE_DQ and TPR_PLAN_MASKED. */
#define TPR_PLAN_RECOMPUTE_DQ 1
#define TPR_PLAN_MASKED 2
#define TPR_DS_STORE_DEFAULT (-1)
#define TPR_DS_STORE_DEFAULT_BYTES (INT64_C(8) << 30)
typedef struct TprTreeDesc {
  int32_t num_leaves;
  int32_t num_nodes;
  int32_t max_depth;
  int32_t num_q_heads;
  int32_t num_kv_heads;
  int32_t head_dim;
  int32_t dtype; /* TprDtype */
  int32_t flags; /* 0, TPR_PLAN_RECOMPUTE_DQ, TPR_PLAN_MASKED */
  const int32_t* cu_seqlens_q;
  const int32_t* node_offsets;
  const int32_t* leaf_ancestors;
  int64_t ds_store_max_bytes; /* dS store budget: 0, TPR_DS_STORE_DEFAULT or > 0 bytes */
} TprTreeDesc;

/* Forward: out = softmax(scale * q [prefix_k; k]^T + mask) [prefix_v; v], and
 * lse. Replaces one npu_fusion_attention call per sibling
 * (rectangular_attention.py:187-204) by one launch over all siblings. */
typedef struct TprFwdParams {
  int32_t abi_version; /* must be TPR_ATTN_ABI_VERSION */
  int32_t reserved;
  float softmax_scale; /* finite, > 0 (rectangular_attention.py:169-172) */
  float reserved_f;
  const int32_t* plan_host;   /* plan blob written by tpr_attn_plan (host copy) */
  const int32_t* plan_device; /* identical blob in device memory */
  const void* q;
  const void* k;
  const void* v;
  const void* prefix_k;
  const void* prefix_v;
  void* out;
  float* lse;
  /* Token (row) strides of q, k and v in elements; 0 = packed (Hq*D for q,
   * Hkv*D for k and v). They let q, k and v be read as views of a wider
   * buffer, e.g. the column slices of a fused QKV projection
   * [tokens, (Hq + 2 Hkv) * D], without a copy. A stride must be at least the
   * packed one, give rows of a multiple of 16 bytes and at most 32 MiB; the
   * heads of a row stay packed (head stride D). Every other tensor is packed. */
  int64_t q_row_stride;
  int64_t k_row_stride;
  int64_t v_row_stride;
  /* Physical key mask of a TPR_PLAN_MASKED plan (NULL with any other plan):
   * bytes, nonzero = hidden, one row per query token (the rows of q), row r
   * at mask + r * mask_row_stride. Column c of a row of leaf s is key c of
   * that leaf's key sequence cat(ancestor nodes root first, own suffix), the
   * columns of the reference's [Sq, Skv] bool mask for one leaf. A row reads
   * only its leaf's columns; mask_row_stride (bytes, 0 = the minimum) must be
   * at least the longest key sequence of any leaf. A query row that sees no
   * key gets out = 0, lse = -inf and zero gradients. */
  const uint8_t* mask;
  int64_t mask_row_stride;
} TprFwdParams;

/* Backward: dq, dk, dv for the suffix tokens, and dprefix_k/dprefix_v summed
 * over every descendant leaf of each node in leaf order (fixed-order
 * reduction, the deterministic counterpart of prefix_state.py:565-573).
 * delta is caller-provided scratch of lse's shape; workspace is caller-provided
 * scratch of at least tpr_attn_bwd_workspace_bytes() bytes, 256-byte aligned
 * (TPR_ERR_INVALID_ARGUMENT otherwise; may be NULL when that size is 0).
 *
 * flags = TPR_BWD_ACCUMULATE_PREFIX_F32: dprefix_k/dprefix_v are fp32 buffers
 * of [total_prefix, Hkv, D] whatever the dtype, and each node's gradient
 * (still the fixed-order sum over its leaves) is ADDED to them instead of
 * written. This is the gradient relay of KVPrefixState.accumulate_layer_gradients
 * (prefix_state.py:546-573), where every backward that reads a prefix state
 * adds its gradient to that state's buffer, with the buffer kept in fp32 and
 * the add fused into the kernel's final write. One writer per element per
 * call, so calls on one stream accumulate deterministically. */
#define TPR_BWD_ACCUMULATE_PREFIX_F32 1
typedef struct TprBwdParams {
  int32_t abi_version;
  int32_t flags; /* 0 or TPR_BWD_ACCUMULATE_PREFIX_F32 */
  float softmax_scale;
  float reserved_f;
  const int32_t* plan_host;
  const int32_t* plan_device;
  const void* q;
  const void* k;
  const void* v;
  const void* prefix_k;
  const void* prefix_v;
  const void* out;
  const void* dout;
  const float* lse;
  float* delta;
  void* dq;
  void* dk;
  void* dv;
  void* dprefix_k;
  void* dprefix_v;
  void* workspace;        /* 256-byte aligned */
  size_t workspace_bytes; /* >= tpr_attn_bwd_workspace_bytes(plan_host) */
  /* row strides of q, k and v, as in TprFwdParams (0 = packed); the
   * gradients dq, dk, dv are written packed */
  int64_t q_row_stride;
  int64_t k_row_stride;
  int64_t v_row_stride;
  /* the forward's key mask (TprFwdParams.mask) */
  const uint8_t* mask;
  int64_t mask_row_stride;
} TprBwdParams;

/* ABI version compiled into the library (TPR_ATTN_ABI_VERSION). */
int tpr_attn_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* tpr_attn_last_error(void);

/* Build the launch plan (metadata + work lists) for a tree on the host.
 * With plan == NULL only *words_needed is written. The blob is position
 * independent: copy it unchanged to device memory for plan_device. */
int tpr_attn_plan(const TprTreeDesc* tree, int32_t* plan, int64_t capacity_words,
                  int64_t* words_needed);

/* Bytes of workspace the backward needs for this plan (fp32 statistics and
 * partial sums, and the dS store of a plan that has one). */
size_t tpr_attn_bwd_workspace_bytes(const int32_t* plan_host);

/* Enqueue the forward on `stream` (a hipStream_t; NULL = default stream). */
int tpr_attn_fwd(const TprFwdParams* params, void* stream);

/* Enqueue the backward on `stream` (all phases, in order). */
int tpr_attn_bwd(const TprBwdParams* params, void* stream);

/* Backward phases, for callers that time them separately or run dK/dV and dQ
 * on two streams: TPR_BWD_DELTA must complete before the other two. Those are
 * independent of each other when the plan recomputes dQ; with a dS store
 * (see TprTreeDesc.flags) TPR_BWD_DQ reads what TPR_BWD_DKDV (its tiles step)
 * wrote, so it must run after it. tpr_attn_bwd == all three in this order.
 * TPR_BWD_DKDV is the two steps TPR_BWD_DKDV_TILES then TPR_BWD_DKDV_REDUCE,
 * which may also be enqueued separately (in that order, same workspace). */
#define TPR_BWD_DELTA 1        /* delta = rowsum(dout * out), fp32 [Hq, Tq] */
#define TPR_BWD_DKDV 2         /* dk, dv, dprefix_k, dprefix_v */
#define TPR_BWD_DQ 4           /* dq */
#define TPR_BWD_DKDV_TILES 8   /* dK/dV tiles; split prefix tiles leave fp32 partials in the workspace */
#define TPR_BWD_DKDV_REDUCE 16 /* ordered sum of those partials into dprefix_k / dprefix_v */
int tpr_attn_bwd_phases(const TprBwdParams* params, int phases, void* stream);

/* Allocation-free backward. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). Same as tpr_attn_bwd, except
 * that params->workspace / workspace_bytes are ignored: the workspace is the
 * library's static device scratch array, one per GPU, of
 * tpr_attn_bwd_noalloc_max_workspace_bytes() bytes (64 MiB), held from the
 * library's first use on a GPU until the process ends. A plan whose
 * tpr_attn_bwd_workspace_bytes() exceeds that is rejected with
 * TPR_ERR_UNSUPPORTED. The call allocates and frees nothing; the scratch
 * address is looked up once per device (with that device current) on the
 * first call there, which must not be under stream capture (a capturing
 * first call is refused with TPR_ERR_INVALID_ARGUMENT): make one call per
 * device before capturing it into a graph. Every call on one GPU shares that GPU's scratch: calls
 * that overlap on one GPU (two streams, two threads) race and must be
 * serialised by the caller. Nothing in the scratch needs to start at zero:
 * each call writes every workspace element it later reads. */
int tpr_attn_bwd_noalloc(const TprBwdParams* params, void* stream);

/* Bytes of static scratch tpr_attn_bwd_noalloc has per GPU. */
size_t tpr_attn_bwd_noalloc_max_workspace_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* TPR_ATTN_H */
