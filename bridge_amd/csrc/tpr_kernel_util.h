// tpr_kernel_util.h -- device helpers shared by the bf16 MFMA kernel families
// (tpr_mfma.hip: head_dim 128; tpr_mfma16.hip: head_dim 64 and 256): the
// forward / dQ key stream (ancestor key runs + causal suffix, in 64-row
// tiles), the global -> LDS DMA copy helpers and small compile-time tools.
#pragma once

#include <type_traits>
#include <utility>

#include "tpr_device.h"

namespace tpr {
namespace {

constexpr int kTileRows = 64;  // rows per staged K/V/Q/dO tile

// Key stream of a forward/dQ workgroup: the leaf's ancestor key runs (fully
// visible; the plan's run table) and its own suffix (right-down causal), cut
// into 64-row tiles. SegTable holds up to kMfmaRegRuns runs, read from the
// plan once, before the tile loop, in (uniform) registers; RunList serves
// launches whose longest run list is longer, and reads a run's (row, len)
// from the plan when the cursor enters it.
struct SegTable {
  int row[kMfmaRegRuns];    // first row of run e in prefix_k/v
  int len[kMfmaRegRuns];    // rows of run e (0 past the leaf's runs)
  int suffix_row;           // first row of the leaf in k/v
  int suffix_keys;          // suffix keys the workgroup needs
  int ntiles;
};

struct RunList {
  const int32_t* runs;      // the leaf's [max_runs][2] = {row, len}; len 0 past its runs
  int nruns;
  int suffix_row;
  int suffix_keys;
  int ntiles;
};

struct TileLoc {
  int64_t row;   // absolute row in prefix_k/v (prefix) or k/v (suffix)
  int len;       // valid rows in this tile (<= 64)
  int pos0;      // position of the first key within its segment
  bool suffix;
};

__device__ __forceinline__ SegTable load_segments(const KernelArgs& a, int leaf, int suffix_keys) {
  const int32_t* runs = a.plan + a.off_runs + 2 * leaf * a.max_runs;
  SegTable t;
  int tiles = 0;
#pragma unroll
  for (int e = 0; e < kMfmaRegRuns; e++) {
    const bool have = e < a.max_runs;
    const int r = have ? runs[2 * e] : 0;
    const int l = have ? runs[2 * e + 1] : 0;
    t.row[e] = r;
    t.len[e] = l;
    tiles += (l + kTileRows - 1) / kTileRows;
  }
  t.suffix_row = a.plan[a.off_cu + leaf];
  t.suffix_keys = suffix_keys;
  t.ntiles = tiles + (suffix_keys + kTileRows - 1) / kTileRows;
  return t;
}

__device__ __forceinline__ RunList load_runs(const KernelArgs& a, int leaf, int suffix_keys) {
  RunList t;
  t.runs = a.plan + a.off_runs + 2 * leaf * a.max_runs;
  int n = 0, tiles = 0;
  for (; n < a.max_runs; n++) {
    const int l = t.runs[2 * n + 1];
    if (l == 0) break;  // runs are non-empty; {0, 0} pads the list
    tiles += (l + kTileRows - 1) / kTileRows;
  }
  t.nruns = n;
  t.suffix_row = a.plan[a.off_cu + leaf];
  t.suffix_keys = suffix_keys;
  t.ntiles = tiles + (suffix_keys + kTileRows - 1) / kTileRows;
  return t;
}

template <bool kRunList>
__device__ __forceinline__ auto load_keys(const KernelArgs& a, int leaf, int suffix_keys) {
  if constexpr (kRunList) return load_runs(a, leaf, suffix_keys);
  else return load_segments(a, leaf, suffix_keys);
}

__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(p)));
}

// One dword per lane, lane l's landing at lds_dst + 4*l (global_load_lds_dword).
__device__ __forceinline__ void dma4(const void* src, uint32_t lds_dst) {
  lds_dst = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_dst)));
  __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(uintptr_t)lds_dst, 4, 0, 0);
}

// Direct global -> LDS copy (gfx950 global_load_lds_dwordx4) of one 1 KiB
// block of a swizzled 64 x 256 B tile: lane l of the block lands at
// lds_dst + 16 l, i.e. at (row 4 blk + l/16, physical chunk l%16), so the
// lane fetches the logical chunk that swizzles there. No registers hold the
// data, and the wave's vmcnt covers the copy. The source is a uniform 64-bit
// base (SGPRs) plus a per-lane 32-bit byte offset, so the tile loop does no
// 64-bit address arithmetic.
// The copy is issued from inline asm (M0 = wave-uniform LDS destination,
// restored afterwards): the compiler does not track it, so it does not
// serialise the next tile's copy against the current tile's LDS reads;
// wait_dma() before the barrier that publishes the tile is the only wait it
// needs. vmcnt retires in order, so the compiler's own waits on its loads
// stay correct (they can only become stricter). The asm needs no memory
// clobber: the kernel never writes the global data it reads, and the LDS it
// writes is read only after wait_dma() and a barrier.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_dst) {
  // readfirstlane returns a signed int: go through uint32_t, or the low word
  // would be sign-extended into the high word of the address.
  const uint64_t b = reinterpret_cast<uint64_t>(sbase);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xffffffffu)));
  const uint64_t bs = (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo);
  sbase = reinterpret_cast<const void*>(bs);
  lds_dst = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_dst)));
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(sbase), "s"(lds_dst));
}

// The same copy through the compiler's builtin, which manages M0 itself (no
// save/restore around every copy); its placement is left to the scheduler.
__device__ __forceinline__ void dma16sb(const void* sbase, uint32_t voff, uint32_t lds_dst) {
  const uint64_t b = reinterpret_cast<uint64_t>(sbase);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xffffffffu)));
  const char* bs = reinterpret_cast<const char*>((static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo));
  lds_dst = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(lds_dst)));
  __builtin_amdgcn_global_load_lds(bs + voff, (__attribute__((address_space(3))) void*)(uintptr_t)lds_dst, 16, 0, 0);
}

// Four 1 KiB global -> LDS copies (global_load_lds_dwordx4) of one wave, block
// j landing at lds_dst + 1024 j from the uniform base `sbase` (SGPRs) plus the
// lane's 32-bit offset vj, with M0 saved and restored once around the group.
// Like dma16s, the compiler does not track these loads; the wait_dma()
// before the barrier that publishes the tile is their only wait.
//
// dma_blocks4 writes M0 once: blocks 1-3 use the instruction offset (1024 j),
// which applies to both the LDS and the global address, so their lane offsets
// are passed as vj - 1024 j. That needs vj >= 1024 j in every lane (the
// offset is an unsigned 32-bit VGPR): true for a full tile, whose block j
// starts at row 4 j of rows of at least 256 bytes; NOT for a tile whose rows
// are clamped to a short tile's last row -- those use dma_blocks4_m0, which
// steps M0 between the blocks instead.
__device__ __forceinline__ void dma_blocks4(const char* sbase, uint32_t v0, uint32_t v1, uint32_t v2, uint32_t v3,
                                            uint32_t lds_dst) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %5\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %6\n\t"
      "global_load_lds_dwordx4 %2, %6 offset:1024\n\t"
      "global_load_lds_dwordx4 %3, %6 offset:2048\n\t"
      "global_load_lds_dwordx4 %4, %6 offset:3072\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(v0), "v"(v1 - 1024u), "v"(v2 - 2048u), "v"(v3 - 3072u), "s"(lds_dst), "s"(sbase));
}

// dma_blocks4 with the streaming (nt) hint, for data read once: it keeps
// the last-level cache for the data that is read again.
__device__ __forceinline__ void dma_blocks4_nt(const char* sbase, uint32_t v0, uint32_t v1, uint32_t v2, uint32_t v3,
                                               uint32_t lds_dst) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %5\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %6 nt\n\t"
      "global_load_lds_dwordx4 %2, %6 offset:1024 nt\n\t"
      "global_load_lds_dwordx4 %3, %6 offset:2048 nt\n\t"
      "global_load_lds_dwordx4 %4, %6 offset:3072 nt\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(v0), "v"(v1 - 1024u), "v"(v2 - 2048u), "v"(v3 - 3072u), "s"(lds_dst), "s"(sbase));
}

__device__ __forceinline__ void dma_blocks4_m0(const char* sbase, uint32_t v0, uint32_t v1, uint32_t v2, uint32_t v3,
                                               uint32_t lds_dst) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %5\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %6\n\t"
      "s_add_u32 m0, m0, 0x400\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %2, %6\n\t"
      "s_add_u32 m0, m0, 0x400\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %3, %6\n\t"
      "s_add_u32 m0, m0, 0x400\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %4, %6\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(v0), "v"(v1), "v"(v2), "v"(v3), "s"(lds_dst), "s"(sbase)
      : "scc");  // s_add_u32 sets SCC
}

// One dword per lane from a per-lane address, landing at lds_dst + 4 l
// (global_load_lds_dword), untracked by the compiler like dma_blocks4.
__device__ __forceinline__ void dma4_lane(const float* src, uint32_t lds_dst) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dword %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(src), "s"(lds_dst));
}

// Cursor over a forward / dQ workgroup's key stream: the leaf's own suffix
// first, then its ancestor nodes (root first). Reading the shared prefix
// last in every workgroup leaves it the most recently used data in the XCD's
// L2 when the next workgroups (other query blocks and siblings of the same
// KV head) start on their suffix, so their suffix tiles evict older suffix
// lines rather than the prefix. The rows a workgroup reads or writes once
// (Q, dO, O, dQ) go through non-temporal loads and stores for the same
// reason. It only changes segment at segment ends, so the common step is a
// compare.
struct Cursor {
  int d;     // position in the stream: 0 = suffix, 1 + e = ancestor node e
  int lt;    // tile within the segment
  int row;   // first row of the segment
  int len;   // rows of the segment (0 past the stream's end)
};

__device__ __forceinline__ void cursor_load(const SegTable& t, Cursor& c) {
  int row = t.suffix_row, len = c.d == 0 ? t.suffix_keys : 0;
#pragma unroll
  for (int e = 0; e < kMfmaRegRuns; e++) {
    row = c.d == e + 1 ? t.row[e] : row;
    len = c.d == e + 1 ? t.len[e] : len;
  }
  c.row = row;
  c.len = len;
}

// Reads run c.d - 1 of the plan only when it is one of the leaf's runs.
__device__ __forceinline__ void cursor_load(const RunList& t, Cursor& c) {
  int row = t.suffix_row, len = c.d == 0 ? t.suffix_keys : 0;
  if (c.d > 0 && c.d <= t.nruns) {
    row = t.runs[2 * (c.d - 1)];
    len = t.runs[2 * (c.d - 1) + 1];
  }
  c.row = row;
  c.len = len;
}

template <typename Keys>
__device__ __forceinline__ Cursor cursor_begin(const Keys& t) {
  Cursor c{0, 0, 0, 0};  // the suffix holds at least one key
  cursor_load(t, c);
  return c;
}

// Past the last run the cursor stays at an empty segment (len 0).
template <typename Keys>
__device__ __forceinline__ void cursor_next(const Keys& t, Cursor& c) {
  c.lt++;
  if (c.lt * kTileRows >= c.len) {
    c.lt = 0;
    do {
      c.d++;
      cursor_load(t, c);
    } while (c.len == 0 && c.d < kMfmaRegRuns);
  }
}

__device__ __forceinline__ TileLoc cursor_tile(const Cursor& c) {
  return TileLoc{static_cast<int64_t>(c.row) + c.lt * kTileRows, min(kTileRows, c.len - c.lt * kTileRows),
                 c.lt * kTileRows, c.d == 0};
}

// The same key stream as Cursor, carrying the current tile's K and V source
// addresses: the step inside a segment is a few scalar adds (no 64-bit
// multiply per tile), and only a segment change reads the key table. A
// cursor whose addresses are never read (a mask cursor) compiles to its
// position fields alone.
struct KvSources {
  const char* k;   // suffix K / V of the workgroup's KV head (row 0)
  const char* v;
  const char* pk;  // prefix K / V of the KV head (row 0)
  const char* pv;
  uint32_t k_rb, v_rb, p_rb;  // row bytes of k, v and the packed prefix
};

struct KvCursor {
  const char* k;   // K rows of the current tile (uniform)
  const char* v;   // V rows of the current tile
  int64_t kstep, vstep;  // bytes of one tile of the current segment
  uint32_t krb, vrb;     // row bytes of the current segment
  int rem;         // rows of the segment from the current tile on (0 past the stream's end)
  int pos0;        // position of the tile's first key within its segment
  int d;           // 0 = suffix, 1 + e = key run e
};

template <typename Keys>
__device__ __forceinline__ void kv_enter(const Keys& t, const KvSources& s, KvCursor& c) {
  Cursor seg{c.d, 0, 0, 0};
  cursor_load(t, seg);
  const bool suffix = c.d == 0;
  c.krb = suffix ? s.k_rb : s.p_rb;
  c.vrb = suffix ? s.v_rb : s.p_rb;
  c.kstep = static_cast<int64_t>(c.krb) * kTileRows;
  c.vstep = static_cast<int64_t>(c.vrb) * kTileRows;
  c.k = (suffix ? s.k : s.pk) + static_cast<int64_t>(seg.row) * c.krb;
  c.v = (suffix ? s.v : s.pv) + static_cast<int64_t>(seg.row) * c.vrb;
  c.rem = seg.len;
  c.pos0 = 0;
}

template <typename Keys>
__device__ __forceinline__ KvCursor kv_begin(const Keys& t, const KvSources& s) {
  KvCursor c;
  c.d = 0;  // the suffix holds at least one key
  kv_enter(t, s, c);
  return c;
}

// Past the last run the cursor stays at an empty segment (rem 0).
template <typename Keys>
__device__ __forceinline__ void kv_next(const Keys& t, const KvSources& s, KvCursor& c) {
  c.rem -= kTileRows;
  c.pos0 += kTileRows;
  c.k += c.kstep;
  c.v += c.vstep;
  if (c.rem <= 0) {
    do {
      c.d++;
      kv_enter(t, s, c);
    } while (c.rem == 0 && c.d < kMfmaRegRuns);
  }
}

__device__ __forceinline__ int kv_len(const KvCursor& c) { return min(kTileRows, c.rem); }

// A plan word read through the scalar cache (s_load_dword) at a uniform
// address, waited for here. The compiler reads plan words it cannot prove
// unclobbered with vector loads, and its vmcnt(0) wait for one of those also
// drains every global->LDS copy in flight; a scalar load is counted by
// lgkmcnt instead.
__device__ __forceinline__ int plan_word(const int32_t* p) {
  const uint64_t b = reinterpret_cast<uint64_t>(p);
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b >> 32)));
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(b & 0xffffffffu)));
  const uint64_t bs = (static_cast<uint64_t>(hi) << 32) | static_cast<uint64_t>(lo);
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(bs));
  return v;
}

// Wait until this wave's outstanding global->LDS copies have landed.
// Ordered before the __syncthreads() that follows it (both have side effects);
// the barrier is what orders the LDS reads of the copied tile.
__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)"); }


__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Make the compiler complete the load of `x` here. Operands loaded before a
// tile loop are waited for once, before it, instead of at their first use
// inside it -- a wait there would also drain the in-flight tile copies.
template <typename T>
__device__ __forceinline__ void settle(const T& x) {
  asm volatile("" ::"v"(x));
}
// Keep `x` in accumulation registers (AGPRs) at this point. Used on the
// dK/dV accumulators at the end of each stage so that every path through the
// stage hands them over in the registers the MFMAs write, instead of the
// allocator parking them in VGPRs and copying them back each stage.
template <typename T>
__device__ __forceinline__ void settle_acc(T& x) {
  asm volatile("" : "+a"(x));
}
// Make `x` final here: its computation stays before this point (it cannot be
// sunk into a later block, e.g. past a workgroup barrier, towards its use).
template <typename T>
__device__ __forceinline__ void pin(T& x) {
  asm volatile("" : "+v"(x));
}


// Calls f(std::integral_constant<int, i>) for i = 0 .. N-1, unrolled at
// compile time (array indices derived from i are constants).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace
}  // namespace tpr
