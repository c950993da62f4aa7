// tpr_lanes.h -- per-lane byte offsets of the grouped global -> LDS copies,
// as plain integer functions: the kernels compute their copy offsets with
// them, and a host test (tests/test_dma_lanes.py) evaluates the same
// functions for every lane, wave and row stride.
//
// The grouped copy dma_blocks4 / dma_blocks4_nt (tpr_kernel_util.h) sets M0
// once and reaches blocks 1-3 through the instruction offset 1024 j, which
// applies to both the LDS and the global address; a lane's register then
// holds v_j - 1024 j, an unsigned 32-bit offset. Every lane must have
// v_j >= 1024 j (blocks4_lane_ok), or the register wraps to about 4 GB and
// the load reads far out of bounds. Tiles whose rows are clamped to a short
// tile's last row break that and use dma_blocks4_m0 (M0 stepped, offsets
// passed as they are).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define TPR_HD __host__ __device__ __forceinline__
#else
#define TPR_HD inline
#endif

namespace tpr {

// 16-byte chunk swizzle of a [rows][128 bf16] LDS tile (256 B rows):
// physical chunk = logical chunk ^ f(row), with f swapping the two 2-bit
// fields of row % 16. Rows r..r+15 at one logical chunk land in 16 distinct
// chunks (conflict-free ds_read_b128 over 16 lanes), and 4 consecutive rows
// (r % 4 == 0) x 4 consecutive chunks land in 16 distinct chunks
// (conflict-free ds_read_tr16_b64 over 32 lanes).
TPR_HD int swz_chunk(int row, int chunk) { return chunk ^ (((row & 3) << 2) | ((row >> 2) & 3)); }

// A 64-row x 256-byte tile copied by 4 waves, 4 x 1 KiB blocks each: lane l
// of wave w moves, in block j, row 16 w + 4 j + l / 16 and the source chunk
// that swizzles to physical chunk l % 16 (the swizzle is its own inverse):
// swz_chunk(row, l % 16), which for these rows is (l % 16) ^ ((l / 16) << 2)
// ^ j. The dK/dV kernel forms it the first way, the dQ kernel the second
// (each keeps the instructions it was tuned with); the host test checks that
// the two agree for every lane and wave.
TPR_HD int tile4_row(int wave, int lane, int j) { return 16 * wave + 4 * j + (lane >> 4); }
TPR_HD uint32_t tile4_chunk_bytes_swz(int wave, int lane, int j) {
  return static_cast<uint32_t>(swz_chunk(tile4_row(wave, lane, j), lane & 15)) * 16u;
}
TPR_HD uint32_t tile4_chunk_bytes(int lane, int j) {
  return static_cast<uint32_t>(16 * ((lane & 15) ^ ((lane >> 4) << 2))) ^ (16u * static_cast<uint32_t>(j));
}
// byte offset of that lane's 16 bytes in a full tile of `row_bytes`-byte rows
TPR_HD uint32_t tile4_lane_bytes_swz(int wave, int lane, uint32_t row_bytes, int j) {
  return static_cast<uint32_t>(tile4_row(wave, lane, j)) * row_bytes + tile4_chunk_bytes_swz(wave, lane, j);
}
TPR_HD uint32_t tile4_lane_bytes(int wave, int lane, uint32_t row_bytes, int j) {
  return (static_cast<uint32_t>(tile4_row(wave, lane, 0)) + 4u * static_cast<uint32_t>(j)) * row_bytes +
         tile4_chunk_bytes(lane, j);
}

// dS store, head_dim 128: one 32-query half of a dQ wave's 8 KiB block of a
// 64-key half is the slot's wave blocks kb = 0, 1 (4 KiB apart) x 16-query
// quarters qc = 0, 1 (1 KiB apart) of that 32-query half; copy block j =
// 2 kb + qc, and lane l fetches the chunk that lands at l after the swizzle
// l ^ (8 (l / 32) + 4 qc). The wave copies its two 32-query halves from
// sources 2 KiB apart.
TPR_HD uint32_t dqs_ds_lane_bytes(int lane, int j) {
  const int kb = j >> 1, qc = j & 1;
  return static_cast<uint32_t>(kb * 4096 + qc * 1024 + 16 * (lane ^ (8 * (lane >> 5) + 4 * qc)));
}
// the copies' sources lie at most 8 KiB (the second 64-key half) plus 2 KiB
// (the second 32-query half) into the slot's 16 KiB head block
constexpr int kDqsDsSpanBytes = 8192 + 2048;

// dS store, head_dim 256: a slot's 64-key tile of one head is four 2 KiB
// wave blocks (16 keys each); a dQ wave copies its 32-query half (1 KiB, at
// +1024 for the second half) of each, block j from wave block j, lane l
// fetching the chunk that lands at l ^ 4 ((l / 16) % 2).
TPR_HD uint32_t m16_dqs_ds_lane_bytes(int lane, int j) {
  return static_cast<uint32_t>(2048 * j + 16 * (lane ^ (4 * ((lane >> 4) & 1))));
}

// The register a grouped copy passes for block j: v_j - 1024 j, valid only
// when it does not wrap.
TPR_HD bool blocks4_lane_ok(uint32_t v, int j) { return v >= 1024u * static_cast<uint32_t>(j); }

}  // namespace tpr
