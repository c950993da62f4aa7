// Host check of the grouped-copy lane offsets (bridge_amd/csrc/tpr_lanes.h),
// built and run by tests/test_dma_lanes.py with g++: the functions the
// kernels compute their copy offsets with, evaluated for every lane and
// wave. Arguments: the row strides in bytes of the tiles the kernels copy
// with grouped copies (packed K/V rows Hkv * 256 and packed Q/dO rows
// Hq * 256 of every plan the caller lists). Prints the number of checks and
// "ok"; exits 1 at the first violation. "--clamped LEN STRIDE" checks the
// offsets of a partial tile instead.
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "tpr_lanes.h"

using namespace tpr;

static int fail(const char* what, int a, int b, int c, long long v) {
  std::printf("FAIL %s (%d, %d, %d): %lld\n", what, a, b, c, v);
  return 1;
}

// A tile of `len` < 64 rows whose rows at or beyond len re-read row len - 1
// (the partial tiles, which the kernels copy with dma_blocks4_m0): the
// offsets that dma_blocks4 would be given for it, checked the same way.
static int check_clamped(int len, unsigned rb) {
  for (int w = 0; w < 4; w++)
    for (int l = 0; l < 64; l++)
      for (int j = 0; j < 4; j++) {
        const int row = tile4_row(w, l, j) < len ? tile4_row(w, l, j) : len - 1;
        const unsigned v = static_cast<unsigned>(row) * rb + tile4_chunk_bytes(l, j);
        if (!blocks4_lane_ok(v, j)) return fail("clamped tile wraps", w, l, j, static_cast<long long>(v) - 1024 * j);
      }
  std::printf("ok\n");
  return 0;
}

int main(int argc, char** argv) {
  if (argc == 4 && std::string(argv[1]) == "--clamped")
    return check_clamped(std::atoi(argv[2]), static_cast<unsigned>(std::strtoul(argv[3], nullptr, 10)));
  std::vector<unsigned> strides;
  for (int i = 1; i < argc; i++) strides.push_back(static_cast<unsigned>(std::strtoul(argv[i], nullptr, 10)));
  long long checks = 0;
  // full 64-row tiles (dK/dV Q/dO stages, recomputing dQ K/V tiles): every
  // block's register v_j - 1024 j does not wrap; the lane reads 16 bytes of
  // its row's first 256; rows 0..63 each once per chunk; both forms agree
  for (unsigned rb : strides) {
    if (rb < 256 || rb % 16) return fail("row stride", static_cast<int>(rb), 0, 0, rb);
    std::vector<int> seen(64 * 16, 0);
    for (int w = 0; w < 4; w++)
      for (int l = 0; l < 64; l++)
        for (int j = 0; j < 4; j++) {
          const unsigned v = tile4_lane_bytes(w, l, rb, j);
          if (v != tile4_lane_bytes_swz(w, l, rb, j)) return fail("tile4 forms differ", w, l, j, v);
          if (!blocks4_lane_ok(v, j)) return fail("tile4 wraps", w, l, j, static_cast<long long>(v) - 1024 * j);
          const int row = tile4_row(w, l, j);
          const unsigned chunk = tile4_chunk_bytes(l, j);
          if (row < 0 || row >= 64 || chunk + 16 > 256 || v != row * rb + chunk)
            return fail("tile4 bounds", w, l, j, v);
          // the lane's 16 bytes land at LDS block (4 w + j), lane l: physical chunk l % 16 of the row
          if (swz_chunk(row, static_cast<int>(chunk / 16)) != (l & 15)) return fail("tile4 swizzle", w, l, j, chunk);
          seen[row * 16 + static_cast<int>(chunk / 16)]++;
          checks++;
        }
    for (int c : seen)
      if (c != 1) return fail("tile4 coverage", static_cast<int>(rb), c, 0, 0);
  }
  // dS blocks of the head_dim-128 dQ kernel: within the wave's 4 KiB of the
  // half, each 16-byte chunk once, no wrap, inside the head's 16 KiB
  {
    std::vector<int> seen(4096 / 16, 0);
    for (int l = 0; l < 64; l++)
      for (int j = 0; j < 4; j++) {
        const unsigned v = dqs_ds_lane_bytes(l, j);
        if (!blocks4_lane_ok(v, j)) return fail("dqs dS wraps", l, j, 0, static_cast<long long>(v) - 1024 * j);
        // block j covers 1 KiB of slot wave block j / 2 (4 KiB apart), quarter j % 2
        const unsigned rel = v - (j >> 1) * 4096u - (j & 1) * 1024u;
        if (rel >= 1024 || v + 16 + kDqsDsSpanBytes > 16384) return fail("dqs dS bounds", l, j, 0, v);
        seen[(j * 1024 + rel) / 16]++;
        checks++;
      }
    for (int c : seen)
      if (c != 1) return fail("dqs dS coverage", c, 0, 0, 0);
  }
  // dS blocks of the head_dim-256 dQ kernel: 1 KiB of each 2 KiB wave block
  {
    std::vector<int> seen(4096 / 16, 0);
    for (int l = 0; l < 64; l++)
      for (int j = 0; j < 4; j++) {
        const unsigned v = m16_dqs_ds_lane_bytes(l, j);
        if (!blocks4_lane_ok(v, j)) return fail("m16 dS wraps", l, j, 0, static_cast<long long>(v) - 1024 * j);
        const unsigned rel = v - 2048u * j;
        if (rel >= 1024 || v + 16 + 1024 > 8192) return fail("m16 dS bounds", l, j, 0, v);
        seen[(j * 1024 + rel) / 16]++;
        checks++;
      }
    for (int c : seen)
      if (c != 1) return fail("m16 dS coverage", c, 0, 0, 0);
  }
  std::printf("checks %lld\nok\n", checks);
  return 0;
}
