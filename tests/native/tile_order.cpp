// Checks the workgroup -> tile order of the kernels (csrc/sr_tile_order.h) on
// the host: for every launch size tried, the workgroups of padded_grid(tiles)
// cover each tile in [0, tiles) exactly once, padding stays below one eighth
// of the grid (or one chunk round for small launches), and each XCD's
// workgroups walk whole chunks of 2^chunk_shift consecutive tiles.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "sr_tile_order.h"

int check(uint32_t tiles) {
  const uint64_t grid = sr::padded_grid(tiles);
  const uint32_t s = sr::chunk_shift(tiles);
  const uint64_t unit = static_cast<uint64_t>(sr::kXcds) << s;
  if (grid % unit != 0 || grid < tiles || grid - tiles >= unit) return 1;
  if (tiles >= 64 && (grid - tiles) * 8 > tiles) return 2;
  std::vector<uint8_t> seen(tiles, 0);
  for (uint64_t b = 0; b < grid; ++b) {
    const uint32_t t = sr::tile_of(static_cast<uint32_t>(b), tiles);
    if (t >= grid) return 3;
    if (t < tiles && seen[t]++) return 4;
    // Consecutive workgroups of one XCD stay in one chunk of 2^s tiles.
    const uint64_t k = b / sr::kXcds;
    if ((k & ((1u << s) - 1u)) != 0) {
      const uint32_t previous = sr::tile_of(static_cast<uint32_t>(b - sr::kXcds), tiles);
      if (t != previous + 1) return 5;
    }
  }
  for (uint32_t t = 0; t < tiles; ++t) {
    if (!seen[t]) return 6;
  }
  return 0;
}

int main() {
  int failures = 0;
  std::vector<uint32_t> sizes;
  for (uint32_t n = 1; n <= 5000; ++n) sizes.push_back(n);
  for (uint32_t n : {32767u, 32768u, 32769u, 65535u, 65536u, 121524u, 1000003u, 1511424u, 4871168u}) {
    sizes.push_back(n);
  }
  for (uint32_t n : sizes) {
    if (int rc = check(n)) {
      std::printf("tiles %u: failure %d\n", n, rc);
      ++failures;
    }
  }
  if (sr::chunk_shift(63) != 0 || sr::chunk_shift(64) != 0 || sr::chunk_shift(128) != 1 ||
      sr::chunk_shift(32767) != 8 || sr::chunk_shift(32768) != 9 || sr::chunk_shift(0xFFFFFFFFu) != 9) {
    std::printf("chunk_shift breakpoints moved\n");
    ++failures;
  }
  std::printf("%zu launch sizes, %d failures\n", sizes.size(), failures);
  return failures != 0;
}
