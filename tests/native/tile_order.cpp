// Checks the workgroup -> tile order of the kernels (csrc/sr_tile_order.h) on
// the host: for every launch size tried, the workgroups of padded_grid(tiles)
// cover each tile in [0, tiles) exactly once, padding stays below one eighth
// of the grid (or one chunk round for small launches), and each XCD's
// workgroups walk whole chunks of 2^chunk_shift consecutive tiles.  It also
// checks launch_shape: one row when the padded grid fits the per-dimension
// work-item limit, otherwise rows of whole chunk rounds whose workgroups,
// numbered row by row, still cover each tile exactly once.  Finally it pins
// resident_cap, the resident-workgroup cap of large optimizer launches, and
// resident_cap_override, the parse of its environment override.
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

// launch_shape under a per-dimension limit of `max_items` work-items.
int check_shape(uint32_t tiles, uint32_t block, uint64_t max_items, bool walk) {
  const sr::LaunchShape shape = sr::launch_shape(tiles, block, max_items);
  const uint64_t grid = sr::padded_grid(tiles);
  const uint64_t unit = static_cast<uint64_t>(sr::kXcds) << sr::chunk_shift(tiles);
  const uint64_t total = static_cast<uint64_t>(shape.x) * shape.y;
  if (grid * block <= max_items) return shape.x == grid && shape.y == 1 ? 0 : 11;
  if (static_cast<uint64_t>(shape.x) * block > max_items && shape.x != unit) return 12;
  if (shape.x % unit != 0 || shape.y < 2 || total < grid || total - grid >= shape.x) return 13;
  if (total + 3584 >= (1ull << 32)) return 14;
  if (!walk) {
    // Only the workgroups past the padded grid: all padding, none wrapped.
    for (uint64_t b = grid; b < total; ++b) {
      const uint32_t t = sr::tile_of(static_cast<uint32_t>(b), tiles);
      if (t < tiles || t + 3584ull < b) return 15;
    }
    return 0;
  }
  std::vector<uint8_t> seen(tiles, 0);
  for (uint64_t b = 0; b < total; ++b) {
    const uint32_t t = sr::tile_of(static_cast<uint32_t>(b), tiles);
    if (b >= grid && t < tiles) return 16;
    if (t < tiles && seen[t]++) return 17;
  }
  for (uint32_t t = 0; t < tiles; ++t) {
    if (!seen[t]) return 18;
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
  int shapes = 0;
  for (uint32_t tiles : {1u, 63u, 64u, 4095u, 4096u, 4097u, 32769u, 121524u, 1000003u}) {
    for (uint32_t block : {64u, 128u, 256u, 1024u}) {
      for (uint64_t limit : {1ull << 16, 1ull << 20, (1ull << 24) + 4096 * 64, 0xFFFFFFFFull}) {
        ++shapes;
        if (int rc = check_shape(tiles, block, limit, true)) {
          std::printf("tiles %u block %u limit %llu: failure %d\n", tiles, block, (unsigned long long)limit, rc);
          ++failures;
        }
      }
    }
  }
  // At the real limit: 2^34 + 2^20 elements in 512-element tiles (two rows),
  // and the largest tile count a launch accepts.
  struct Big { uint32_t tiles, block; bool walk; };
  for (const Big& big : {Big{33556480u, 128u, true}, Big{0x7FFFF000u, 1024u, false}, Big{0x7FFFF000u, 64u, false}}) {
    ++shapes;
    const sr::LaunchShape shape = sr::launch_shape(big.tiles, big.block);
    if (shape.y < 2) {
      std::printf("tiles %u block %u: expected several rows\n", big.tiles, big.block);
      ++failures;
    } else if (int rc = check_shape(big.tiles, big.block, 0xFFFFFFFFull, big.walk)) {
      std::printf("tiles %u block %u: failure %d\n", big.tiles, big.block, rc);
      ++failures;
    }
  }
  // resident_cap: round(in-flight bytes / tile bytes) for FP32-parameter
  // launches of at least 2^16 tiles, when that is 1..14; otherwise none (0).
  struct Cap { uint32_t tiles, block, bytes; bool fp32; uint32_t want; };
  for (const Cap& c : {Cap{3022848u, 128u, 20u, true, 8u},   // north star: 80 KiB / 10 KiB
                       Cap{65536u, 128u, 20u, true, 8u},     // smallest capped launch
                       Cap{65535u, 128u, 20u, true, 0u},     // one tile fewer
                       Cap{3022848u, 128u, 20u, false, 0u},  // BF16 parameters
                       Cap{3022848u, 128u, 18u, true, 9u},   // 8.89
                       Cap{3022848u, 128u, 16u, true, 10u},
                       Cap{3022848u, 128u, 28u, true, 6u},   // 5.71
                       Cap{3022848u, 128u, 24u, true, 7u},   // 6.67
                       Cap{3022848u, 128u, 14u, true, 11u},  // 11.43
                       Cap{3022848u, 128u, 13u, true, 12u},  // 12.31
                       Cap{3022848u, 128u, 12u, true, 13u},  // 13.33
                       Cap{3022848u, 128u, 11u, true, 0u},   // 14.55 rounds to 15: above the largest cap
                       Cap{3022848u, 256u, 20u, true, 4u},
                       Cap{3022848u, 1024u, 20u, true, 1u},
                       Cap{3022848u, 1024u, 40u, true, 1u},  // 0.5 rounds up
                       Cap{3022848u, 64u, 20u, true, 0u},    // 16
                       Cap{0xFFFFFFFFu, 128u, 20u, true, 8u}}) {
    const uint32_t got = sr::resident_cap(c.tiles, c.block, 4, c.bytes, c.fp32);
    if (got != c.want) {
      std::printf("resident_cap(%u, %u, 4, %u, %d) = %u, expected %u\n", c.tiles, c.block, c.bytes, c.fp32, got,
                  c.want);
      ++failures;
    }
  }
  // The budgets by launch family, and the caps they give at 128 lanes.
  if (sr::adamw_in_flight(false, false) != 80u * 1024u || sr::adamw_in_flight(false, true) != 96u * 1024u ||
      sr::adamw_in_flight(true, false) != 96u * 1024u || sr::adamw_in_flight(true, true) != 0u ||
      sr::sgdm_in_flight(false) != 88u * 1024u || sr::sgdm_in_flight(true) != 72u * 1024u) {
    std::printf("in-flight budgets differ from 80/96/96/0 and 88/72 KiB\n");
    ++failures;
  }
  struct Budget { uint32_t in_flight, bytes, want; };
  for (const Budget& c : {Budget{96u * 1024u, 20u, 10u},  // AdamW, two FP16-SR moments
                          Budget{96u * 1024u, 16u, 12u},  // two FP8-SR moments
                          Budget{96u * 1024u, 18u, 11u},  // BF16 gradient, BF16 moments (10.67)
                          Budget{96u * 1024u, 26u, 7u},   // BF16 gradient, FP32 moments (7.38)
                          Budget{96u * 1024u, 15u, 13u},  // 12.8
                          Budget{96u * 1024u, 14u, 14u},  // 13.71
                          Budget{96u * 1024u, 13u, 0u},   // 14.77 rounds to 15
                          Budget{0u, 18u, 0u},            // no budget: no cap
                          Budget{88u * 1024u, 16u, 11u},  // SGDM, 2-byte momentum
                          Budget{88u * 1024u, 20u, 9u},   // SGDM, FP32 momentum (8.8)
                          Budget{88u * 1024u, 14u, 13u},  // SGDM, FP8 momentum (12.57)
                          Budget{72u * 1024u, 16u, 9u}}) {  // SGDM, FP16-SR momentum
    const uint32_t got = sr::resident_cap(3022848u, 128u, 4, c.bytes, true, c.in_flight);
    if (got != c.want) {
      std::printf("resident_cap(%u B in flight, %u B) = %u, expected %u\n", c.in_flight, c.bytes, got, c.want);
      ++failures;
    }
  }
  // resident_cap_override: the text of SR_STATES_RESIDENT_CAP, -1 = the rule.
  struct Override { const char* text; int want; };
  for (const Override& c : {Override{nullptr, -1}, Override{"", -1}, Override{"0", 0}, Override{"8", 8},
                            Override{"16", 16}, Override{"017", -1}, Override{"17", -1}, Override{"-1", -1},
                            Override{"8 ", -1}, Override{"x", -1}, Override{"99999999999", -1}}) {
    const int got = sr::resident_cap_override(c.text);
    if (got != c.want) {
      std::printf("resident_cap_override(%s) = %d, expected %d\n", c.text ? c.text : "null", got, c.want);
      ++failures;
    }
  }
  std::printf("%zu launch sizes, %d launch shapes, %d failures\n", sizes.size(), shapes, failures);
  return failures != 0;
}
