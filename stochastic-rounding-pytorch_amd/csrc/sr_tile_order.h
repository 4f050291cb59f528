// sr_tile_order.h -- which tile each workgroup of a launch processes.
//
// Shared by the kernels and by the host code that sizes the grid, and plain
// C++ otherwise, so it also compiles on the host alone.  It also holds the
// rule for how many workgroups of a large optimizer launch stay resident
// per CU (resident_cap, at the end).
//
// The dispatcher hands workgroup b to XCD (b mod 8).  Tiles are dealt to the
// XCDs in chunks of 2^s consecutive tiles: XCD x takes chunks x, x + 8,
// x + 16, ..., and its k-th workgroup takes tile (k mod 2^s) of its
// (k >> s)-th chunk.  The tiles in flight on one XCD therefore stay within a
// few neighbouring chunks, and the eight XCDs stream eight neighbouring
// chunks.  s is at most 9 (512-tile chunks) and small enough that 64 chunks
// fit in the launch, so padding the grid to a multiple of 8 chunks adds less
// than one eighth of it.  Measured on MI355X for the fused update's
// 12-byte-read / 8-byte-write pattern, 512-tile chunks beat both plain order
// and one contiguous eighth of the tiles per XCD.
#pragma once

#include <cstdint>

#if defined(__HIPCC__)
#define SR_HOST_DEVICE __host__ __device__
#else
#define SR_HOST_DEVICE
#endif

namespace sr {

constexpr uint32_t kXcds = 8;
constexpr uint32_t kMaxChunkShift = 9;

// log2 of the chunk size for a launch of `tiles` tiles.
SR_HOST_DEVICE inline uint32_t chunk_shift(uint32_t tiles) {
  const uint32_t chunks = tiles >> 6;
  if (chunks == 0) return 0;
  const uint32_t s = 31u - static_cast<uint32_t>(__builtin_clz(chunks));
  return s < kMaxChunkShift ? s : kMaxChunkShift;
}

// Workgroups launched for `tiles` tiles: a multiple of 8 chunks.
SR_HOST_DEVICE inline uint64_t padded_grid(uint32_t tiles) {
  const uint64_t unit = static_cast<uint64_t>(kXcds) << chunk_shift(tiles);
  return (static_cast<uint64_t>(tiles) + unit - 1) / unit * unit;
}

// Tile of workgroup b; values >= tiles mark padding.  The result is
// b - x + x * 2^s - 7 * (k mod 2^s), within 7 * 2^s of b, so it does not wrap
// for b < 2^32 - 3584; every b at or past padded_grid(tiles) maps to padding.
SR_HOST_DEVICE inline uint32_t tile_of(uint32_t b, uint32_t tiles) {
  const uint32_t s = chunk_shift(tiles);
  const uint32_t k = b / kXcds, x = b % kXcds;
  return (((k >> s) * kXcds + x) << s) | (k & ((1u << s) - 1u));
}

// A dispatch packet holds the grid size in work-items as a 32-bit number per
// dimension, so one dimension carries fewer than 2^32 work-items (HIP
// rejects larger launches).  Launches whose padded grid exceeds that are
// laid out as `y` rows of `x` workgroups; x is a whole number of chunk
// rounds (a multiple of 8 << chunk_shift), so workgroup b = y_index * x +
// x_index still runs on XCD b mod 8 and the tile order above is unchanged.
// Workgroups past padded_grid(tiles) map to padding.  `max_items` is the
// per-dimension work-item limit; tests pass smaller values.
struct LaunchShape {
  uint32_t x, y;
};

SR_HOST_DEVICE inline LaunchShape launch_shape(uint32_t tiles, uint32_t block,
                                               uint64_t max_items = 0xFFFFFFFFull) {
  const uint64_t grid = padded_grid(tiles);
  if (grid * block <= max_items) return {static_cast<uint32_t>(grid), 1u};
  const uint64_t unit = static_cast<uint64_t>(kXcds) << chunk_shift(tiles);
  uint64_t per_row = max_items / block / unit * unit;
  if (per_row == 0) per_row = unit;  // only for limits below one chunk round
  return {static_cast<uint32_t>(per_row), static_cast<uint32_t>((grid + per_row - 1) / per_row)};
}

// Resident workgroups per CU of a large optimizer launch.  The fused updates
// use few registers, so 16 of their 128-lane workgroups fit on a CU, and
// that many keep more memory requests in flight than HBM can serve: the
// surplus only adds contention.  Measured on MI355X (every cap exact,
// interleaved in one process, through the library's multi-tensor launches),
// the rate peaks with about 80 KiB of tiles in flight per CU, i.e. cap =
// round(80 KiB / tile bytes):
//   north star (FP32 p/g, BF16-SR m/v, 20 B):  6.21 -> 6.40 TB/s at 8
//   2^26-element tensor, same streams:           6.45 -> 6.71 at 8
//   E4M3-SR m + BF16-SR v (18 B): 6.20 -> 6.38 at 9
//   SGDM, FP16-SR momentum (16 B): 6.31 -> 6.44 at the rule's 10 (6.53 at 9)
//   FP32 moments (28 B): 6.03 -> 6.18-6.26 at the rule's 6 (6.24 at 7)
// AdamW launches whose two moments both round stochastically to FP16 or FP8
// spend longer in each workgroup's arithmetic (two minifloat encoders per
// element) and peak nearer 96 KiB: FP16-SR m/v (20 B) 6.18 -> 6.33 at 10
// (6.20 at 8), E4M3-SR m/v (16 B) 6.22 -> 6.35 at 12 (6.25 at 10), E5M2-SR
// m/v 6.28 -> 6.34 at 12 (6.22 at 10).
// Launches with BF16 parameters spend more of a workgroup's life in
// arithmetic; caps of 11 to 15 moved them by under 1%, so they stay
// uncapped, as do launches of fewer than 2^16 tiles (2^25 elements at 128
// lanes), whose tail the cap lengthens (2^24 elements: 6.50 -> 6.46;
// 2^25: 6.53 -> 6.62), and the casts (every cap slower).
constexpr uint32_t kInFlightBytesPerCu = 80u * 1024u;
constexpr uint32_t kInFlightBytesPerCuTwoMinifloatSr = 96u * 1024u;
constexpr uint32_t kResidentCapMinTiles = 1u << 16;
constexpr uint32_t kResidentCapMax = 12;

// Workgroups per CU to leave resident for an optimizer launch of `tiles`
// tiles of `block` lanes times `lanes` elements, moving `bytes_per_element`
// bytes per element with `in_flight` bytes of tiles in flight per CU, or 0
// for no cap.
SR_HOST_DEVICE inline uint32_t resident_cap(uint32_t tiles, uint32_t block, uint32_t lanes,
                                            uint32_t bytes_per_element, bool fp32_params,
                                            uint32_t in_flight = kInFlightBytesPerCu) {
  if (!fp32_params || tiles < kResidentCapMinTiles) return 0;
  const uint64_t tile_bytes = static_cast<uint64_t>(block) * lanes * bytes_per_element;
  if (tile_bytes == 0) return 0;
  const uint64_t cap = (in_flight + tile_bytes / 2) / tile_bytes;
  return cap >= 1 && cap <= kResidentCapMax ? static_cast<uint32_t>(cap) : 0u;
}

// The environment can replace the rule: SR_STATES_RESIDENT_CAP=k caps every
// optimizer launch of at least 2^16 tiles (any parameter dtype) at k
// workgroups per CU, 1 <= k <= kResidentCapOverrideMax, and 0 leaves them
// all uncapped.  For measuring the rule and for workloads whose best cap
// differs; results never depend on it.  resident_cap_override parses the
// variable's text: the override, or -1 for "use the rule" (unset, empty or
// not a number in range).
constexpr int kResidentCapOverrideMax = 16;

inline int resident_cap_override(const char* text) {
  if (text == nullptr || *text == '\0') return -1;
  int value = 0;
  for (const char* c = text; *c; ++c) {
    if (*c < '0' || *c > '9') return -1;
    value = value * 10 + (*c - '0');
    if (value > kResidentCapOverrideMax) return -1;
  }
  return value;
}

}  // namespace sr
