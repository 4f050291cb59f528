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
// surplus only adds contention.  The cap is round(budget / tile bytes), the
// budget being the bytes of tiles in flight per CU at which the rate peaked
// on MI355X.  Every cap exact, each launch family swept through the
// library's own launches (SR_STATES_RESIDENT_CAP, two runs per cap), TB/s
// uncapped -> at the cap:
//   AdamW, FP32 gradients: 80 KiB.  North star (FP32 p/g, BF16-SR m/v,
//     20 B) 6.22 -> 6.42 at 8; one 2^26-element tensor 6.46 -> 6.64 at 8;
//     E4M3-SR m + BF16-SR v (18 B) 6.22 -> 6.41 at 9; FP32 moments (28 B)
//     6.01 -> 6.23 at 6; BF16-, FP16- and FP8-nearest moments peak at 8,
//     8 and 10.
//   AdamW, BF16 gradients (GPT-2 shapes): 96 KiB.  BF16-SR m/v (18 B)
//     6.29 -> 6.36 at 11, 6.27 at 80 KiB's 9 (on another machine 6.34 at
//     9, 6.40 at 11); BF16-RN, FP16-RN and FP32 moments also peak at 11,
//     11 and 7.
//   AdamW whose two moments both round stochastically to FP16 or FP8 (two
//     minifloat encoders per element lengthen each workgroup's life): 96 KiB
//     with FP32 gradients (FP16-SR m/v 6.20 -> 6.32 at 10, E4M3-SR and
//     E5M2-SR 6.23 -> 6.28 at 12); with BF16 gradients none at all (FP16-SR
//     6.31 uncapped, 6.22 at 11; FP8-SR 6.36-6.39 uncapped, 5.97 at 12).
//   SGDM: 88 KiB (BF16-SR, BF16-RN and FP16-RN momentum, 16 B: 6.36-6.38 ->
//     6.47-6.49 at 11; FP32: 6.21 -> 6.43 at 9; FP8: best at 12-13), except
//     FP16-SR momentum at 72 KiB (6.35-6.38 -> 6.58-6.61 at 9, against
//     6.50-6.54 at 10 and 6.48 at 11, on three machines).
// Launches with BF16 parameters spend more of a workgroup's life in
// arithmetic; caps of 11 to 15 moved them by under 1%, so they stay
// uncapped, as do launches of fewer than 2^16 tiles (2^25 elements at 128
// lanes), whose tail the cap lengthens (2^24 elements: 6.50 -> 6.46;
// 2^25: 6.53 -> 6.62), and the casts (every cap slower).  A budget that
// rounds to more than kResidentCapMax workgroups also means no cap.
constexpr uint32_t kInFlightAdamW = 80u * 1024u;
constexpr uint32_t kInFlightAdamWWide = 96u * 1024u;
constexpr uint32_t kInFlightSgdm = 88u * 1024u;
constexpr uint32_t kInFlightSgdmF16Sr = 72u * 1024u;
constexpr uint32_t kResidentCapMinTiles = 1u << 16;
constexpr uint32_t kResidentCapMax = 14;

// In-flight budget of an AdamW launch with FP32 parameters, or 0 for no cap.
SR_HOST_DEVICE constexpr uint32_t adamw_in_flight(bool bf16_gradient, bool two_minifloat_sr) {
  return bf16_gradient ? (two_minifloat_sr ? 0u : kInFlightAdamWWide)
                       : (two_minifloat_sr ? kInFlightAdamWWide : kInFlightAdamW);
}

// In-flight budget of a momentum-SGD launch with FP32 parameters.
SR_HOST_DEVICE constexpr uint32_t sgdm_in_flight(bool f16_sr_momentum) {
  return f16_sr_momentum ? kInFlightSgdmF16Sr : kInFlightSgdm;
}

// Workgroups per CU to leave resident for an optimizer launch of `tiles`
// tiles of `block` lanes times `lanes` elements, moving `bytes_per_element`
// bytes per element with `in_flight` bytes of tiles in flight per CU, or 0
// for no cap (also for in_flight 0).
SR_HOST_DEVICE inline uint32_t resident_cap(uint32_t tiles, uint32_t block, uint32_t lanes,
                                            uint32_t bytes_per_element, bool fp32_params,
                                            uint32_t in_flight = kInFlightAdamW) {
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
