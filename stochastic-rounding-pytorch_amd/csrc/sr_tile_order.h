// sr_tile_order.h -- which tile each workgroup of a launch processes.
//
// Shared by the kernels and by the host code that sizes the grid, and plain
// C++ otherwise, so it also compiles on the host alone.
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

// Tile of workgroup b < padded_grid(tiles); values >= tiles mark padding.
SR_HOST_DEVICE inline uint32_t tile_of(uint32_t b, uint32_t tiles) {
  const uint32_t s = chunk_shift(tiles);
  const uint32_t k = b / kXcds, x = b % kXcds;
  return (((k >> s) * kXcds + x) << s) | (k & ((1u << s) - 1u));
}

}  // namespace sr
