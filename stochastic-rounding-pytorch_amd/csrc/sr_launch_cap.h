// sr_launch_cap.h -- the dynamic LDS that caps resident workgroups per CU.
//
// Host code over the HIP runtime, shared by the library's launches and the
// bandwidth-ceiling helper so that both apply the same launch policy.  How
// many workgroups to leave resident is sr::resident_cap (sr_tile_order.h);
// this header turns a cap into the LDS reservation that enforces it.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>

#include "sr_tile_order.h"

namespace sr {

constexpr uint32_t kLdsPerCu = 160u * 1024u;  // gfx950
constexpr int kCapMaxBlock = 1024;
constexpr uint32_t kCapLdsMax = static_cast<uint32_t>(kResidentCapOverrideMax);

// Dynamic LDS per workgroup that leaves at most `cap` workgroups of `block`
// lanes resident per CU; 0 for cap 0.  The kernels it serves use no LDS, so
// the reservation only limits residency.  The allocation granularity is the
// hardware's, so the smallest such size (a multiple of 256 bytes) is found
// with the runtime's occupancy calculator, once per (block, cap): for every
// kernel without static LDS whose registers alone allow more than `cap`
// workgroups, the answer depends on the LDS alone and is shared.  A kernel
// whose registers already hold it to `cap` needs none (and the shared size
// changes nothing for it).  0 when the calculator fails: the launch then
// runs uncapped, and the failure is cleared from the runtime's last error so
// that no later, unrelated error check reports it.
inline size_t cap_lds(const void* fn, int block, uint32_t cap) {
  static std::atomic<uint32_t> known[kCapMaxBlock / 64][kCapLdsMax + 1];
  if (cap == 0 || cap > kCapLdsMax || block < 64 || block > kCapMaxBlock || block % 64) return 0;
  std::atomic<uint32_t>& slot = known[block / 64 - 1][cap];
  const uint32_t kept = slot.load(std::memory_order_relaxed);
  if (kept != 0) return static_cast<size_t>(kept - 1) * 256;
  auto resident_with = [&](size_t lds, int* resident) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(resident, fn, block, lds) == hipSuccess) return true;
    (void)hipGetLastError();
    return false;
  };
  int uncapped = 0;
  if (!resident_with(0, &uncapped) || uncapped <= static_cast<int>(cap)) return 0;
  uint32_t lo = 1, hi = kLdsPerCu / 256;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) / 2;
    int resident = 0;
    if (!resident_with(static_cast<size_t>(mid) * 256, &resident)) return 0;
    if (resident <= static_cast<int>(cap)) hi = mid;
    else lo = mid + 1;
  }
  slot.store(lo + 1, std::memory_order_relaxed);
  return static_cast<size_t>(lo) * 256;
}

}  // namespace sr
