// sr_kernels.h -- gfx950 kernels of the stochastic-rounding optimizer path.
//
// All kernels are persistent grid-stride loops over tiles of
// blockDim.x * SR_ELEMENTS_PER_THREAD elements.  A thread owns 8 consecutive
// elements of a tile, so FP32 operands move as two 128-bit accesses, 16-bit
// states as one 128-bit access and 8-bit states as one 64-bit access.  Rows
// whose pointers are not all 16-byte aligned, and the partial last tile of a
// row, take a coalesced scalar path (element k*blockDim.x + tid of the tile).
//
// Multi-tensor launches read a table of sr_row records.  Each workgroup
// stages the rows' tile ends in LDS once, then finds the row of each tile by
// binary search starting from the previous row (tiles arrive in increasing
// order), and loads the row record through the scalar path only when the row
// changes.  The random stream of an element depends only on its row's key,
// its shard start and its index, never on the launch shape.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/sr_states_hip.h"
#include "sr_math.h"

namespace sr {

constexpr int kVec = SR_ELEMENTS_PER_THREAD;
static_assert(kVec == 8, "the vector paths below move 8 elements per thread");
constexpr int kMaxBlock = 1024;
// Rows staged per launch (4 bytes of LDS each).  Hosts split larger buckets.
constexpr int kMaxRows = 4096;

struct AdamWArgs {
  const sr_row* rows;  // device table; nullptr selects `inline_row`
  sr_row inline_row;
  AdamWScalars s;
  uint32_t nrows;
  uint32_t total_tiles;
  uint32_t seed_lo, seed_hi, step_lo, step_hi;
};

struct SgdmArgs {
  const sr_row* rows;
  sr_row inline_row;
  SgdmScalars s;
  uint32_t nrows;
  uint32_t total_tiles;
  uint32_t seed_lo, seed_hi, step_lo, step_hi;
};

struct CastArgs {
  const float* x;
  void* y;
  int64_t n;
  uint32_t counter_base;  // seed + offset (mod 2^32)
  uint32_t total_tiles;
  uint32_t vector_ok;     // x and y 16-byte aligned
};

// ---------------------------------------------------------------------------
// Element I/O.  Raw storage words are zero-extended into 32-bit lanes.  The
// table holds plain integers, so pointers are cast to the global address
// space explicitly; otherwise every access would be a flat access.
// ---------------------------------------------------------------------------
#if defined(__HIP_DEVICE_COMPILE__)
#define SR_GLOBAL __attribute__((address_space(1)))
#else
#define SR_GLOBAL
#endif

template <class T>
__device__ __forceinline__ const SR_GLOBAL T* gptr(const void* p) {
  return (const SR_GLOBAL T*)(p);
}
template <class T>
__device__ __forceinline__ SR_GLOBAL T* gptr_mut(void* p) {
  return (SR_GLOBAL T*)(p);
}

template <int ENC>
__device__ __forceinline__ void load8(const void* base, int64_t i, uint32_t (&raw)[kVec]) {
  constexpr int W = enc_bytes(ENC);
  const char* ptr = static_cast<const char*>(base) + i * W;
  if constexpr (W == 4) {
    const uint4 a = *gptr<uint4>(ptr);
    const uint4 b = *gptr<uint4>(ptr + 16);
    raw[0] = a.x; raw[1] = a.y; raw[2] = a.z; raw[3] = a.w;
    raw[4] = b.x; raw[5] = b.y; raw[6] = b.z; raw[7] = b.w;
  } else if constexpr (W == 2) {
    const uint4 a = *gptr<uint4>(ptr);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      raw[2 * k] = w[k] & 0xFFFFu;
      raw[2 * k + 1] = w[k] >> 16;
    }
  } else {
    const uint2 a = *gptr<uint2>(ptr);
    const uint32_t w[2] = {a.x, a.y};
#pragma unroll
    for (int k = 0; k < 2; ++k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) raw[4 * k + j] = (w[k] >> (8 * j)) & 0xFFu;
    }
  }
}

template <int ENC>
__device__ __forceinline__ void store8(void* base, int64_t i, const uint32_t (&raw)[kVec]) {
  constexpr int W = enc_bytes(ENC);
  char* ptr = static_cast<char*>(base) + i * W;
  if constexpr (W == 4) {
    *gptr_mut<uint4>(ptr) = make_uint4(raw[0], raw[1], raw[2], raw[3]);
    *gptr_mut<uint4>(ptr + 16) = make_uint4(raw[4], raw[5], raw[6], raw[7]);
  } else if constexpr (W == 2) {
    *gptr_mut<uint4>(ptr) =
        make_uint4(raw[0] | (raw[1] << 16), raw[2] | (raw[3] << 16), raw[4] | (raw[5] << 16),
                   raw[6] | (raw[7] << 16));
  } else {
    *gptr_mut<uint2>(ptr) =
        make_uint2(raw[0] | (raw[1] << 8) | (raw[2] << 16) | (raw[3] << 24),
                   raw[4] | (raw[5] << 8) | (raw[6] << 16) | (raw[7] << 24));
  }
}

template <int ENC>
__device__ __forceinline__ uint32_t load1(const void* base, int64_t i) {
  constexpr int W = enc_bytes(ENC);
  if constexpr (W == 4) return gptr<uint32_t>(base)[i];
  else if constexpr (W == 2) return gptr<uint16_t>(base)[i];
  else return gptr<uint8_t>(base)[i];
}

template <int ENC>
__device__ __forceinline__ void store1(void* base, int64_t i, uint32_t v) {
  constexpr int W = enc_bytes(ENC);
  if constexpr (W == 4) gptr_mut<uint32_t>(base)[i] = v;
  else if constexpr (W == 2) gptr_mut<uint16_t>(base)[i] = static_cast<uint16_t>(v);
  else gptr_mut<uint8_t>(base)[i] = static_cast<uint8_t>(v);
}

__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

// ---------------------------------------------------------------------------
// Row walking shared by the optimizer kernels.
// ---------------------------------------------------------------------------
struct RowCursor {
  uint32_t index;     // row of the current tile
  uint32_t tile_end;  // one past the row's last tile
};

template <class Args>
__device__ __forceinline__ const sr_row& row_at(const Args& a, uint32_t r) {
  return a.rows ? a.rows[r] : a.inline_row;
}

// Stage every row's tile end in LDS (one 32-bit word per row).
template <class Args>
__device__ __forceinline__ void stage_tile_ends(const Args& a, uint32_t* s_end) {
  for (uint32_t r = threadIdx.x; r < a.nrows; r += blockDim.x) s_end[r] = row_at(a, r).tile_end;
  __syncthreads();
}

// Smallest row >= `from` whose tile range contains t.  s_end is increasing
// and its last entry is the launch's tile count, so the search terminates.
__device__ __forceinline__ uint32_t find_row(const uint32_t* s_end, uint32_t from, uint32_t nrows,
                                             uint32_t t) {
  uint32_t lo = from, hi = nrows - 1;
  while (lo < hi) {
    const uint32_t mid = (lo + hi) >> 1;
    if (uniform(s_end[mid]) > t) hi = mid;
    else lo = mid + 1;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// Fused AdamW.
// ---------------------------------------------------------------------------
template <int PE, int GE, int ME, int VE>
__device__ __forceinline__ void adamw_vector(char* p, const char* g, char* m, char* v, int64_t i,
                                             uint32_t cm, uint32_t cv, const AdamWScalars& s) {
  uint32_t rp[kVec], rg[kVec], rm[kVec], rv[kVec];
  load8<PE>(p, i, rp);
  load8<GE>(g, i, rg);
  load8<ME>(m, i, rm);
  load8<VE>(v, i, rv);
  const uint32_t base = static_cast<uint32_t>(i);
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    float po, mo, vo;
    adamw_update(decode<PE>(rp[k]), decode<GE>(rg[k]), decode<ME>(rm[k]), decode<VE>(rv[k]), s,
                 po, mo, vo);
    rp[k] = encode<PE>(po, 0);
    rm[k] = encode<ME>(mo, cm + base + k);
    rv[k] = encode<VE>(vo, cv + base + k);
  }
  store8<PE>(p, i, rp);
  store8<ME>(m, i, rm);
  store8<VE>(v, i, rv);
}

template <int PE, int GE, int ME, int VE>
__device__ __forceinline__ void adamw_scalar(char* p, const char* g, char* m, char* v, int64_t i,
                                             uint32_t cm, uint32_t cv, const AdamWScalars& s) {
  float po, mo, vo;
  adamw_update(decode<PE>(load1<PE>(p, i)), decode<GE>(load1<GE>(g, i)),
               decode<ME>(load1<ME>(m, i)), decode<VE>(load1<VE>(v, i)), s, po, mo, vo);
  const uint32_t base = static_cast<uint32_t>(i);
  store1<PE>(p, i, encode<PE>(po, 0));
  store1<ME>(m, i, encode<ME>(mo, cm + base));
  store1<VE>(v, i, encode<VE>(vo, cv + base));
}

template <int PE, int GE, int ME, int VE>
__global__ __launch_bounds__(kMaxBlock) void adamw_kernel(const AdamWArgs a) {
  extern __shared__ uint32_t s_end[];
  stage_tile_ends(a, s_end);
  const uint32_t tile = blockDim.x * kVec;
  RowCursor cur{0, 0};
  char *p = nullptr, *m = nullptr, *v = nullptr;
  const char* g = nullptr;
  int64_t numel = 0;
  uint32_t tile_begin = 0, vector_ok = 0, cm = 0, cv = 0;
  bool first = true;
  for (uint32_t t = blockIdx.x; t < a.total_tiles; t += gridDim.x) {
    if (first || t >= cur.tile_end) {
      cur.index = find_row(s_end, first ? 0u : cur.index + 1, a.nrows, t);
      first = false;
      const sr_row& r = row_at(a, cur.index);
      cur.tile_end = r.tile_end;
      tile_begin = r.tile_begin;
      numel = r.numel;
      vector_ok = r.flags & SR_ROW_VECTOR;
      p = reinterpret_cast<char*>(r.ptr[0]);
      g = reinterpret_cast<const char*>(r.ptr[1]);
      m = reinterpret_cast<char*>(r.ptr[2]);
      v = reinterpret_cast<char*>(r.ptr[3]);
      const uint32_t key = (r.flags & SR_ROW_KEYED)
                               ? r.param_index
                               : update_key(a.seed_lo, a.seed_hi, a.step_lo, a.step_hi, r.param_index);
      cm = state_key(key, 0) + r.shard_start;
      cv = state_key(key, 1) + r.shard_start;
    }
    const int64_t start = static_cast<int64_t>(t - tile_begin) * tile;
    if (vector_ok && start + tile <= numel) {
      adamw_vector<PE, GE, ME, VE>(p, g, m, v, start + static_cast<int64_t>(threadIdx.x) * kVec, cm,
                                   cv, a.s);
    } else {
#pragma unroll
      for (int k = 0; k < kVec; ++k) {
        const int64_t i = start + static_cast<int64_t>(k) * blockDim.x + threadIdx.x;
        if (i < numel) adamw_scalar<PE, GE, ME, VE>(p, g, m, v, i, cm, cv, a.s);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Fused momentum SGD.
// ---------------------------------------------------------------------------
template <int PE, int GE, int UE>
__device__ __forceinline__ void sgdm_vector(char* p, const char* g, char* u, int64_t i, uint32_t cu,
                                            const SgdmScalars& s) {
  uint32_t rp[kVec], rg[kVec], ru[kVec];
  load8<PE>(p, i, rp);
  load8<GE>(g, i, rg);
  load8<UE>(u, i, ru);
  const uint32_t base = static_cast<uint32_t>(i);
#pragma unroll
  for (int k = 0; k < kVec; ++k) {
    float po, uo;
    sgdm_update(decode<PE>(rp[k]), decode<GE>(rg[k]), decode<UE>(ru[k]), s, po, uo);
    rp[k] = encode<PE>(po, 0);
    ru[k] = encode<UE>(uo, cu + base + k);
  }
  store8<PE>(p, i, rp);
  store8<UE>(u, i, ru);
}

template <int PE, int GE, int UE>
__device__ __forceinline__ void sgdm_scalar(char* p, const char* g, char* u, int64_t i, uint32_t cu,
                                            const SgdmScalars& s) {
  float po, uo;
  sgdm_update(decode<PE>(load1<PE>(p, i)), decode<GE>(load1<GE>(g, i)), decode<UE>(load1<UE>(u, i)),
              s, po, uo);
  store1<PE>(p, i, encode<PE>(po, 0));
  store1<UE>(u, i, encode<UE>(uo, cu + static_cast<uint32_t>(i)));
}

template <int PE, int GE, int UE>
__global__ __launch_bounds__(kMaxBlock) void sgdm_kernel(const SgdmArgs a) {
  extern __shared__ uint32_t s_end[];
  stage_tile_ends(a, s_end);
  const uint32_t tile = blockDim.x * kVec;
  RowCursor cur{0, 0};
  char *p = nullptr, *u = nullptr;
  const char* g = nullptr;
  int64_t numel = 0;
  uint32_t tile_begin = 0, vector_ok = 0, cu = 0;
  bool first = true;
  for (uint32_t t = blockIdx.x; t < a.total_tiles; t += gridDim.x) {
    if (first || t >= cur.tile_end) {
      cur.index = find_row(s_end, first ? 0u : cur.index + 1, a.nrows, t);
      first = false;
      const sr_row& r = row_at(a, cur.index);
      cur.tile_end = r.tile_end;
      tile_begin = r.tile_begin;
      numel = r.numel;
      vector_ok = r.flags & SR_ROW_VECTOR;
      p = reinterpret_cast<char*>(r.ptr[0]);
      g = reinterpret_cast<const char*>(r.ptr[1]);
      u = reinterpret_cast<char*>(r.ptr[2]);
      const uint32_t key = (r.flags & SR_ROW_KEYED)
                               ? r.param_index
                               : update_key(a.seed_lo, a.seed_hi, a.step_lo, a.step_hi, r.param_index);
      cu = state_key(key, 0) + r.shard_start;
    }
    const int64_t start = static_cast<int64_t>(t - tile_begin) * tile;
    if (vector_ok && start + tile <= numel) {
      sgdm_vector<PE, GE, UE>(p, g, u, start + static_cast<int64_t>(threadIdx.x) * kVec, cu, a.s);
    } else {
#pragma unroll
      for (int k = 0; k < kVec; ++k) {
        const int64_t i = start + static_cast<int64_t>(k) * blockDim.x + threadIdx.x;
        if (i < numel) sgdm_scalar<PE, GE, UE>(p, g, u, i, cu, a.s);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Standalone cast: y = round(x), counter = index + seed + offset.
// ---------------------------------------------------------------------------
template <int ENC>
__global__ __launch_bounds__(kMaxBlock) void cast_kernel(const CastArgs a) {
  const uint32_t tile = blockDim.x * kVec;
  for (uint32_t t = blockIdx.x; t < a.total_tiles; t += gridDim.x) {
    const int64_t start = static_cast<int64_t>(t) * tile;
    if (a.vector_ok && start + tile <= a.n) {
      const int64_t i = start + static_cast<int64_t>(threadIdx.x) * kVec;
      uint32_t r[kVec];
      load8<ENC_F32>(a.x, i, r);
      const uint32_t base = a.counter_base + static_cast<uint32_t>(i);
#pragma unroll
      for (int k = 0; k < kVec; ++k) r[k] = encode<ENC>(bits_f32(r[k]), base + k);
      store8<ENC>(a.y, i, r);
    } else {
#pragma unroll
      for (int k = 0; k < kVec; ++k) {
        const int64_t i = start + static_cast<int64_t>(k) * blockDim.x + threadIdx.x;
        if (i < a.n) {
          const float x = bits_f32(load1<ENC_F32>(a.x, i));
          store1<ENC>(a.y, i, encode<ENC>(x, a.counter_base + static_cast<uint32_t>(i)));
        }
      }
    }
  }
}

// Kernel tables (host stub addresses), filled by the instantiating units.
// Index order: [param enc][grad enc][state enc...]; param/grad enc is 0 for
// FP32 and 1 for BF16.
using KernelTableAdamW = const void* [2][2][ENC_COUNT][ENC_COUNT];
using KernelTableSgdm = const void* [2][2][ENC_COUNT];
using KernelTableCast = const void* [ENC_COUNT];

void register_adamw_m0(KernelTableAdamW&);
void register_adamw_m1(KernelTableAdamW&);
void register_adamw_m2(KernelTableAdamW&);
void register_adamw_m3(KernelTableAdamW&);
void register_adamw_m4(KernelTableAdamW&);
void register_adamw_m5(KernelTableAdamW&);
void register_adamw_m6(KernelTableAdamW&);
void register_adamw_m7(KernelTableAdamW&);
void register_adamw_m8(KernelTableAdamW&);
void register_sgdm(KernelTableSgdm&);
void register_cast(KernelTableCast&);

}  // namespace sr
