// sr_kernels.h -- gfx950 kernels of the stochastic-rounding optimizer path.
//
// Work decomposition.  Every launch covers a range of tiles; a tile is
// blockDim.x * E consecutive elements of one tensor and is processed by
// exactly one workgroup (no persistent loop).  A lane owns E consecutive
// elements.  Optimizer launches use E = 4 (FP32 operands move as one 128-bit
// access per lane), casts E = 8.  Measured on MI355X with the non-temporal
// accesses below, E = 4 is the faster optimizer width for every combination
// tried (E4M3 + BF16 moments 6.03 vs 5.41 TB/s at E = 8, BF16 parameters
// and momentum 6.47 vs 6.21) and E = 8 the faster cast width (BF16 output
// 6.08 vs 5.81 TB/s).  Rows whose pointers are not all 16-byte
// aligned, and the partial last tile of a row, take a coalesced scalar path
// (element k*blockDim.x + lane of the tile).
//
// XCD-aware order.  Workgroups map to tiles through sr_tile_order.h: each
// XCD takes chunks of up to 512 consecutive tiles in turn, so the tiles in
// flight on one XCD stay close together.  Measured on MI355X for the
// 12-byte-read / 8-byte-write pattern of the fused update, this order and one
// tile per workgroup beat persistent grid-stride loops.
//
// Multi-tensor launches.  `tile_rows[t]` names the row (tensor) of tile t
// and `rows[row]` is its 64-byte sr_row record: both are read once per
// workgroup with uniform (scalar) loads.  The random stream of an element
// depends only on its row's key, its shard start and its index, never on the
// launch shape.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/sr_states_hip.h"
#include "sr_math.h"
#include "sr_tile_order.h"

namespace sr {

// Elements per lane of an optimizer launch whose operands have encodings
// p, g, a, b (the host's sr_lane_elements() applies the same rule to dtypes).
// Every combination currently uses SR_LANE_ELEMENTS; the operands stay part
// of the contract so that a combination can move without an ABI change.
constexpr int lane_elements(int /*p*/, int /*g*/, int /*a*/, int /*b*/) {
  return SR_LANE_ELEMENTS;
}
static_assert(SR_LANE_ELEMENTS == 4 && SR_LANE_ELEMENTS_NARROW == 8, "lanes move 4 or 8 elements");
constexpr int kMaxBlock = 1024;

struct AdamWArgs {
  const sr_row* rows;        // device table; nullptr selects `inline_row`
  const uint32_t* tile_rows; // row of each tile; nullptr with `inline_row`
  // Per-row (neg_step_size, correction2_sqrt) pairs when the rows' AdamW
  // steps differ; nullptr: every row uses s.neg_step_size, s.correction2_sqrt.
  const float* row_scalars;
  sr_row inline_row;
  AdamWScalars s;
  uint32_t total_tiles;
  uint32_t key_prefix;  // update_key_prefix(seed, rng_step), computed by the host
};

struct SgdmArgs {
  const sr_row* rows;
  const uint32_t* tile_rows;
  sr_row inline_row;
  SgdmScalars s;
  uint32_t total_tiles;
  uint32_t key_prefix;  // update_key_prefix(seed, rng_step), computed by the host
};

struct CastArgs {
  const float* x;
  void* y;
  int64_t n;
  uint32_t counter_base;  // seed + offset (mod 2^32)
  uint32_t total_tiles;
  uint32_t vector_ok;     // x and y 16-byte aligned
};

// Logical tile of this workgroup; >= total_tiles for the padding workgroups.
// The host launches launch_shape(total_tiles, block): one row of
// padded_grid(total_tiles) workgroups, or several rows when that many would
// exceed the dispatch packet's 32-bit work-item count.
__device__ __forceinline__ uint32_t logical_tile(uint32_t total_tiles) {
  return tile_of(blockIdx.y * gridDim.x + blockIdx.x, total_tiles);
}

// ---------------------------------------------------------------------------
// Element I/O.  Raw storage words are zero-extended into 32-bit lanes.  Table
// entries are plain integers, so pointers are cast to the global address
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

// Streaming accesses.  Every operand is read once and written at most once
// per launch, so every global load and store carries the non-temporal hint.
// Measured on MI355X: north star 5.64 -> 6.13 TB/s, SGDM 5.87 -> 6.41 TB/s;
// the hint on loads alone is slower (5.51) and on stores alone neutral.
typedef uint32_t stream_v4 __attribute__((ext_vector_type(4)));
typedef uint32_t stream_v2 __attribute__((ext_vector_type(2)));

template <class T>
__device__ __forceinline__ T stream_load(const void* p) {
  return __builtin_nontemporal_load(gptr<T>(p));
}
template <class T>
__device__ __forceinline__ void stream_store(void* p, T v) {
  __builtin_nontemporal_store(v, gptr_mut<T>(p));
}

// E elements at index i (i a multiple of E, base 16-byte aligned), moved as
// one access of E * width bytes (two for 32 bytes).  kCached keeps a 16-byte
// load under the normal cache policy (the small casts' input, below).
template <int BYTES, bool kCached = false>
__device__ __forceinline__ void load_words(const char* ptr, uint32_t* w) {
  static_assert(!kCached || BYTES == 16, "cached loads are 16-byte loads");
  if constexpr (kCached) {
    const stream_v4 a = *gptr<stream_v4>(ptr);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (BYTES == 32) {
    const stream_v4 a = stream_load<stream_v4>(ptr), b = stream_load<stream_v4>(ptr + 16);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w; w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  } else if constexpr (BYTES == 16) {
    const stream_v4 a = stream_load<stream_v4>(ptr);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  } else if constexpr (BYTES == 8) {
    const stream_v2 a = stream_load<stream_v2>(ptr);
    w[0] = a.x; w[1] = a.y;
  } else if constexpr (BYTES == 4) {
    w[0] = stream_load<uint32_t>(ptr);
  } else {
    static_assert(BYTES == 2, "unsupported access width");
    w[0] = stream_load<uint16_t>(ptr);
  }
}

template <int BYTES>
__device__ __forceinline__ void store_words(char* ptr, const uint32_t* w) {
  if constexpr (BYTES == 32) {
    stream_store(ptr, stream_v4{w[0], w[1], w[2], w[3]});
    stream_store(ptr + 16, stream_v4{w[4], w[5], w[6], w[7]});
  } else if constexpr (BYTES == 16) {
    stream_store(ptr, stream_v4{w[0], w[1], w[2], w[3]});
  } else if constexpr (BYTES == 8) {
    stream_store(ptr, stream_v2{w[0], w[1]});
  } else if constexpr (BYTES == 4) {
    stream_store(ptr, w[0]);
  } else {
    static_assert(BYTES == 2, "unsupported access width");
    stream_store(ptr, static_cast<uint16_t>(w[0]));
  }
}

// The storage words of the group of four elements at index i (a multiple
// of four, base 16-byte aligned), moved as one access.
template <int ENC, bool kCached = false>
__device__ __forceinline__ void load_group(const void* base, int64_t i, uint32_t (&words)[group_words(ENC)]) {
  load_words<kGroup * enc_bytes(ENC), kCached>(static_cast<const char*>(base) + i * enc_bytes(ENC), words);
}

template <int ENC>
__device__ __forceinline__ void store_group(void* base, int64_t i, const uint32_t (&words)[group_words(ENC)]) {
  store_words<kGroup * enc_bytes(ENC)>(static_cast<char*>(base) + i * enc_bytes(ENC), words);
}

// The same with a workgroup-uniform tile base and the lane's group index j
// below 2^30: the address is a scalar base plus a 32-bit lane offset, which
// the loads and stores take as such (no per-lane 64-bit address arithmetic).
template <int ENC>
__device__ __forceinline__ void load_lane_group(const char* tile, uint32_t j, uint32_t (&words)[group_words(ENC)]) {
  load_words<kGroup * enc_bytes(ENC)>(tile + j * static_cast<uint32_t>(kGroup * enc_bytes(ENC)), words);
}

template <int ENC>
__device__ __forceinline__ void store_lane_group(char* tile, uint32_t j, const uint32_t (&words)[group_words(ENC)]) {
  // The offset is recomputed behind an empty asm: sharing it with the load
  // of the same tile made the compiler form full 64-bit store addresses.
  uint32_t offset = j * static_cast<uint32_t>(kGroup * enc_bytes(ENC));
  __asm__("" : "+v"(offset));
  store_words<kGroup * enc_bytes(ENC)>(tile + offset, words);
}

template <int ENC>
__device__ __forceinline__ uint32_t load1(const void* base, int64_t i) {
  constexpr int W = enc_bytes(ENC);
  const char* p = static_cast<const char*>(base) + i * W;
  if constexpr (W == 4) return stream_load<uint32_t>(p);
  else if constexpr (W == 2) return stream_load<uint16_t>(p);
  else return stream_load<uint8_t>(p);
}

template <int ENC>
__device__ __forceinline__ void store1(void* base, int64_t i, uint32_t v) {
  constexpr int W = enc_bytes(ENC);
  char* p = static_cast<char*>(base) + i * W;
  if constexpr (W == 4) stream_store(p, v);
  else if constexpr (W == 2) stream_store(p, static_cast<uint16_t>(v));
  else stream_store(p, static_cast<uint8_t>(v));
}

// The row record of this workgroup's tile, read once with uniform loads.
template <class Args>
__device__ __forceinline__ uint32_t tile_row_index(const Args& a, uint32_t t) {
  return a.rows ? a.tile_rows[t] : 0u;
}

// The row record, copied once: one wide uniform load from the table (or the
// kernel argument) instead of a load per field behind its own branch.
template <class Args>
__device__ __forceinline__ sr_row row_record(const Args& a, uint32_t row) {
  if (a.rows) return a.rows[row];
  return a.inline_row;
}

template <class Args>
__device__ __forceinline__ uint32_t row_key(const Args& a, const sr_row& r) {
  return (r.flags & SR_ROW_KEYED)
             ? r.param_index
             : update_key_from_prefix(a.key_prefix, r.param_index);
}

// ---------------------------------------------------------------------------
// Fused AdamW.
// ---------------------------------------------------------------------------
// One lane's group of a full vector tile: p, g, m, v point at the tile's
// first element (workgroup-uniform), j is the lane's group in the tile and
// `index` the flat index (mod 2^32) of its first element.
template <int PE, int GE, int ME, int VE>
__device__ __forceinline__ void adamw_vector(char* p, const char* g, char* m, char* v, uint32_t j,
                                             uint32_t index, uint32_t cm, uint32_t cv, const AdamWScalars& s) {
  constexpr int E = lane_elements(PE, GE, ME, VE);
  static_assert(E == kGroup, "a lane's elements are one group");
  uint32_t wp[group_words(PE)], wg[group_words(GE)], wm[group_words(ME)], wv[group_words(VE)];
  load_lane_group<PE>(p, j, wp);
  load_lane_group<GE>(g, j, wg);
  load_lane_group<ME>(m, j, wm);
  load_lane_group<VE>(v, j, wv);
  float pf[E], gf[E], mf[E], vf[E];
  decode_group<PE>(wp, pf);
  decode_group<GE>(wg, gf);
  decode_group<ME>(wm, mf);
  decode_group<VE>(wv, vf);
  float mo[E], vo[E], root[E];
  bool tiny = false;
#pragma unroll
  for (int k = 0; k < E; ++k) {
    adamw_moments(gf[k], mf[k], vf[k], s, mo[k], vo[k]);
    root[k] = sqrt_rn_wide(vo[k]);
    tiny |= sqrt_needs_library(vo[k]);
  }
  // One branch for the lane's E square roots; whole waves skip it.
  if (tiny) {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      if (sqrt_needs_library(vo[k])) root[k] = sqrt_library(vo[k]);
    }
  }
  // numer / den through div_short where its domain holds: eps, uniform, in
  // its range and every |q0| in range (an infinite or NaN denominator fails
  // the latter).  Otherwise the lane computes its E denominators and
  // quotients again, exactly, with the library division (one branch, which
  // whole waves skip).
  float numer[E], den[E], quotient[E];
  bool divide_again = !short_division_eps(s.eps);
#pragma unroll
  for (int k = 0; k < E; ++k) {
    numer[k] = s.neg_step_size * mo[k];
    den[k] = adamw_denominator_finite(root[k], s);
    bool ok;
    quotient[k] = div_short(numer[k], den[k], ok);
    divide_again |= !ok;
  }
  if (divide_again) {
#pragma unroll
    for (int k = 0; k < E; ++k) quotient[k] = div_library(numer[k], adamw_denominator(root[k], s));
  }
#pragma unroll
  for (int k = 0; k < E; ++k) pf[k] = pf[k] * s.decay + quotient[k];
  encode_group<PE>(pf, 0u, wp);
  encode_group<ME>(mo, cm + index, wm);
  encode_group<VE>(vo, cv + index, wv);
  store_lane_group<PE>(p, j, wp);
  store_lane_group<ME>(m, j, wm);
  store_lane_group<VE>(v, j, wv);
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
  constexpr int E = lane_elements(PE, GE, ME, VE);
  const uint32_t t = logical_tile(a.total_tiles);
  if (t >= a.total_tiles) return;
  const uint32_t row = tile_row_index(a, t);
  const sr_row r = row_record(a, row);
  AdamWScalars s = a.s;
  if (a.row_scalars) {
    s.neg_step_size = a.row_scalars[2 * row];
    s.correction2_sqrt = a.row_scalars[2 * row + 1];
    s.inv_correction2_sqrt = 1.0f / s.correction2_sqrt;
  }
  char* p = reinterpret_cast<char*>(r.ptr[0]);
  const char* g = reinterpret_cast<const char*>(r.ptr[1]);
  char* m = reinterpret_cast<char*>(r.ptr[2]);
  char* v = reinterpret_cast<char*>(r.ptr[3]);
  const int64_t numel = r.numel;
  const uint32_t key = row_key(a, r);
  const uint32_t cm = state_key(key, 0) + r.shard_start;
  const uint32_t cv = state_key(key, 1) + r.shard_start;
  const uint32_t tile = blockDim.x * E;
  const int64_t start = static_cast<int64_t>(t - r.tile_begin) * tile;
  if ((r.flags & SR_ROW_VECTOR) && start + tile <= numel) {
    adamw_vector<PE, GE, ME, VE>(p + start * enc_bytes(PE), g + start * enc_bytes(GE), m + start * enc_bytes(ME),
                                 v + start * enc_bytes(VE), threadIdx.x,
                                 static_cast<uint32_t>(start) + threadIdx.x * E, cm, cv, s);
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int64_t i = start + static_cast<int64_t>(k) * blockDim.x + threadIdx.x;
      if (i < numel) adamw_scalar<PE, GE, ME, VE>(p, g, m, v, i, cm, cv, s);
    }
  }
}

// ---------------------------------------------------------------------------
// Fused momentum SGD.
// ---------------------------------------------------------------------------
// One lane's group of a full vector tile, as adamw_vector.
template <int PE, int GE, int UE>
__device__ __forceinline__ void sgdm_vector(char* p, const char* g, char* u, uint32_t j, uint32_t index,
                                            uint32_t cu, const SgdmScalars& s) {
  constexpr int E = lane_elements(PE, GE, UE, UE);
  static_assert(E == kGroup, "a lane's elements are one group");
  uint32_t wp[group_words(PE)], wg[group_words(GE)], wu[group_words(UE)];
  load_lane_group<PE>(p, j, wp);
  load_lane_group<GE>(g, j, wg);
  load_lane_group<UE>(u, j, wu);
  float pf[E], gf[E], uf[E];
  decode_group<PE>(wp, pf);
  decode_group<GE>(wg, gf);
  decode_group<UE>(wu, uf);
#pragma unroll
  for (int k = 0; k < E; ++k) sgdm_update(pf[k], gf[k], uf[k], s, pf[k], uf[k]);
  encode_group<PE>(pf, 0u, wp);
  encode_group<UE>(uf, cu + index, wu);
  store_lane_group<PE>(p, j, wp);
  store_lane_group<UE>(u, j, wu);
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
  constexpr int E = lane_elements(PE, GE, UE, UE);
  const uint32_t t = logical_tile(a.total_tiles);
  if (t >= a.total_tiles) return;
  const sr_row r = row_record(a, tile_row_index(a, t));
  char* p = reinterpret_cast<char*>(r.ptr[0]);
  const char* g = reinterpret_cast<const char*>(r.ptr[1]);
  char* u = reinterpret_cast<char*>(r.ptr[2]);
  const int64_t numel = r.numel;
  const uint32_t cu = state_key(row_key(a, r), 0) + r.shard_start;
  const uint32_t tile = blockDim.x * E;
  const int64_t start = static_cast<int64_t>(t - r.tile_begin) * tile;
  if ((r.flags & SR_ROW_VECTOR) && start + tile <= numel) {
    sgdm_vector<PE, GE, UE>(p + start * enc_bytes(PE), g + start * enc_bytes(GE), u + start * enc_bytes(UE),
                            threadIdx.x, static_cast<uint32_t>(start) + threadIdx.x * E, cu, a.s);
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int64_t i = start + static_cast<int64_t>(k) * blockDim.x + threadIdx.x;
      if (i < numel) sgdm_scalar<PE, GE, UE>(p, g, u, i, cu, a.s);
    }
  }
}

// ---------------------------------------------------------------------------
// Standalone cast: y = round(x), counter = index + seed + offset.
// ---------------------------------------------------------------------------
// Casts move 8 elements per lane whatever the output width, as two groups
// of 4 a workgroup-width apart: every load instruction then reads
// blockDim * 16 contiguous bytes, and every store writes a contiguous span
// too.  With the lane's 8 elements adjacent (two 16-byte loads per lane,
// each instruction reading every other 16 bytes of its span), the same
// streams reach 5.55 TB/s at 2^24 elements; grouped, 6.03-6.06 (trivial
// arithmetic, 256 threads).  At 4 elements per lane: 5.42.
constexpr int kCastLaneElements = SR_LANE_ELEMENTS_NARROW;
constexpr int kCastGroup = 4;

// Inputs of up to 2^23 elements (32 MiB) are loaded under the normal cache
// policy (kCachedLoads), larger ones non-temporally; stores stay
// non-temporal.  Measured on MI355X for the BF16 SR cast, back-to-back
// calls: at 2^22 elements 5.39 -> 4.66 us over eight rotating buffers and
// 3.55 -> 2.91 us on one; at 2^23 9.21 -> 8.19 and 7.19 -> 6.66; at 2^24
// the non-temporal loads win (16.71 against 17.68 us over eight buffers).
constexpr int64_t kCachedCastMaxElements = int64_t{1} << 23;

template <int ENC, bool kCachedLoads>
__global__ __launch_bounds__(kMaxBlock) void cast_kernel(const CastArgs a) {
  constexpr int E = kCastLaneElements, G = kCastGroup;
  const uint32_t t = logical_tile(a.total_tiles);
  if (t >= a.total_tiles) return;
  const uint32_t tile = blockDim.x * E;
  const int64_t start = static_cast<int64_t>(t) * tile;
  if (a.vector_ok && start + tile <= a.n) {
    static_assert(G == kGroup, "cast groups are encoder groups");
    uint32_t r[E / G][G];
#pragma unroll
    for (int k = 0; k < E / G; ++k) {
      load_group<ENC_F32, kCachedLoads>(a.x, start + static_cast<int64_t>(k * blockDim.x + threadIdx.x) * G, r[k]);
    }
#pragma unroll
    for (int k = 0; k < E / G; ++k) {
      const int64_t i = start + static_cast<int64_t>(k * blockDim.x + threadIdx.x) * G;
      float x[G];
#pragma unroll
      for (int j = 0; j < G; ++j) x[j] = bits_f32(r[k][j]);
      uint32_t words[group_words(ENC)];
      encode_group<ENC, true>(x, a.counter_base + static_cast<uint32_t>(i), words);
      store_group<ENC>(a.y, i, words);
    }
  } else {
#pragma unroll
    for (int k = 0; k < E; ++k) {
      const int64_t i = start + static_cast<int64_t>(k) * blockDim.x + threadIdx.x;
      if (i < a.n) {
        const float x = bits_f32(load1<ENC_F32>(a.x, i));
        store1<ENC>(a.y, i, encode<ENC>(x, a.counter_base + static_cast<uint32_t>(i)));
      }
    }
  }
}

// Ordered neighbours of each FP32 input in the format of ENC (one of the
// nearest encodings BF16_RN, F16_RN, E4M3_RN, E5M2_RN), a checking helper
// (sr_states/_bf16.py:77-101, sr_states/_minifloat.py:73-99).  A grid-stride
// loop: every lane leaves once its index passes n, whatever the grid.
struct NeighborArgs {
  const float* x;
  void* lower;
  void* upper;
  int64_t n;
};

constexpr int kNeighborBlock = 256;

template <int ENC>
__global__ __launch_bounds__(kNeighborBlock) void neighbors_kernel(const NeighborArgs a) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < a.n; i += stride) {
    uint32_t lower, upper;
    neighbor_bits<ENC>(load1<ENC_F32>(a.x, i), lower, upper);
    store1<ENC>(a.lower, i, lower);
    store1<ENC>(a.upper, i, upper);
  }
}

// Kernel tables (host stub addresses), filled by the instantiating units.
// Index order: [param enc][grad enc][state enc...]; param/grad enc is 0 for
// FP32 and 1 for BF16.
using KernelTableAdamW = const void* [2][2][ENC_COUNT][ENC_COUNT];
using KernelTableSgdm = const void* [2][2][ENC_COUNT];
using KernelTableCast = const void* [2][ENC_COUNT];  // [kCachedLoads][encoding]
using KernelTableNeighbors = const void* [ENC_COUNT];  // nearest encodings only

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
void register_neighbors(KernelTableNeighbors&);

}  // namespace sr
