// Bandwidth matrix of the fused AdamW step's streams, measured in one process.
//
// The north star moves, per element, an FP32 parameter read and written, an
// FP32 gradient read and two BF16 moments read and written: 12 bytes read and
// 8 written over seven streams.  Every kernel here has trivial arithmetic
// (XOR folds) and moves a subset or a rearrangement of those streams over
// the same buffers, with the product's tile shape (128 lanes x 4 elements),
// its XCD-chunked tile order (sr_tile_order.h) and non-temporal accesses
// unless a variant says otherwise.  Interleaved timing of all variants over
// one set of allocations tells which structure the memory system rewards:
//
//   - read-only, write-only and copy patterns bound what reads and writes
//     reach on their own;
//   - patterns with one, two and three written streams separate the read:
//     write mix from the number of written streams;
//   - the product's pattern with K tiles per workgroup, in registers or
//     staged through LDS with gfx950's global_load_lds (no VGPRs held), all
//     loads before any store or software-pipelined, test whether more bytes
//     in flight or longer write bursts per workgroup help.
//
// Measurement helper only: bench.py --workload bandwidth_matrix prints the
// rates.  It allocates its own buffers and frees them before returning.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <utility>

#include "../../stochastic-rounding-pytorch_amd/csrc/sr_tile_order.h"

namespace {

constexpr int kBlock = 128;
constexpr int kLanes = 4;
constexpr uint32_t kTile = kBlock * kLanes;
constexpr uint32_t kMaxK = 8;

typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
#define SR_LDS __attribute__((address_space(3)))

#define SR_GLOBAL __attribute__((address_space(1)))

// Addressing as the fused kernels address a tile: a workgroup-uniform tile
// base plus the lane's 32-bit byte offset, in the global address space, each
// store's offset in a fresh register (a shared one makes the compiler form
// full 64-bit store addresses).
template <class T>
__device__ __forceinline__ T ld(const char* tile, uint32_t offset) {
  return __builtin_nontemporal_load((const SR_GLOBAL T*)(tile + offset));
}
template <class T>
__device__ __forceinline__ void st(char* tile, uint32_t offset, T v) {
  __asm__("" : "+v"(offset));
  __builtin_nontemporal_store(v, (SR_GLOBAL T*)(tile + offset));
}
__device__ __forceinline__ uint32_t fold(u4 w) { return w.x ^ w.y ^ w.z ^ w.w; }
__device__ __forceinline__ uint32_t fold(u2 w) { return w.x ^ w.y; }

// p: 4n bytes, g: 4n, m: 4n (2n used except by the interleaved variant), v: 2n.
struct Buffers {
  char* p;
  char* g;
  char* m;
  char* v;
  uint32_t* sink;
  uint32_t groups;  // work units of the launch: K tiles each
};

__device__ __forceinline__ uint32_t unit_of(uint32_t groups) {
  return sr::tile_of(blockIdx.y * gridDim.x + blockIdx.x, groups);
}

// The seven-stream pattern with K tiles per workgroup held in registers
// (all loads first), and its read-only / write-only halves.
enum Role { MIXED = 0, READ_ONLY = 1, WRITE_ONLY = 2 };

template <int ROLE, int K>
__global__ __launch_bounds__(kBlock) void seven_streams(Buffers b) {
  const uint32_t unit = unit_of(b.groups);
  if (unit >= b.groups) return;
  const uint64_t first = static_cast<uint64_t>(unit) * K * kTile;
  const uint32_t lane = threadIdx.x * kLanes;
  u4 wp[K], wg[K];
  u2 wm[K], wv[K];
  if constexpr (ROLE != WRITE_ONLY) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const uint64_t t = first + static_cast<uint64_t>(k) * kTile;
      wp[k] = ld<u4>(b.p + t * 4, lane * 4);
      wg[k] = ld<u4>(b.g + t * 4, lane * 4);
      wm[k] = ld<u2>(b.m + t * 2, lane * 2);
      wv[k] = ld<u2>(b.v + t * 2, lane * 2);
    }
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const uint64_t t = first + static_cast<uint64_t>(k) * kTile;
    if constexpr (ROLE == WRITE_ONLY) {
      const uint32_t h = static_cast<uint32_t>(t + lane) * 0x9E3779B9u;
      st<u4>(b.p + t * 4, lane * 4, u4{h, h + 1, h + 2, h + 3});
      st<u2>(b.m + t * 2, lane * 2, u2{h, h + 5});
      st<u2>(b.v + t * 2, lane * 2, u2{h + 7, h});
    } else {
      const uint32_t h = fold(wp[k]) ^ fold(wg[k]) ^ fold(wm[k]) ^ fold(wv[k]);
      if constexpr (ROLE == READ_ONLY) {
        // Practically never true (and harmless: the sink is real memory),
        // but the compiler cannot know, so the loads stay.
        if (h == b.groups * 7919u + 1u) b.sink[threadIdx.x & 15] = h;
      } else {
        st<u4>(b.p + t * 4, lane * 4, wp[k] ^ h);
        st<u2>(b.m + t * 2, lane * 2, wm[k] ^ h);
        st<u2>(b.v + t * 2, lane * 2, wv[k] ^ h);
      }
    }
  }
}

// Other stream sets, one tile per workgroup.
enum Shape {
  COPY_IN_PLACE = 0,  // p read and written: 4R:4W, one stream
  COPY_TWO = 1,       // g read, p written: 4R:4W, two streams
  ONE_WRITTEN = 2,    // p read and written, g read: 8R:4W
  TWO_WRITTEN = 3,    // p and m read and written, g read: 10R:6W
  NO_GRADIENT = 4,    // p, m, v read and written: 8R:8W
  MV_PAIRED = 5       // p read and written, g read, m and v interleaved as one 4-byte stream: 12R:8W
};

template <int SHAPE>
__global__ __launch_bounds__(kBlock) void stream_set(Buffers b) {
  const uint32_t unit = unit_of(b.groups);
  if (unit >= b.groups) return;
  const uint64_t t = static_cast<uint64_t>(unit) * kTile;
  const uint32_t l4 = threadIdx.x * kLanes * 4, l2 = threadIdx.x * kLanes * 2;
  char* const p = b.p + t * 4;
  char* const g = b.g + t * 4;
  char* const m2 = b.m + t * 2;
  char* const m4 = b.m + t * 4;
  char* const v = b.v + t * 2;
  if constexpr (SHAPE == COPY_IN_PLACE) {
    const u4 wp = ld<u4>(p, l4);
    st<u4>(p, l4, wp ^ fold(wp));
  } else if constexpr (SHAPE == COPY_TWO) {
    const u4 wg = ld<u4>(g, l4);
    st<u4>(p, l4, wg ^ fold(wg));
  } else if constexpr (SHAPE == ONE_WRITTEN) {
    const u4 wp = ld<u4>(p, l4), wg = ld<u4>(g, l4);
    st<u4>(p, l4, wp ^ (fold(wp) ^ fold(wg)));
  } else if constexpr (SHAPE == TWO_WRITTEN) {
    const u4 wp = ld<u4>(p, l4), wg = ld<u4>(g, l4);
    const u2 wm = ld<u2>(m2, l2);
    const uint32_t h = fold(wp) ^ fold(wg) ^ fold(wm);
    st<u4>(p, l4, wp ^ h);
    st<u2>(m2, l2, wm ^ h);
  } else if constexpr (SHAPE == NO_GRADIENT) {
    const u4 wp = ld<u4>(p, l4);
    const u2 wm = ld<u2>(m2, l2), wv = ld<u2>(v, l2);
    const uint32_t h = fold(wp) ^ fold(wm) ^ fold(wv);
    st<u4>(p, l4, wp ^ h);
    st<u2>(m2, l2, wm ^ h);
    st<u2>(v, l2, wv ^ h);
  } else {
    static_assert(SHAPE == MV_PAIRED, "unknown stream set");
    const u4 wp = ld<u4>(p, l4), wg = ld<u4>(g, l4), wmv = ld<u4>(m4, l4);
    const uint32_t h = fold(wp) ^ fold(wg) ^ fold(wmv);
    st<u4>(p, l4, wp ^ h);
    st<u4>(m4, l4, wmv ^ h);
  }
}

// The seven-stream pattern staged through LDS.  Each wave copies its 256
// elements of a tile (p and g: 1 KB each, m and v: 512 B each) straight into
// LDS with global_load_lds_dwordx4, which holds no VGPRs while in flight;
// lane l's 16 bytes land at offset 16 l of the wave's slot, so each lane
// reads back exactly what it loaded and no barrier is needed (m and v use
// the first 32 lanes: 512 bytes).  DEPTH 0: the workgroup's K tiles are all
// requested before any is stored; DEPTH d > 0: tile k + d is requested just
// before tile k is stored, from a ring of d + 1 slots.  The waits count
// vector-memory instructions (each tile issues 4 loads and 3 stores per
// wave, and gfx950 counts both, retiring them in order), so a wait covers
// exactly the loads of the tile about to be stored.
constexpr int kSlotBytes = 3072;

constexpr int vmcnt_wait(int n) { return (n & 0xF) | ((n >> 4) << 14) | (7 << 4) | (0xF << 8); }
constexpr int kLgkmWait0 = 0xC07F;  // lgkmcnt(0), other counters unchecked

template <int K, int DEPTH, int k>
constexpr int in_flight_after() {
  if (DEPTH == 0) return 4 * (K - 1 - k) + 3 * k;
  const int last = (k + DEPTH < K - 1) ? k + DEPTH : K - 1;
  return 4 * (last - k) + 3 * (k < DEPTH ? k : DEPTH);
}

template <int K, int DEPTH>
struct Staged {
  static constexpr int kSlots = DEPTH == 0 ? K : DEPTH + 1;
  static_assert(K <= static_cast<int>(kMaxK) && DEPTH < K, "K tiles, prefetched at most K - 1 ahead");
  const Buffers* b;
  char* slots;
  uint64_t first;  // first element of the workgroup's K tiles
  int wave, lane;

  __device__ __forceinline__ char* slot(int k) const { return slots + (DEPTH == 0 ? k : k % kSlots) * kSlotBytes; }

  __device__ __forceinline__ void request(int k) const {
    char* s = slot(k);
    const uint64_t w0 = first + static_cast<uint64_t>(k) * kTile + wave * (kTile / 2);
    const uint32_t offset = static_cast<uint32_t>(lane) * 16u;
    __builtin_amdgcn_global_load_lds((const SR_GLOBAL void*)(b->p + w0 * 4 + offset), (SR_LDS void*)(s), 16, 0, 2);
    __builtin_amdgcn_global_load_lds((const SR_GLOBAL void*)(b->g + w0 * 4 + offset), (SR_LDS void*)(s + 1024), 16, 0, 2);
    if (lane < 32) {
      __builtin_amdgcn_global_load_lds((const SR_GLOBAL void*)(b->m + w0 * 2 + offset), (SR_LDS void*)(s + 2048), 16, 0, 2);
      __builtin_amdgcn_global_load_lds((const SR_GLOBAL void*)(b->v + w0 * 2 + offset), (SR_LDS void*)(s + 2560), 16, 0, 2);
    }
  }

  __device__ __forceinline__ void store(int k) const {
    const char* s = slot(k);
    const u4 wp = *reinterpret_cast<const u4*>(s + lane * 16);
    const u4 wg = *reinterpret_cast<const u4*>(s + 1024 + lane * 16);
    const u2 wm = *reinterpret_cast<const u2*>(s + 2048 + lane * 8);
    const u2 wv = *reinterpret_cast<const u2*>(s + 2560 + lane * 8);
    const uint32_t h = fold(wp) ^ fold(wg) ^ fold(wm) ^ fold(wv);
    const uint64_t t = first + static_cast<uint64_t>(k) * kTile;
    const uint32_t l = static_cast<uint32_t>(wave * 64 + lane) * kLanes;
    st<u4>(b->p + t * 4, l * 4, wp ^ h);
    st<u2>(b->m + t * 2, l * 2, wm ^ h);
    st<u2>(b->v + t * 2, l * 2, wv ^ h);
  }

  template <int k>
  __device__ __forceinline__ void step() const {
    if constexpr (DEPTH > 0 && k + DEPTH < K) request(k + DEPTH);
    __builtin_amdgcn_s_waitcnt(vmcnt_wait(in_flight_after<K, DEPTH, k>()));
    store(k);
    // The slot's LDS reads finish before a later request refills it.
    if constexpr (DEPTH > 0) __builtin_amdgcn_s_waitcnt(kLgkmWait0);
  }

  template <int... ks>
  __device__ __forceinline__ void run(std::integer_sequence<int, ks...>) const {
    ((DEPTH == 0 || ks < DEPTH ? request(ks) : void()), ...);
    (step<ks>(), ...);
  }
};

template <int K, int DEPTH>
__global__ __launch_bounds__(kBlock) void staged_streams(Buffers b) {
  constexpr int kWaves = kBlock / 64;
  __shared__ __attribute__((aligned(16))) char lds[kWaves * Staged<K, DEPTH>::kSlots * kSlotBytes];
  const uint32_t unit = unit_of(b.groups);
  if (unit >= b.groups) return;
  Staged<K, DEPTH> s;
  s.b = &b;
  s.wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  s.lane = threadIdx.x % 64;
  s.slots = lds + s.wave * Staged<K, DEPTH>::kSlots * kSlotBytes;
  s.first = static_cast<uint64_t>(unit) * K * kTile;
  s.run(std::make_integer_sequence<int, K>{});
}

typedef void (*Kernel)(Buffers);

struct Variant {
  const char* name;
  Kernel kernel;
  int tiles_per_workgroup;
  int bytes_per_element;  // algorithmic reads + writes
};

const Variant kVariants[] = {
    {"seven_streams (the fused update's pattern)", seven_streams<MIXED, 1>, 1, 20},
    {"read_only_12B (its four read streams)", seven_streams<READ_ONLY, 1>, 1, 12},
    {"write_only_8B (its three written streams)", seven_streams<WRITE_ONLY, 1>, 1, 8},
    {"copy_in_place_4R4W", stream_set<COPY_IN_PLACE>, 1, 8},
    {"copy_two_buffers_4R4W", stream_set<COPY_TWO>, 1, 8},
    {"one_written_stream_8R4W", stream_set<ONE_WRITTEN>, 1, 12},
    {"two_written_streams_10R6W", stream_set<TWO_WRITTEN>, 1, 16},
    {"three_written_streams_no_gradient_8R8W", stream_set<NO_GRADIENT>, 1, 16},
    {"moments_interleaved_12R8W", stream_set<MV_PAIRED>, 1, 20},
    {"seven_streams_2_tiles_in_registers", seven_streams<MIXED, 2>, 2, 20},
    {"seven_streams_4_tiles_in_registers", seven_streams<MIXED, 4>, 4, 20},
    {"seven_streams_lds_1_tile", staged_streams<1, 0>, 1, 20},
    {"seven_streams_lds_2_tiles", staged_streams<2, 0>, 2, 20},
    {"seven_streams_lds_4_tiles", staged_streams<4, 0>, 4, 20},
    {"seven_streams_lds_8_tiles", staged_streams<8, 0>, 8, 20},
    {"seven_streams_lds_4_tiles_prefetch_1", staged_streams<4, 1>, 4, 20},
    {"seven_streams_lds_8_tiles_prefetch_1", staged_streams<8, 1>, 8, 20},
    {"seven_streams_lds_8_tiles_prefetch_2", staged_streams<8, 2>, 8, 20},
};
constexpr int kVariantCount = sizeof(kVariants) / sizeof(kVariants[0]);

}  // namespace

// Number of variants; name and algorithmic bytes per element of variant v.
extern "C" int sr_bandwidth_variants(void) { return kVariantCount; }

extern "C" int sr_bandwidth_variant(int v, const char** name, int* bytes_per_element) {
  if (v < 0 || v >= kVariantCount || !name || !bytes_per_element) return 1;
  *name = kVariants[v].name;
  *bytes_per_element = kVariants[v].bytes_per_element;
  return 0;
}

// Times every variant over n elements (a positive multiple of 4096, so that
// every tile count divides; at most 2^31 tiles): `rounds` interleaved
// rounds, each timing `reps` back-to-back launches of each variant after two
// untimed ones.  ms[round * count + v] receives the average milliseconds per
// launch.  Returns 0, 1 for an invalid argument, 2 for a HIP error (buffers
// are freed either way).
extern "C" int sr_bandwidth_matrix(uint64_t n, int reps, int rounds, float* ms, int count) {
  if (n == 0 || n % (kMaxK * kTile) || n / kTile > 0x7FFFF000ull || reps < 1 || rounds < 1 || !ms ||
      count != kVariantCount)
    return 1;
  Buffers b{};
  const size_t sizes[4] = {n * 4, n * 4, n * 4, n * 2};
  char** bufs[4] = {&b.p, &b.g, &b.m, &b.v};
  hipEvent_t start = nullptr, stop = nullptr;
  int rc = 2;
  do {
    if (hipDeviceSynchronize() != hipSuccess) break;
    bool ok = hipMalloc(reinterpret_cast<void**>(&b.sink), 64) == hipSuccess;
    for (int k = 0; k < 4 && ok; ++k) {
      ok = hipMalloc(reinterpret_cast<void**>(bufs[k]), sizes[k]) == hipSuccess &&
           hipMemset(*bufs[k], 0x3A + k, sizes[k]) == hipSuccess;
    }
    if (!ok || hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) break;
    bool failed = false;
    for (int r = 0; r < rounds && !failed; ++r) {
      for (int v = 0; v < kVariantCount && !failed; ++v) {
        const uint32_t tiles = static_cast<uint32_t>(n / kTile);
        b.groups = tiles / kVariants[v].tiles_per_workgroup;
        const sr::LaunchShape shape = sr::launch_shape(b.groups, kBlock);
        auto launch = [&] {
          hipLaunchKernelGGL(kVariants[v].kernel, dim3(shape.x, shape.y), dim3(kBlock), 0, nullptr, b);
        };
        launch();
        launch();
        if (hipGetLastError() != hipSuccess || hipEventRecord(start, nullptr) != hipSuccess) {
          failed = true;
          break;
        }
        for (int i = 0; i < reps; ++i) launch();
        float t = 0.0f;
        failed = hipGetLastError() != hipSuccess || hipEventRecord(stop, nullptr) != hipSuccess ||
                 hipEventSynchronize(stop) != hipSuccess || hipEventElapsedTime(&t, start, stop) != hipSuccess;
        ms[r * kVariantCount + v] = t / reps;
      }
    }
    if (!failed) rc = 0;
  } while (false);
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  (void)hipDeviceSynchronize();
  for (char** buf : bufs)
    if (*buf) (void)hipFree(*buf);
  if (b.sink) (void)hipFree(b.sink);
  return rc;
}
