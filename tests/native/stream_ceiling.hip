// The bandwidth ceiling of a fused update's access pattern, measured.
//
// A kernel with trivial arithmetic (XORs) that moves exactly the streams of
// one fused-update launch: a parameter (FP32 or BF16) read and written, a
// gradient read, and one or two states read and written, with the product's
// tile shape (128 lanes x 4 elements), its XCD-chunked tile order
// (sr_tile_order.h), its addressing (a scalar tile base plus a 32-bit lane
// offset), its non-temporal accesses and its resident-workgroup cap
// (sr::resident_cap, enforced with sr::cap_lds as the library's launches
// do).  Whatever rate this kernel reaches for n elements is what the memory
// system gives that access pattern at that footprint; the fused kernels do
// strictly more work per byte, so their rate over this one says how much of
// the reachable bandwidth their arithmetic and table lookups cost.
//
// sr_cast_ceiling does the same for the cast's pattern (FP32 in, a 2- or
// 1-byte format out) with the cast's launch shape.
//
// sr_launch_cap_sweep times this kernel beside the library's own fused AdamW
// kernel (FP32 parameter and gradient, BF16 stochastic moments: the north
// star's instantiation, on one tensor) at caller-chosen resident-workgroup
// caps, to show what the cap rule gains at a given footprint.
//
// Measurement helper only: bench.py reports it beside the fused kernel's
// rate and tests/test_gpu_stream_ceiling.py checks the fused kernels against
// it.  It allocates its own buffers, so it never touches caller memory.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../stochastic-rounding-pytorch_amd/csrc/sr_kernels.h"
#include "../../stochastic-rounding-pytorch_amd/csrc/sr_launch_cap.h"
#include "../../stochastic-rounding-pytorch_amd/csrc/sr_tile_order.h"

namespace {

constexpr int kBlock = 128;
constexpr int kLanes = 4;
constexpr uint32_t kTile = kBlock * kLanes;

typedef uint32_t word4 __attribute__((ext_vector_type(4)));
typedef uint32_t word2 __attribute__((ext_vector_type(2)));

// The access type of kLanes elements of `BYTES` bytes each.
template <int BYTES> struct Access;
template <> struct Access<4> { typedef word4 type; };
template <> struct Access<2> { typedef word2 type; };
template <> struct Access<1> { typedef uint32_t type; };

// Every word of every load feeds a value that every stored word depends on,
// so the compiler can neither drop nor narrow an access.
__device__ __forceinline__ uint32_t fold(const word4& w) { return w.x ^ w.y ^ w.z ^ w.w; }
__device__ __forceinline__ uint32_t fold(const word2& w) { return w.x ^ w.y; }
__device__ __forceinline__ uint32_t fold(uint32_t w) { return w; }

// Addressing as the fused kernels address a tile: a workgroup-uniform tile
// base (scalar registers) plus the lane's 32-bit byte offset, in the global
// address space, and each store's offset in a fresh register (a shared one
// makes the compiler form full 64-bit store addresses).
#define SR_GLOBAL __attribute__((address_space(1)))

template <int BYTES>
__device__ __forceinline__ typename Access<BYTES>::type load(const char* tile, uint32_t offset) {
  return __builtin_nontemporal_load((const SR_GLOBAL typename Access<BYTES>::type*)(tile + offset));
}
template <int BYTES>
__device__ __forceinline__ void store(char* tile, uint32_t offset, typename Access<BYTES>::type w) {
  __asm__("" : "+v"(offset));
  __builtin_nontemporal_store(w, (SR_GLOBAL typename Access<BYTES>::type*)(tile + offset));
}

// P, G, M, V: bytes per element of the parameter, the gradient and the two
// states (V = 0: one state).  Tile t covers elements [t * kTile, (t + 1) *
// kTile) < n.
template <int P, int G, int M, int V>
__global__ __launch_bounds__(kBlock) void streams(void* p, const void* g, void* m, void* v, uint32_t tiles) {
  const uint32_t t = sr::tile_of(blockIdx.y * gridDim.x + blockIdx.x, tiles);
  if (t >= tiles) return;
  const uint64_t first = static_cast<uint64_t>(t) * kTile;
  const uint32_t lane = threadIdx.x * kLanes;
  char* tp = static_cast<char*>(p) + first * P;
  const char* tg = static_cast<const char*>(g) + first * G;
  char* tm = static_cast<char*>(m) + first * M;
  char* tv = static_cast<char*>(v) + first * (V > 0 ? V : 1);
  // Every load is issued before any store, as in the fused kernels: the
  // pointers may alias as far as the compiler knows, so a load placed after
  // a store would wait for it.
  auto wp = load<P>(tp, lane * P);
  auto wg = load<G>(tg, lane * G);
  auto wm = load<M>(tm, lane * M);
  typename Access<(V > 0 ? V : 1)>::type wv{};
  if constexpr (V > 0) wv = load<V>(tv, lane * V);
  const uint32_t h = fold(wg) ^ fold(wp) ^ fold(wm) ^ fold(wv);
  wp ^= h;
  wm ^= h;
  wv ^= h;
  store<P>(tp, lane * P, wp);
  store<M>(tm, lane * M, wm);
  if constexpr (V > 0) store<V>(tv, lane * V, wv);
}

// The cast's pattern: 8 FP32 elements read and 8 narrower ones written per
// lane (OUT = 2 or 1 bytes), in workgroups of kCastBlock lanes as the cast
// kernel launches them.  Every output word takes bits of every input word.
constexpr int kCastBlock = 256;
constexpr int kCastLanes = 8;
constexpr uint32_t kCastTile = kCastBlock * kCastLanes;

template <int OUT>
__global__ __launch_bounds__(kCastBlock) void cast_streams(const void* x, void* y, uint32_t tiles) {
  const uint32_t t = sr::tile_of(blockIdx.y * gridDim.x + blockIdx.x, tiles);
  if (t >= tiles) return;
  // The cast's lane layout: two groups of 4 elements a workgroup-width apart.
  const uint64_t first = static_cast<uint64_t>(t) * kCastTile;
  const uint32_t i0 = threadIdx.x * kLanes, i1 = i0 + kCastBlock * kLanes;
  const char* tx = static_cast<const char*>(x) + first * 4;
  char* ty = static_cast<char*>(y) + first * OUT;
  const word4 a = load<4>(tx, i0 * 4), b = load<4>(tx, i1 * 4);
  if constexpr (OUT == 2) {
    store<2>(ty, i0 * 2, word2{(a.x >> 16) | (a.y & 0xFFFF0000u), (a.z >> 16) | (a.w & 0xFFFF0000u)});
    store<2>(ty, i1 * 2, word2{(b.x >> 16) | (b.y & 0xFFFF0000u), (b.z >> 16) | (b.w & 0xFFFF0000u)});
  } else {
    store<1>(ty, i0, (a.x >> 24) | ((a.y >> 16) & 0xFF00u) | ((a.z >> 8) & 0xFF0000u) | (a.w & 0xFF000000u));
    store<1>(ty, i1, (b.x >> 24) | ((b.y >> 16) & 0xFF00u) | ((b.z >> 8) & 0xFF0000u) | (b.w & 0xFF000000u));
  }
}

typedef void (*Kernel)(void*, const void*, void*, void*, uint32_t);

Kernel pick(int p, int g, int m, int v) {
  if (p == 4) {
    if (g == 4 && m == 2 && v == 2) return streams<4, 4, 2, 2>;
    if (g == 2 && m == 2 && v == 2) return streams<4, 2, 2, 2>;
    if (g == 4 && m == 1 && v == 2) return streams<4, 4, 1, 2>;
    if (g == 4 && m == 2 && v == 0) return streams<4, 4, 2, 0>;
    if (g == 4 && m == 4 && v == 4) return streams<4, 4, 4, 4>;
    if (g == 4 && m == 1 && v == 1) return streams<4, 4, 1, 1>;
    if (g == 4 && m == 4 && v == 0) return streams<4, 4, 4, 0>;
    if (g == 4 && m == 1 && v == 0) return streams<4, 4, 1, 0>;
  } else if (p == 2) {
    if (g == 2 && m == 2 && v == 2) return streams<2, 2, 2, 2>;
    if (g == 2 && m == 1 && v == 2) return streams<2, 2, 1, 2>;
    if (g == 2 && m == 2 && v == 0) return streams<2, 2, 2, 0>;
  }
  return nullptr;
}

// The placements the ceiling tries: gaps between consecutive stream bases in
// one allocation.  Where the streams land relative to each other moves the
// rate of this pattern by a few percent, so the ceiling is the best of
// several.
constexpr uint64_t kCeilingGaps[] = {0, 4096, 65536, 16ull << 20};
constexpr uint64_t kMaxGap = 16ull << 20;

// Times the trivial kernel for one placement: streams p, g, m, v (widths
// w[0..3], w[3] = 0 for one state) laid out from `slab` with `gap` bytes
// after each (every base a multiple of 256 bytes).  Returns the milliseconds
// per launch over `reps` launches after two untimed ones, or a negative
// value on a HIP error.
float time_placement(Kernel kernel, char* slab, const uint64_t (&bytes)[4], uint64_t gap, uint32_t tiles, int reps,
                     size_t lds, hipEvent_t start, hipEvent_t stop) {
  void* bases[4] = {nullptr, nullptr, nullptr, nullptr};
  uint64_t at = 0;
  for (int k = 0; k < 4; ++k) {
    if (bytes[k] == 0) continue;
    bases[k] = slab + at;
    at += (bytes[k] + 255) / 256 * 256 + gap;
  }
  const sr::LaunchShape shape = sr::launch_shape(tiles, kBlock);
  auto launch = [&] {
    hipLaunchKernelGGL(kernel, dim3(shape.x, shape.y), dim3(kBlock), lds, nullptr, bases[0], bases[1], bases[2],
                       bases[3], tiles);
  };
  launch();
  launch();
  if (hipGetLastError() != hipSuccess || hipEventRecord(start, nullptr) != hipSuccess) return -1.0f;
  for (int r = 0; r < reps; ++r) launch();
  float ms = 0.0f;
  if (hipGetLastError() != hipSuccess || hipEventRecord(stop, nullptr) != hipSuccess ||
      hipEventSynchronize(stop) != hipSuccess || hipEventElapsedTime(&ms, start, stop) != hipSuccess)
    return -1.0f;
  return ms / reps;
}

// Times `kernel` over n elements at each gap in gaps[0..count) (every gap at
// most kMaxGap) and each resident-workgroup cap in caps[0..ncaps) (0: none),
// writing milliseconds per launch to ms[cap_index * count + gap_index].
// Returns 0, or 2 for a HIP error (buffers are freed either way).
int time_placements(Kernel kernel, uint64_t n, const int (&widths)[4], const uint64_t* gaps, int count,
                    const uint32_t* caps, int ncaps, int reps, float* ms) {
  const uint32_t tiles = static_cast<uint32_t>(n / kTile);
  const uint64_t bytes[4] = {n * widths[0], n * widths[1], n * widths[2], n * widths[3]};
  uint64_t total = 0;
  for (uint64_t b : bytes) total += b ? (b + 255) / 256 * 256 + kMaxGap : 0;
  char* slab = nullptr;
  hipEvent_t start = nullptr, stop = nullptr;
  int rc = 2;
  do {
    if (hipDeviceSynchronize() != hipSuccess) break;
    if (hipMalloc(reinterpret_cast<void**>(&slab), total) != hipSuccess ||
        hipMemset(slab, 0x3A, total) != hipSuccess)
      break;
    if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) break;
    bool failed = false;
    for (int c = 0; c < ncaps && !failed; ++c) {
      const size_t lds = sr::cap_lds(reinterpret_cast<const void*>(kernel), kBlock, caps[c]);
      for (int i = 0; i < count && !failed; ++i) {
        float& out = ms[c * count + i];
        out = time_placement(kernel, slab, bytes, gaps[i], tiles, reps, lds, start, stop);
        failed = out < 0.0f;
      }
    }
    if (!failed) rc = 0;
  } while (false);
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  (void)hipDeviceSynchronize();
  if (slab) (void)hipFree(slab);
  return rc;
}

bool valid_streams(uint64_t n, int reps) { return n != 0 && n % kTile == 0 && n / kTile <= 0x7FFFF000ull && reps >= 1; }

// Parameters ~ U(-0.02, 0.02) and gradients ~ U(-1e-3, 1e-3) from a hash of
// the index: finite values that keep the fused update on its common path.
__global__ void fill_update_inputs(float* p, float* g, uint64_t n) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    const uint32_t h = sr::h32(static_cast<uint32_t>(i) ^ 0x5EEDu), k = sr::h32(h ^ 0x9E3779B9u);
    p[i] = ((h >> 8) * 0x1p-24f - 0.5f) * 0.04f;
    g[i] = ((k >> 8) * 0x1p-24f - 0.5f) * 2e-3f;
  }
}

}  // namespace

// Average milliseconds per launch of the trivial kernel over n elements with
// a parameter of p_bytes, a gradient of g_bytes and states of m_bytes and
// v_bytes per element (v_bytes 0: one state), over `reps` launches after two
// untimed ones, at the best of the placements kCeilingGaps and of three
// launch policies: no resident-workgroup cap, the cap of an 80 KiB budget
// for this pattern (sr::resident_cap, the library's for FP32 gradients) and
// half of it.  (With no arithmetic to wait
// for, the trivial kernel's workgroups are short-lived and it keeps enough
// bytes in flight with fewer of them: the north star's streams at 31 GB ran
// at 6.18 TB/s uncapped, 6.31 at 8 per CU and 6.38 at 4.)  Supported
// (p, g, m, v) patterns: FP32 parameters with (4,2,2), (2,2,2), (4,1,2),
// (4,2,0), (4,4,4), (4,1,1), (4,4,0), (4,1,0); BF16 parameters with (2,2,2),
// (2,1,2), (2,2,0).  n must be a positive multiple of 512 with n / 512 <=
// 2^31 - 4096 (the fused launches' tile limit); the grid is laid out as the
// fused launches lay it out (sr::launch_shape).  Returns 0, or 1 for an
// unsupported argument, 2 for a HIP error (buffers are freed either way).
extern "C" int sr_stream_ceiling_p(uint64_t n, int p_bytes, int g_bytes, int m_bytes, int v_bytes, int reps,
                                   float* avg_ms) {
  const Kernel kernel = pick(p_bytes, g_bytes, m_bytes, v_bytes);
  if (!kernel || !valid_streams(n, reps) || !avg_ms) return 1;
  const uint32_t per_element = 2 * p_bytes + g_bytes + 2 * m_bytes + 2 * v_bytes;
  const uint32_t rule =
      sr::resident_cap(static_cast<uint32_t>(n / kTile), kBlock, kLanes, per_element, p_bytes == 4);
  uint32_t caps[3] = {0, rule, rule / 2};
  const int ncaps = rule == 0 ? 1 : (rule / 2 == 0 ? 2 : 3);
  constexpr int kCount = sizeof(kCeilingGaps) / sizeof(kCeilingGaps[0]);
  float ms[3 * kCount];
  const int rc = time_placements(kernel, n, {p_bytes, g_bytes, m_bytes, v_bytes}, kCeilingGaps, kCount, caps, ncaps,
                                 reps, ms);
  if (rc != 0) return rc;
  float best = ms[0];
  for (int i = 0; i < ncaps * kCount; ++i) best = ms[i] < best ? ms[i] : best;
  *avg_ms = best;
  return 0;
}

// sr_stream_ceiling_p with an FP32 parameter.
extern "C" int sr_stream_ceiling(uint64_t n, int g_bytes, int m_bytes, int v_bytes, int reps, float* avg_ms) {
  return sr_stream_ceiling_p(n, 4, g_bytes, m_bytes, v_bytes, reps, avg_ms);
}

// Average milliseconds per launch of the cast-pattern kernel over n FP32
// elements written as out_bytes-wide ones (2 or 1), rotating through
// `buffers` input/output pairs (1-16) so that a pair is reused only after
// the others have passed through the caches, over `reps` launches after
// one untimed round.  n must be a positive multiple of 2048 with
// n / 2048 <= 2^31 - 4096.  Returns 0, 1 for an unsupported argument, or 2
// for a HIP error (buffers are freed either way).
extern "C" int sr_cast_ceiling(uint64_t n, int out_bytes, int buffers, int reps, float* avg_ms) {
  if ((out_bytes != 1 && out_bytes != 2) || buffers < 1 || buffers > 16 || n == 0 || n % kCastTile ||
      n / kCastTile > 0x7FFFF000ull || reps < 1 || !avg_ms)
    return 1;
  const uint32_t tiles = static_cast<uint32_t>(n / kCastTile);
  const sr::LaunchShape shape = sr::launch_shape(tiles, kCastBlock);
  void (*kernel)(const void*, void*, uint32_t) = out_bytes == 2 ? cast_streams<2> : cast_streams<1>;
  void* in[16] = {};
  void* out[16] = {};
  hipEvent_t start = nullptr, stop = nullptr;
  int rc = 2;
  do {
    if (hipDeviceSynchronize() != hipSuccess) break;
    bool ok = true;
    for (int k = 0; k < buffers && ok; ++k) {
      ok = hipMalloc(&in[k], n * 4) == hipSuccess && hipMemset(in[k], 0x3A, n * 4) == hipSuccess &&
           hipMalloc(&out[k], n * out_bytes) == hipSuccess;
    }
    if (!ok) break;
    if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) break;
    int turn = 0;
    auto launch = [&] {
      hipLaunchKernelGGL(kernel, dim3(shape.x, shape.y), dim3(kCastBlock), 0, nullptr, in[turn], out[turn], tiles);
      turn = (turn + 1) % buffers;
    };
    for (int k = 0; k < buffers; ++k) launch();
    if (hipGetLastError() != hipSuccess || hipEventRecord(start, nullptr) != hipSuccess) break;
    for (int r = 0; r < reps; ++r) launch();
    if (hipGetLastError() != hipSuccess || hipEventRecord(stop, nullptr) != hipSuccess ||
        hipEventSynchronize(stop) != hipSuccess)
      break;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, start, stop) != hipSuccess) break;
    *avg_ms = ms / reps;
    rc = 0;
  } while (false);
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  (void)hipDeviceSynchronize();
  for (int k = 0; k < 16; ++k) {
    if (in[k]) (void)hipFree(in[k]);
    if (out[k]) (void)hipFree(out[k]);
  }
  return rc;
}

// Milliseconds per launch of the trivial kernel (ms_trivial[i]) and of the
// library's fused AdamW kernel (ms_fused[i]) over one FP32 parameter and
// gradient and two BF16 moments of n elements (20 bytes per element), at
// resident-workgroup cap caps[i]: -1 for the library's rule
// (sr::resident_cap), 0 for none, 1-16 for that many workgroups per CU;
// resident[i] receives the workgroups per CU the fused launch allowed (the
// runtime's occupancy calculator).  Each is averaged over `reps` launches
// after two untimed ones; the two kernels alternate cap by cap.  n must be a
// positive multiple of 512 with n / 512 <= 2^31 - 4096, 1 <= ncaps <= 32.
// The buffers are allocated and freed here.  Returns 0, 1 for an
// unsupported argument, or 2 for a HIP error.
extern "C" int sr_launch_cap_sweep(uint64_t n, int reps, const int* caps, int ncaps, float* ms_trivial,
                                   float* ms_fused, int* resident) {
  if (!valid_streams(n, reps) || !caps || ncaps < 1 || ncaps > 32 || !ms_trivial || !ms_fused || !resident) return 1;
  for (int i = 0; i < ncaps; ++i)
    if (caps[i] < -1 || caps[i] > sr::kResidentCapOverrideMax) return 1;
  const uint32_t tiles = static_cast<uint32_t>(n / kTile);
  const sr::LaunchShape shape = sr::launch_shape(tiles, kBlock);
  auto fused = sr::adamw_kernel<sr::ENC_F32, sr::ENC_F32, sr::ENC_BF16_SR, sr::ENC_BF16_SR>;
  auto trivial = streams<4, 4, 2, 2>;
  char* slab = nullptr;
  hipEvent_t start = nullptr, stop = nullptr;
  int rc = 2;
  do {
    if (hipDeviceSynchronize() != hipSuccess || hipMalloc(reinterpret_cast<void**>(&slab), n * 12) != hipSuccess)
      break;
    float* p = reinterpret_cast<float*>(slab);
    float* g = p + n;
    char* m = slab + n * 8;
    char* v = m + n * 2;
    hipLaunchKernelGGL(fill_update_inputs, dim3(4096), dim3(256), 0, nullptr, p, g, n);
    if (hipGetLastError() != hipSuccess || hipMemset(m, 0, n * 4) != hipSuccess) break;
    if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) break;
    sr::AdamWArgs a{};
    a.inline_row.ptr[0] = reinterpret_cast<uint64_t>(p);
    a.inline_row.ptr[1] = reinterpret_cast<uint64_t>(g);
    a.inline_row.ptr[2] = reinterpret_cast<uint64_t>(m);
    a.inline_row.ptr[3] = reinterpret_cast<uint64_t>(v);
    a.inline_row.numel = static_cast<int64_t>(n);
    a.inline_row.tile_end = tiles;
    a.inline_row.param_index = 7;
    a.inline_row.flags = SR_ROW_VECTOR | SR_ROW_KEYED;
    // lr 3e-4, betas (0.9, 0.999), eps 1e-8, weight decay 0.01 at step 1.
    a.s = {0.9f, 0.999f, 0.1f, 0.001f, -3e-3f, 0.0316227766f, 1.0f - 3e-6f, 1e-8f, 1.0f / 0.0316227766f};
    a.total_tiles = tiles;
    bool failed = false;
    for (int i = 0; i < ncaps && !failed; ++i) {
      const uint32_t cap = caps[i] < 0 ? sr::resident_cap(tiles, kBlock, kLanes, 20, true) : caps[i];
      for (int kind = 0; kind < 2 && !failed; ++kind) {
        const void* fn = kind ? reinterpret_cast<const void*>(fused) : reinterpret_cast<const void*>(trivial);
        const size_t lds = sr::cap_lds(fn, kBlock, cap);
        if (kind && hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident[i], fn, kBlock, lds) != hipSuccess) {
          failed = true;
          break;
        }
        auto launch = [&] {
          if (kind) hipLaunchKernelGGL(fused, dim3(shape.x, shape.y), dim3(kBlock), lds, nullptr, a);
          else hipLaunchKernelGGL(trivial, dim3(shape.x, shape.y), dim3(kBlock), lds, nullptr, p, g, m, v, tiles);
        };
        launch();
        launch();
        float ms = 0.0f;
        if (hipGetLastError() != hipSuccess || hipEventRecord(start, nullptr) != hipSuccess) {
          failed = true;
          break;
        }
        for (int r = 0; r < reps; ++r) launch();
        if (hipGetLastError() != hipSuccess || hipEventRecord(stop, nullptr) != hipSuccess ||
            hipEventSynchronize(stop) != hipSuccess || hipEventElapsedTime(&ms, start, stop) != hipSuccess) {
          failed = true;
          break;
        }
        (kind ? ms_fused : ms_trivial)[i] = ms / reps;
      }
    }
    if (!failed) rc = 0;
  } while (false);
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  (void)hipDeviceSynchronize();
  if (slab) (void)hipFree(slab);
  return rc;
}
