// The bandwidth ceiling of a fused update's access pattern, measured.
//
// A kernel with trivial arithmetic (XORs) that moves exactly the
// streams of one fused-update launch: a parameter (FP32 or BF16) read and
// written, a gradient read, and one or two states read and written, with the product's
// tile shape (128 lanes x 4 elements), its XCD-chunked tile order
// (sr_tile_order.h) and its non-temporal accesses.  Whatever rate this
// kernel reaches for n elements is what the memory system gives that access
// pattern at that footprint; the fused kernels do strictly more work per
// byte, so their rate over this one says how much of the reachable
// bandwidth their arithmetic and table lookups cost.
//
// sr_cast_ceiling does the same for the cast's pattern (FP32 in, a 2- or
// 1-byte format out) with the cast's launch shape.
//
// Measurement helper only: bench.py reports it beside the fused kernel's
// rate and tests/test_gpu_stream_ceiling.py checks the fused kernels against
// it.  It allocates its own buffers, so it never touches caller memory.
#include <hip/hip_runtime.h>

#include <cstdint>

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

template <int BYTES>
__device__ __forceinline__ typename Access<BYTES>::type load(const void* base, uint64_t i) {
  return __builtin_nontemporal_load(
      reinterpret_cast<const typename Access<BYTES>::type*>(static_cast<const char*>(base) + i * BYTES));
}
template <int BYTES>
__device__ __forceinline__ void store(void* base, uint64_t i, typename Access<BYTES>::type w) {
  __builtin_nontemporal_store(
      w, reinterpret_cast<typename Access<BYTES>::type*>(static_cast<char*>(base) + i * BYTES));
}

// P, G, M, V: bytes per element of the parameter, the gradient and the two
// states (V = 0: one state).  Tile t covers elements [t * kTile, (t + 1) *
// kTile) < n.
template <int P, int G, int M, int V>
__global__ __launch_bounds__(kBlock) void streams(void* p, const void* g, void* m, void* v, uint32_t tiles) {
  const uint32_t t = sr::tile_of(blockIdx.y * gridDim.x + blockIdx.x, tiles);
  if (t >= tiles) return;
  const uint64_t i = static_cast<uint64_t>(t) * kTile + threadIdx.x * kLanes;
  // Every load is issued before any store, as in the fused kernels: the
  // pointers may alias as far as the compiler knows, so a load placed after
  // a store would wait for it.
  auto wp = load<P>(p, i);
  auto wg = load<G>(g, i);
  auto wm = load<M>(m, i);
  typename Access<(V > 0 ? V : 1)>::type wv{};
  if constexpr (V > 0) wv = load<V>(v, i);
  const uint32_t h = fold(wg) ^ fold(wp) ^ fold(wm) ^ fold(wv);
  wp ^= h;
  wm ^= h;
  wv ^= h;
  store<P>(p, i, wp);
  store<M>(m, i, wm);
  if constexpr (V > 0) store<V>(v, i, wv);
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
  const uint64_t i0 = static_cast<uint64_t>(t) * kCastTile + threadIdx.x * kLanes;
  const uint64_t i1 = i0 + kCastBlock * kLanes;
  const word4 a = load<4>(x, i0), b = load<4>(x, i1);
  if constexpr (OUT == 2) {
    __builtin_nontemporal_store(word2{(a.x >> 16) | (a.y & 0xFFFF0000u), (a.z >> 16) | (a.w & 0xFFFF0000u)},
                                reinterpret_cast<word2*>(static_cast<char*>(y) + i0 * 2));
    __builtin_nontemporal_store(word2{(b.x >> 16) | (b.y & 0xFFFF0000u), (b.z >> 16) | (b.w & 0xFFFF0000u)},
                                reinterpret_cast<word2*>(static_cast<char*>(y) + i1 * 2));
  } else {
    __builtin_nontemporal_store((a.x >> 24) | ((a.y >> 16) & 0xFF00u) | ((a.z >> 8) & 0xFF0000u) | (a.w & 0xFF000000u),
                                reinterpret_cast<uint32_t*>(static_cast<char*>(y) + i0));
    __builtin_nontemporal_store((b.x >> 24) | ((b.y >> 16) & 0xFF00u) | ((b.z >> 8) & 0xFF0000u) | (b.w & 0xFF000000u),
                                reinterpret_cast<uint32_t*>(static_cast<char*>(y) + i1));
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

}  // namespace

// Average milliseconds per launch of the trivial kernel over n elements with
// a parameter of p_bytes, a gradient of g_bytes and states of m_bytes and
// v_bytes per element (v_bytes 0: one state), over `reps` launches after two
// untimed ones.  Supported (p, g, m, v) patterns: FP32 parameters with
// (4,2,2), (2,2,2), (4,1,2), (4,2,0), (4,4,4), (4,1,1), (4,4,0), (4,1,0);
// BF16 parameters with (2,2,2), (2,1,2), (2,2,0).  n must be a positive
// multiple of 512 with n / 512 <= 2^31 - 4096 (the fused launches' tile
// limit); the grid is laid out as the fused launches lay it out
// (sr::launch_shape).  Returns 0, or 1 for an unsupported argument, 2 for a
// HIP error (buffers are freed either way).
extern "C" int sr_stream_ceiling_p(uint64_t n, int p_bytes, int g_bytes, int m_bytes, int v_bytes, int reps,
                                   float* avg_ms) {
  const Kernel kernel = pick(p_bytes, g_bytes, m_bytes, v_bytes);
  if (!kernel || n == 0 || n % kTile || n / kTile > 0x7FFFF000ull || reps < 1 || !avg_ms) return 1;
  const uint32_t tiles = static_cast<uint32_t>(n / kTile);
  const sr::LaunchShape shape = sr::launch_shape(tiles, kBlock);
  const size_t bytes[4] = {n * p_bytes, n * g_bytes, n * m_bytes, n * v_bytes};
  void* buf[4] = {nullptr, nullptr, nullptr, nullptr};
  hipEvent_t start = nullptr, stop = nullptr;
  int rc = 2;
  do {
    if (hipDeviceSynchronize() != hipSuccess) break;
    bool ok = true;
    for (int k = 0; k < 4 && ok; ++k) {
      if (bytes[k] == 0) continue;
      ok = hipMalloc(&buf[k], bytes[k]) == hipSuccess && hipMemset(buf[k], 0x3A, bytes[k]) == hipSuccess;
    }
    if (!ok) break;
    if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) break;
    auto launch = [&] {
      hipLaunchKernelGGL(kernel, dim3(shape.x, shape.y), dim3(kBlock), 0, nullptr, buf[0], buf[1], buf[2], buf[3],
                         tiles);
    };
    launch();
    launch();
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
  for (void* b : buf)
    if (b) (void)hipFree(b);
  return rc;
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
