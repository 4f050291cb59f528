// sr_abi.hip -- extern "C" entry points of libsr_states_hip.so.
//
// Validation of dtypes, rules, sizes and launch shapes happens here; the
// Python layer validates tensors, layouts and hyperparameters before it
// calls in.  Launches go through hipLaunchKernel with the kernel's host stub
// so that instantiations can live in separately compiled units.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/sr_states_hip.h"
#include "sr_kernels.h"
#include "sr_launch_cap.h"

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(hipError_t err, const char* what) {
  return fail(SR_ERR_HIP, "%s failed: %s (%d)", what, hipGetErrorString(err), static_cast<int>(err));
}

struct Tables {
  sr::KernelTableAdamW adamw{};
  sr::KernelTableSgdm sgdm{};
  sr::KernelTableCast cast{};
  sr::KernelTableNeighbors neighbors{};
};

const Tables& tables() {
  static const Tables t = [] {
    Tables r{};
    sr::register_adamw_m0(r.adamw);
    sr::register_adamw_m1(r.adamw);
    sr::register_adamw_m2(r.adamw);
    sr::register_adamw_m3(r.adamw);
    sr::register_adamw_m4(r.adamw);
    sr::register_adamw_m5(r.adamw);
    sr::register_adamw_m6(r.adamw);
    sr::register_adamw_m7(r.adamw);
    sr::register_adamw_m8(r.adamw);
    sr::register_sgdm(r.sgdm);
    sr::register_cast(r.cast);
    sr::register_neighbors(r.neighbors);
    return r;
  }();
  return t;
}

// (dtype, rule) -> storage encoding index, or -1.
int state_enc(int dtype, int rule) {
  if (rule != SR_NEAREST && rule != SR_STOCHASTIC) return -1;
  switch (dtype) {
    case SR_F32: return sr::ENC_F32;
    case SR_BF16: return rule == SR_STOCHASTIC ? sr::ENC_BF16_SR : sr::ENC_BF16_RN;
    case SR_F16: return rule == SR_STOCHASTIC ? sr::ENC_F16_SR : sr::ENC_F16_RN;
    case SR_E4M3: return rule == SR_STOCHASTIC ? sr::ENC_E4M3_SR : sr::ENC_E4M3_RN;
    case SR_E5M2: return rule == SR_STOCHASTIC ? sr::ENC_E5M2_SR : sr::ENC_E5M2_RN;
    default: return -1;
  }
}

// Parameter / gradient storage -> table index (FP32 0, BF16 1), or -1.
int pg_index(int dtype) { return dtype == SR_F32 ? 0 : (dtype == SR_BF16 ? 1 : -1); }

// Encoding of a parameter or gradient table index (FP32, or BF16 nearest).
int param_enc(int index) { return index == 0 ? sr::ENC_F32 : sr::ENC_BF16_RN; }

bool valid_block(int block) { return block >= 64 && block <= sr::kMaxBlock && block % 64 == 0; }

// One workgroup per tile; the grid is padded to a whole number of XCD chunk
// rounds so that the kernels' tile order (sr_tile_order.h) is a permutation,
// and split into rows when one dimension would carry 2^32 or more
// work-items (2^34 elements at four per lane).  `tiles` must equal the
// total_tiles the kernel argument carries.  `cap` > 0 limits the resident
// workgroups per CU to that many (sr::cap_lds).
int launch(const void* fn, int block, uint32_t tiles, void* arg, void* stream, uint32_t cap = 0) {
  if (sr::padded_grid(tiles) > 0x7FFFFFFFull) return fail(SR_ERR_ARGUMENT, "%u tiles exceed the grid limit", tiles);
  const sr::LaunchShape shape = sr::launch_shape(tiles, static_cast<uint32_t>(block));
  void* args[] = {arg};
  hipError_t err = hipLaunchKernel(fn, dim3(shape.x, shape.y), dim3(block), args, sr::cap_lds(fn, block, cap),
                                   static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return hip_fail(err, "hipLaunchKernel");
  return SR_OK;
}

// SR_STATES_RESIDENT_CAP, read once (sr::resident_cap_override): the cap of
// every launch of at least 2^16 tiles, or -1 for the rule.
int cap_override() {
  static const int value = sr::resident_cap_override(std::getenv("SR_STATES_RESIDENT_CAP"));
  return value;
}

// Whether an encoding rounds stochastically to FP16 or FP8.
bool minifloat_sr(int enc) { return enc == sr::ENC_F16_SR || enc == sr::ENC_E4M3_SR || enc == sr::ENC_E5M2_SR; }

// Resident-workgroup cap of an AdamW launch (sr::resident_cap).
uint32_t adamw_cap(int pi, int gi, int me, int ve, int block, uint32_t tiles) {
  if (cap_override() >= 0) return tiles >= sr::kResidentCapMinTiles ? static_cast<uint32_t>(cap_override()) : 0u;
  const int bytes = 2 * sr::enc_bytes(param_enc(pi)) + sr::enc_bytes(param_enc(gi)) + 2 * sr::enc_bytes(me) +
                    2 * sr::enc_bytes(ve);
  const uint32_t in_flight = sr::adamw_in_flight(gi == 1, minifloat_sr(me) && minifloat_sr(ve));
  return sr::resident_cap(tiles, static_cast<uint32_t>(block),
                          static_cast<uint32_t>(sr::lane_elements(param_enc(pi), param_enc(gi), me, ve)),
                          static_cast<uint32_t>(bytes), pi == 0, in_flight);
}

// Resident-workgroup cap of a momentum-SGD launch.
uint32_t sgdm_cap(int pi, int gi, int ue, int block, uint32_t tiles) {
  if (cap_override() >= 0) return tiles >= sr::kResidentCapMinTiles ? static_cast<uint32_t>(cap_override()) : 0u;
  const int bytes = 2 * sr::enc_bytes(param_enc(pi)) + sr::enc_bytes(param_enc(gi)) + 2 * sr::enc_bytes(ue);
  return sr::resident_cap(tiles, static_cast<uint32_t>(block),
                          static_cast<uint32_t>(sr::lane_elements(param_enc(pi), param_enc(gi), ue, ue)),
                          static_cast<uint32_t>(bytes), pi == 0, sr::sgdm_in_flight(ue == sr::ENC_F16_SR));
}

// Tiles of block * lanes elements covering n elements, or fail if they do
// not fit 32-bit tile indices.
int tiles_for(int64_t n, int block, int lanes, uint32_t* tiles) {
  const int64_t tile = static_cast<int64_t>(block) * lanes;
  const int64_t count = (n + tile - 1) / tile;
  if (count > 0xFFFFFFFFll) return fail(SR_ERR_ARGUMENT, "%lld elements exceed the tile index range", (long long)n);
  *tiles = static_cast<uint32_t>(count);
  return SR_OK;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

sr::AdamWScalars adamw_scalars(const sr_adamw_hparams& h) {
  return {h.beta1, h.beta2, h.one_minus_beta1, h.one_minus_beta2,
          h.neg_step_size, h.correction2_sqrt, h.decay, h.eps, 1.0f / h.correction2_sqrt};
}

// correction2_sqrt in [2^-27, 1] (sr_math.h, div_by_constant); NaN fails.
bool valid_correction(const sr_adamw_hparams& h) {
  return h.correction2_sqrt >= sr::kMinCorrection2Sqrt && h.correction2_sqrt <= 1.0f;
}

// ---------------------------------------------------------------------------
// Scratch of the entry point that allocates nothing (sr_adamw_multi_noalloc).
// One static device array per GPU holds the bucket's row records, its per-row
// scalars and the tile-to-row map, in that order; each call overwrites the
// parts it uses, so nothing needs clearing.  Calls that overlap on one GPU
// share it and race.
// ---------------------------------------------------------------------------
constexpr size_t kScratchRowBytes = size_t{SR_NOALLOC_MAX_ROWS} * sizeof(sr_row);
constexpr size_t kScratchScalarBytes = size_t{SR_NOALLOC_MAX_ROWS} * 2 * sizeof(float);
constexpr size_t kScratchTileBytes = size_t{SR_NOALLOC_MAX_TILES} * sizeof(uint32_t);
static_assert(kScratchRowBytes % 256 == 0 && kScratchScalarBytes % 256 == 0, "regions stay 256-byte aligned");

static __device__ __align__(256) unsigned char scratch[kScratchRowBytes + kScratchScalarBytes + kScratchTileBytes];

// Device address of `scratch` on each GPU, looked up once per device with
// that device current.  The array's name in host code is only a handle for
// the lookup, never an address to pass to a kernel or a copy.
constexpr int kMaxDevices = 64;

struct ScratchSlot {
  std::once_flag once;
  void* base = nullptr;
  hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kMaxDevices];

int scratch_base(void* stream, unsigned char** base) {
  int device = 0;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) return hip_fail(err, "hipGetDevice");
  if (device < 0 || device >= kMaxDevices) return fail(SR_ERR_ARGUMENT, "device %d has no scratch slot", device);
  if (stream) {
    hipDevice_t owner = 0;
    err = hipStreamGetDevice(static_cast<hipStream_t>(stream), &owner);
    if (err != hipSuccess) return hip_fail(err, "hipStreamGetDevice");
    if (owner != device)
      return fail(SR_ERR_ARGUMENT, "stream belongs to device %d, but device %d is current", owner, device);
  }
  ScratchSlot& slot = g_scratch[device];
  std::call_once(slot.once, [&slot] { slot.err = hipGetSymbolAddress(&slot.base, HIP_SYMBOL(scratch)); });
  if (slot.err != hipSuccess) return hip_fail(slot.err, "hipGetSymbolAddress(scratch)");
  *base = static_cast<unsigned char*>(slot.base);
  return SR_OK;
}

// tile_rows[t] = the row whose tile range holds t, found by binary search
// over the rows' first tiles (host-checked: they start at 0, increase and
// cover [0, total_tiles) without gaps).  The threads of a wave hold
// neighbouring tiles and mostly read the same records.
constexpr int kFillBlock = 256;

__global__ __launch_bounds__(kFillBlock) void fill_tile_rows(const sr_row* rows, int nrows, uint32_t* tile_rows,
                                                             uint32_t total_tiles) {
  const uint32_t t = blockIdx.x * kFillBlock + threadIdx.x;
  if (t >= total_tiles) return;
  int lo = 0, hi = nrows - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (rows[mid].tile_begin <= t) lo = mid;
    else hi = mid - 1;
  }
  tile_rows[t] = static_cast<uint32_t>(lo);
}

// Under stream capture the copies of the host tables become graph nodes that
// read the tables again at every replay, so they must be pinned (page-locked)
// host memory that outlives the graph; pageable tables are refused before
// anything is recorded.  Eager calls take either kind.
int check_capture_tables(hipStream_t stream, const void* rows, const void* row_scalars) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  hipError_t err = hipStreamIsCapturing(stream, &status);
  if (err != hipSuccess) return hip_fail(err, "hipStreamIsCapturing");
  if (status == hipStreamCaptureStatusNone) return SR_OK;
  const void* tables[2] = {rows, row_scalars};
  for (const void* table : tables) {
    if (!table) continue;
    hipPointerAttribute_t attributes{};
    err = hipPointerGetAttributes(&attributes, table);
    if (err != hipSuccess) (void)hipGetLastError();  // an unknown pointer: not pinned
    if (err != hipSuccess || attributes.type != hipMemoryTypeHost)
      return fail(SR_ERR_ARGUMENT,
                  "under stream capture, rows and row_scalars must be pinned host memory that stays unchanged "
                  "while the graph can replay");
  }
  return SR_OK;
}

// The checks sr_adamw_multi leaves to its caller, made on the host copy.
int check_host_rows(const sr_row* rows, const float* row_scalars, int nrows, uint32_t total_tiles,
                    int64_t tile_elements) {
  uint32_t next = 0;
  for (int r = 0; r < nrows; ++r) {
    const sr_row& row = rows[r];
    if (row.numel < 1) return fail(SR_ERR_ARGUMENT, "row %d: numel %lld below 1", r, (long long)row.numel);
    if (row.tile_begin != next) return fail(SR_ERR_ARGUMENT, "row %d: tiles start at %u, expected %u", r, row.tile_begin, next);
    const int64_t tiles = (row.numel + tile_elements - 1) / tile_elements;
    if (static_cast<int64_t>(row.tile_end) - row.tile_begin != tiles)
      return fail(SR_ERR_ARGUMENT, "row %d: %u tiles for %lld elements, expected %lld", r,
                  row.tile_end - row.tile_begin, (long long)row.numel, (long long)tiles);
    if (row.flags & ~(SR_ROW_VECTOR | SR_ROW_KEYED)) return fail(SR_ERR_ARGUMENT, "row %d: unknown flags %#x", r, row.flags);
    for (int k = 0; k < 4; ++k) {
      if (!row.ptr[k]) return fail(SR_ERR_ARGUMENT, "row %d: null pointer %d", r, k);
      if ((row.flags & SR_ROW_VECTOR) && (row.ptr[k] & 15u))
        return fail(SR_ERR_ARGUMENT, "row %d: pointer %d not 16-byte aligned on a vector row", r, k);
    }
    if (row_scalars) {
      const float c = row_scalars[2 * r + 1];
      if (!(c >= sr::kMinCorrection2Sqrt && c <= 1.0f))
        return fail(SR_ERR_ARGUMENT, "row %d: correction2_sqrt %g outside [2^-27, 1]", r, (double)c);
    }
    next = row.tile_end;
  }
  if (next != total_tiles) return fail(SR_ERR_ARGUMENT, "rows cover %u tiles, total_tiles is %u", next, total_tiles);
  return SR_OK;
}

}  // namespace

extern "C" {

int sr_abi_version(void) { return SR_ABI_VERSION; }

const char* sr_last_error(void) { return g_error.c_str(); }

int sr_lane_elements(int p_dtype, int g_dtype, int state0_dtype, int state1_dtype) {
  // Rounding rules do not change widths; the nearest-rule encodings stand in.
  const int p = state_enc(p_dtype, SR_NEAREST), g = state_enc(g_dtype, SR_NEAREST);
  const int a = state_enc(state0_dtype, SR_NEAREST), b = state_enc(state1_dtype, SR_NEAREST);
  if (p < 0 || g < 0 || a < 0 || b < 0) return 0;
  return sr::lane_elements(p, g, a, b);
}

uint32_t sr_update_key(uint64_t seed, uint64_t step, uint32_t param_index) {
  return sr::update_key(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32),
                        static_cast<uint32_t>(step), static_cast<uint32_t>(step >> 32), param_index);
}

uint32_t sr_state_key(uint32_t key, uint32_t state_index) { return sr::state_key(key, state_index); }

int sr_cast(const void* x, void* y, int64_t n, int dtype, int rule, uint32_t seed, uint32_t offset,
            int block_size, void* stream) {
  const int enc = state_enc(dtype, rule);
  if (enc < 0) return fail(SR_ERR_ARGUMENT, "unsupported cast dtype %d / rule %d", dtype, rule);
  if (!valid_block(block_size)) return fail(SR_ERR_ARGUMENT, "invalid block size %d", block_size);
  if (n < 0) return fail(SR_ERR_ARGUMENT, "negative element count");
  if (n == 0) return SR_OK;
  if (!x || !y) return fail(SR_ERR_ARGUMENT, "null pointer");
  sr::CastArgs a{};
  a.x = static_cast<const float*>(x);
  a.y = y;
  a.n = n;
  a.counter_base = seed + offset;
  a.vector_ok = aligned16(x) && aligned16(y);
  if (int rc = tiles_for(n, block_size, sr::kCastLaneElements, &a.total_tiles)) return rc;
  const bool cached_loads = n <= sr::kCachedCastMaxElements;
  return launch(tables().cast[cached_loads][enc], block_size, a.total_tiles, &a, stream);
}

int sr_neighbors(const void* x, void* lower, void* upper, int64_t n, int dtype, void* stream) {
  if (dtype != SR_BF16 && dtype != SR_F16 && dtype != SR_E4M3 && dtype != SR_E5M2)
    return fail(SR_ERR_ARGUMENT, "neighbors support BF16, FP16, E4M3 and E5M2, not dtype %d", dtype);
  if (n < 0) return fail(SR_ERR_ARGUMENT, "negative element count");
  if (n == 0) return SR_OK;
  if (!x || !lower || !upper) return fail(SR_ERR_ARGUMENT, "null pointer");
  sr::NeighborArgs a{static_cast<const float*>(x), lower, upper, n};
  // Enough workgroups to fill the chip; the kernel's grid-stride loop covers
  // any n with them.
  constexpr int64_t kMaxGroups = 8192;
  const int64_t groups = (n + sr::kNeighborBlock - 1) / sr::kNeighborBlock;
  void* args[] = {&a};
  const hipError_t err =
      hipLaunchKernel(tables().neighbors[state_enc(dtype, SR_NEAREST)],
                      dim3(static_cast<uint32_t>(groups < kMaxGroups ? groups : kMaxGroups)),
                      dim3(sr::kNeighborBlock), args, 0, static_cast<hipStream_t>(stream));
  if (err != hipSuccess) return hip_fail(err, "hipLaunchKernel");
  return SR_OK;
}

int sr_adamw_step(void* p, const void* g, void* m, void* v, int64_t n, int p_dtype, int g_dtype,
                  int m_dtype, int m_rule, int v_dtype, int v_rule, const sr_adamw_hparams* hp,
                  uint32_t key, uint32_t offset, int block_size, void* stream) {
  const int pi = pg_index(p_dtype), gi = pg_index(g_dtype);
  const int me = state_enc(m_dtype, m_rule), ve = state_enc(v_dtype, v_rule);
  if (pi < 0 || gi < 0) return fail(SR_ERR_ARGUMENT, "parameter and gradient must be FP32 or BF16");
  if (me < 0 || ve < 0) return fail(SR_ERR_ARGUMENT, "unsupported state dtype or rule");
  if (!valid_block(block_size)) return fail(SR_ERR_ARGUMENT, "invalid block size %d", block_size);
  if (!hp) return fail(SR_ERR_ARGUMENT, "null hyperparameters");
  if (!valid_correction(*hp))
    return fail(SR_ERR_ARGUMENT, "correction2_sqrt %g outside [2^-27, 1]", (double)hp->correction2_sqrt);
  if (n < 0) return fail(SR_ERR_ARGUMENT, "negative element count");
  if (n == 0) return SR_OK;
  if (!p || !g || !m || !v) return fail(SR_ERR_ARGUMENT, "null pointer");
  sr::AdamWArgs a{};
  a.rows = nullptr;
  a.tile_rows = nullptr;
  a.s = adamw_scalars(*hp);
  const int lanes = sr::lane_elements(param_enc(pi), param_enc(gi), me, ve);
  if (int rc = tiles_for(n, block_size, lanes, &a.total_tiles)) return rc;
  sr_row& r = a.inline_row;
  r.ptr[0] = reinterpret_cast<uint64_t>(p);
  r.ptr[1] = reinterpret_cast<uint64_t>(g);
  r.ptr[2] = reinterpret_cast<uint64_t>(m);
  r.ptr[3] = reinterpret_cast<uint64_t>(v);
  r.numel = n;
  r.tile_begin = 0;
  r.tile_end = a.total_tiles;
  r.param_index = key;
  r.shard_start = offset;
  r.flags = SR_ROW_KEYED |
            ((aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v)) ? SR_ROW_VECTOR : 0u);
  return launch(tables().adamw[pi][gi][me][ve], block_size, a.total_tiles, &a, stream,
                adamw_cap(pi, gi, me, ve, block_size, a.total_tiles));
}

int sr_adamw_multi(const sr_row* rows, const uint32_t* tile_rows, const float* row_scalars,
                   int nrows, uint32_t total_tiles,
                   int p_dtype, int g_dtype,
                   int m_dtype, int m_rule, int v_dtype, int v_rule, const sr_adamw_hparams* hp,
                   uint64_t seed, uint64_t rng_step, int block_size, void* stream) {
  const int pi = pg_index(p_dtype), gi = pg_index(g_dtype);
  const int me = state_enc(m_dtype, m_rule), ve = state_enc(v_dtype, v_rule);
  if (pi < 0 || gi < 0) return fail(SR_ERR_ARGUMENT, "parameter and gradient must be FP32 or BF16");
  if (me < 0 || ve < 0) return fail(SR_ERR_ARGUMENT, "unsupported state dtype or rule");
  if (!valid_block(block_size)) return fail(SR_ERR_ARGUMENT, "invalid block size %d", block_size);
  if (!hp || !rows || !tile_rows) return fail(SR_ERR_ARGUMENT, "null argument");
  if (!valid_correction(*hp))
    return fail(SR_ERR_ARGUMENT, "correction2_sqrt %g outside [2^-27, 1]", (double)hp->correction2_sqrt);
  if (nrows < 1) return fail(SR_ERR_ARGUMENT, "row count %d below 1", nrows);
  if (total_tiles == 0) return fail(SR_ERR_ARGUMENT, "empty tile range");
  sr::AdamWArgs a{};
  a.rows = rows;
  a.tile_rows = tile_rows;
  a.row_scalars = row_scalars;
  a.total_tiles = total_tiles;
  a.s = adamw_scalars(*hp);
  a.key_prefix = sr::update_key_prefix(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32),
                                       static_cast<uint32_t>(rng_step),
                                       static_cast<uint32_t>(rng_step >> 32));
  return launch(tables().adamw[pi][gi][me][ve], block_size, total_tiles, &a, stream,
                adamw_cap(pi, gi, me, ve, block_size, total_tiles));
}

int sr_sgdm_step(void* p, const void* g, void* u, int64_t n, int p_dtype, int g_dtype, int u_dtype,
                 int u_rule, const sr_sgdm_hparams* hp, uint32_t key, uint32_t offset,
                 int block_size, void* stream) {
  const int pi = pg_index(p_dtype), gi = pg_index(g_dtype);
  const int ue = state_enc(u_dtype, u_rule);
  if (pi < 0 || gi < 0) return fail(SR_ERR_ARGUMENT, "parameter and gradient must be FP32 or BF16");
  if (ue < 0) return fail(SR_ERR_ARGUMENT, "unsupported state dtype or rule");
  if (!valid_block(block_size)) return fail(SR_ERR_ARGUMENT, "invalid block size %d", block_size);
  if (!hp) return fail(SR_ERR_ARGUMENT, "null hyperparameters");
  if (n < 0) return fail(SR_ERR_ARGUMENT, "negative element count");
  if (n == 0) return SR_OK;
  if (!p || !g || !u) return fail(SR_ERR_ARGUMENT, "null pointer");
  sr::SgdmArgs a{};
  a.rows = nullptr;
  a.tile_rows = nullptr;
  a.s = {hp->momentum, hp->neg_lr};
  const int lanes = sr::lane_elements(param_enc(pi), param_enc(gi), ue, ue);
  if (int rc = tiles_for(n, block_size, lanes, &a.total_tiles)) return rc;
  sr_row& r = a.inline_row;
  r.ptr[0] = reinterpret_cast<uint64_t>(p);
  r.ptr[1] = reinterpret_cast<uint64_t>(g);
  r.ptr[2] = reinterpret_cast<uint64_t>(u);
  r.ptr[3] = 0;
  r.numel = n;
  r.tile_begin = 0;
  r.tile_end = a.total_tiles;
  r.param_index = key;
  r.shard_start = offset;
  r.flags = SR_ROW_KEYED | ((aligned16(p) && aligned16(g) && aligned16(u)) ? SR_ROW_VECTOR : 0u);
  return launch(tables().sgdm[pi][gi][ue], block_size, a.total_tiles, &a, stream,
                sgdm_cap(pi, gi, ue, block_size, a.total_tiles));
}

int sr_sgdm_multi(const sr_row* rows, const uint32_t* tile_rows, int nrows, uint32_t total_tiles,
                  int p_dtype, int g_dtype,
                  int u_dtype, int u_rule, const sr_sgdm_hparams* hp, uint64_t seed,
                  uint64_t rng_step, int block_size, void* stream) {
  const int pi = pg_index(p_dtype), gi = pg_index(g_dtype);
  const int ue = state_enc(u_dtype, u_rule);
  if (pi < 0 || gi < 0) return fail(SR_ERR_ARGUMENT, "parameter and gradient must be FP32 or BF16");
  if (ue < 0) return fail(SR_ERR_ARGUMENT, "unsupported state dtype or rule");
  if (!valid_block(block_size)) return fail(SR_ERR_ARGUMENT, "invalid block size %d", block_size);
  if (!hp || !rows || !tile_rows) return fail(SR_ERR_ARGUMENT, "null argument");
  if (nrows < 1) return fail(SR_ERR_ARGUMENT, "row count %d below 1", nrows);
  if (total_tiles == 0) return fail(SR_ERR_ARGUMENT, "empty tile range");
  sr::SgdmArgs a{};
  a.rows = rows;
  a.tile_rows = tile_rows;
  a.total_tiles = total_tiles;
  a.s = {hp->momentum, hp->neg_lr};
  a.key_prefix = sr::update_key_prefix(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32),
                                       static_cast<uint32_t>(rng_step),
                                       static_cast<uint32_t>(rng_step >> 32));
  return launch(tables().sgdm[pi][gi][ue], block_size, total_tiles, &a, stream,
                sgdm_cap(pi, gi, ue, block_size, total_tiles));
}

int sr_adamw_multi_noalloc(const sr_row* rows, const float* row_scalars, int nrows, uint32_t total_tiles,
                           int p_dtype, int g_dtype, int m_dtype, int m_rule, int v_dtype, int v_rule,
                           const sr_adamw_hparams* hp, uint64_t seed, uint64_t rng_step, int block_size,
                           void* stream) {
  const int pi = pg_index(p_dtype), gi = pg_index(g_dtype);
  const int me = state_enc(m_dtype, m_rule), ve = state_enc(v_dtype, v_rule);
  if (pi < 0 || gi < 0) return fail(SR_ERR_ARGUMENT, "parameter and gradient must be FP32 or BF16");
  if (me < 0 || ve < 0) return fail(SR_ERR_ARGUMENT, "unsupported state dtype or rule");
  if (!valid_block(block_size)) return fail(SR_ERR_ARGUMENT, "invalid block size %d", block_size);
  if (!hp || !rows) return fail(SR_ERR_ARGUMENT, "null argument");
  if (!valid_correction(*hp))
    return fail(SR_ERR_ARGUMENT, "correction2_sqrt %g outside [2^-27, 1]", (double)hp->correction2_sqrt);
  if (nrows < 1 || nrows > SR_NOALLOC_MAX_ROWS)
    return fail(SR_ERR_ARGUMENT, "row count %d outside [1, %d] (the scratch holds %d rows)", nrows,
                SR_NOALLOC_MAX_ROWS, SR_NOALLOC_MAX_ROWS);
  if (total_tiles == 0 || total_tiles > SR_NOALLOC_MAX_TILES)
    return fail(SR_ERR_ARGUMENT, "%u tiles outside [1, %u] (the scratch holds %u tiles)", total_tiles,
                (unsigned)SR_NOALLOC_MAX_TILES, (unsigned)SR_NOALLOC_MAX_TILES);
  const int64_t tile_elements =
      static_cast<int64_t>(block_size) * sr::lane_elements(param_enc(pi), param_enc(gi), me, ve);
  if (int rc = check_host_rows(rows, row_scalars, nrows, total_tiles, tile_elements)) return rc;
  if (int rc = check_capture_tables(static_cast<hipStream_t>(stream), rows, row_scalars)) return rc;
  unsigned char* base = nullptr;
  if (int rc = scratch_base(stream, &base)) return rc;
  sr_row* rows_dev = reinterpret_cast<sr_row*>(base);
  float* scalars_dev = reinterpret_cast<float*>(base + kScratchRowBytes);
  uint32_t* tiles_dev = reinterpret_cast<uint32_t*>(base + kScratchRowBytes + kScratchScalarBytes);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t err = hipMemcpyAsync(rows_dev, rows, sizeof(sr_row) * nrows, hipMemcpyHostToDevice, s);
  if (err != hipSuccess) return hip_fail(err, "hipMemcpyAsync(rows)");
  if (row_scalars) {
    err = hipMemcpyAsync(scalars_dev, row_scalars, 2 * sizeof(float) * nrows, hipMemcpyHostToDevice, s);
    if (err != hipSuccess) return hip_fail(err, "hipMemcpyAsync(row_scalars)");
  }
  const uint32_t fill_groups = (total_tiles + kFillBlock - 1) / kFillBlock;
  hipLaunchKernelGGL(fill_tile_rows, dim3(fill_groups), dim3(kFillBlock), 0, s, rows_dev, nrows, tiles_dev,
                     total_tiles);
  err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(err, "fill_tile_rows launch");
  sr::AdamWArgs a{};
  a.rows = rows_dev;
  a.tile_rows = tiles_dev;
  a.row_scalars = row_scalars ? scalars_dev : nullptr;
  a.total_tiles = total_tiles;
  a.s = adamw_scalars(*hp);
  a.key_prefix = sr::update_key_prefix(static_cast<uint32_t>(seed), static_cast<uint32_t>(seed >> 32),
                                       static_cast<uint32_t>(rng_step),
                                       static_cast<uint32_t>(rng_step >> 32));
  return launch(tables().adamw[pi][gi][me][ve], block_size, total_tiles, &a, stream,
                adamw_cap(pi, gi, me, ve, block_size, total_tiles));
}

}  // extern "C"
