/*
 * sr_states_hip.h -- C ABI of the MI355X (gfx950) backend for sr_states.
 *
 * This is the drop-in boundary for the fused stochastic-rounding optimizer
 * step and the standalone cast.  Every entry point takes plain device
 * pointers, element counts, scalars and a HIP stream handle; no torch types
 * cross the boundary.  Each declaration names the reference interface it
 * replaces (paths relative to the reference repository root).
 *
 * Conventions
 *   - Return value: 0 on success, otherwise a nonzero SR_ERR_* code.  The
 *     message for the most recent failure on the calling thread is returned
 *     by sr_last_error().
 *   - `stream` is a hipStream_t passed as void* (0 = the null stream).  All
 *     launches are asynchronous on that stream; nothing synchronizes.
 *   - Pointers are borrowed for the duration of the launch; the caller keeps
 *     the memory alive until the stream has consumed it.
 *   - Counters are 32-bit: every seed/offset/step word is taken modulo 2^32,
 *     exactly as the reference masks them (sr_states/_hash.py:5-50).
 *   - Optimizer launches of 2^16 tiles or more with FP32 parameters reserve
 *     dynamic LDS that their kernels never touch, to keep a measured budget
 *     of tiles in flight per CU: AdamW 80 KiB, or 96 KiB with BF16
 *     gradients or with two FP16/FP8 stochastic moments (none with both);
 *     SGDM 88 KiB, or 72 KiB with FP16 stochastic momentum.  Kernels of
 *     other streams running beside such a launch find that LDS taken on the
 *     CUs it occupies.  The environment
 *     variable SR_STATES_RESIDENT_CAP=k (0-16, read once per process)
 *     replaces that rule for every optimizer launch of 2^16 tiles or more:
 *     at most k workgroups per CU, none reserved for k = 0.  Results do
 *     not depend on either.
 */
#ifndef SR_STATES_HIP_H
#define SR_STATES_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SR_ABI_VERSION 5

/* Storage dtypes (torch.float32, bfloat16, float16, float8_e4m3fn,
 * float8_e5m2).  The set mirrors the built-in rounding table of the
 * reference (sr_states/rounding.py:135-142). */
enum sr_dtype {
  SR_F32 = 0,
  SR_BF16 = 1,
  SR_F16 = 2,
  SR_E4M3 = 3,
  SR_E5M2 = 4
};

/* Rounding rules ("nearest", "stochastic"); FP32 ignores the rule, as the
 * reference maps both FP32 rules to the identity (sr_states/rounding.py:135-136). */
enum sr_rule {
  SR_NEAREST = 0,
  SR_STOCHASTIC = 1
};

enum sr_error {
  SR_OK = 0,
  SR_ERR_ARGUMENT = 1,   /* invalid dtype / rule / size / block size */
  SR_ERR_HIP = 2,        /* a HIP runtime call failed (message has details) */
  SR_ERR_UNSUPPORTED = 3 /* combination not compiled into this library */
};

/* Elements one lane moves per tile.  A tile is block_size * (this many)
 * consecutive elements of one tensor and is processed by one workgroup.
 * Optimizer launches currently all use SR_LANE_ELEMENTS (FP32 operands move
 * as one 128-bit access per lane) and casts SR_LANE_ELEMENTS_NARROW (two
 * groups of four a workgroup-width apart, so that every access instruction
 * covers a contiguous span).  sr_lane_elements() returns the width of an
 * optimizer launch; hosts must use it rather than assume a width. */
#define SR_LANE_ELEMENTS 4
#define SR_LANE_ELEMENTS_NARROW 8

/* Row flag: every pointer of the row is 16-byte aligned, so full tiles take
 * the 128-bit vector path.  Rows without it take the coalesced scalar path. */
#define SR_ROW_VECTOR 1u
/* Row flag: `param_index` already holds the update key (functional API);
 * the kernel then skips the on-device key derivation. */
#define SR_ROW_KEYED 2u

/* One parameter of a multi-tensor bucket (64 bytes, device memory).
 * Together with a per-tile row map (uint32 row index per tile) it replaces
 * the reference's tables `meta`, `chunks` and `pointers`
 * (built by sr_states/triton/_multi_tensor.py:43-47, 64-134, consumed by
 * sr_states/triton/_common.py:47-60). */
typedef struct sr_row {
  uint64_t ptr[4];      /* parameter, gradient, state 0, state 1 (0 for SGDM) */
  int64_t numel;        /* elements of this parameter (>= 1) */
  uint32_t tile_begin;  /* first tile of this row in the bucket's tile space */
  uint32_t tile_end;    /* one past its last tile; tiles are contiguous */
  uint32_t param_index; /* global parameter index, or the key if SR_ROW_KEYED */
  uint32_t shard_start; /* flat index of the first local element (mod 2^32) */
  uint32_t flags;       /* SR_ROW_* */
  uint32_t reserved;
} sr_row;

/* AdamW launch scalars, already rounded to FP32 by the host exactly as the
 * eager reference rounds its Python-double scalars
 * (sr_states/reference/adamw.py:86-96; triton/adamw.py:224-234). */
typedef struct sr_adamw_hparams {
  float beta1;            /* f32(beta1) */
  float beta2;            /* f32(beta2) */
  float one_minus_beta1;  /* f32(1 - beta1) */
  float one_minus_beta2;  /* f32(1 - beta2) */
  float neg_step_size;    /* f32(-lr / (1 - beta1^step)) */
  float correction2_sqrt; /* f32(sqrt(1 - beta2^step)), in [2^-27, 1] for
                             0 <= beta2 < 1 and step >= 1; the AdamW entry
                             points fail with SR_ERR_ARGUMENT outside it */
  float decay;            /* f32(1 - lr * weight_decay) */
  float eps;              /* f32(eps) */
} sr_adamw_hparams;

/* Momentum-SGD launch scalars (sr_states/reference/sgd.py:62-64). */
typedef struct sr_sgdm_hparams {
  float momentum; /* f32(momentum_factor) */
  float neg_lr;   /* f32(-lr) */
} sr_sgdm_hparams;

/* ---- library ---------------------------------------------------------- */

/* Returns SR_ABI_VERSION. */
int sr_abi_version(void);

/* Message of the last failure on this thread ("" if none). */
const char* sr_last_error(void);

/* Elements per lane (SR_LANE_ELEMENTS or SR_LANE_ELEMENTS_NARROW) of an
 * optimizer launch with these operand dtypes: parameter, gradient and the
 * two AdamW moments, or for SGDM the momentum dtype twice.  Hosts lay out
 * the tile ranges of sr_row tables with tiles of
 * block_size * sr_lane_elements(...) elements.  (Casts lay out their own
 * tiles and always move SR_LANE_ELEMENTS_NARROW elements per lane.)  Returns 0 for
 * an unknown dtype.  No reference counterpart: the reference's Triton
 * launches take BLOCK_SIZE elements per program
 * (sr_states/triton/_common.py:47-60). */
int sr_lane_elements(int p_dtype, int g_dtype, int state0_dtype, int state1_dtype);

/* ---- counter-hash keys (host) ----------------------------------------- */

/* Replaces sr_states/_hash.py:18-23 `update_key(seed, step, param_index)`;
 * seed and step are their low 64 bits (two's complement). */
uint32_t sr_update_key(uint64_t seed, uint64_t step, uint32_t param_index);

/* Replaces sr_states/_hash.py:26-28 `state_key(key, state_index)`. */
uint32_t sr_state_key(uint32_t key, uint32_t state_index);

/* ---- standalone cast -------------------------------------------------- */

/* y[i] = round(x[i]) for i < n, counter = i + seed + offset (mod 2^32).
 * x: contiguous FP32; y: contiguous storage of `dtype`; x and y disjoint.
 * Replaces the `_cast_kernel` launch of sr_states/triton/cast.py:47-60 and
 * `_sr_cast_bf16_kernel` of sr_states/triton/sr_cast.py:55-86, 131-164; its
 * arithmetic is sr_states/rounding.py:97-142. */
int sr_cast(const void* x, void* y, int64_t n, int dtype, int rule,
            uint32_t seed, uint32_t offset, int block_size, void* stream);

/* lower[i], upper[i] = the two `dtype` values stochastic rounding chooses
 * between for x[i], ordered, for i < n; both the nearest-even value when
 * x[i] is representable, Inf or NaN.  Saturating FP8 formats clamp |x| to
 * their maximum first; FP16 brackets finite magnitudes above 65504 by 65504
 * and Inf.  dtype: SR_BF16, SR_F16, SR_E4M3 or SR_E5M2.  x: contiguous
 * FP32; lower, upper: contiguous storage of `dtype`, disjoint from x.
 * Replaces `bf16_neighbors` (sr_states/_bf16.py:77-101) and
 * `minifloat_neighbors` (sr_states/_minifloat.py:73-99), which
 * sr_states/reference/rounding.py:1-9 exports. */
int sr_neighbors(const void* x, void* lower, void* upper, int64_t n, int dtype, void* stream);

/* ---- fused AdamW ------------------------------------------------------ */

/* One tensor.  p, g: FP32 or BF16; m, v: any sr_dtype.  `key` is the
 * parameter's update key; `offset` the flat shard start.
 * Replaces `_fused_adamw_kernel` (sr_states/triton/adamw.py:59-100) and its
 * launch by `triton_adamw_step_` (sr_states/triton/adamw.py:160-221). */
int sr_adamw_step(void* p, const void* g, void* m, void* v, int64_t n,
                  int p_dtype, int g_dtype, int m_dtype, int m_rule,
                  int v_dtype, int v_rule, const sr_adamw_hparams* hp,
                  uint32_t key, uint32_t offset, int block_size, void* stream);

/* One bucket: `rows` is a device table of nrows sr_row records whose tile
 * ranges cover [0, total_tiles) in order, and `tile_rows` a device array of
 * total_tiles row indices (tile_rows[t] = the row whose range holds t).
 * `row_scalars` is NULL when every row has the same AdamW step (hp then
 * holds its scalars), or a device array of 2 * nrows floats holding each
 * row's (neg_step_size, correction2_sqrt), each correction2_sqrt in
 * [2^-27, 1] as in hp (not checked: the table is device memory); the other
 * scalars come from hp.
 * The reference launches once per distinct step instead
 * (sr_states/triton/_multi_tensor.py:22-36); the per-row pair keeps one
 * launch per bucket with the same FP32 scalars per row.
 * Row r spans ceil(numel / T) tiles of T = block_size *
 * sr_lane_elements(p_dtype, g_dtype, m_dtype, v_dtype) elements.  The
 * tables live in device memory and are not checked: tables that break these
 * rules make the kernel access memory out of bounds.  total_tiles may be up
 * to 2^31 - 4096 (SR_ERR_ARGUMENT beyond); launches whose grid would carry
 * 2^32 or more work-items in one dimension are split into rows of
 * workgroups, so one call covers buckets past 2^34 elements.
 * Keys are derived on the device from (seed, rng_step, param_index).
 * Replaces `_multi_adamw_kernel` and its launch
 * (sr_states/triton/adamw.py:102-157, 289-319). */
int sr_adamw_multi(const sr_row* rows, const uint32_t* tile_rows, const float* row_scalars,
                   int nrows, uint32_t total_tiles,
                   int p_dtype, int g_dtype, int m_dtype, int m_rule,
                   int v_dtype, int v_rule, const sr_adamw_hparams* hp,
                   uint64_t seed, uint64_t rng_step, int block_size, void* stream);

/* Limits of sr_adamw_multi_noalloc: its static device scratch holds this
 * many rows and tiles (16.3 MiB per GPU). */
#define SR_NOALLOC_MAX_ROWS 4096
#define SR_NOALLOC_MAX_TILES (1u << 22)

/* sr_adamw_multi without any device allocation by the caller or the library.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts
 * whose harness forbids hipMalloc).
 *
 * `rows` (nrows records) and `row_scalars` (NULL, or 2 * nrows floats as in
 * sr_adamw_multi) are HOST memory.  The library checks them on the host
 * (tile ranges that start at 0, follow each other and cover [0, total_tiles)
 * with ceil(numel / T) tiles per row, non-null pointers, 16-byte alignment
 * of vector rows, known flags, every correction2_sqrt in [2^-27, 1]), copies
 * them into a static device array of the library, builds the tile-to-row map
 * there with a small kernel, and launches the same kernel as sr_adamw_multi,
 * all on `stream`.  Results equal sr_adamw_multi's for the same tables.
 *
 * Limits: 1 <= nrows <= SR_NOALLOC_MAX_ROWS and 1 <= total_tiles <=
 * SR_NOALLOC_MAX_TILES (2^22 tiles: 2.1 G elements at 128-thread
 * workgroups); larger buckets fail with SR_ERR_ARGUMENT before any device
 * work.  The array is one per GPU and keeps the last call's contents: calls
 * that overlap on one GPU (on different streams or threads) race, so a
 * caller serializes them, for example on one stream.  The stream must belong
 * to the current device.  Eager calls: pageable `rows`/`row_scalars` may be
 * reused when the call returns; pinned ones must stay unchanged until the
 * stream has passed the call.  Under HIP stream capture the two table copies
 * become graph nodes that read the host tables again at every replay: the
 * tables must then be pinned host memory (hipHostMalloc) that stays valid
 * and unchanged for as long as the graph can replay, and pageable ones fail
 * with SR_ERR_ARGUMENT before anything is recorded.  Each replay restages
 * the tables in the scratch, so replays race with other calls on the GPU
 * as calls do. */
int sr_adamw_multi_noalloc(const sr_row* rows, const float* row_scalars, int nrows, uint32_t total_tiles,
                           int p_dtype, int g_dtype, int m_dtype, int m_rule, int v_dtype, int v_rule,
                           const sr_adamw_hparams* hp, uint64_t seed, uint64_t rng_step, int block_size,
                           void* stream);

/* ---- fused momentum SGD ----------------------------------------------- */

/* Replaces `_fused_sgdm_kernel` (sr_states/triton/sgd.py:47-72) and its launch
 * by `triton_sgdm_step_` (sr_states/triton/sgd.py:115-171). */
int sr_sgdm_step(void* p, const void* g, void* u, int64_t n,
                 int p_dtype, int g_dtype, int u_dtype, int u_rule,
                 const sr_sgdm_hparams* hp, uint32_t key, uint32_t offset,
                 int block_size, void* stream);

/* Same table layout as sr_adamw_multi (state 1 pointer unused); tiles are
 * block_size * sr_lane_elements(p_dtype, g_dtype, u_dtype, u_dtype) elements.
 * Replaces `_multi_sgdm_kernel` and its launch
 * (sr_states/triton/sgd.py:74-112, 214-237). */
int sr_sgdm_multi(const sr_row* rows, const uint32_t* tile_rows, int nrows, uint32_t total_tiles,
                  int p_dtype, int g_dtype, int u_dtype, int u_rule,
                  const sr_sgdm_hparams* hp, uint64_t seed, uint64_t rng_step,
                  int block_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SR_STATES_HIP_H */
