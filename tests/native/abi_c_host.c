/* A plain C host of the C ABI: no Python, no torch.
 *
 * Allocates device buffers with the HIP runtime, runs sr_cast (BF16 and
 * E4M3 stochastic, FP16 nearest), sr_adamw_step (FP32 parameters, BF16-SR
 * moments), sr_sgdm_step (FP16-SR momentum) and sr_adamw_multi (three rows
 * with the row table and tile map built here) on the default stream,
 * copies the results back and compares them byte for byte with the C
 * oracle (oracle/sr_oracle.c, test infrastructure linked in as the
 * checker).  sr_neighbors (BF16) is checked against the definition of the
 * pair.  Also checks that a bad argument comes back as SR_ERR_ARGUMENT
 * with a message.  Prints one line per check and "abi_c_host ok" at the
 * end; exits nonzero on the first failure.
 *
 * Built and run by tests/test_gpu_abi_c_host.py.
 */
#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/sr_states_hip.h"

/* oracle/sr_oracle.c */
void oc_cast(const float* x, void* y, int64_t n, int dtype, int rule, uint32_t seed, uint32_t offset);
void oc_adamw(void* p, int p_dtype, const void* g, int g_dtype, void* m, int m_dtype, int m_rule, void* v,
              int v_dtype, int v_rule, int64_t n, const float* hp, uint32_t key, uint32_t offset);
void oc_sgdm(void* p, int p_dtype, const void* g, int g_dtype, void* u, int u_dtype, int u_rule, int64_t n,
             float momentum, float neg_lr, uint32_t key, uint32_t offset);

#define N 1000003 /* full tiles and a scalar tail */

static int check_hip(hipError_t err, const char* what) {
  if (err != hipSuccess) {
    printf("FAIL %s: %s\n", what, hipGetErrorString(err));
    return 1;
  }
  return 0;
}

static int check_rc(int rc, const char* what) {
  if (rc != SR_OK) {
    printf("FAIL %s: rc %d (%s)\n", what, rc, sr_last_error());
    return 1;
  }
  return 0;
}

static int same(const void* a, const void* b, size_t bytes, const char* what) {
  if (memcmp(a, b, bytes) != 0) {
    const unsigned char *x = a, *y = b;
    size_t k = 0;
    while (x[k] == y[k]) ++k;
    printf("FAIL %s: first differing byte %zu\n", what, k);
    return 1;
  }
  printf("ok %s (%zu bytes)\n", what, bytes);
  return 0;
}

/* Deterministic inputs: x_i = sin(i) * scale, spread over several binades. */
static void fill(float* x, size_t n, float scale) {
  for (size_t i = 0; i < n; ++i) x[i] = (float)(sin((double)i * 0.7 + 0.3) * scale * (1 + (i % 7)));
}

int main(void) {
  if (sr_abi_version() != SR_ABI_VERSION) {
    printf("FAIL abi version %d, header %d\n", sr_abi_version(), SR_ABI_VERSION);
    return 1;
  }
  float *x = malloc(N * 4), *p = malloc(N * 4), *g = malloc(N * 4);
  unsigned char *host = malloc(N * 4), *want = malloc(N * 4), *m = malloc(N * 2), *v = malloc(N * 2);
  if (!x || !p || !g || !host || !want || !m || !v) return 1;
  fill(x, N, 1.0f);
  fill(p, N, 0.02f);
  fill(g, N, 1e-3f);

  void *dx, *dy, *dp, *dg, *dm, *dv;
  if (check_hip(hipMalloc(&dx, N * 4), "hipMalloc") || check_hip(hipMalloc(&dy, N * 4), "hipMalloc") ||
      check_hip(hipMalloc(&dp, N * 4), "hipMalloc") || check_hip(hipMalloc(&dg, N * 4), "hipMalloc") ||
      check_hip(hipMalloc(&dm, N * 2), "hipMalloc") || check_hip(hipMalloc(&dv, N * 2), "hipMalloc"))
    return 1;
  if (check_hip(hipMemcpy(dx, x, N * 4, hipMemcpyHostToDevice), "copy x")) return 1;

  /* Casts: (dtype, rule, bytes per element). */
  const int casts[3][3] = {{SR_BF16, SR_STOCHASTIC, 2}, {SR_E4M3, SR_STOCHASTIC, 1}, {SR_F16, SR_NEAREST, 2}};
  for (int c = 0; c < 3; ++c) {
    const int dtype = casts[c][0], rule = casts[c][1], width = casts[c][2];
    char what[64];
    snprintf(what, sizeof what, "sr_cast dtype %d rule %d", dtype, rule);
    if (check_rc(sr_cast(dx, dy, N, dtype, rule, 7u, 3u, 256, NULL), what)) return 1;
    if (check_hip(hipMemcpy(host, dy, (size_t)N * width, hipMemcpyDeviceToHost), "copy y")) return 1;
    oc_cast(x, want, N, dtype, rule, 7u, 3u);
    if (same(host, want, (size_t)N * width, what)) return 1;
  }

  /* Neighbours in BF16: each pair brackets x, carries x's sign, is two
   * adjacent encodings or one, and is one exactly when x is a BF16 value. */
  {
    void* dz;
    if (check_hip(hipMalloc(&dz, N * 2), "hipMalloc")) return 1;
    if (check_rc(sr_neighbors(dx, dy, dz, N, SR_BF16, NULL), "sr_neighbors")) return 1;
    uint16_t* lower = (uint16_t*)host;
    uint16_t* upper = (uint16_t*)want;
    if (check_hip(hipMemcpy(lower, dy, N * 2, hipMemcpyDeviceToHost), "copy lower") ||
        check_hip(hipMemcpy(upper, dz, N * 2, hipMemcpyDeviceToHost), "copy upper"))
      return 1;
    hipFree(dz);
    for (size_t i = 0; i < N; ++i) {
      uint32_t xb, lb = (uint32_t)lower[i] << 16, ub = (uint32_t)upper[i] << 16;
      float lo, hi;
      memcpy(&xb, &x[i], 4);
      memcpy(&lo, &lb, 4);
      memcpy(&hi, &ub, 4);
      const uint32_t sign = xb >> 31, lm = lower[i] & 0x7FFFu, um = upper[i] & 0x7FFFu;
      const uint32_t step = sign ? lm - um : um - lm;
      const int exact = (xb & 0xFFFFu) == 0;
      if (!(lo <= x[i] && x[i] <= hi) || (lb >> 31) != sign || (ub >> 31) != sign || step > 1u ||
          (step == 0u) != exact) {
        printf("FAIL sr_neighbors bf16 at %zu: x %08x lower %04x upper %04x\n", i, xb, lower[i], upper[i]);
        return 1;
      }
    }
    printf("ok sr_neighbors bf16 (%d inputs)\n", N);
  }

  /* AdamW: FP32 p/g, BF16-SR moments from zero, step 3. */
  const double lr = 3e-4, beta1 = 0.9, beta2 = 0.999, eps = 1e-8, wd = 0.01;
  const int step = 3;
  sr_adamw_hparams hp = {(float)beta1, (float)beta2, (float)(1 - beta1), (float)(1 - beta2),
                         (float)(-lr / (1 - pow(beta1, step))), (float)sqrt(1 - pow(beta2, step)),
                         (float)(1 - lr * wd), (float)eps};
  const float hp_array[8] = {hp.beta1, hp.beta2, hp.one_minus_beta1, hp.one_minus_beta2,
                             hp.neg_step_size, hp.correction2_sqrt, hp.decay, hp.eps};
  const uint32_t key = sr_update_key(7u, 5u, 2u), offset = 11u;
  memset(m, 0, N * 2);
  memset(v, 0, N * 2);
  if (check_hip(hipMemcpy(dp, p, N * 4, hipMemcpyHostToDevice), "copy p") ||
      check_hip(hipMemcpy(dg, g, N * 4, hipMemcpyHostToDevice), "copy g") ||
      check_hip(hipMemcpy(dm, m, N * 2, hipMemcpyHostToDevice), "copy m") ||
      check_hip(hipMemcpy(dv, v, N * 2, hipMemcpyHostToDevice), "copy v"))
    return 1;
  if (check_rc(sr_adamw_step(dp, dg, dm, dv, N, SR_F32, SR_F32, SR_BF16, SR_STOCHASTIC, SR_BF16, SR_STOCHASTIC,
                             &hp, key, offset, 128, NULL),
               "sr_adamw_step"))
    return 1;
  oc_adamw(p, 0, g, 0, m, 1, 1, v, 1, 1, N, hp_array, key, offset);
  if (check_hip(hipMemcpy(host, dp, N * 4, hipMemcpyDeviceToHost), "copy p")) return 1;
  if (same(host, p, N * 4, "sr_adamw_step parameter")) return 1;
  if (check_hip(hipMemcpy(host, dm, N * 2, hipMemcpyDeviceToHost), "copy m")) return 1;
  if (same(host, m, N * 2, "sr_adamw_step exp_avg")) return 1;
  if (check_hip(hipMemcpy(host, dv, N * 2, hipMemcpyDeviceToHost), "copy v")) return 1;
  if (same(host, v, N * 2, "sr_adamw_step exp_avg_sq")) return 1;

  /* Momentum SGD: FP32 p/g, FP16-SR momentum from the AdamW parameters. */
  sr_sgdm_hparams sp = {0.9f, -0.1f};
  memset(m, 0, N * 2);
  if (check_hip(hipMemcpy(dm, m, N * 2, hipMemcpyHostToDevice), "copy u")) return 1;
  if (check_rc(sr_sgdm_step(dp, dg, dm, N, SR_F32, SR_F32, SR_F16, SR_STOCHASTIC, &sp, key, offset, 256, NULL),
               "sr_sgdm_step"))
    return 1;
  oc_sgdm(p, 0, g, 0, m, 2, 1, N, sp.momentum, sp.neg_lr, key, offset);
  if (check_hip(hipMemcpy(host, dp, N * 4, hipMemcpyDeviceToHost), "copy p")) return 1;
  if (same(host, p, N * 4, "sr_sgdm_step parameter")) return 1;
  if (check_hip(hipMemcpy(host, dm, N * 2, hipMemcpyDeviceToHost), "copy u")) return 1;
  if (same(host, m, N * 2, "sr_sgdm_step momentum")) return 1;

  /* Multi-tensor AdamW: three rows (three parameters of one bucket) carved
   * out of the device buffers, one with an unaligned start, with the row
   * table and tile map a C host builds (the layout sr_row documents). */
  {
    const int64_t sizes[3] = {4099, 65536, 777};
    const int64_t starts[3] = {0, 4104, 69641}; /* element offsets; 69641 is not 16-byte aligned */
    const uint32_t param_index[3] = {0, 3, 4}, shard_start[3] = {0, 1000, 4294967000u};
    const int lanes = sr_lane_elements(SR_F32, SR_F32, SR_BF16, SR_BF16), block = 128;
    const uint32_t tile = (uint32_t)(block * lanes);
    sr_row rows[3];
    uint32_t tiles = 0;
    for (int r = 0; r < 3; ++r) {
      const uint32_t count = (uint32_t)((sizes[r] + tile - 1) / tile);
      rows[r].ptr[0] = (uint64_t)(uintptr_t)((float*)dp + starts[r]);
      rows[r].ptr[1] = (uint64_t)(uintptr_t)((float*)dg + starts[r]);
      rows[r].ptr[2] = (uint64_t)(uintptr_t)((uint16_t*)dm + starts[r]);
      rows[r].ptr[3] = (uint64_t)(uintptr_t)((uint16_t*)dv + starts[r]);
      rows[r].numel = sizes[r];
      rows[r].tile_begin = tiles;
      rows[r].tile_end = tiles + count;
      rows[r].param_index = param_index[r];
      rows[r].shard_start = shard_start[r];
      rows[r].flags = (starts[r] % 8 == 0) ? SR_ROW_VECTOR : 0u; /* 16-byte aligned FP32 and BF16 */
      rows[r].reserved = 0;
      tiles += count;
    }
    uint32_t* tile_rows = malloc(tiles * sizeof(uint32_t));
    if (!tile_rows) return 1;
    for (int r = 0; r < 3; ++r)
      for (uint32_t t = rows[r].tile_begin; t < rows[r].tile_end; ++t) tile_rows[t] = (uint32_t)r;
    void *drows, *dtiles;
    memset(m, 0, N * 2);
    memset(v, 0, N * 2);
    fill(p, N, 0.02f);
    if (check_hip(hipMalloc(&drows, sizeof rows), "hipMalloc rows") ||
        check_hip(hipMalloc(&dtiles, tiles * sizeof(uint32_t)), "hipMalloc tiles") ||
        check_hip(hipMemcpy(drows, rows, sizeof rows, hipMemcpyHostToDevice), "copy rows") ||
        check_hip(hipMemcpy(dtiles, tile_rows, tiles * sizeof(uint32_t), hipMemcpyHostToDevice), "copy tiles") ||
        check_hip(hipMemcpy(dp, p, N * 4, hipMemcpyHostToDevice), "copy p") ||
        check_hip(hipMemcpy(dm, m, N * 2, hipMemcpyHostToDevice), "copy m") ||
        check_hip(hipMemcpy(dv, v, N * 2, hipMemcpyHostToDevice), "copy v"))
      return 1;
    const uint64_t seed = 0x123456789ull, rng_step = 4;
    if (check_rc(sr_adamw_multi((const sr_row*)drows, (const uint32_t*)dtiles, NULL, 3, tiles, SR_F32, SR_F32,
                                SR_BF16, SR_STOCHASTIC, SR_BF16, SR_STOCHASTIC, &hp, seed, rng_step, block, NULL),
                 "sr_adamw_multi"))
      return 1;
    for (int r = 0; r < 3; ++r) {
      const uint32_t row_key = sr_update_key(seed, rng_step, param_index[r]);
      oc_adamw(p + starts[r], 0, g + starts[r], 0, (uint16_t*)m + starts[r], 1, 1, (uint16_t*)v + starts[r], 1, 1,
               sizes[r], hp_array, row_key, shard_start[r]);
    }
    if (check_hip(hipMemcpy(host, dp, N * 4, hipMemcpyDeviceToHost), "copy p")) return 1;
    if (same(host, p, N * 4, "sr_adamw_multi parameters (3 rows and untouched gaps)")) return 1;
    if (check_hip(hipMemcpy(host, dm, N * 2, hipMemcpyDeviceToHost), "copy m")) return 1;
    if (same(host, m, N * 2, "sr_adamw_multi exp_avg")) return 1;
    if (check_hip(hipMemcpy(host, dv, N * 2, hipMemcpyDeviceToHost), "copy v")) return 1;
    if (same(host, v, N * 2, "sr_adamw_multi exp_avg_sq")) return 1;
    hipFree(drows);
    hipFree(dtiles);
    free(tile_rows);
  }

  /* Errors come back as codes with a message; nothing is launched. */
  if (sr_cast(dx, dy, N, 9, SR_NEAREST, 0u, 0u, 256, NULL) != SR_ERR_ARGUMENT || strlen(sr_last_error()) == 0) {
    printf("FAIL bad dtype not refused\n");
    return 1;
  }
  printf("ok bad dtype refused: %s\n", sr_last_error());

  if (check_hip(hipDeviceSynchronize(), "synchronize")) return 1;
  hipFree(dx); hipFree(dy); hipFree(dp); hipFree(dg); hipFree(dm); hipFree(dv);
  free(x); free(p); free(g); free(host); free(want); free(m); free(v);
  printf("abi_c_host ok\n");
  return 0;
}
