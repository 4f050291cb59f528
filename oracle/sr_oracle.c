/*
 * sr_oracle.c -- plain-C restatement of the reference's stochastic-rounding
 * arithmetic, used as a CHECKER ONLY.
 *
 * TEST INFRASTRUCTURE.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only to check or time against
 * it.  The product (libsr_states_hip.so and the sr_states package) never
 * links, loads or calls it.
 *
 * The formulation deliberately differs from the product kernels: minifloat
 * rounding follows the reference's floating-point grid (power-of-two scale,
 * floor, remainder, 24-bit threshold compared as floats) and encodes the
 * result with frexpf/ldexpf, where the product works on integer shifts of the
 * significand.  FP32 recurrences use libm's correctly rounded sqrtf and IEEE
 * division, with fmaf exactly where torch's CPU kernels fuse.  Build with
 * -ffp-contract=off (see oracle/Makefile).
 *
 * Reference files followed (paths in the reference repository):
 *   sr_states/_hash.py:5-50         hash, update_key, state_key, counters
 *   sr_states/_bf16.py:37-74        FP32 -> BF16 stochastic rounding
 *   sr_states/_minifloat.py:10-70   E4M3 / E5M2 / FP16 nearest and stochastic
 *   sr_states/rounding.py:97-142    rule table (FP32 identity, BF16/torch RN)
 *   sr_states/reference/adamw.py:54-105, reference/sgd.py:44-72  recurrences
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { D_F32 = 0, D_BF16 = 1, D_F16 = 2, D_E4M3 = 3, D_E5M2 = 4 };
enum { R_NEAREST = 0, R_STOCHASTIC = 1 };

static uint32_t fbits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

static float bitsf(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* ---- counter hash (sr_states/_hash.py:10-50) ------------------------- */

static uint32_t h32(uint32_t v) {
  v ^= v >> 16;
  v *= 0x7FEB352Du;
  v ^= v >> 15;
  v *= 0x846CA68Bu;
  return v ^ (v >> 16);
}

uint32_t oc_hash(uint32_t counter) { return h32(counter); }

uint32_t oc_update_key(uint64_t seed, uint64_t step, uint32_t param_index) {
  const uint32_t words[4] = {(uint32_t)(seed >> 32), (uint32_t)step, (uint32_t)(step >> 32),
                             param_index};
  uint32_t key = h32((uint32_t)seed ^ 0x9E3779B9u);
  for (int i = 0; i < 4; ++i) key = h32(key ^ words[i]);
  return key;
}

uint32_t oc_state_key(uint32_t key, uint32_t state_index) { return h32(key ^ state_index); }

/* ---- BF16 (sr_states/_bf16.py:37-74; torch float->bfloat16) ---------- */

static uint32_t bf16_stochastic(float x, uint32_t hash) {
  const uint32_t bits = fbits(x);
  const uint32_t truncated = bits & 0xFFFF0000u;
  uint32_t rounded = (uint32_t)(((uint64_t)bits + (hash & 0xFFFFu)) & 0xFFFF0000u);
  if ((bits & 0x7F800000u) == 0x7F800000u) {
    rounded = (bits & 0x007FFFFFu) ? (truncated | 0x00400000u) : truncated;
  }
  return rounded >> 16;
}

static uint32_t bf16_nearest(float x) {
  const uint32_t bits = fbits(x);
  if (isnan(x)) return 0x7FC0u;
  return (uint32_t)(((uint64_t)bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

/* ---- minifloats (sr_states/_minifloat.py:10-70) ------------------------ */

typedef struct {
  int mant;     /* mantissa bits */
  int emin;     /* minimum normal exponent */
  float max;    /* largest finite magnitude */
  int saturate; /* FP8: overflow and Inf go to +-max */
  int width;    /* storage bits */
} mf_t;

static const mf_t MF_E4M3 = {3, -6, 448.0f, 1, 8};
static const mf_t MF_E5M2 = {2, -14, 57344.0f, 1, 8};
static const mf_t MF_F16 = {10, -14, 65504.0f, 0, 16};

/* a = (q + rem) * ulp with integer q, ulp = 2^(max(e, emin) - mant). */
static void mf_grid(float a, const mf_t* f, float* q, float* rem, float* ulp) {
  int e = (int)((fbits(a) >> 23) & 0xFFu) - 127;
  if (e < f->emin) e = f->emin;
  *ulp = ldexpf(1.0f, e - f->mant);
  const float scaled = a * ldexpf(1.0f, f->mant - e); /* exact: power-of-two scale */
  *q = floorf(scaled);
  *rem = scaled - *q;
}

/* Magnitude after the format's saturation, with specials mapped to 0. */
static float mf_safe(float x, const mf_t* f) {
  float a = fabsf(x);
  if (f->saturate && a > f->max) a = f->max; /* NaN compares false and stays NaN */
  return isfinite(a) ? a : 0.0f;
}

static float mf_finish(float rounded, float x, const mf_t* f) {
  rounded = copysignf(rounded, x);
  if (!f->saturate && isinf(x)) rounded = x;
  if (isnan(x)) rounded = x;
  return rounded;
}

static float mf_stochastic_value(float x, const mf_t* f, uint32_t hash) {
  float q, rem, ulp;
  mf_grid(mf_safe(x, f), f, &q, &rem, &ulp);
  const float threshold = floorf(rem * 16777216.0f);
  const float k = (float)(hash >> 8);
  return mf_finish((q + (k < threshold ? 1.0f : 0.0f)) * ulp, x, f);
}

/* Nearest-even on the same grid.  For FP16 (no saturation) this restates
 * IEEE round-to-nearest-even, torch's Tensor.to(torch.float16). */
static float mf_nearest_value(float x, const mf_t* f) {
  float q, rem, ulp;
  mf_grid(mf_safe(x, f), f, &q, &rem, &ulp);
  const int odd = fmodf(q, 2.0f) == 1.0f;
  const float up = (rem > 0.5f || (rem == 0.5f && odd)) ? 1.0f : 0.0f;
  return mf_finish((q + up) * ulp, x, f);
}

/* Encode a value that lies on the format's grid (or NaN / Inf / an FP16
 * overflow that rounds to Inf). */
static uint32_t mf_encode(float v, const mf_t* f) {
  const uint32_t sign = signbit(v) ? (1u << (f->width - 1)) : 0u;
  if (isnan(v)) return sign | (f->width == 16 ? 0x7E00u : 0x7Fu);
  const float a = fabsf(v);
  const int exp_bits = f->width - 1 - f->mant;
  const int emax = (1 << exp_bits) - 2 - ((1 << (exp_bits - 1)) - 1);
  if (!f->saturate && a >= ldexpf(1.0f, emax + 1)) return sign | 0x7C00u;
  if (a == 0.0f) return sign;
  int e;
  frexpf(a, &e); /* a = fr * 2^e, fr in [0.5, 1) */
  const int E = e - 1;
  if (E < f->emin) return sign | (uint32_t)ldexpf(a, f->mant - f->emin);
  const uint32_t frac = (uint32_t)(ldexpf(a, f->mant - E) - ldexpf(1.0f, f->mant));
  return sign | ((uint32_t)(E - f->emin + 1) << f->mant) | frac;
}

static float mf_decode(uint32_t enc, const mf_t* f) {
  const int exp_bits = f->width - 1 - f->mant;
  const uint32_t E = (enc >> f->mant) & ((1u << exp_bits) - 1u);
  const uint32_t frac = enc & ((1u << f->mant) - 1u);
  const float sign = (enc >> (f->width - 1)) ? -1.0f : 1.0f;
  if (f->mant == 3) { /* E4M3 (fn): only all-ones is special, and it is NaN */
    if (E == 15u && frac == 7u) return NAN;
  } else if (E == (1u << exp_bits) - 1u) {
    return frac ? NAN : sign * INFINITY;
  }
  if (E == 0) return sign * ldexpf((float)frac, f->emin - f->mant);
  return sign * ldexpf((float)((1u << f->mant) + frac), (int)E - 1 + f->emin - f->mant);
}

static const mf_t* mf_of(int dtype) {
  return dtype == D_F16 ? &MF_F16 : (dtype == D_E4M3 ? &MF_E4M3 : &MF_E5M2);
}

/* ---- storage access ----------------------------------------------------- */

static int width_of(int dtype) { return dtype == D_F32 ? 4 : (dtype <= D_F16 ? 2 : 1); }

static uint32_t load_raw(const void* base, int64_t i, int dtype) {
  switch (width_of(dtype)) {
    case 4: return ((const uint32_t*)base)[i];
    case 2: return ((const uint16_t*)base)[i];
    default: return ((const uint8_t*)base)[i];
  }
}

static void store_raw(void* base, int64_t i, int dtype, uint32_t v) {
  switch (width_of(dtype)) {
    case 4: ((uint32_t*)base)[i] = v; break;
    case 2: ((uint16_t*)base)[i] = (uint16_t)v; break;
    default: ((uint8_t*)base)[i] = (uint8_t)v; break;
  }
}

static float decode(uint32_t raw, int dtype) {
  if (dtype == D_F32) return bitsf(raw);
  if (dtype == D_BF16) return bitsf(raw << 16);
  return mf_decode(raw, mf_of(dtype));
}

/* Storage bits of x under (dtype, rule); `counter` feeds stochastic rules. */
static uint32_t encode(float x, int dtype, int rule, uint32_t counter) {
  if (dtype == D_F32) return fbits(x);
  if (dtype == D_BF16) return rule == R_STOCHASTIC ? bf16_stochastic(x, h32(counter)) : bf16_nearest(x);
  const mf_t* f = mf_of(dtype);
  const float v = rule == R_STOCHASTIC ? mf_stochastic_value(x, f, h32(counter)) : mf_nearest_value(x, f);
  return mf_encode(v, f);
}

/* ---- entry points ------------------------------------------------------- */

uint32_t oc_encode(float x, int dtype, int rule, uint32_t counter) {
  return encode(x, dtype, rule, counter);
}

float oc_decode(uint32_t raw, int dtype) { return decode(raw, dtype); }

/* y[i] = round(x[i]), counter = i + seed + offset (sr_states/rounding.py:97-124). */
void oc_cast(const float* x, void* y, int64_t n, int dtype, int rule, uint32_t seed,
             uint32_t offset) {
  for (int64_t i = 0; i < n; ++i)
    store_raw(y, i, dtype, encode(x[i], dtype, rule, (uint32_t)i + seed + offset));
}

/* hp = {beta1, beta2, 1-beta1, 1-beta2, -lr/(1-beta1^t), sqrt(1-beta2^t),
 *       1-lr*wd, eps}, each already rounded to FP32. */
void oc_adamw(void* p, int p_dtype, const void* g, int g_dtype, void* m, int m_dtype,
              int m_rule, void* v, int v_dtype, int v_rule, int64_t n, const float* hp,
              uint32_t key, uint32_t offset) {
  const uint32_t base_m = h32(key ^ 0u) + offset, base_v = h32(key ^ 1u) + offset;
  for (int64_t i = 0; i < n; ++i) {
    const float p32 = decode(load_raw(p, i, p_dtype), p_dtype);
    const float g32 = decode(load_raw(g, i, g_dtype), g_dtype);
    const float m32 = decode(load_raw(m, i, m_dtype), m_dtype);
    const float v32 = decode(load_raw(v, i, v_dtype), v_dtype);
    /* exp_avg.mul(beta1).add(g, alpha=1-beta1): torch fuses the add */
    const float m_new = fmaf(g32, hp[2], m32 * hp[0]);
    /* exp_avg_sq.mul(beta2).addcmul(g, g, value=1-beta2) */
    const float v_new = fmaf(hp[3] * g32, g32, v32 * hp[1]);
    /* v.sqrt().div_(sqrt(bc2)).add_(eps) */
    const float den = sqrtf(v_new) / hp[5] + hp[7];
    /* p.mul(1-lr*wd).addcdiv_(m, den, value=-lr/bc1) */
    const float p_new = p32 * hp[6] + (hp[4] * m_new) / den;
    store_raw(p, i, p_dtype, encode(p_new, p_dtype, R_NEAREST, 0));
    store_raw(m, i, m_dtype, encode(m_new, m_dtype, m_rule, (uint32_t)i + base_m));
    store_raw(v, i, v_dtype, encode(v_new, v_dtype, v_rule, (uint32_t)i + base_v));
  }
}

void oc_sgdm(void* p, int p_dtype, const void* g, int g_dtype, void* u, int u_dtype, int u_rule,
             int64_t n, float momentum, float neg_lr, uint32_t key, uint32_t offset) {
  const uint32_t base = h32(key ^ 0u) + offset;
  for (int64_t i = 0; i < n; ++i) {
    const float p32 = decode(load_raw(p, i, p_dtype), p_dtype);
    const float g32 = decode(load_raw(g, i, g_dtype), g_dtype);
    const float u32 = decode(load_raw(u, i, u_dtype), u_dtype);
    /* momentum.mul(mu).add(g); p.add(u, alpha=-lr) (torch fuses the latter) */
    const float u_new = u32 * momentum + g32;
    const float p_new = fmaf(u_new, neg_lr, p32);
    store_raw(p, i, p_dtype, encode(p_new, p_dtype, R_NEAREST, 0));
    store_raw(u, i, u_dtype, encode(u_new, u_dtype, u_rule, (uint32_t)i + base));
  }
}
