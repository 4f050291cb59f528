// sr_math.h -- element arithmetic of the stochastic-rounding optimizer path.
//
// Everything here is a pure function of its arguments, usable on the host
// (key derivation, CPU-side unit checks) and on gfx950.  Encoders work on the
// IEEE-754 bit patterns with integer ALU, except that the device finishes
// BF16 stochastic rounding with gfx950's stochastic convert, BF16 nearest
// rounding with its nearest convert, and the minifloat encodings with a
// hardware convert of an exactly representable value; all are checked
// exhaustively against the integer forms on the device.  The FP32 recurrences use explicit fmaf() exactly where the
// reference's eager CPU kernels fuse, and must be compiled with
// -ffp-contract=off so that no other multiply-add is contracted.
#pragma once

#include <stdint.h>

#include <type_traits>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define SR_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#define SR_HD static inline
#endif

namespace sr {

// ---------------------------------------------------------------------------
// Counter hash and keys (sr_states/_hash.py:5-50).
// ---------------------------------------------------------------------------
constexpr uint32_t kHashMul1 = 0x7FEB352Du;
constexpr uint32_t kHashMul2 = 0x846CA68Bu;
constexpr uint32_t kKeySalt = 0x9E3779B9u;

// 32-bit avalanche finalizer: two multiplies, three xor-shifts, mod 2^32.
SR_HD uint32_t h32(uint32_t x) {
  x ^= x >> 16;
  x *= kHashMul1;
  x ^= x >> 15;
  x *= kHashMul2;
  return x ^ (x >> 16);
}

// Update key of one parameter at one optimizer RNG step.  The seed and step
// enter as their low and high 32-bit words (sr_states/_hash.py:18-23).
// The first four rounds depend only on (seed, step), so a launch computes
// them once (update_key_prefix) and each row adds its parameter index.
SR_HD uint32_t update_key_prefix(uint32_t seed_lo, uint32_t seed_hi, uint32_t step_lo,
                                 uint32_t step_hi) {
  uint32_t key = h32(seed_lo ^ kKeySalt);
  key = h32(key ^ seed_hi);
  key = h32(key ^ step_lo);
  return h32(key ^ step_hi);
}

SR_HD uint32_t update_key_from_prefix(uint32_t prefix, uint32_t param_index) {
  return h32(prefix ^ param_index);
}

SR_HD uint32_t update_key(uint32_t seed_lo, uint32_t seed_hi, uint32_t step_lo,
                          uint32_t step_hi, uint32_t param_index) {
  return update_key_from_prefix(update_key_prefix(seed_lo, seed_hi, step_lo, step_hi), param_index);
}

// Per-state counter base (sr_states/_hash.py:26-28).
SR_HD uint32_t state_key(uint32_t key, uint32_t state_index) { return h32(key ^ state_index); }

// ---------------------------------------------------------------------------
// Storage encodings.  `Enc` values index the kernel instantiation tables.
// ---------------------------------------------------------------------------
enum Enc : int {
  ENC_F32 = 0,
  ENC_BF16_RN = 1,
  ENC_BF16_SR = 2,
  ENC_F16_RN = 3,
  ENC_F16_SR = 4,
  ENC_E4M3_RN = 5,
  ENC_E4M3_SR = 6,
  ENC_E5M2_RN = 7,
  ENC_E5M2_SR = 8,
  ENC_COUNT = 9
};

// Storage width in bytes of an encoding.
constexpr int enc_bytes(int enc) {
  return enc == ENC_F32 ? 4 : (enc <= ENC_F16_SR ? 2 : 1);
}
constexpr bool enc_stochastic(int enc) {
  return enc == ENC_BF16_SR || enc == ENC_F16_SR || enc == ENC_E4M3_SR || enc == ENC_E5M2_SR;
}

SR_HD uint32_t f32_bits(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __float_as_uint(x);
#else
  union { float f; uint32_t u; } v;
  v.f = x;
  return v.u;
#endif
}

SR_HD float bits_f32(uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __uint_as_float(b);
#else
  union { float f; uint32_t u; } v;
  v.u = b;
  return v.f;
#endif
}

// FP32 -> BF16 stochastic rounding (sr_states/_bf16.py:37-74).  For finite
// input the low 16 bits of the FP32 pattern are the position between the
// two BF16 neighbours; adding 16 uniform bits and truncating rounds away from
// zero with exactly that probability.  A carry may reach the next binade or
// +-Inf.  Inf needs no special case: its low 16 bits are zero, so the sum
// keeps the Inf pattern.  NaN gets its quiet bit forced so that truncation
// cannot turn it into Inf.  Written as a select so that it stays branch-free.
SR_HD uint32_t bf16_sr_bits(uint32_t b, uint32_t hash) {
  const uint32_t rounded = b + (hash & 0xFFFFu);
  const uint32_t quieted = b | 0x00400000u;
  const bool nan = (b & 0x7FFFFFFFu) > 0x7F800000u;
  return (nan ? quieted : rounded) >> 16;
}

// The same rounding with gfx950's stochastic convert.  v_cvt_sr_bf16_f32
// adds the upper 16 bits of its random operand below the BF16 mantissa and
// truncates, so it equals bf16_sr_bits when given the 16 random bits in the
// upper half.  Checked exactly, NaN payloads included, over every FP32 input
// at the random values where the decision flips, and over every pair of low
// input half and random value for the special and ordinary upper halves
// (tests/native/bf16_sr_check.hip).  Host builds use bf16_sr_bits.
SR_HD uint32_t bf16_sr(uint32_t b, uint32_t hash) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  // An empty asm hides the hash from the optimizer (it emits nothing).
  // Otherwise LLVM folds the shift below through the hash's last xor-shift
  // into its second multiply: y*C << 16 becomes y*(C << 16), one more
  // quarter-rate v_mul_lo_u32 per element where a shift would do.
  __asm__("" : "+v"(hash));
  const bf16x2 out =
      __builtin_amdgcn_cvt_sr_bf16_f32(bf16x2{}, __builtin_bit_cast(float, b), hash << 16, false);
  return __builtin_bit_cast(uint32_t, out) & 0xFFFFu;
#else
  return bf16_sr_bits(b, hash);
#endif
}

// FP32 -> BF16 round to nearest, ties to even (torch's Tensor.to(bfloat16)).
SR_HD uint32_t bf16_rn_bits(uint32_t b) {
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}

// bf16_rn_bits on the device: gfx950's v_cvt_pk_bf16_f32 rounds to nearest
// even in the kernels' rounding mode and keeps subnormals; NaN becomes the
// reference's 0x7FC0.  Checked against bf16_rn_bits on every FP32 input.
SR_HD uint32_t bf16_rn(uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float x = __builtin_bit_cast(float, b);
  const uint32_t rounded = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
  return x != x ? 0x7FC0u : rounded;
#else
  return bf16_rn_bits(b);
#endif
}

// Minifloat formats: mantissa bits M, minimum normal exponent EMIN, FP32
// bits of the largest finite magnitude, saturation policy and storage width
// (sr_states/_minifloat.py:10-14).
template <int M, int EMIN, uint32_t MAX_BITS, bool SAT, int WIDTH, uint32_t NAN_ENC, uint32_t INF_ENC>
struct Minifloat {
  static constexpr int kM = M;
  static constexpr int kEmin = EMIN;
  static constexpr uint32_t kMaxBits = MAX_BITS;
  static constexpr bool kSat = SAT;
  static constexpr int kWidth = WIDTH;
  static constexpr uint32_t kNan = NAN_ENC;
  static constexpr uint32_t kInf = INF_ENC;  // unused when saturating
};
using E4M3 = Minifloat<3, -6, 0x43E00000u /*448*/, true, 8, 0x7Fu, 0u>;
using E5M2 = Minifloat<2, -14, 0x47600000u /*57344*/, true, 8, 0x7Fu, 0u>;
using F16 = Minifloat<10, -14, 0x477FE000u /*65504*/, false, 16, 0x7E00u, 0x7C00u>;

// FP32 -> minifloat with nearest-even (STOCH=false) or 24-bit-grid
// stochastic rounding (STOCH=true), computed on the integer significand.
//
// With a = |x| (clamped to the format maximum when saturating) and
// e = max(exponent(a), EMIN), the target spacing is 2^(e-M).  Writing
// a / 2^(e-M) = q + r with integer q and 0 <= r < 1:
//   stochastic: round up iff (hash >> 8) < floor(r * 2^24)
//   nearest:    round up iff r > 1/2, or r == 1/2 and q is odd
// (sr_states/_minifloat.py:17-70).  a / 2^(e-M) equals sig * 2^-s for the
// 24-bit FP32 significand sig and shift s = 150 - M + e - E', so q, r and
// floor(r * 2^24) are exact integer shifts of sig.  The encoding of the
// result value (q + up) * 2^(e-M) is ((e - EMIN) << M) + q + up for every
// finite result: the carry q + up = 2^(M+1) lands on the next binade's
// encoding, and subnormals (e == EMIN, q < 2^M) need no special case.
template <class F, bool STOCH>
SR_HD uint32_t minifloat_bits(uint32_t b, uint32_t hash) {
  const uint32_t sign = (b >> 31) << (F::kWidth - 1);
  uint32_t a = b & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return F::kNan | sign;
  if (F::kSat) {
    a = a < F::kMaxBits ? a : F::kMaxBits;  // also maps +-Inf to +-max
  } else if (a == 0x7F800000u) {
    return F::kInf | sign;
  }
  const int E = (int)(a >> 23);
  const uint32_t sig = E ? ((a & 0x007FFFFFu) | 0x00800000u) : a;
  const int e_raw = (E ? E : 1) - 127;  // exponent of the significand's unit bit
  const int e = (E - 127) > F::kEmin ? (E - 127) : F::kEmin;
  const int s = 23 - F::kM + (e - e_raw);  // >= 23 - M >= 13
  uint32_t q, up;
  if (s <= 24) {
    q = sig >> s;
    const uint32_t rem = sig & ((1u << s) - 1u);
    if (STOCH) {
      up = (hash >> 8) < (rem << (24 - s)) ? 1u : 0u;
    } else {
      const uint32_t half = 1u << (s - 1);
      up = (rem > half || (rem == half && (q & 1u))) ? 1u : 0u;
    }
  } else {
    // a / spacing < 2^(24 - s) <= 1/2: q = 0 and nearest never rounds up.
    q = 0;
    const int t = s - 24;
    up = (STOCH && t < 24 && (hash >> 8) < (sig >> t)) ? 1u : 0u;
  }
  uint32_t enc = ((uint32_t)(e - F::kEmin) << F::kM) + q + up;
  if (!F::kSat) enc = enc < F::kInf ? enc : F::kInf;  // IEEE overflow to Inf
  return enc | sign;
}

// FP32 bits -> F rounded to nearest even, with IEEE overflow to Inf for
// FP16 (the FP8 callers clamp to the format maximum first): one hardware
// convert on the device, the integer nearest form on the host.  Exact for
// values F represents.  The empty asm makes the input opaque: otherwise,
// where the bits are those of an FMA result, the compiler may fuse the FMA
// and the convert into one mixed-precision instruction that rounds once,
// straight to F, instead of to FP32 first.
template <class F>
SR_HD uint32_t nearest_convert(uint32_t bits) {
#if defined(__HIP_DEVICE_COMPILE__)
  __asm__("" : "+v"(bits));
  const float v = __builtin_bit_cast(float, bits);
  if constexpr (F::kWidth == 16) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  } else if constexpr (F::kM == 3) {
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(v, 0.0f, 0, false)) & 0xFFu;
  } else {
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(v, 0.0f, 0, false)) & 0xFFu;
  }
#else
  return minifloat_bits<F, false>(bits, 0u);
#endif
}

// minifloat_bits on the device, bit for bit, with fewer instructions.
// Nearest even is the convert's own rounding, applied to the (clamped)
// input.  Stochastic: with D = s the number of dropped significand bits,
// "round up iff (hash >> 8) < rem * 2^(24-D)" equals "iff T < rem" for
// T = (hash >> 8) >> (24 - D), and for D <= 23 the dropped bits are the low
// D bits of the FP32 pattern, so the rounded value's FP32 bits are
//   (a + 2^D - 1 - T) & ~(2^D - 1)
// with the carry into the exponent doing what q + up does in the integer
// form.  For D >= 24 the result is 0 or the smallest subnormal, decided as
// in minifloat_bits.  That value is exactly representable (or, for FP16, at
// least 65536 and taken to Inf), so the convert finishes the encoding
// exactly.  tests/native/minifloat_check.hip compares the two on every FP32
// input: nearest once, stochastic at the random values where each input's
// decision flips and at the extremes.
template <class F, bool STOCH>
SR_HD uint32_t minifloat_bits_fast(uint32_t b, uint32_t hash) {
  const uint32_t sign = b & 0x80000000u;
  uint32_t a = b & 0x7FFFFFFFu;
  const bool nan = a > 0x7F800000u;
  if (F::kSat) a = a < F::kMaxBits ? a : F::kMaxBits;  // also maps +-Inf to +-max
  if constexpr (!STOCH) {
    // Nearest even on the target grid, with IEEE overflow to Inf for FP16,
    // is the convert's own rounding; the FP8 formats saturate by the clamp.
    const uint32_t enc = nearest_convert<F>(a | sign);
    return nan ? (F::kNan | (sign >> (32 - F::kWidth))) : enc;
  }
  // D dropped significand bits: 23 - M on normal results, one more per
  // binade below the smallest normal.  The code works with s = 32 - D and
  // the complemented hash: (~hash) >> k = (2^(32-k) - 1) - (hash >> k).
  // An FP32 subnormal (E = 0) is far below F's smallest subnormal; taking
  // its exponent as 0 instead of 1 keeps it in the second branch, where it
  // never rounds up, as in the integer form.  The two branches stay real
  // branches: waves whose elements all take one side skip the other, which
  // measured 3-6% faster on FP8 casts than computing both sides with
  // selects.
  const int E = static_cast<int>(a >> 23);
  const int s_below = E - (118 + F::kEmin - F::kM);
  const int s = s_below < 9 + F::kM ? s_below : 9 + F::kM;
  const uint32_t sign_bit = sign >> (32 - F::kWidth);
  if (s >= 9) {  // D <= 23
    // With T = (hash >> 8) >> (24 - D) = hash >> s and mask = 2^D - 1:
    // mask - T = ~hash >> s, and mask = 0xFFFFFFFF >> s.
    const uint32_t r = (a + (~hash >> s)) & ~(0xFFFFFFFFu >> s);
    const uint32_t enc = nearest_convert<F>(r | sign);  // exact: r is on the grid
    return nan ? (F::kNan | sign_bit) : enc;            // NaN has E = 255: only here
  }
  // D >= 24: 0, or the smallest subnormal (encoding 1) when the random
  // value's upper 24 bits fall below sig / 2^(D - 24); no NaN reaches here.
  // Shifts of 24 to 31 leave nothing of the 24-bit significand, so D - 24
  // is clamped to 31 instead of tested.
#if defined(__HIP_DEVICE_COMPILE__)
  // The compiler drops the skip over a divergent block this short, so
  // waves with no such element would still issue it; an asm statement
  // (even an empty one) keeps the skip.
  __asm__ volatile("");
#endif
  const uint32_t sig = (a & 0x007FFFFFu) | 0x00800000u;
  const int t = 8 - s;  // D - 24
  const bool up = (hash >> 8) < (sig >> (t < 31 ? t : 31));
  return sign_bit | (up ? 1u : 0u);
}

// The minifloat encoders: the integer form on the host, its bit-exact
// hardware-finished form on the device.
template <class F, bool STOCH>
SR_HD uint32_t minifloat_encode(uint32_t b, uint32_t hash) {
#if defined(__HIP_DEVICE_COMPILE__)
  return minifloat_bits_fast<F, STOCH>(b, hash);
#else
  return minifloat_bits<F, STOCH>(b, hash);
#endif
}

// ---------------------------------------------------------------------------
// Ordered neighbours: for each FP32 input, the two storage values that
// stochastic rounding chooses between, lower <= x <= upper.  A checking
// helper beside the encoders, not used by the updates.
// ---------------------------------------------------------------------------

// BF16 (sr_states/_bf16.py:77-101).  Dropping the low 16 bits moves toward
// zero, and one more in the truncated BF16 word moves away from zero for
// either sign (from the largest finite magnitude to Inf).  Inputs BF16
// represents, Inf and NaN give their nearest-even conversion twice.
SR_HD void bf16_neighbor_bits(uint32_t b, uint32_t& lower, uint32_t& upper) {
  if ((b & 0xFFFFu) == 0u || (b & 0x7F800000u) == 0x7F800000u) {
    lower = upper = bf16_rn_bits(b);
    return;
  }
  const uint32_t toward = b >> 16;
  const uint32_t away = toward + 1u;
  const bool negative = (b >> 31) != 0u;
  lower = negative ? away : toward;
  upper = negative ? toward : away;
}

// The minifloat formats after their saturation policy
// (sr_states/_minifloat.py:73-99).  With q and the spacing of
// minifloat_bits, the value toward zero is q * spacing, whose encoding is
// ((e - EMIN) << M) + q, and the one away from zero one encoding further
// unless x lies on the grid: every nonzero remainder counts, however small,
// also where the stochastic rule's 24-bit threshold is 0.  Saturating
// formats clamp |x| (Inf included) to the maximum first.  FP16 brackets
// finite magnitudes above its maximum by the maximum and Inf, and keeps
// Inf.  NaN gives F's NaN twice.
template <class F>
SR_HD void minifloat_neighbor_bits(uint32_t b, uint32_t& lower, uint32_t& upper) {
  const uint32_t sign = (b >> 31) << (F::kWidth - 1);
  uint32_t a = b & 0x7FFFFFFFu;
  if (a > 0x7F800000u) {
    lower = upper = F::kNan | sign;
    return;
  }
  if (F::kSat) a = a < F::kMaxBits ? a : F::kMaxBits;
  uint32_t toward, away;
  if (!F::kSat && a > F::kMaxBits) {
    toward = a == 0x7F800000u ? F::kInf : F::kInf - 1u;  // Inf, or the largest finite
    away = F::kInf;
  } else {
    const int E = static_cast<int>(a >> 23);
    const uint32_t sig = E ? ((a & 0x007FFFFFu) | 0x00800000u) : a;
    const int e_raw = (E ? E : 1) - 127;
    const int e = (E - 127) > F::kEmin ? (E - 127) : F::kEmin;
    const int s = 23 - F::kM + (e - e_raw);  // >= 23 - M
    const uint32_t q = s < 32 ? sig >> s : 0u;
    const bool inexact = s < 32 ? (sig & ((1u << s) - 1u)) != 0u : sig != 0u;
    toward = (static_cast<uint32_t>(e - F::kEmin) << F::kM) + q;
    away = toward + (inexact ? 1u : 0u);
  }
  const bool negative = sign != 0u;
  lower = (negative ? away : toward) | sign;
  upper = (negative ? toward : away) | sign;
}

template <int ENC>
SR_HD void neighbor_bits(uint32_t b, uint32_t& lower, uint32_t& upper) {
  if constexpr (ENC == ENC_BF16_RN) {
    bf16_neighbor_bits(b, lower, upper);
  } else if constexpr (ENC == ENC_F16_RN) {
    minifloat_neighbor_bits<F16>(b, lower, upper);
  } else if constexpr (ENC == ENC_E4M3_RN) {
    minifloat_neighbor_bits<E4M3>(b, lower, upper);
  } else {
    static_assert(ENC == ENC_E5M2_RN, "neighbours exist for BF16, FP16, E4M3 and E5M2");
    minifloat_neighbor_bits<E5M2>(b, lower, upper);
  }
}

// Encode an FP32 value into the storage bits of `ENC` with the counter's
// hash.  The hash is only evaluated for stochastic encodings.
template <int ENC>
SR_HD uint32_t encode(float x, uint32_t counter) {
  const uint32_t b = f32_bits(x);
  if constexpr (ENC == ENC_F32) {
    return b;
  } else if constexpr (ENC == ENC_BF16_RN) {
    return bf16_rn(b);
  } else if constexpr (ENC == ENC_BF16_SR) {
    return bf16_sr(b, h32(counter));
  } else if constexpr (ENC == ENC_F16_RN) {
    return minifloat_encode<F16, false>(b, 0);
  } else if constexpr (ENC == ENC_F16_SR) {
    return minifloat_encode<F16, true>(b, h32(counter));
  } else if constexpr (ENC == ENC_E4M3_RN) {
    return minifloat_encode<E4M3, false>(b, 0);
  } else if constexpr (ENC == ENC_E4M3_SR) {
    return minifloat_encode<E4M3, true>(b, h32(counter));
  } else if constexpr (ENC == ENC_E5M2_RN) {
    return minifloat_encode<E5M2, false>(b, 0);
  } else {
    static_assert(ENC == ENC_E5M2_SR, "unknown encoding");
    return minifloat_encode<E5M2, true>(b, h32(counter));
  }
}

// Exact decode of a minifloat encoding to FP32 (torch's Tensor.float()).
template <class F>
SR_HD float minifloat_value(uint32_t v) {
  constexpr int kExpBits = F::kWidth - 1 - F::kM;
  constexpr uint32_t kExpMask = (1u << kExpBits) - 1u;
  const uint32_t sign = (v >> (F::kWidth - 1)) << 31;
  const uint32_t E = (v >> F::kM) & kExpMask;
  const uint32_t man = v & ((1u << F::kM) - 1u);
  if (F::kSat && F::kM == 3) {  // E4M3 (fn): only S.1111.111 is special (NaN)
    if (E == kExpMask && man == ((1u << F::kM) - 1u)) return bits_f32(sign | 0x7FC00000u);
  } else if (E == kExpMask) {  // E5M2 / FP16: IEEE Inf and NaN
    return bits_f32(sign | 0x7F800000u | (man << (23 - F::kM)) | (man ? 0x00400000u : 0u));
  }
  if (E == 0) {
    // man * 2^(EMIN - M): a small integer times a power of two, exact.
    const float mag = (float)man * bits_f32((uint32_t)(127 + F::kEmin - F::kM) << 23);
    return bits_f32(f32_bits(mag) | sign);
  }
  return bits_f32(sign | ((E - 1u + (uint32_t)(127 + F::kEmin)) << 23) | (man << (23 - F::kM)));
}

// minifloat_value on the device with one hardware convert: equal for every
// encoding that is not a NaN, and a NaN for every NaN encoding (payloads are
// not part of the contract), checked for every encoding by
// tests/native/minifloat_check.hip.
template <class F>
SR_HD float minifloat_decode(uint32_t v) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (F::kWidth == 16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(v)));
  } else if constexpr (F::kM == 3) {
    return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(v), 0);
  } else {
    return __builtin_amdgcn_cvt_f32_bf8(static_cast<int>(v), 0);
  }
#else
  return minifloat_value<F>(v);
#endif
}

// Decode storage bits of `ENC` to the exact FP32 value.
template <int ENC>
SR_HD float decode(uint32_t v) {
  if constexpr (ENC == ENC_F32) {
    return bits_f32(v);
  } else if constexpr (ENC == ENC_BF16_RN || ENC == ENC_BF16_SR) {
    return bits_f32(v << 16);
  } else if constexpr (ENC == ENC_F16_RN || ENC == ENC_F16_SR) {
    return minifloat_decode<F16>(v);
  } else if constexpr (ENC == ENC_E4M3_RN || ENC == ENC_E4M3_SR) {
    return minifloat_decode<E4M3>(v);
  } else {
    return minifloat_decode<E5M2>(v);
  }
}

// ---------------------------------------------------------------------------
// Groups of four consecutive elements.
//
// The kernels' vector paths move four consecutive elements per lane as one
// access, so they decode and encode whole storage words (element k of a
// group at byte k * width, little-endian).  On the device two elements share
// one hardware convert where gfx950 has a paired form: v_cvt_pk_f32_fp8 /
// _bf8 to decode, v_cvt_pk_fp8_f32 / _bf8_f32, v_cvt_pk_f16_f32 and
// v_cvt_pk_bf16_f32 to encode, and v_cvt_sr_bf16_f32 writing either half of
// its destination.  The bits equal the single-element forms' for every
// input in every position of a group (tests/native/minifloat_check.hip and
// tests/native/bf16_sr_check.hip check both sides on the device); on the
// host the groups are the single-element forms.
// ---------------------------------------------------------------------------
constexpr int kGroup = 4;

// Storage words of one group of encoding ENC.
constexpr int group_words(int enc) { return enc_bytes(enc) * kGroup / 4; }

constexpr float pow2f(int e) {
  float r = 1.0f;
  for (; e > 0; --e) r *= 2.0f;
  for (; e < 0; ++e) r *= 0.5f;
  return r;
}

// Element codes (one per 32-bit lane) packed into storage words, and back.
template <int ENC>
SR_HD void pack_group(const uint32_t (&codes)[kGroup], uint32_t (&words)[group_words(ENC)]) {
  constexpr int W = enc_bytes(ENC);
#pragma unroll
  for (int j = 0; j < group_words(ENC); ++j) words[j] = 0u;
#pragma unroll
  for (int k = 0; k < kGroup; ++k) words[k * W / 4] |= codes[k] << (8 * ((k * W) % 4));
}

template <int ENC>
SR_HD void unpack_group(const uint32_t (&words)[group_words(ENC)], uint32_t (&codes)[kGroup]) {
  constexpr int W = enc_bytes(ENC);
  constexpr uint32_t mask = W == 4 ? 0xFFFFFFFFu : (1u << (8 * W)) - 1u;
#pragma unroll
  for (int k = 0; k < kGroup; ++k) codes[k] = (words[k * W / 4] >> (8 * ((k * W) % 4))) & mask;
}

// The value minifloat_bits<F, STOCH> rounds b to, as FP32 bits, for every b
// that is not a NaN (NaN gives an unspecified value; callers treat NaN
// groups apart).  Nearest: the clamped input, which the convert rounds.
// Stochastic with D <= 23 dropped bits: the grid value of
// minifloat_bits_fast.  Below F's smallest subnormal 2^(EMIN - M) (D >= 24):
// that subnormal when (hash >> 8) < floor(|b| 2^(24 - EMIN + M)), else 0 --
// the integer form's threshold sig >> (D - 24), here one exact product (a
// power of two; the result is below 2^24) and a truncating convert.  Every
// result is exactly representable in F (or, for FP16, at least 65536 and
// taken to Inf by the convert).
template <class F>
constexpr uint32_t kSubnormalBits = static_cast<uint32_t>(127 + F::kEmin - F::kM) << 23;

// `subnormal` is kSubnormalBits<F>, passed in so that a caller encoding
// several elements holds the constant in one register.
template <class F, bool STOCH>
SR_HD uint32_t minifloat_grid_bits(uint32_t b, uint32_t hash, uint32_t subnormal = kSubnormalBits<F>) {
  const uint32_t sign = b & 0x80000000u;
  uint32_t a = b & 0x7FFFFFFFu;
  if (F::kSat) a = a < F::kMaxBits ? a : F::kMaxBits;  // also maps +-Inf to +-max
  if constexpr (!STOCH) {
    (void)hash;
    return a | sign;
  } else {
    constexpr float kScale = pow2f(24 - F::kEmin + F::kM);
    uint32_t rounded;
    if (a >= subnormal) {
#if defined(__HIP_DEVICE_COMPILE__)
      // Each branch keeps its skip, so a wave whose elements all take one
      // side never issues the other (the compiler drops skips over short
      // blocks; an asm statement, even an empty one, keeps them).
      __asm__ volatile("");
#endif
      const int E = static_cast<int>(a >> 23);
      const int s_below = E - (118 + F::kEmin - F::kM);
      const int s = s_below < 9 + F::kM ? s_below : 9 + F::kM;
      rounded = (a + (~hash >> s)) & ~(0xFFFFFFFFu >> s);
    } else {
#if defined(__HIP_DEVICE_COMPILE__)
      __asm__ volatile("");
#endif
      const uint32_t threshold = static_cast<uint32_t>(bits_f32(a) * kScale);
      rounded = (hash >> 8) < threshold ? subnormal : 0u;
    }
    return rounded | sign;
  }
}

// The stochastic grid value of minifloat_grid_bits<F, true> for the FP8
// formats (M <= 3) in one computation, with no branch between the normal
// and the subnormal range.  |b|, clamped to the largest finite value, is
// scaled by the power of two that makes the grid spacing there -- 2^(e-M) in
// the binade of 2^e, 2^(emin-M) below 2^emin -- equal to 2^24.  The product
// is exact and below 2^(25+M) <= 2^28, so its truncated integer y holds the
// grid index above bit 24 and, below it, the integer form's 24-bit threshold
// T (the dropped fraction times 2^24, truncated).  (y + (~hash >> 8)) >> 24
// is then the index plus one iff (hash >> 8) < T, and the rounded value is
// that index times the spacing (exact: the index is at most 2^(M+1)).  For
// every b that is not a NaN (NaN gives an unspecified value).  `low24` and
// `magnitude` are the constants 0x00FFFFFF and 0x7FFFFFFF; a caller encoding
// several elements passes them in scalar registers, where the three-operand
// instructions that fold the xor into the add and the sign merge take them
// (these instructions take no literal operand).
template <class F>
SR_HD uint32_t fp8_sr_grid_bits(uint32_t b, uint32_t hash, uint32_t low24 = 0x00FFFFFFu,
                                uint32_t magnitude = 0x7FFFFFFFu) {
  static_assert(F::kWidth == 8 && F::kSat && F::kM <= 3, "FP8 formats only");
  // Scale exponent 151 + M - e in the binade of 2^e (from the exponent field),
  // at most 151 - emin + M; spacing exponent 24 less than minus the scale's.
  constexpr uint32_t kScaleOfExponent = (278u + F::kM) << 23;
  constexpr uint32_t kScaleBelowNormal = static_cast<uint32_t>(151 - F::kEmin + F::kM) << 23;
  constexpr uint32_t kSpacingOfScale = 278u << 23;
  // |b| clamped to the largest finite value (+-Inf to it as well).
  const float clamped = fminf(fabsf(bits_f32(b)), bits_f32(F::kMaxBits));
  const uint32_t from_exponent = kScaleOfExponent - (f32_bits(clamped) & 0x7F800000u);
  const uint32_t scale = from_exponent < kScaleBelowNormal ? from_exponent : kScaleBelowNormal;
  const uint32_t y = static_cast<uint32_t>(clamped * bits_f32(scale));
  // ~hash >> 8 is the 24-bit complement of hash >> 8.
  const uint32_t index = (((hash >> 8) ^ low24) + y) >> 24;
  const float value = static_cast<float>(index) * bits_f32(kSpacingOfScale - scale);
  return b ^ ((b ^ f32_bits(value)) & magnitude);  // value's magnitude, b's sign
}

// Decodes one group of storage words of ENC.
template <int ENC>
SR_HD void decode_group(const uint32_t (&words)[group_words(ENC)], float (&x)[kGroup]) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (ENC == ENC_E4M3_RN || ENC == ENC_E4M3_SR || ENC == ENC_E5M2_RN || ENC == ENC_E5M2_SR) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    constexpr bool kE4M3 = ENC == ENC_E4M3_RN || ENC == ENC_E4M3_SR;
    const int w = static_cast<int>(words[0]);
    const f2 lo = kE4M3 ? __builtin_amdgcn_cvt_pk_f32_fp8(w, false) : __builtin_amdgcn_cvt_pk_f32_bf8(w, false);
    const f2 hi = kE4M3 ? __builtin_amdgcn_cvt_pk_f32_fp8(w, true) : __builtin_amdgcn_cvt_pk_f32_bf8(w, true);
    x[0] = lo.x;
    x[1] = lo.y;
    x[2] = hi.x;
    x[3] = hi.y;
    return;
  }
#endif
  uint32_t codes[kGroup];
  unpack_group<ENC>(words, codes);
#pragma unroll
  for (int k = 0; k < kGroup; ++k) x[k] = decode<ENC>(codes[k]);
}

// Encodes one group of FP32 values (bits b) with the random words
// hash[k] (ignored by nearest encodings) into storage words of ENC.
// kFromMemory: the values were loaded as they are (the casts), so no FMA
// result can fuse into a convert and the group needs no barrier against it.
template <int ENC, bool kFromMemory = false>
SR_HD void encode_group_with(const uint32_t (&b)[kGroup], const uint32_t (&hash)[kGroup],
                             uint32_t (&words)[group_words(ENC)]) {
#if defined(__HIP_DEVICE_COMPILE__)
  if constexpr (ENC == ENC_F32) {
#pragma unroll
    for (int k = 0; k < kGroup; ++k) words[k] = b[k];
  } else if constexpr (ENC == ENC_BF16_SR) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t h0 = hash[2 * j], h1 = hash[2 * j + 1];
      // As in bf16_sr: the empty asm keeps each shift a shift.
      __asm__("" : "+v"(h0));
      __asm__("" : "+v"(h1));
      bf16x2 pair = __builtin_amdgcn_cvt_sr_bf16_f32(bf16x2{}, __builtin_bit_cast(float, b[2 * j]), h0 << 16, false);
      pair = __builtin_amdgcn_cvt_sr_bf16_f32(pair, __builtin_bit_cast(float, b[2 * j + 1]), h1 << 16, true);
      words[j] = __builtin_bit_cast(uint32_t, pair);
    }
  } else if constexpr (ENC == ENC_BF16_RN) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    // The sum of the group is NaN if any element is (or for opposite
    // infinities): then every element takes the integer form bf16_rn_bits,
    // whose NaN is the reference's 0x7FC0 whatever the payload (rare; whole
    // waves skip it; a convert there would be shared with the pairs below
    // and split them).
    uint32_t bits[kGroup];
    float x[kGroup];
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      // The empty asm keeps an FMA producing b from fusing with the convert.
      // Loaded values need none, and there it made the compiler wait for a
      // group's load before issuing the next one.
      bits[k] = b[k];
      if constexpr (!kFromMemory) __asm__("" : "+v"(bits[k]));
      x[k] = __builtin_bit_cast(float, bits[k]);
    }
    const float sum = (x[0] + x[1]) + (x[2] + x[3]);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const bf16x2 pair = {static_cast<__bf16>(x[2 * j]), static_cast<__bf16>(x[2 * j + 1])};
      words[j] = __builtin_bit_cast(uint32_t, pair);
    }
    if (sum != sum) {
      __asm__ volatile("");
      uint32_t codes[kGroup];
#pragma unroll
      for (int k = 0; k < kGroup; ++k) codes[k] = bf16_rn_bits(bits[k]);
      pack_group<ENC>(codes, words);
    }
  } else {
    using F = typename std::conditional<ENC == ENC_F16_RN || ENC == ENC_F16_SR, F16,
              typename std::conditional<ENC == ENC_E4M3_RN || ENC == ENC_E4M3_SR, E4M3, E5M2>::type>::type;
    constexpr bool kStoch = enc_stochastic(ENC);
    uint32_t grid[kGroup];
    bool nan = false;
    uint32_t subnormal = kSubnormalBits<F>, low24 = 0x00FFFFFFu, magnitude = 0x7FFFFFFFu;
    if constexpr (kStoch && F::kWidth == 8) {
      __asm__("" : "+s"(low24), "+s"(magnitude));  // one scalar register each
    } else {
      __asm__("" : "+v"(subnormal));  // one register for the group's four selects
    }
#pragma unroll
    for (int k = 0; k < kGroup; ++k) {
      nan |= bits_f32(b[k]) != bits_f32(b[k]);
      if constexpr (kStoch && F::kWidth == 8) grid[k] = fp8_sr_grid_bits<F>(b[k], hash[k], low24, magnitude);
      else grid[k] = minifloat_grid_bits<F, kStoch>(b[k], hash[k], subnormal);
      __asm__("" : "+v"(grid[k]));  // no fusing of an FMA into the convert
    }
    float g[kGroup];
#pragma unroll
    for (int k = 0; k < kGroup; ++k) g[k] = __builtin_bit_cast(float, grid[k]);
    if constexpr (F::kWidth == 16) {
      typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const f16x2 pair = {static_cast<_Float16>(g[2 * j]), static_cast<_Float16>(g[2 * j + 1])};
        words[j] = __builtin_bit_cast(uint32_t, pair);
      }
    } else if constexpr (F::kM == 3) {
      int w = __builtin_amdgcn_cvt_pk_fp8_f32(g[0], g[1], 0, false);
      words[0] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(g[2], g[3], w, true));
    } else {
      int w = __builtin_amdgcn_cvt_pk_bf8_f32(g[0], g[1], 0, false);
      words[0] = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(g[2], g[3], w, true));
    }
    if (nan) {
      // A NaN anywhere in the group: every element through the single-element
      // form (rare; whole waves skip it).
      __asm__ volatile("");
      uint32_t codes[kGroup];
#pragma unroll
      for (int k = 0; k < kGroup; ++k) codes[k] = minifloat_bits_fast<F, kStoch>(b[k], hash[k]);
      pack_group<ENC>(codes, words);
    }
  }
#else
  uint32_t codes[kGroup];
#pragma unroll
  for (int k = 0; k < kGroup; ++k) {
    if constexpr (ENC == ENC_F32) codes[k] = b[k];
    else if constexpr (ENC == ENC_BF16_RN) codes[k] = bf16_rn_bits(b[k]);
    else if constexpr (ENC == ENC_BF16_SR) codes[k] = bf16_sr_bits(b[k], hash[k]);
    else if constexpr (ENC == ENC_F16_RN) codes[k] = minifloat_bits<F16, false>(b[k], 0u);
    else if constexpr (ENC == ENC_F16_SR) codes[k] = minifloat_bits<F16, true>(b[k], hash[k]);
    else if constexpr (ENC == ENC_E4M3_RN) codes[k] = minifloat_bits<E4M3, false>(b[k], 0u);
    else if constexpr (ENC == ENC_E4M3_SR) codes[k] = minifloat_bits<E4M3, true>(b[k], hash[k]);
    else if constexpr (ENC == ENC_E5M2_RN) codes[k] = minifloat_bits<E5M2, false>(b[k], 0u);
    else codes[k] = minifloat_bits<E5M2, true>(b[k], hash[k]);
  }
  pack_group<ENC>(codes, words);
#endif
}

// Encodes one group with counters counter0 + k: the hash of each counter
// for stochastic encodings (sr_states/_hash.py:31-50), nothing for nearest.
template <int ENC, bool kFromMemory = false>
SR_HD void encode_group(const float (&x)[kGroup], uint32_t counter0, uint32_t (&words)[group_words(ENC)]) {
  uint32_t b[kGroup], hash[kGroup];
#pragma unroll
  for (int k = 0; k < kGroup; ++k) {
    b[k] = f32_bits(x[k]);
    hash[k] = enc_stochastic(ENC) ? h32(counter0 + static_cast<uint32_t>(k)) : 0u;
  }
  encode_group_with<ENC, kFromMemory>(b, hash, words);
}

// ---------------------------------------------------------------------------
// FP32 recurrences in the eager reference's operation order.
// ---------------------------------------------------------------------------
struct AdamWScalars {
  float beta1, beta2, one_minus_beta1, one_minus_beta2;
  float neg_step_size, correction2_sqrt, decay, eps;
  float inv_correction2_sqrt;  // RN(1 / correction2_sqrt)
};

// Domain of correction2_sqrt = f32(sqrt(1 - beta2^t)) for 0 <= beta2 < 1
// (a double) and t >= 1: 1 - beta2^t >= 2^-53, so it lies in [2^-27, 1].
constexpr float kMinCorrection2Sqrt = 0x1p-27f;

// IEEE square root, correctly rounded, for |v| >= 2^-96, zero, infinite
// and NaN v.  On the device: y = the hardware 1/sqrt(v) estimate,
// s0 = RN(v y), and one Newton step with the exact residual,
// RN(s0 + RN(v - s0^2) * RN(y / 2)).  A device check found this equal to
// the correctly rounded root for every v in [2^-96, +Inf); zero and +Inf,
// where s0 is 0 * Inf, return v itself, and negative v and NaN give NaN
// through y.  Below 2^-96 the residual loses bits: sqrt_needs_library()
// marks those inputs, for which the caller takes sqrtf.  Checked, with that
// fallback, against sqrtf on every FP32 input.
SR_HD float sqrt_rn_wide(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float y = __builtin_amdgcn_rsqf(v);
  const float s0 = v * y;
  const float root = fmaf(fmaf(-s0, s0, v), 0.5f * y, s0);
  constexpr int kZeroOrInf = 32 | 64 | 512;  // -0, +0, +Inf
  return __builtin_amdgcn_classf(v, kZeroOrInf) ? v : root;
#else
  return sqrtf(v);
#endif
}

SR_HD bool sqrt_needs_library(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_fabsf(v) < 0x1p-96f && v != 0.0f;
#else
  (void)v;
  return false;
#endif
}

// sqrtf behind a side effect the compiler may not hoist, so that the
// library's scaled sequence stays behind its branch instead of being
// computed for every input and selected.
SR_HD float sqrt_library(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
  __asm__ volatile("" : "+v"(v));
#endif
  return sqrtf(v);
}

// Correctly rounded square root of any float.
SR_HD float sqrt_rn(float v) {
  float root = sqrt_rn_wide(v);
  if (sqrt_needs_library(v)) root = sqrt_library(v);
  return root;
}

// x / c, correctly rounded, for c in [2^-27, 1] with r = RN(1/c), and x
// zero, infinite, NaN or in [2^-75, 2^64] (every square root of a float).
// On the device: q0 = RN(x r) and one correction by the exact remainder
// x - q0 c (Markstein's step).  Scaling x or c by a power of two scales
// every intermediate exactly in that domain, so agreement on every pair of
// significands is agreement everywhere; a device check covers all 2^46
// pairs.  Zero, infinite and NaN quotients keep q0, as x / c gives them.
SR_HD float div_by_constant(float x, float c, float r) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float q0 = x * r;
  const float q = fmaf(fmaf(-q0, c, x), r, q0);
  constexpr int kFinite = 8 | 16 | 128 | 256;  // negative/positive normal and subnormal
  return __builtin_amdgcn_classf(q0, kFinite) ? q : q0;
#else
  (void)r;
  return x / c;
#endif
}

// sr_states/reference/adamw.py:86-96:
//   m' = m*beta1 + (1-beta1)*g          -> fma(g, 1-beta1, m*beta1)
//   v' = v*beta2 + (1-beta2)*g*g        -> fma((1-beta2)*g, g, v*beta2)
//   den = sqrt(v') / sqrt(1-beta2^t) + eps
//   p' = p*(1-lr*wd) + (-lr/(1-beta1^t) * m') / den
// Every operation is rounded to FP32 on its own; division and square root
// are IEEE correctly rounded (the division by sqrt(1-beta2^t) through its
// reciprocal, exactly).  The parameter uses the unrounded m'.
SR_HD void adamw_moments(float g, float m, float v, const AdamWScalars& s, float& m_out,
                         float& v_out) {
  const float m_scaled = m * s.beta1;
  m_out = fmaf(g, s.one_minus_beta1, m_scaled);
  const float g_scaled = s.one_minus_beta2 * g;
  const float v_scaled = v * s.beta2;
  v_out = fmaf(g_scaled, g, v_scaled);
}

// The denominator sqrt(v') / sqrt(1-beta2^t) + eps from root = sqrt(v').
SR_HD float adamw_denominator(float root, const AdamWScalars& s) {
  return div_by_constant(root, s.correction2_sqrt, s.inv_correction2_sqrt) + s.eps;
}

// The same without div_by_constant's selection of q0: equal to it for every
// finite root when eps > 0 (the selection matters for an infinite root, and
// for the sign of a zero root, which adding a positive eps removes).  The
// vector path's division falls back, recomputing adamw_denominator, wherever
// the result is infinite or NaN.
SR_HD float adamw_denominator_finite(float root, const AdamWScalars& s) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float q0 = root * s.inv_correction2_sqrt;
  return fmaf(fmaf(-q0, s.correction2_sqrt, root), s.inv_correction2_sqrt, q0) + s.eps;
#else
  return adamw_denominator(root, s);
#endif
}

// The parameter from the unrounded m' and root = sqrt(v').
SR_HD float adamw_parameter(float p, float m_out, float root, const AdamWScalars& s) {
  const float numer = s.neg_step_size * m_out;
  const float p_decayed = p * s.decay;
  return p_decayed + numer / adamw_denominator(root, s);
}

// Domain of div_short for the AdamW denominator: with eps in [2^-60, 2^100]
// every finite denominator sqrt(v') / c + eps lies in [2^-60, 2^101), since
// sqrt(v') < 2^64 and c >= 2^-27.  A launch-uniform test on eps's bits.
SR_HD bool short_division_eps(float eps) {
  const uint32_t e = f32_bits(eps);
  return e >= 0x21800000u && e <= 0x71800000u;  // 2^-60 .. 2^100
}

// RN(1/b) for every b in [2^-126, 2^126): the hardware reciprocal estimate
// y0 and one Newton step, RN(y0 + RN(1 - b y0) y0).  A device check compares
// it with 1.0f / b on every float of that range.
SR_HD float rcp_rn(float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float y0 = __builtin_amdgcn_rcpf(b);
  return fmaf(fmaf(-b, y0, 1.0f), y0, y0);
#else
  return 1.0f / b;
#endif
}

// a / b, correctly rounded, wherever `ok` comes back true, for b in
// [2^-60, 2^101).  On the device: y = rcp_rn(b) = RN(1/b), q0 = RN(a y),
// and Markstein's correction by the exact remainder a - b q0.  `ok` is false unless |q0| lies in [2^-40, 2^100): there q0,
// the quotient and the remainder stay clear of underflow and overflow
// (|a| >= 2^-101), so scaling a or b by a power of two scales every
// intermediate exactly, and a device check of every pair of significands
// covers the whole domain.  Zero, infinite and NaN quotients come back with
// ok false.  The caller divides again with the library where ok is false.
SR_HD float div_short(float a, float b, bool& ok) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float y = rcp_rn(b);
  const float q0 = a * y;
  ok = __builtin_fabsf(q0) >= 0x1p-40f && __builtin_fabsf(q0) < 0x1p100f;
  return fmaf(fmaf(-b, q0, a), y, q0);
#else
  ok = true;
  return a / b;
#endif
}

// a / b through the library's correctly rounded sequence, behind a side
// effect the compiler may not hoist (as sqrt_library).
SR_HD float div_library(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
  __asm__ volatile("" : "+v"(a));
#endif
  return a / b;
}

SR_HD void adamw_update(float p, float g, float m, float v, const AdamWScalars& s,
                        float& p_out, float& m_out, float& v_out) {
  adamw_moments(g, m, v, s, m_out, v_out);
  p_out = adamw_parameter(p, m_out, sqrt_rn(v_out), s);
}

struct SgdmScalars {
  float momentum, neg_lr;
};

// sr_states/reference/sgd.py:62-64:
//   u' = u*momentum + g                 (two roundings)
//   p' = p + (-lr)*u'                   -> fma(u', -lr, p)
SR_HD void sgdm_update(float p, float g, float u, const SgdmScalars& s, float& p_out,
                       float& u_out) {
  const float u_scaled = u * s.momentum;
  u_out = u_scaled + g;
  p_out = fmaf(u_out, s.neg_lr, p);
}

}  // namespace sr
