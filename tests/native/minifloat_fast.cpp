// Host check of the bit arithmetic of sr::minifloat_bits_fast against the
// integer form sr::minifloat_bits, for FP16, E4M3 and E5M2.  On the host the
// final convert is the integer nearest form applied to the exactly
// representable rounded value, so this checks the rounding algebra apart
// from the hardware converts (which tests/native/minifloat_check.hip covers
// exhaustively on the device).  Every 257th FP32 input (16.7 M inputs, all
// exponents and both signs) is rounded to nearest once and stochastically
// at the random values where its decision flips and at the extremes.
#include <cstdint>
#include <cstdio>

#include "sr_math.h"

template <class F>
uint32_t threshold(uint32_t b) {  // the integer form rounds up iff (hash >> 8) < threshold
  uint32_t a = b & 0x7FFFFFFFu;
  if (F::kSat) a = a < F::kMaxBits ? a : F::kMaxBits;
  const int E = static_cast<int>(a >> 23);
  const uint32_t sig = E ? ((a & 0x007FFFFFu) | 0x00800000u) : a;
  const int e_raw = (E ? E : 1) - 127;
  const int e = (E - 127) > F::kEmin ? (E - 127) : F::kEmin;
  const int s = 23 - F::kM + (e - e_raw);
  if (s <= 24) return (sig & ((1u << s) - 1u)) << (24 - s);
  const int t = s - 24;
  return t < 24 ? sig >> t : 0u;
}

template <class F>
unsigned long long sweep(const char* name) {
  unsigned long long mismatches = 0, checks = 0;
  for (uint64_t x = 0; x < (1ull << 32); x += 257) {
    const uint32_t b = static_cast<uint32_t>(x);
    mismatches += sr::minifloat_bits_fast<F, false>(b, 0u) != sr::minifloat_bits<F, false>(b, 0u);
    const uint32_t th = threshold<F>(b);
    const uint32_t randoms[6] = {th ? ((th - 1u) << 8) | 0xFFu : 0u, th << 8, (th << 8) | 0xFFu, 0u,
                                 0xFFFFFFFFu, sr::h32(b ^ 0x5bd1e995u)};
    for (uint32_t r : randoms) mismatches += sr::minifloat_bits_fast<F, true>(b, r) != sr::minifloat_bits<F, true>(b, r);
    checks += 7;
  }
  std::printf("%s: %llu mismatches of %llu\n", name, mismatches, checks);
  return mismatches;
}

// sr::fp8_sr_grid_bits (the kernels' single-form FP8 stochastic rounding)
// gives the rounded value; its encoding, by the integer nearest form (the
// value is exactly representable), must equal the integer stochastic form's.
template <class F>
unsigned long long sweep_fp8(const char* name) {
  unsigned long long mismatches = 0, checks = 0;
  for (uint64_t x = 0; x < (1ull << 32); x += 257) {
    const uint32_t b = static_cast<uint32_t>(x);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) continue;  // NaN groups take the single-element form
    const uint32_t th = threshold<F>(b);
    const uint32_t randoms[6] = {th ? ((th - 1u) << 8) | 0xFFu : 0u, th << 8, (th << 8) | 0xFFu, 0u,
                                 0xFFFFFFFFu, sr::h32(b ^ 0x5bd1e995u)};
    for (uint32_t r : randoms) {
      mismatches += sr::minifloat_bits<F, false>(sr::fp8_sr_grid_bits<F>(b, r), 0u) != sr::minifloat_bits<F, true>(b, r);
    }
    checks += 6;
  }
  std::printf("%s grid: %llu mismatches of %llu\n", name, mismatches, checks);
  return mismatches;
}

int main() {
  const unsigned long long bad = sweep<sr::F16>("F16") + sweep<sr::E4M3>("E4M3") + sweep<sr::E5M2>("E5M2") +
                                 sweep_fp8<sr::E4M3>("E4M3") + sweep_fp8<sr::E5M2>("E5M2");
  return bad != 0;
}
