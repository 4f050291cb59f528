// Exhaustive device check of the minifloat encoders and decoders: the
// device paths sr::minifloat_bits_fast (bit arithmetic finished by a
// hardware convert) and sr::minifloat_decode (one hardware convert) against
// the integer forms sr::minifloat_bits and sr::minifloat_value, for FP16,
// E4M3 and E5M2.
//   decode:     every encoding; equal bits, or NaN for NaN;
//   nearest:    every FP32 input;
//   stochastic: every FP32 input with six random values: the two values
//               where its rounding decision flips (threshold - 1 and
//               threshold, in the upper 24 bits, with low bytes 0xFF and
//               0x00), 0, 0xFFFFFFFF and a hashed value.  Both forms round
//               up exactly when (random >> 8) is below a threshold of the
//               input, so agreement at the flip and the extremes is
//               agreement for every random value.
// The group forms the kernels' vector paths use (sr::encode_group_with,
// sr::decode_group: four elements per storage word set, two per paired
// convert) are checked the same way in every position of a group
// (sr_check_minifloat_groups): each FP32 input at each of the four
// positions, beside finite companions (the paired-convert path) and beside a
// NaN companion (the path that re-encodes the group element by element),
// nearest once and stochastic at its six random values, every element of the
// group compared with the integer form; and every encoding at every position
// through the group decoder.
// Built by __graft_entry__.build() into tests/native/libminifloat_check.so and
// run by tests/test_gpu_minifloat_check.py.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../stochastic-rounding-pytorch_amd/csrc/sr_math.h"

namespace {

__device__ unsigned long long wave_sum(unsigned long long x) {
  for (int offset = 32; offset > 0; offset >>= 1) x += __shfl_xor(x, offset, 64);
  return x;
}

__device__ void add(unsigned long long* counters, unsigned long long mismatches,
                    unsigned long long checks) {
  const unsigned long long m = wave_sum(mismatches), c = wave_sum(checks);
  if ((threadIdx.x & 63) == 0) {
    if (m) atomicAdd(&counters[0], m);
    atomicAdd(&counters[1], c);
  }
}

// The 24-bit threshold of input b: the integer form rounds up iff
// (hash >> 8) < threshold (its s <= 24 and s > 24 branches).
template <class F>
__device__ uint32_t threshold(uint32_t b) {
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

// One launch covers 2^31 inputs starting at `base`.
template <class F>
__global__ void every_input(uint32_t base, unsigned long long* counters) {
  const uint32_t b = base + blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long mismatches =
      sr::minifloat_bits_fast<F, false>(b, 0u) != sr::minifloat_bits<F, false>(b, 0u);
  const uint32_t th = threshold<F>(b);
  const uint32_t below = th ? ((th - 1u) << 8) | 0xFFu : 0u;
  const uint32_t randoms[6] = {below, th << 8, th << 8 | 0xFFu, 0u, 0xFFFFFFFFu, sr::h32(b ^ 0x5bd1e995u)};
  for (uint32_t r : randoms) {
    mismatches += sr::minifloat_bits_fast<F, true>(b, r) != sr::minifloat_bits<F, true>(b, r);
  }
  add(counters, mismatches, 7);
}

// Every encoding of F: the hardware decode equals the integer one, or both
// are NaN.
template <class F>
__global__ void every_code(unsigned long long* counters) {
  const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = v < (1u << F::kWidth);
  unsigned long long mismatch = 0;
  if (valid) {
    const float want = sr::minifloat_value<F>(v), got = sr::minifloat_decode<F>(v);
    mismatch = want != want ? !(got != got) : sr::f32_bits(got) != sr::f32_bits(want);
  }
  add(counters, mismatch, valid ? 1 : 0);
}

// The six random values of the stochastic check for input b (as in
// every_input).
template <class F>
__device__ void randoms_of(uint32_t b, uint32_t (&r)[6]) {
  const uint32_t th = threshold<F>(b);
  r[0] = th ? ((th - 1u) << 8) | 0xFFu : 0u;
  r[1] = th << 8;
  r[2] = th << 8 | 0xFFu;
  r[3] = 0u;
  r[4] = 0xFFFFFFFFu;
  r[5] = sr::h32(b ^ 0x5bd1e995u);
}

template <class F> struct Encodings;
template <> struct Encodings<sr::F16> { static constexpr int kRn = sr::ENC_F16_RN, kSr = sr::ENC_F16_SR; };
template <> struct Encodings<sr::E4M3> { static constexpr int kRn = sr::ENC_E4M3_RN, kSr = sr::ENC_E4M3_SR; };
template <> struct Encodings<sr::E5M2> { static constexpr int kRn = sr::ENC_E5M2_RN, kSr = sr::ENC_E5M2_SR; };

// Elements of the group whose encoding differs from the integer form's.
template <class F, bool STOCH>
__device__ unsigned long long group_mismatches(const uint32_t (&b)[sr::kGroup], const uint32_t (&r)[sr::kGroup]) {
  constexpr int ENC = STOCH ? Encodings<F>::kSr : Encodings<F>::kRn;
  uint32_t words[sr::group_words(ENC)], got[sr::kGroup];
  sr::encode_group_with<ENC>(b, r, words);
  sr::unpack_group<ENC>(words, got);
  unsigned long long mismatches = 0;
  for (int k = 0; k < sr::kGroup; ++k) mismatches += got[k] != sr::minifloat_bits<F, STOCH>(b[k], r[k]);
  return mismatches;
}

// Input x = base + thread at each position of a group: beside three finite
// companions (bit 30 cleared: exponent below 255), and beside one NaN
// companion.  Per position: nearest, and stochastic with each of the six
// random values of every element; then nearest and the first random value
// with the NaN companion.  4 * (7 + 2) groups of 4 elements per thread.
template <class F>
__global__ void every_input_group(uint32_t base, unsigned long long* counters) {
  const uint32_t x = base + blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long mismatches = 0;
  for (int p = 0; p < sr::kGroup; ++p) {
    uint32_t b[sr::kGroup];
    for (int k = 0; k < sr::kGroup; ++k) b[k] = k == p ? x : (sr::h32(x + 0x9E3779B9u * (k + 1)) & 0xBFFFFFFFu);
    uint32_t zero[sr::kGroup] = {};
    mismatches += group_mismatches<F, false>(b, zero);
    uint32_t rand[sr::kGroup][6];
    for (int k = 0; k < sr::kGroup; ++k) randoms_of<F>(b[k], rand[k]);
    for (int j = 0; j < 6; ++j) {
      const uint32_t r[sr::kGroup] = {rand[0][j], rand[1][j], rand[2][j], rand[3][j]};
      mismatches += group_mismatches<F, true>(b, r);
    }
    b[(p + 1) % sr::kGroup] = 0x7FC00000u | (x & 0x803FFFFFu);  // a NaN of either sign
    mismatches += group_mismatches<F, false>(b, zero);
    const uint32_t r[sr::kGroup] = {rand[0][0], rand[1][0], rand[2][0], rand[3][0]};
    mismatches += group_mismatches<F, true>(b, r);
  }
  add(counters, mismatches, 4ull * 9 * sr::kGroup);
}

// Every encoding v at every position of a group (companions v + 37 k,
// wrapped) through the group decoder: equal bits, or NaN for NaN.
template <class F>
__global__ void every_code_group(unsigned long long* counters) {
  constexpr int ENC = Encodings<F>::kRn;
  constexpr uint32_t kMask = (1u << F::kWidth) - 1u;
  const uint32_t v = blockIdx.x * blockDim.x + threadIdx.x;
  const bool valid = v < (1u << F::kWidth);
  unsigned long long mismatches = 0;
  if (valid) {
    for (int p = 0; p < sr::kGroup; ++p) {
      uint32_t codes[sr::kGroup], words[sr::group_words(ENC)];
      for (int k = 0; k < sr::kGroup; ++k) codes[k] = (v + 37u * ((k - p + sr::kGroup) % sr::kGroup)) & kMask;
      sr::pack_group<ENC>(codes, words);
      float got[sr::kGroup];
      sr::decode_group<ENC>(words, got);
      for (int k = 0; k < sr::kGroup; ++k) {
        const float want = sr::minifloat_value<F>(codes[k]);
        mismatches += want != want ? !(got[k] != got[k]) : sr::f32_bits(got[k]) != sr::f32_bits(want);
      }
    }
  }
  add(counters, mismatches, valid ? 4ull * sr::kGroup : 0ull);
}

template <class F>
hipError_t sweep_groups(unsigned long long* counters) {
  hipLaunchKernelGGL(every_code_group<F>, dim3(256), dim3(256), 0, 0, counters);
  const dim3 grid(1u << 23), block(256);  // 2^31 threads per launch
  hipError_t err = hipGetLastError();
  for (uint32_t half = 0; err == hipSuccess && half < 2; ++half) {
    hipLaunchKernelGGL(every_input_group<F>, grid, block, 0, 0, half << 31, counters);
    err = hipGetLastError();
  }
  return err;
}

template <class F>
hipError_t sweep(unsigned long long* counters) {
  hipLaunchKernelGGL(every_code<F>, dim3(256), dim3(256), 0, 0, counters);
  const dim3 grid(1u << 23), block(256);  // 2^31 threads per launch
  hipError_t err = hipGetLastError();
  for (uint32_t half = 0; err == hipSuccess && half < 2; ++half) {
    hipLaunchKernelGGL(every_input<F>, grid, block, 0, 0, half << 31, counters);
    err = hipGetLastError();
  }
  return err;
}

}  // namespace

// format: 0 FP16, 1 E4M3, 2 E5M2; groups: 0 the single-element forms, 1 the
// group forms.  counters_host[0] = mismatches, [1] = comparisons.  Returns
// 0, a hipError_t, or -1 for an unknown format.
static int check(int format, int groups, unsigned long long* counters_host) {
  if (format < 0 || format > 2) return -1;
  unsigned long long* counters = nullptr;
  hipError_t err = hipMalloc(&counters, 2 * sizeof(unsigned long long));
  if (err == hipSuccess) err = hipMemset(counters, 0, 2 * sizeof(unsigned long long));
  if (err == hipSuccess && groups) {
    err = format == 0 ? sweep_groups<sr::F16>(counters)
          : format == 1 ? sweep_groups<sr::E4M3>(counters) : sweep_groups<sr::E5M2>(counters);
  } else if (err == hipSuccess) {
    err = format == 0 ? sweep<sr::F16>(counters) : format == 1 ? sweep<sr::E4M3>(counters) : sweep<sr::E5M2>(counters);
  }
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err == hipSuccess) {
    err = hipMemcpy(counters_host, counters, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  }
  if (counters) (void)hipFree(counters);
  return static_cast<int>(err);
}

extern "C" int sr_check_minifloat(int format, unsigned long long* counters_host) {
  return check(format, 0, counters_host);
}

extern "C" int sr_check_minifloat_groups(int format, unsigned long long* counters_host) {
  return check(format, 1, counters_host);
}
