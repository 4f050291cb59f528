// Exhaustive device check of the AdamW update's square root and divisions:
// sr::sqrt_rn, sr::div_by_constant (by sqrt(1 - beta2^t)) and sr::div_short
// (by the denominator) against the IEEE correctly rounded sqrtf and
// division (this file is built, like the library, with
// -fhip-fp32-correctly-rounded-divide-sqrt).
//   sqrt_rn:         every FP32 input; equal bits, or NaN for NaN.
//   div_by_constant: every pair of significands, x in [1, 2) and c in
//                    [1/2, 1), with r = 1 / c correctly rounded; in the
//                    function's domain (c in [2^-27, 1], x zero, infinite,
//                    NaN or in [2^-75, 2^64]) scaling x or c by a power of
//                    two scales every intermediate exactly, so these pairs
//                    stand for all.  A second kernel runs x = 0, infinity
//                    and NaN, and both ends of the exponent ranges.
//   div_short:       every pair of significands (a and b in [1, 2)), where
//                    the result must be accepted and equal a / b; in its
//                    domain (b in [2^-60, 2^101), |q0| in [2^-40, 2^100))
//                    scaling a or b by a power of two scales every
//                    intermediate exactly, so these pairs stand for all;
//                    rcp_rn on every float of [2^-126, 2^126); and hashed
//                    cases over the whole domain, special dividends and
//                    divisors, and first quotients at both ends of the range.
// Built by tests/native/build_checks.py into tests/native/libdivsqrt_check.so
// and run by tests/test_gpu_divsqrt_check.py.
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

__device__ bool same(float got, float want) {
  return want != want ? got != got : __builtin_bit_cast(uint32_t, got) == __builtin_bit_cast(uint32_t, want);
}

// One launch covers 2^31 inputs starting at `base`.
__global__ void every_sqrt(uint32_t base, unsigned long long* counters) {
  const uint32_t b = base + blockIdx.x * blockDim.x + threadIdx.x;
  const float v = __builtin_bit_cast(float, b);
  add(counters, !same(sr::sqrt_rn(v), sqrtf(v)), 1);
}

constexpr int kXShift = 9;  // 2^9 threads per divisor, 2^14 dividends each

// Thread t: divisor significand c_first + (t >> 9), dividends
// [(t & 511) << 14, ((t & 511) + 1) << 14).
__global__ void every_pair(uint32_t c_first, unsigned long long* counters) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const float c = __builtin_bit_cast(float, 0x3F000000u | (c_first + (t >> kXShift)));
  const float r = 1.0f / c;
  const uint32_t x_first = (t & ((1u << kXShift) - 1u)) << (23 - kXShift);
  unsigned long long mismatches = 0;
  for (uint32_t k = 0; k < (1u << (23 - kXShift)); ++k) {
    const float x = __builtin_bit_cast(float, 0x3F800000u | (x_first + k));
    mismatches += !same(sr::div_by_constant(x, c, r), x / c);
  }
  add(counters, mismatches, 1u << (23 - kXShift));
}

// Thread t: divisor significand (t >> 9) * 32771 mod 2^23 at exponents -27
// and -1, against x = +-0, +inf, NaN and, over 2^14 significands each, x in
// [2^-75, 2^-74) and [2^63, 2^64).
__global__ void edges(unsigned long long* counters) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t c_sig = ((t >> kXShift) * 32771u) & 0x7FFFFFu;
  const uint32_t x_first = (t & ((1u << kXShift) - 1u)) << (23 - kXShift);
  unsigned long long mismatches = 0, checks = 0;
  for (uint32_t c_exp : {127u - 27u, 126u}) {
    const float c = __builtin_bit_cast(float, (c_exp << 23) | c_sig);
    const float r = 1.0f / c;
    for (float x : {0.0f, -0.0f, __builtin_inff(), __builtin_nanf("")}) {
      mismatches += !same(sr::div_by_constant(x, c, r), x / c);
      ++checks;
    }
    for (uint32_t x_exp : {127u - 75u, 127u + 63u}) {
      for (uint32_t k = 0; k < (1u << (23 - kXShift)); ++k) {
        const float x = __builtin_bit_cast(float, (x_exp << 23) | (x_first + k));
        mismatches += !same(sr::div_by_constant(x, c, r), x / c);
        ++checks;
      }
    }
  }
  add(counters, mismatches, checks);
}

// div_short (the AdamW update's division by its denominator) on every pair
// of significands: thread t takes divisor significand b_first + (t >> 9) and
// 2^14 dividends, as every_pair.  In [1, 2) x [1, 2) every first quotient is
// in range, so `ok` must hold; counters[2] counts where it does not.
__global__ void every_short_pair(uint32_t b_first, unsigned long long* counters) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  const float b = __builtin_bit_cast(float, 0x3F800000u | (b_first + (t >> kXShift)));
  const uint32_t a_first = (t & ((1u << kXShift) - 1u)) << (23 - kXShift);
  unsigned long long mismatches = 0, refused = 0;
  for (uint32_t k = 0; k < (1u << (23 - kXShift)); ++k) {
    const float a = __builtin_bit_cast(float, 0x3F800000u | (a_first + k));
    bool ok;
    const float q = sr::div_short(a, b, ok);
    mismatches += ok && !same(q, a / b);
    refused += !ok;
  }
  add(counters, mismatches + refused, 1u << (23 - kXShift));
}

// rcp_rn on every float in [2^-126, 2^126) (2^31 threads from `base`).
__global__ void every_reciprocal(uint32_t base, unsigned long long* counters) {
  const uint32_t bits = base + blockIdx.x * blockDim.x + threadIdx.x;
  const bool in_range = bits >= 0x00800000u && bits < 0x7E800000u;
  const float b = __builtin_bit_cast(float, bits);
  add(counters, in_range && !same(sr::rcp_rn(b), 1.0f / b), in_range);
}

// div_short over its whole domain, 2^9 cases per thread from hashed bits:
// divisors in [2^-60, 2^101), dividends of every exponent, where `ok` holds
// the quotient must equal a / b; dividends 0, +-Inf and NaN, and infinite
// and NaN divisors, must come back with ok false; and first quotients next
// to both ends of the range, 2^-40 and 2^100.  counters[0] counts wrong
// quotients with ok and special cases with ok; [1] the cases; [2] those
// with ok.
__global__ void short_domain(unsigned long long* counters, unsigned long long* accepted) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long bad = 0, cases = 0, oks = 0;
  for (uint32_t k = 0; k < 512; ++k) {
    const uint32_t h1 = sr::h32(t * 512u + k), h2 = sr::h32(h1 ^ 0x85EBCA6Bu), h3 = sr::h32(h2 + 0x68E31DA4u);
    const uint32_t b_exp = 127u - 60u + (h1 >> 24) % 161u;  // 2^-60 .. 2^100
    const float b = __builtin_bit_cast(float, (b_exp << 23) | (h2 & 0x7FFFFFu));
    // Dividends of every exponent, and dividends that put q0 at the ends.
    float a = __builtin_bit_cast(float, (h3 & 0x80000000u) | (((h1 >> 8) % 255u) << 23) | (h3 & 0x7FFFFFu));
    if ((k & 3u) == 1u) a = b * (0x1p-40f * (1.0f + (h3 & 0xFFu) * 0x1p-22f - 0x1p-16f));
    if ((k & 3u) == 2u) a = b * (0x1p100f * (1.0f + (h3 & 0xFFu) * 0x1p-22f - 0x1p-16f));
    bool ok;
    const float q = sr::div_short(a, b, ok);
    bad += ok && !same(q, a / b);
    oks += ok;
    ++cases;
    const float specials[4] = {0.0f, __builtin_inff(), -__builtin_inff(), __builtin_nanf("")};
    const float sa = (h1 & 1u) ? -specials[k & 3u] : specials[k & 3u];
    (void)sr::div_short(sa, b, ok);
    bad += ok;
    const float sb = (k & 4u) ? __builtin_inff() : __builtin_nanf("");
    (void)sr::div_short(a, sb, ok);
    bad += ok;
    cases += 2;
  }
  add(counters, bad, cases);
  const unsigned long long o = wave_sum(oks);
  if ((threadIdx.x & 63) == 0) atomicAdd(accepted, o);
}

hipError_t run(unsigned long long* counters_host, hipError_t (*launches)(unsigned long long*)) {
  unsigned long long* counters = nullptr;
  hipError_t err = hipMalloc(&counters, 2 * sizeof(unsigned long long));
  if (err == hipSuccess) err = hipMemset(counters, 0, 2 * sizeof(unsigned long long));
  if (err == hipSuccess) err = launches(counters);
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err == hipSuccess) {
    err = hipMemcpy(counters_host, counters, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  }
  if (counters) (void)hipFree(counters);
  return err;
}

uint32_t g_c_first, g_c_count;

}  // namespace

// counters_host[0] = mismatches, [1] = comparisons.  Each returns 0 or a
// hipError_t (-1 for arguments outside the ranges below).

// Every FP32 input (2^32 comparisons).
extern "C" int sr_check_sqrt(unsigned long long* counters_host) {
  return static_cast<int>(run(counters_host, [](unsigned long long* counters) {
    hipError_t err = hipSuccess;
    for (uint32_t half = 0; err == hipSuccess && half < 2; ++half) {
      hipLaunchKernelGGL(every_sqrt, dim3(1u << 23), dim3(256), 0, 0, half << 31, counters);
      err = hipGetLastError();
    }
    return err;
  }));
}

// Divisor significands [c_first, c_first + c_count) against every dividend
// significand (c_count * 2^23 comparisons); c_count at least 1 and
// c_first + c_count at most 2^23.
extern "C" int sr_check_div_by_constant(uint32_t c_first, uint32_t c_count, unsigned long long* counters_host) {
  if (c_count == 0 || c_first > (1u << 23) || c_count > (1u << 23) - c_first) return -1;
  g_c_first = c_first;
  g_c_count = c_count;
  return static_cast<int>(run(counters_host, [](unsigned long long* counters) {
    // 2^9 threads per divisor, 256 threads per workgroup.
    hipLaunchKernelGGL(every_pair, dim3(g_c_count << kXShift >> 8), dim3(256), 0, 0, g_c_first, counters);
    return hipGetLastError();
  }));
}

// div_short: divisor significands [b_first, b_first + b_count) against every
// dividend significand (b_count * 2^23 comparisons; mismatches include
// refusals); ranges as sr_check_div_by_constant.
extern "C" int sr_check_div_short(uint32_t b_first, uint32_t b_count, unsigned long long* counters_host) {
  if (b_count == 0 || b_first > (1u << 23) || b_count > (1u << 23) - b_first) return -1;
  g_c_first = b_first;
  g_c_count = b_count;
  return static_cast<int>(run(counters_host, [](unsigned long long* counters) {
    hipLaunchKernelGGL(every_short_pair, dim3(g_c_count << kXShift >> 8), dim3(256), 0, 0, g_c_first, counters);
    return hipGetLastError();
  }));
}

// rcp_rn on every float in [2^-126, 2^126) (0x7E000000 comparisons).
extern "C" int sr_check_rcp_rn(unsigned long long* counters_host) {
  return static_cast<int>(run(counters_host, [](unsigned long long* counters) {
    hipError_t err = hipSuccess;
    for (uint32_t half = 0; err == hipSuccess && half < 2; ++half) {
      hipLaunchKernelGGL(every_reciprocal, dim3(1u << 23), dim3(256), 0, 0, half << 31, counters);
      err = hipGetLastError();
    }
    return err;
  }));
}

// div_short over its domain: 2^16 threads x 512 cases x 3 (counters_host[0]
// bad, [1] cases), and counters_host[2] = the random cases accepted (ok).
extern "C" int sr_check_div_short_domain(unsigned long long* counters_host) {
  unsigned long long* counters = nullptr;
  hipError_t err = hipMalloc(&counters, 3 * sizeof(unsigned long long));
  if (err == hipSuccess) err = hipMemset(counters, 0, 3 * sizeof(unsigned long long));
  if (err == hipSuccess) {
    hipLaunchKernelGGL(short_domain, dim3(256), dim3(256), 0, 0, counters, counters + 2);
    err = hipGetLastError();
  }
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err == hipSuccess) err = hipMemcpy(counters_host, counters, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  if (counters) (void)hipFree(counters);
  return static_cast<int>(err);
}

// Zero, infinite and NaN dividends (once per thread) and both ends of the
// exponent ranges, for 2^14 divisor significands at two exponents
// (2^14 * 2 * (2^9 * 4 + 2 * 2^23) comparisons).
extern "C" int sr_check_div_edges(unsigned long long* counters_host) {
  return static_cast<int>(run(counters_host, [](unsigned long long* counters) {
    hipLaunchKernelGGL(edges, dim3((1u << 14) << kXShift >> 8), dim3(256), 0, 0, counters);
    return hipGetLastError();
  }));
}
