// Exhaustive device check of the BF16 stochastic-rounding encoder: the
// product's device path sr::bf16_sr (gfx950's v_cvt_sr_bf16_f32) against the
// portable formula sr::bf16_sr_bits, compared bit for bit, NaN payloads
// included.
//   sweep 1: every FP32 input with five random values each: the two values
//            where its rounding decision flips, 0, 0xFFFF and a hashed value;
//   sweep 2: for twelve upper halves (zeros, subnormals, ordinary values, the
//            largest finite value, Inf and NaN patterns, both signs), every
//            pair of low input half and 16-bit random value.
// The nearest encoder's device path sr::bf16_rn (v_cvt_pk_bf16_f32) is
// compared with sr::bf16_rn_bits on every FP32 input (sr_check_bf16_rn).
// The group forms of the kernels' vector paths (sr::encode_group_with for
// BF16 SR and nearest: two elements per convert, the second written to the
// high half of the first's destination) are checked in every position of a
// group (sr_check_bf16_groups): every FP32 input at each of the four
// positions beside hashed companions, stochastic with its five random values
// and nearest once, and the twelve upper halves' (low half, random value)
// pairs at each position.
// Built by __graft_entry__.build() into tests/native/libbf16_sr_check.so and
// run by tests/test_gpu_bf16_sr_check.py.
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

// One launch covers 2^31 inputs starting at `base`.
__global__ void every_input(uint32_t base, unsigned long long* counters) {
  const uint32_t b = base + blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t lo = b & 0xFFFFu;
  const uint32_t randoms[5] = {(0x10000u - lo) & 0xFFFFu, (0xFFFFu - lo) & 0xFFFFu, 0u, 0xFFFFu,
                               sr::h32(b ^ 0x5bd1e995u)};
  unsigned long long mismatches = 0;
  for (uint32_t r : randoms) mismatches += sr::bf16_sr(b, r) != sr::bf16_sr_bits(b, r);
  add(counters, mismatches, 5);
}

// One launch covers 2^31 inputs starting at `base`.
__global__ void every_input_nearest(uint32_t base, unsigned long long* counters) {
  const uint32_t b = base + blockIdx.x * blockDim.x + threadIdx.x;
  add(counters, sr::bf16_rn(b) != sr::bf16_rn_bits(b), 1);
}

// One launch covers 2^15 random values x 2^16 low halves for upper half `hi`;
// each thread also takes the random value with bit 15 set.
__global__ void every_pair(uint32_t hi, unsigned long long* counters) {
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t b = (hi << 16) | (idx & 0xFFFFu);
  const uint32_t r = (idx >> 16) & 0x7FFFu;
  unsigned long long mismatches = 0;
  for (uint32_t random : {r, r | 0x8000u}) {
    mismatches += sr::bf16_sr(b, random) != sr::bf16_sr_bits(b, random);
  }
  add(counters, mismatches, 2);
}

// Elements of a group whose BF16 encoding differs from the integer forms'.
// kFromMemory selects the casts' form of the group encoder.
template <int ENC, bool kFromMemory = false>
__device__ unsigned long long group_mismatches(const uint32_t (&b)[sr::kGroup], const uint32_t (&r)[sr::kGroup]) {
  uint32_t words[sr::group_words(ENC)], got[sr::kGroup];
  sr::encode_group_with<ENC, kFromMemory>(b, r, words);
  sr::unpack_group<ENC>(words, got);
  unsigned long long mismatches = 0;
  for (int k = 0; k < sr::kGroup; ++k) {
    const uint32_t want = ENC == sr::ENC_BF16_SR ? sr::bf16_sr_bits(b[k], r[k]) : sr::bf16_rn_bits(b[k]);
    mismatches += got[k] != want;
  }
  return mismatches;
}

__device__ void randoms_of(uint32_t b, uint32_t (&r)[5]) {
  const uint32_t lo = b & 0xFFFFu;
  r[0] = (0x10000u - lo) & 0xFFFFu;
  r[1] = (0xFFFFu - lo) & 0xFFFFu;
  r[2] = 0u;
  r[3] = 0xFFFFu;
  r[4] = sr::h32(b ^ 0x5bd1e995u);
}

// Input x = base + thread at each position of a group beside hashed
// companions: stochastic with each of the five random values of every
// element, and nearest in both the optimizers' and the casts' form.
// 4 * 7 groups of 4 elements per thread.
__global__ void every_input_group(uint32_t base, unsigned long long* counters) {
  const uint32_t x = base + blockIdx.x * blockDim.x + threadIdx.x;
  unsigned long long mismatches = 0;
  for (int p = 0; p < sr::kGroup; ++p) {
    uint32_t b[sr::kGroup], rand[sr::kGroup][5];
    for (int k = 0; k < sr::kGroup; ++k) {
      b[k] = k == p ? x : sr::h32(x + 0x9E3779B9u * (k + 1));
      randoms_of(b[k], rand[k]);
    }
    for (int j = 0; j < 5; ++j) {
      const uint32_t r[sr::kGroup] = {rand[0][j], rand[1][j], rand[2][j], rand[3][j]};
      mismatches += group_mismatches<sr::ENC_BF16_SR>(b, r);
    }
    const uint32_t zero[sr::kGroup] = {};
    mismatches += group_mismatches<sr::ENC_BF16_RN>(b, zero);
    mismatches += group_mismatches<sr::ENC_BF16_RN, true>(b, zero);
  }
  add(counters, mismatches, 4ull * 7 * sr::kGroup);
}

// every_pair at each position of a group, the other elements hashed inputs
// with hashed random values.
__global__ void every_pair_group(uint32_t hi, unsigned long long* counters) {
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t x = (hi << 16) | (idx & 0xFFFFu);
  const uint32_t r = (idx >> 16) & 0x7FFFu;
  unsigned long long mismatches = 0;
  for (int p = 0; p < sr::kGroup; ++p) {
    for (uint32_t random : {r, r | 0x8000u}) {
      uint32_t b[sr::kGroup], rs[sr::kGroup];
      for (int k = 0; k < sr::kGroup; ++k) {
        b[k] = k == p ? x : sr::h32(x ^ (idx * (k + 7)));
        rs[k] = k == p ? random : sr::h32(idx + k);
      }
      mismatches += group_mismatches<sr::ENC_BF16_SR>(b, rs);
    }
  }
  add(counters, mismatches, 4ull * 2 * sr::kGroup);
}

}  // namespace

// The group forms: counters_host[0] = mismatches, [1] = comparisons.
// Returns 0 or a hipError_t.
extern "C" int sr_check_bf16_groups(unsigned long long* counters_host) {
  unsigned long long* counters = nullptr;
  hipError_t err = hipMalloc(&counters, 2 * sizeof(unsigned long long));
  if (err == hipSuccess) err = hipMemset(counters, 0, 2 * sizeof(unsigned long long));
  const dim3 grid(1u << 23), block(256);  // 2^31 threads per launch
  for (uint32_t half = 0; err == hipSuccess && half < 2; ++half) {
    hipLaunchKernelGGL(every_input_group, grid, block, 0, 0, half << 31, counters);
    err = hipGetLastError();
  }
  const uint32_t highs[] = {0x0000u, 0x0001u, 0x007Fu, 0x0080u, 0x3F80u, 0x4B7Fu,
                            0x7F7Fu, 0x7F80u, 0x7FC0u, 0x8000u, 0xBF80u, 0xFF7Fu};
  for (uint32_t hi : highs) {
    if (err != hipSuccess) break;
    hipLaunchKernelGGL(every_pair_group, grid, block, 0, 0, hi, counters);
    err = hipGetLastError();
  }
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err == hipSuccess) {
    err = hipMemcpy(counters_host, counters, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  }
  if (counters) (void)hipFree(counters);
  return static_cast<int>(err);
}

// counters_host[0] = mismatches, [1] = comparisons.  Returns 0 or a hipError_t.
extern "C" int sr_check_bf16_sr(unsigned long long* counters_host) {
  unsigned long long* counters = nullptr;
  hipError_t err = hipMalloc(&counters, 2 * sizeof(unsigned long long));
  if (err == hipSuccess) err = hipMemset(counters, 0, 2 * sizeof(unsigned long long));
  const dim3 grid(1u << 23), block(256);  // 2^31 threads per launch
  for (uint32_t half = 0; err == hipSuccess && half < 2; ++half) {
    hipLaunchKernelGGL(every_input, grid, block, 0, 0, half << 31, counters);
    err = hipGetLastError();
  }
  const uint32_t highs[] = {0x0000u, 0x0001u, 0x007Fu, 0x0080u, 0x3F80u, 0x4B7Fu,
                            0x7F7Fu, 0x7F80u, 0x7FC0u, 0x8000u, 0xBF80u, 0xFF7Fu};
  for (uint32_t hi : highs) {
    if (err != hipSuccess) break;
    hipLaunchKernelGGL(every_pair, grid, block, 0, 0, hi, counters);
    err = hipGetLastError();
  }
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err == hipSuccess) {
    err = hipMemcpy(counters_host, counters, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  }
  if (counters) (void)hipFree(counters);
  return static_cast<int>(err);
}

// Every FP32 input through the nearest encoder: counters_host[0] =
// mismatches, [1] = comparisons (2^32).  Returns 0 or a hipError_t.
extern "C" int sr_check_bf16_rn(unsigned long long* counters_host) {
  unsigned long long* counters = nullptr;
  hipError_t err = hipMalloc(&counters, 2 * sizeof(unsigned long long));
  if (err == hipSuccess) err = hipMemset(counters, 0, 2 * sizeof(unsigned long long));
  for (uint32_t half = 0; err == hipSuccess && half < 2; ++half) {
    hipLaunchKernelGGL(every_input_nearest, dim3(1u << 23), dim3(256), 0, 0, half << 31, counters);
    err = hipGetLastError();
  }
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err == hipSuccess) {
    err = hipMemcpy(counters_host, counters, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
  }
  if (counters) (void)hipFree(counters);
  return static_cast<int>(err);
}
