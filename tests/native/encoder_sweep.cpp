// Sweep FP32 bit patterns through the product's encoders (sr_math.h, compiled
// for the host) and the C oracle (oracle/sr_oracle.c); count mismatches.
// NaN results compare as equal whatever their payload.  Usage:
//   encoder_sweep [stride]      stride 1 = all 2^32 inputs (minutes on 8 cores)
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <cmath>
#include <thread>
#include <vector>
#include <atomic>

#include "sr_math.h"

extern "C" uint32_t oc_encode(float x, int dtype, int rule, uint32_t counter);
extern "C" float oc_decode(uint32_t raw, int dtype);

namespace {

bool is_nan_enc(uint32_t e, int dtype) {
  switch (dtype) {
    case 1: return (e & 0x7FFF) > 0x7F80;
    case 2: return (e & 0x7FFF) > 0x7C00;
    case 3: return (e & 0x7F) == 0x7F;
    default: return (e & 0x7F) > 0x7C;
  }
}

template <int ENC>
uint32_t product(float x, uint32_t counter) { return sr::encode<ENC>(x, counter); }

using Fn = uint32_t (*)(float, uint32_t);
struct Case { Fn fn; int dtype, rule; const char* name; };

}  // namespace

int main(int argc, char** argv) {
  const uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
  const Case cases[] = {
      {product<sr::ENC_BF16_RN>, 1, 0, "bf16 nearest"}, {product<sr::ENC_BF16_SR>, 1, 1, "bf16 stochastic"},
      {product<sr::ENC_F16_RN>, 2, 0, "f16 nearest"},   {product<sr::ENC_F16_SR>, 2, 1, "f16 stochastic"},
      {product<sr::ENC_E4M3_RN>, 3, 0, "e4m3 nearest"}, {product<sr::ENC_E4M3_SR>, 3, 1, "e4m3 stochastic"},
      {product<sr::ENC_E5M2_RN>, 4, 0, "e5m2 nearest"}, {product<sr::ENC_E5M2_SR>, 4, 1, "e5m2 stochastic"},
  };
  const unsigned workers = std::max(1u, std::thread::hardware_concurrency());
  uint64_t total_bad = 0;
  for (const Case& c : cases) {
    std::atomic<uint64_t> bad{0};
    std::vector<std::thread> pool;
    for (unsigned w = 0; w < workers; ++w) {
      pool.emplace_back([&, w] {
        for (uint64_t b = uint64_t(w) * stride; b < (uint64_t(1) << 32); b += uint64_t(workers) * stride) {
          const uint32_t u = static_cast<uint32_t>(b);
          float x;
          std::memcpy(&x, &u, 4);
          const uint32_t counter = u * 2654435761u + 12345u;
          const uint32_t p = c.fn(x, counter), o = oc_encode(x, c.dtype, c.rule, counter);
          if (!(p == o || (is_nan_enc(p, c.dtype) && is_nan_enc(o, c.dtype)))) {
            if (bad.fetch_add(1) < 3) std::printf("%s: x=%08x product=%x oracle=%x\n", c.name, u, p, o);
          }
        }
      });
    }
    for (auto& t : pool) t.join();
    std::printf("%s: %llu mismatches\n", c.name, static_cast<unsigned long long>(bad.load()));
    total_bad += bad.load();
  }
  for (int dtype = 1; dtype <= 4; ++dtype) {
    const int n = dtype <= 2 ? 65536 : 256;
    int bad = 0;
    for (int v = 0; v < n; ++v) {
      const float a = dtype == 1 ? sr::decode<sr::ENC_BF16_RN>(v)
                    : dtype == 2 ? sr::decode<sr::ENC_F16_RN>(v)
                    : dtype == 3 ? sr::decode<sr::ENC_E4M3_RN>(v) : sr::decode<sr::ENC_E5M2_RN>(v);
      const float b = oc_decode(v, dtype);
      if (!((std::isnan(a) && std::isnan(b)) || std::memcmp(&a, &b, 4) == 0)) ++bad;
    }
    std::printf("decode dtype %d: %d mismatches\n", dtype, bad);
    total_bad += bad;
  }
  return total_bad != 0;
}
