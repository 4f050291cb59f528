// AdamW kernel instantiations for one first-moment encoding.  The build
// compiles this file once per encoding with -DSR_M_ENC=<0..8> so the 324
// (param, grad, m, v) combinations compile in parallel.
#include <utility>

#include "sr_kernels.h"

#ifndef SR_M_ENC
#error "compile with -DSR_M_ENC=<encoding index>"
#endif

#define SR_CAT2(a, b) a##b
#define SR_CAT(a, b) SR_CAT2(a, b)

namespace sr {
namespace {

constexpr int pg_enc(int index) { return index ? ENC_BF16_RN : ENC_F32; }

template <int PI, int GI, int... VE>
void fill(KernelTableAdamW& t, std::integer_sequence<int, VE...>) {
  ((t[PI][GI][SR_M_ENC][VE] =
        reinterpret_cast<const void*>(&adamw_kernel<pg_enc(PI), pg_enc(GI), SR_M_ENC, VE>)),
   ...);
}

}  // namespace

void SR_CAT(register_adamw_m, SR_M_ENC)(KernelTableAdamW& t) {
  using All = std::make_integer_sequence<int, ENC_COUNT>;
  fill<0, 0>(t, All{});
  fill<0, 1>(t, All{});
  fill<1, 0>(t, All{});
  fill<1, 1>(t, All{});
}

}  // namespace sr
