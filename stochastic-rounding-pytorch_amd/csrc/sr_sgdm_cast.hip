// Momentum-SGD, cast and neighbour kernel instantiations.
#include <utility>

#include "sr_kernels.h"

namespace sr {
namespace {

constexpr int pg_enc(int index) { return index ? ENC_BF16_RN : ENC_F32; }

template <int PI, int GI, int... UE>
void fill_sgdm(KernelTableSgdm& t, std::integer_sequence<int, UE...>) {
  ((t[PI][GI][UE] = reinterpret_cast<const void*>(&sgdm_kernel<pg_enc(PI), pg_enc(GI), UE>)), ...);
}

template <int... E>
void fill_cast(KernelTableCast& t, std::integer_sequence<int, E...>) {
  ((t[0][E] = reinterpret_cast<const void*>(&cast_kernel<E, false>)), ...);
  ((t[1][E] = reinterpret_cast<const void*>(&cast_kernel<E, true>)), ...);
}

}  // namespace

void register_sgdm(KernelTableSgdm& t) {
  using All = std::make_integer_sequence<int, ENC_COUNT>;
  fill_sgdm<0, 0>(t, All{});
  fill_sgdm<0, 1>(t, All{});
  fill_sgdm<1, 0>(t, All{});
  fill_sgdm<1, 1>(t, All{});
}

void register_cast(KernelTableCast& t) { fill_cast(t, std::make_integer_sequence<int, ENC_COUNT>{}); }

void register_neighbors(KernelTableNeighbors& t) {
  t[ENC_BF16_RN] = reinterpret_cast<const void*>(&neighbors_kernel<ENC_BF16_RN>);
  t[ENC_F16_RN] = reinterpret_cast<const void*>(&neighbors_kernel<ENC_F16_RN>);
  t[ENC_E4M3_RN] = reinterpret_cast<const void*>(&neighbors_kernel<ENC_E4M3_RN>);
  t[ENC_E5M2_RN] = reinterpret_cast<const void*>(&neighbors_kernel<ENC_E5M2_RN>);
}

}  // namespace sr
