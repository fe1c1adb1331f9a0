// The decode kernel's instances for one head_dim and instance kind (PART),
// included by the kernels_decode_*.hip translation units only.
#pragma once

#include "kernels.hpp"

namespace leap_kernels {

template <int HD, bool PART>
KernelFn pick_decode(int g, bool valu, bool kvs)
{
#define LEAP_CASE(G)                                                                                       \
    if (g == G && !kvs)                                                                                    \
        return valu ? leap::decode_attention_kernel<HD, G, kWaves, false, PART>                            \
                    : leap::decode_attention_kernel<HD, G, kWaves, true, PART>;
    LEAP_CASE(1) LEAP_CASE(2) LEAP_CASE(3) LEAP_CASE(4) LEAP_CASE(8)
#undef LEAP_CASE
    if (g == 8 && kvs)
        return valu ? leap::decode_attention_kernel<HD, 8, kWaves, false, PART, true>
                    : leap::decode_attention_kernel<HD, 8, kWaves, true, PART, true>;
    return nullptr;
}

}  // namespace leap_kernels
