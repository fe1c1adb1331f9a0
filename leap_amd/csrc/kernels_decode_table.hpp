// The decode kernel's instances for one head_dim and instance kind (PART),
// included by the kernels_decode_*.hip translation units only.
#pragma once

#include "kernels.hpp"

namespace leap_kernels {

template <int HD, bool PART>
KernelFn pick_decode(int g, bool valu, bool kvs, int waves)
{
    if constexpr (PART) {
        if (waves == kWavesShort) {
            // with kvs: 8 (4) q heads per KV head as two launch groups of 4 (2)
            if (kvs) {
                if (valu) return nullptr;
                if (g == 4) return leap::decode_attention_kernel<HD, 4, kWavesShort, true, true, true>;
                if (g == 2) return leap::decode_attention_kernel<HD, 2, kWavesShort, true, true, true>;
                return nullptr;
            }
            if (valu || !short_waves_shape(HD, g)) return nullptr;
#define LEAP_CASE(G) \
    if (g == G) return leap::decode_attention_kernel<HD, G, kWavesShort, true, true>;
            LEAP_CASE(1) LEAP_CASE(2) LEAP_CASE(3) LEAP_CASE(4)
#undef LEAP_CASE
            if constexpr (HD == 64)
                if (g == 8) return leap::decode_attention_kernel<64, 8, kWavesShort, true, true>;
            return nullptr;
        }
    }
    if (waves != kWaves) return nullptr;
#define LEAP_CASE(G)                                                                                       \
    if (g == G && !kvs)                                                                                    \
        return valu ? leap::decode_attention_kernel<HD, G, kWaves, false, PART>                            \
                    : leap::decode_attention_kernel<HD, G, kWaves, true, PART>;
    LEAP_CASE(1) LEAP_CASE(2) LEAP_CASE(3) LEAP_CASE(4) LEAP_CASE(8)
#undef LEAP_CASE
    // two launch groups per cache head: 4 and 8 q heads per KV head as two
    // groups of 2 and 4 (MFMA products only), 16 as two groups of 8
    if (g == 2 && kvs && !valu) return leap::decode_attention_kernel<HD, 2, kWaves, true, PART, true>;
    if (g == 4 && kvs && !valu) return leap::decode_attention_kernel<HD, 4, kWaves, true, PART, true>;
    if (g == 8 && kvs)
        return valu ? leap::decode_attention_kernel<HD, 8, kWaves, false, PART, true>
                    : leap::decode_attention_kernel<HD, 8, kWaves, true, PART, true>;
    return nullptr;
}

}  // namespace leap_kernels
