// The decode kernel's instances for one head_dim and instance kind (PART),
// included by the kernels_decode_*.hip translation units only.
#pragma once

#include "kernels.hpp"

namespace leap_kernels {

template <int HD, bool PART>
KernelFn pick_decode(int g, bool valu, int kvs, int waves)
{
    if constexpr (PART) {
        if (waves == kWavesShort) {
            // with kvs: 8 (4) q heads per KV head as two launch groups of 4
            // (2), or 8 as four groups of 2
            if (kvs) {
                if (valu) return nullptr;
                if (kvs == 1 && g == 4) return leap::decode_attention_kernel<HD, 4, kWavesShort, true, true, 1>;
                if (kvs == 1 && g == 2) return leap::decode_attention_kernel<HD, 2, kWavesShort, true, true, 1>;
                if (kvs == 2 && g == 2) return leap::decode_attention_kernel<HD, 2, kWavesShort, true, true, 2>;
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
    // several launch groups per cache head: 4 and 8 q heads per KV head as
    // two groups of 2 and 4, 8 as four groups of 2 (MFMA products only), 16
    // as two groups of 8
    if (kvs == 1 && g == 2 && !valu) return leap::decode_attention_kernel<HD, 2, kWaves, true, PART, 1>;
    if (kvs == 1 && g == 4 && !valu) return leap::decode_attention_kernel<HD, 4, kWaves, true, PART, 1>;
    if (kvs == 2 && g == 2 && !valu) return leap::decode_attention_kernel<HD, 2, kWaves, true, PART, 2>;
    if (kvs == 1 && g == 8)
        return valu ? leap::decode_attention_kernel<HD, 8, kWaves, false, PART, 1>
                    : leap::decode_attention_kernel<HD, 8, kWaves, true, PART, 1>;
    return nullptr;
}

}  // namespace leap_kernels
