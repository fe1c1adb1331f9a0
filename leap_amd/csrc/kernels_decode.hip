// Decode-attention kernel table (see kernels.hpp): the floor kernels and the
// cross-XCD merge here, the decode kernel's instances by head_dim and
// instance kind in kernels_decode_*.hip (compiled in parallel).
#include "kernels.hpp"

namespace leap_kernels {

KernelFn pick_kernel(int hd, int g, int kind, bool valu, bool part, int kvs, int waves)
{
    if (kind == kDecode) {
        if (hd == 64)
            return part ? pick_decode<64, true>(g, valu, kvs, waves) : pick_decode<64, false>(g, valu, kvs, waves);
        if (hd == 128)
            return part ? pick_decode<128, true>(g, valu, kvs, waves) : pick_decode<128, false>(g, valu, kvs, waves);
        return nullptr;
    }
    if ((g != 1 && g != 2 && g != 3 && g != 4 && g != 8) || kvs < 0 || kvs > 2 || (kvs == 1 && g != 8 && g != 4 && g != 2) ||
        (kvs == 2 && g != 2))
        return nullptr;
    if (waves == kWavesShort) {
        // the floors of the 2-wave launches: the same grid and block size
        if (!part || !short_waves_shape(hd, g)) return nullptr;
        if (kvs) {  // two launch groups of 2 or 4 q heads per cache head, or four of 2
#define LEAP_KVS_CASE(HD, G, K)                                                              \
    if (hd == HD && g == G && kvs == K)                                                      \
        return kind == kFloorLaunch   ? leap::floor_launch_kernel<HD, G, kWavesShort>         \
             : kind == kFloorStream ? leap::floor_stream_kernel<HD, G, kWavesShort, K, true> \
                                      : nullptr;
            LEAP_KVS_CASE(64, 2, 1) LEAP_KVS_CASE(64, 4, 1) LEAP_KVS_CASE(128, 2, 1) LEAP_KVS_CASE(128, 4, 1)
            LEAP_KVS_CASE(64, 2, 2) LEAP_KVS_CASE(128, 2, 2)
#undef LEAP_KVS_CASE
            return nullptr;
        }
#define LEAP_CASE(HD, G)                                                                  \
    if (hd == HD && g == G)                                                               \
        return kind == kFloorLaunch   ? leap::floor_launch_kernel<HD, G, kWavesShort>      \
             : kind == kFloorStream ? leap::floor_stream_kernel<HD, G, kWavesShort, false, true> \
                                      : nullptr;
        LEAP_CASE(64, 1) LEAP_CASE(64, 2) LEAP_CASE(64, 3) LEAP_CASE(64, 4) LEAP_CASE(64, 8)
        LEAP_CASE(128, 1) LEAP_CASE(128, 2) LEAP_CASE(128, 3) LEAP_CASE(128, 4)
#undef LEAP_CASE
        return nullptr;
    }
    if (waves != kWaves) return nullptr;
#define LEAP_STREAM(HD, G, K) \
    (part ? leap::floor_stream_kernel<HD, G, kWaves, K, true> : leap::floor_stream_kernel<HD, G, kWaves, K, false>)
#define LEAP_CASE(HD, G)                                                                             \
    if (hd == HD && g == G)                                                                          \
        return kind == kFloorLaunch   ? leap::floor_launch_kernel<HD, G, kWaves>                     \
             : kind == kFloorStream ? (kvs == 2 ? LEAP_STREAM(HD, G, 2) : kvs ? LEAP_STREAM(HD, G, 1) : LEAP_STREAM(HD, G, 0)) \
                                      : nullptr;
    LEAP_CASE(64, 1) LEAP_CASE(64, 2) LEAP_CASE(64, 3) LEAP_CASE(64, 4) LEAP_CASE(64, 8)
    LEAP_CASE(128, 1) LEAP_CASE(128, 2) LEAP_CASE(128, 3) LEAP_CASE(128, 4) LEAP_CASE(128, 8)
#undef LEAP_CASE
#undef LEAP_STREAM
    return nullptr;
}

MergeFn pick_merge(int hd, int g)
{
#define LEAP_CASE(HD, G) \
    if (hd == HD && g == G) return leap::part_merge_kernel<HD, G>;
    LEAP_CASE(64, 1) LEAP_CASE(64, 2) LEAP_CASE(64, 3) LEAP_CASE(64, 4) LEAP_CASE(64, 8)
    LEAP_CASE(128, 1) LEAP_CASE(128, 2) LEAP_CASE(128, 3) LEAP_CASE(128, 4) LEAP_CASE(128, 8)
#undef LEAP_CASE
    return nullptr;
}

}  // namespace leap_kernels
