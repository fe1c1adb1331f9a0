// The library's kernel tables, each instantiated in a translation unit of its
// own so that the build compiles them in parallel:
//   - kernels_decode.hip: the measurement kernels with the decode kernel's
//     grids and the cross-XCD merge; kernels_decode_{64,64p,128,128p}.hip:
//     the decode-attention kernels by head_dim and instance kind;
//   - kernels_gemv.hip: the fp32 projection GEMVs by model width;
//   - kernels_q8.hip: the int8 W8A8 projection GEMVs by width, group size,
//     rows per team and input kind.
// leap_hip_attention.hip holds the host side and picks kernels through these
// functions only.
#pragma once

#include "decode_attention.hpp"
#include "gemv.hpp"
#include "gemv_q8.hpp"

namespace leap_kernels {

// Waves per workgroup of the decode kernel.
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * leap::kWave;
// Waves per workgroup for chunks of at most half a kWaves pass (32 rows):
// the short contexts' half-pass chunks and contexts of up to 32 positions,
// which a 4-wave workgroup covers with two waves of masked rows.  Compiled
// for the matrix-core products, with the PART instance kind, at head_dim 64
// and at head_dim 128 with up to 4 q heads per KV head: the merge gives
// each (head, float4 column) of the group at least one thread, and 128
// threads cover 8 heads of 64 or 4 heads of 128.
constexpr int kWavesShort = 2;

// What a launch runs: the decode kernel, or one of the floor kernels with its
// grid (measurement only).
enum LaunchKind { kDecode = 0, kFloorLaunch = 1, kFloorStream = 2 };

// (the preloaded words, leap::Preload, then the argument block)
using KernelFn = void (*)(const float *, const float *, float *, float *, const float4 *, uint32_t, uint32_t, uint32_t,
                          uint32_t, leap::StepArgs);
using MergeFn = void (*)(leap::StepArgs);

// The decode kernel (or a floor kernel) for head_dim hd and g q heads per
// launch group; nullptr for a shape without one.
//   part: the launch's chunks are near-equal, not whole passes, or 2-8 passes
//         long (leap::part_launch);
//   kvs:  the launch's kv_split k: 2^k launch groups of g heads per cache
//         head (0: one); k = 1 with g = 8 for 16 q heads per KV head, g = 4
//         and 2 (MFMA products) for 8 and 4; k = 2 with g = 2 for 8;
//   valu: the score and weighted-V products as VALU FMAs (the A/B knob);
//   waves: kWaves, or kWavesShort (part only, not valu, with kvs only at
//          g = 2 and 4; short_waves_shape).
KernelFn pick_kernel(int hd, int g, int kind, bool valu, bool part, int kvs, int waves = kWaves);
// Whether a shape has kWavesShort instances.
constexpr bool short_waves_shape(int hd, int g)
{
    return (hd == 64 && (g == 1 || g == 2 || g == 3 || g == 4 || g == 8)) ||
           (hd == 128 && (g == 1 || g == 2 || g == 3 || g == 4));
}
// The decode kernel alone, by head_dim HD and instance kind PART (one
// translation unit per pair).
template <int HD, bool PART>
KernelFn pick_decode(int g, bool valu, int kvs, int waves);
extern template KernelFn pick_decode<64, false>(int, bool, int, int);
extern template KernelFn pick_decode<64, true>(int, bool, int, int);
extern template KernelFn pick_decode<128, false>(int, bool, int, int);
extern template KernelFn pick_decode<128, true>(int, bool, int, int);

// The cross-XCD merge of a spread launch.
MergeFn pick_merge(int hd, int g);

// The fp32 projections by dim = 1024 * NC: *rb rows per workgroup.
// (the fields of leap::QkvArgs and leap::ProjArgs as scalar arguments, which
// the dispatch preloads)
using QkvFn = void (*)(const float *, const float *, const float *, float *, float *, float *, int, int);
using ProjFn = void (*)(const float *, const float *, float *, int);
// (w, rows, sink): the same grid streaming the weights alone (measurement)
using GemvFloorFn = void (*)(const float *, int, float *);
bool pick_proj(int dim, QkvFn *qkv, ProjFn *proj, int *rb, GemvFloorFn *floor = nullptr);

// The int8 projections.
// (x, rms_w, w, ws and rows preloaded, then leap::Q8Args)
using Q8Fn = void (*)(const float *, const float *, const int8_t *, const float *, int, leap::Q8Args);
// True if (dim, gs) has int8 kernels.
bool q8_supported(int dim, int gs);
// The kernel of `kind` (leap::kQ8InRms or leap::kQ8InF32) for `rows` rows:
// the smallest compiled rows-per-team count RPT with kQ8Teams * RPT * n_cu >=
// rows, else the largest; *rpt receives it, and *floor (if not null) the
// kernel with the same grid that streams the weights alone (measurement).
Q8Fn pick_q8(int dim, int gs, int kind, int rows, int n_cu, int *rpt, Q8Fn *floor = nullptr);

}  // namespace leap_kernels
