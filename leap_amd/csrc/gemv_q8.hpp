// Device code for the quantized engine's projections on either side of the
// attention block (gfx950, wave64): W8A8 matrix-vector products with one
// float scale per group of gs consecutive values of a row, as
// QuantizedTransformer::quantize (QuantizedTransformer.cpp:338-357) and
// ::matmul (:359-652) compute them.
//   - q8_gemv_kernel<..., kRms = true,  kResid = false>: xb = rmsnorm(x),
//     quantized per group, then q, k, v = the stacked int8 Wq/Wk/Wv . xb
//     (QuantizedTransformer.cpp:664-678);
//   - q8_gemv_kernel<..., kRms = false, kResid = true>: the attention output
//     quantized per group, then x += Wo . that (the wo matmul and the residual
//     after the attention block).
//
// Each workgroup quantizes the whole input vector itself (it is small and
// reaches every workgroup from L2) while its weight rows are in flight: thread
// t owns the E = n/256 consecutive values [t*E, t*E + E), so a group of gs
// values is L = gs/E adjacent lanes, and a row's int8 load is one contiguous
// E-byte access per thread (1 KiB per wave at n = 4096).
//
// Arithmetic, matched to the reference bit for bit:
//   - group scale sx = max|v| * (1/127) (the reference's release build folds
//     its division by 127 into this product), id = 1/sx rounded to nearest
//     (0 for an all-zero group), q = round-half-away(v * id);
//   - the int8 dot product of a group is exact in int32 (v_dot4_i32_i8), and
//     a row's groups are accumulated in order with one fused multiply-add
//     each: val = fma((float)idot_g, ws_g * sx_g, val).  The group products
//     are formed in parallel and the ordered chain runs in one lane per row.
// The rmsnorm in front of the q/k/v product computes 1/sqrt(mean(x^2) +
// 1e-5) exactly rounded, where the reference uses a hardware reciprocal
// square-root estimate plus one Newton step; the two differ in the last bit
// or two, which can move a quantized value by one step.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gemv.hpp"

namespace leap {

struct Q8Args {
    const float *x;      // [n] input: the residual stream (with rmsnorm) or the attention output
    const float *rms_w;  // [n] rms_att weight of the layer (rmsnorm variant only)
    const int8_t *w;     // [rows][n] int8 weights (Wq, Wk, Wv stacked, or Wo)
    const float *ws;     // [rows][n / gs] group scales
    float *out0;         // rows [0, n0): q, or the residual stream x (x[r] += val)
    float *out1;         // rows [n0, n0 + n1): k
    float *out2;         // rows [n0 + n1, rows): v
    int rows, n0, n1;
    int8_t *xq_out;      // [n] the quantized input as every workgroup computed it (written by workgroup 0)
    float *xs_out;       // [n / gs] its group scales
};

// Butterfly over aligned groups of L lanes (L a power of two <= 16) with the
// DPP patterns of wave_sum; every lane of a group ends with the group's
// result.  Integer sums are exact in any order; max is order-free.
template <int L>
__device__ __forceinline__ int group_sum_i32(int v)
{
    if constexpr (L >= 2) v += __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
    if constexpr (L >= 4) v += __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
    if constexpr (L >= 8) v += __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, true);  // row_half_mirror
    if constexpr (L >= 16) v += __builtin_amdgcn_mov_dpp(v, 0x140, 0xF, 0xF, true); // row_mirror
    return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

template <int L>
__device__ __forceinline__ float group_max(float v)
{
    if constexpr (L >= 2) v = fmaxf(v, dpp_f<0xB1>(v));
    if constexpr (L >= 4) v = fmaxf(v, dpp_f<0x4E>(v));
    if constexpr (L >= 8) v = fmaxf(v, dpp_f<0x141>(v));
    if constexpr (L >= 16) v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}

// E int8 values per thread as E/4 packed words.
template <int E>
struct Q8Row {
    int v[E / 4];
};

template <int E>
__device__ __forceinline__ Q8Row<E> load_row_nt(const int8_t *p)
{
    Q8Row<E> r;
    if constexpr (E == 8) {
        typedef int i2 __attribute__((ext_vector_type(2)));
        const i2 a = __builtin_nontemporal_load(reinterpret_cast<const i2 *>(p));
        r.v[0] = a.x;
        r.v[1] = a.y;
    } else {
        typedef int i4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int c = 0; c < E / 16; c++) {
            const i4 a = __builtin_nontemporal_load(reinterpret_cast<const i4 *>(p) + c);
            r.v[4 * c] = a.x;
            r.v[4 * c + 1] = a.y;
            r.v[4 * c + 2] = a.z;
            r.v[4 * c + 3] = a.w;
        }
    }
    return r;
}

// One workgroup of 256 threads owns rows [row0, row0 + RB).  n = 256 * E,
// gs = L * E, NG = n / gs = 256 / L groups per row.
template <int E, int L, int RB, bool kRms, bool kResid>
__global__ __launch_bounds__(kGemvThreads) void q8_gemv_kernel(Q8Args a)
{
    constexpr int n = kGemvThreads * E;
    constexpr int NG = kGemvThreads / L;
    __shared__ float lds_f[NG * RB];  // (float)idot of (group, row), [group][row]
    __shared__ float lds_c[NG * RB];  // ws * sx of (group, row)
    __shared__ float ss_part[kGemvWaves];
    const int tid = threadIdx.x;
    const int g = tid / L;  // this thread's group
    const int row0 = blockIdx.x * RB;

    // 1. the weight rows and their group scales, before anything waits
    Q8Row<E> wv[RB];
    float sc[RB];
#pragma unroll
    for (int i = 0; i < RB; i++) {
        const int r = row0 + i < a.rows ? row0 + i : a.rows - 1;
        wv[i] = load_row_nt<E>(a.w + (size_t)r * n + tid * E);
    }
#pragma unroll
    for (int i = 0; i < RB; i++) {
        const int r = row0 + i < a.rows ? row0 + i : a.rows - 1;
        sc[i] = __builtin_nontemporal_load(a.ws + (size_t)r * NG + g);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the input values of this thread, rmsnorm-ed if asked
    float v[E];
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x + tid * E);
#pragma unroll
    for (int c = 0; c < E / 4; c++) {
        const float4 t = x4[c];
        v[4 * c] = t.x;
        v[4 * c + 1] = t.y;
        v[4 * c + 2] = t.z;
        v[4 * c + 3] = t.w;
    }
    if constexpr (kRms) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; e++) ss += v[e] * v[e];
        ss = wave_sum(ss);
        if (tid % 64 == 0) ss_part[tid / 64] = ss;
        __syncthreads();
        ss = (ss_part[0] + ss_part[1]) + (ss_part[2] + ss_part[3]);
        const float scale = 1.0f / sqrtf(ss / (float)n + 1e-5f);
        const float4 *g4 = reinterpret_cast<const float4 *>(a.rms_w + tid * E);
#pragma unroll
        for (int c = 0; c < E / 4; c++) {
            const float4 t = g4[c];
            v[4 * c] = t.x * (scale * v[4 * c]);
            v[4 * c + 1] = t.y * (scale * v[4 * c + 1]);
            v[4 * c + 2] = t.z * (scale * v[4 * c + 2]);
            v[4 * c + 3] = t.w * (scale * v[4 * c + 3]);
        }
    }

    // 3. quantize: group max over L lanes, scale, round half away from zero
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < E; e++) m = fmaxf(m, fabsf(v[e]));
    m = group_max<L>(m);
    const float sx = m * (1.0f / 127.0f);
    const float id = sx != 0.0f ? __frcp_rn(sx) : 0.0f;
    int xq[E / 4];
#pragma unroll
    for (int k = 0; k < E / 4; k++) {
        int packed = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) packed |= ((int)roundf(v[4 * k + b] * id) & 0xFF) << (8 * b);
        xq[k] = packed;
    }
    if (blockIdx.x == 0 && a.xq_out) {
        int *dst = reinterpret_cast<int *>(a.xq_out + tid * E);
#pragma unroll
        for (int k = 0; k < E / 4; k++) dst[k] = xq[k];
        if (tid % L == 0) a.xs_out[g] = sx;
    }

    // 4. exact group dot products, one (float, scale product) pair per group
#pragma unroll
    for (int i = 0; i < RB; i++) {
        int d = 0;
#pragma unroll
        for (int k = 0; k < E / 4; k++) d = __builtin_amdgcn_sdot4(xq[k], wv[i].v[k], d, false);
        d = group_sum_i32<L>(d);
        if (tid % L == 0) {
            lds_f[g * RB + i] = (float)d;
            lds_c[g * RB + i] = sc[i] * sx;
        }
    }
    __syncthreads();

    // 5. the ordered accumulation, one lane per row
    if (tid < RB) {
        float val = 0.f;
#pragma unroll 8
        for (int j = 0; j < NG; j++) val = __builtin_fmaf(lds_f[j * RB + tid], lds_c[j * RB + tid], val);
        const int r = row0 + tid;
        if (r < a.rows) {
            if constexpr (kResid) {
                a.out0[r] += val;
            } else {
                if (r < a.n0)
                    a.out0[r] = val;
                else if (r < a.n0 + a.n1)
                    a.out1[r - a.n0] = val;
                else
                    a.out2[r - a.n0 - a.n1] = val;
            }
        }
    }
}

}  // namespace leap
