// Device code for the two fp32 projections on either side of the attention
// block (gfx950, wave64):
//   - qkv_kernel: xb = rmsnorm(x, rms_att_weight[l]) and q, k, v = Wq/Wk/Wv . xb
//     (FloatTransformer.cpp:394-402, rmsnorm :88-213, matmul :240-382), with
//     the three weights stacked as one [dim + 2*kv_dim][dim] matrix per layer;
//   - proj_residual_kernel: x += Wo . xb (FloatTransformer.cpp:664-683).
//
// Both are matrix-vector products that stream the weights once: HBM-bound.  A
// workgroup owns RB consecutive rows; thread t holds the float4 columns
// t, t + 256, ... of the input vector in registers and issues, for every row of
// its block, the loads of the same columns, so each load instruction reads
// 4 KiB of one row contiguously and a workgroup has RB * n * 4 bytes in flight
// before its first FMA.  The (small) input vector is loaded before the rows.  The dot products are reduced across the wave with DPP
// and across the four waves in LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace leap {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / 64;

struct QkvArgs {
    const float *x;      // [dim] residual stream in
    const float *rms_w;  // [dim] rms_att_weight of the layer
    const float *w;      // [dim + 2*kv_dim][dim] stacked Wq, Wk, Wv of the layer
    float *q;            // [dim]    rows [0, dim)
    float *k;            // [kv_dim] rows [dim, dim + kv_dim)
    float *v;            // [kv_dim] rows [dim + kv_dim, dim + 2*kv_dim)
    int dim;
    int kv_dim;
};

struct ProjArgs {
    const float *xb;  // [n] attention output
    const float *w;   // [d][n] Wo of the layer
    float *x;         // [d] residual stream, updated in place
    int d;
};

// Sum over the 64 lanes of a wave; the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v)
{
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));
    const auto lane = [&](int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
    };
    return (lane(0) + lane(16)) + (lane(32) + lane(48));
}

__device__ __forceinline__ float dot4f(float4 a, float4 b)
{
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

typedef float gemv_f4 __attribute__((ext_vector_type(4)));

// Issue the loads of rows [row0, row0 + RB) of w ([rows][n], row-major) at
// this thread's float4 columns tid + 256*c, c < NC (n = 1024 * NC).  Rows at
// or past `rows` read the last row and are dropped by the caller.  Issued
// before anything waits, so the weight stream starts with the kernel; the
// weights are read once per step, so the loads are non-temporal (they do not
// displace the KV rows and partials from L2; measured 0.7 us faster per
// layer-step at Llama-3-8B).
template <int RB, int NC>
__device__ __forceinline__ void issue_rows(const float *w, int rows, int row0, int n, gemv_f4 (&wv)[RB][NC])
{
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < RB; i++) {
        const int r = row0 + i;
        const gemv_f4 *wr = reinterpret_cast<const gemv_f4 *>(w + (size_t)(r < rows ? r : rows - 1) * n);
#pragma unroll
        for (int c = 0; c < NC; c++) wv[i][c] = __builtin_nontemporal_load(wr + tid + kGemvThreads * c);
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every row load ahead of the vector work
}

// Dot products of the issued rows with the vector held as xv[c] = v4[tid +
// 256*c].  Returns, in thread i < RB, the dot product of row row0 + i.
template <int RB, int NC>
__device__ __forceinline__ float finish_dots(const gemv_f4 (&wv)[RB][NC], const float4 (&xv)[NC],
                                             float (*red)[kGemvWaves])
{
    const int tid = threadIdx.x;
    const int lane = tid % 64, wave = tid / 64;
#pragma unroll
    for (int i = 0; i < RB; i++) {
        float s = 0.f;
#pragma unroll
        for (int c = 0; c < NC; c++)
            s += dot4f(make_float4(wv[i][c].x, wv[i][c].y, wv[i][c].z, wv[i][c].w), xv[c]);
        s = wave_sum(s);
        if (lane == 0) red[i][wave] = s;
    }
    __syncthreads();
    float s = 0.f;
    if (tid < RB) {
#pragma unroll
        for (int j = 0; j < kGemvWaves; j++) s += red[tid][j];
    }
    return s;
}

// q, k, v = W . rmsnorm(x).  rmsnorm: o = w * (x / sqrt(mean(x^2) + 1e-5))
// (the reference's rsqrt estimate plus one Newton step rounds to within an
// ulp or two of 1/sqrt).  Every workgroup normalises the (small) vector
// itself while its weight rows are in flight, so no separate launch is needed.
//
// The kernels take their arguments as scalars, not as one struct: the
// dispatch preloads the leading 14 argument words into scalar registers (the
// library is built with -mllvm -amdgpu-kernarg-preload-count=14), so that
// the first loads do not wait for a load of the arguments.
template <int RB, int NC>
__global__ __launch_bounds__(kGemvThreads) void qkv_kernel(const float *x, const float *rms_w, const float *w,
                                                           float *q, float *k, float *v, int dim, int kv_dim)
{
    const QkvArgs a{x, rms_w, w, q, k, v, dim, kv_dim};
    __shared__ float red[RB][kGemvWaves];
    __shared__ float ss_part[kGemvWaves];
    const int tid = threadIdx.x;
    const int n = a.dim;
    const int rows = a.dim + 2 * a.kv_dim;
    const int row0 = blockIdx.x * RB;
    // The input first: load waits count outstanding loads in issue order, so
    // the normalisation can then run while the weight rows stream.
    const float4 *x4 = reinterpret_cast<const float4 *>(a.x);
    const float4 *g4 = reinterpret_cast<const float4 *>(a.rms_w);
    float4 xv[NC], gv[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        xv[c] = x4[tid + kGemvThreads * c];
        gv[c] = g4[tid + kGemvThreads * c];
    }
    __builtin_amdgcn_sched_barrier(0);
    gemv_f4 wv[RB][NC];
    issue_rows<RB, NC>(a.w, rows, row0, n, wv);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < NC; c++) ss += dot4f(xv[c], xv[c]);
    ss = wave_sum(ss);
    if (tid % 64 == 0) ss_part[tid / 64] = ss;
    __syncthreads();
    ss = (ss_part[0] + ss_part[1]) + (ss_part[2] + ss_part[3]);
    const float scale = 1.0f / sqrtf(ss / (float)n + 1e-5f);
#pragma unroll
    for (int c = 0; c < NC; c++)
        xv[c] = make_float4(gv[c].x * (scale * xv[c].x), gv[c].y * (scale * xv[c].y),
                            gv[c].z * (scale * xv[c].z), gv[c].w * (scale * xv[c].w));
    const float dot = finish_dots<RB, NC>(wv, xv, red);
    if (tid < RB) {
        const int r = row0 + tid;
        if (r < a.dim)
            a.q[r] = dot;
        else if (r < a.dim + a.kv_dim)
            a.k[r - a.dim] = dot;
        else if (r < rows)
            a.v[r - a.dim - a.kv_dim] = dot;
    }
}

// x += W . xb
template <int RB, int NC>
__global__ __launch_bounds__(kGemvThreads) void proj_residual_kernel(const float *xb, const float *w, float *x, int d)
{
    const ProjArgs a{xb, w, x, d};
    __shared__ float red[RB][kGemvWaves];
    const int tid = threadIdx.x;
    const int n = NC * 4 * kGemvThreads;
    const int row0 = blockIdx.x * RB;
    const float4 *v4 = reinterpret_cast<const float4 *>(a.xb);
    float4 xv[NC];
#pragma unroll
    for (int c = 0; c < NC; c++) xv[c] = v4[tid + kGemvThreads * c];
    __builtin_amdgcn_sched_barrier(0);
    gemv_f4 wv[RB][NC];
    issue_rows<RB, NC>(a.w, a.d, row0, n, wv);
    const float dot = finish_dots<RB, NC>(wv, xv, red);
    if (tid < RB) {
        const int r = row0 + tid;
        if (r < a.d) a.x[r] += dot;
    }
}

// The weights alone (measurement only): the grid, block size and row loads of
// qkv_kernel / proj_residual_kernel over w [rows][n], summed and kept only
// behind a test that real data never meets.  The launch plus the bare weight
// stream of one projection.
template <int RB, int NC>
__global__ __launch_bounds__(kGemvThreads) void gemv_floor_kernel(const float *w, int rows, float *sink)
{
    gemv_f4 wv[RB][NC];
    issue_rows<RB, NC>(w, rows, blockIdx.x * RB, NC * 4 * kGemvThreads, wv);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < RB; i++)
#pragma unroll
        for (int c = 0; c < NC; c++) s += (wv[i][c].x + wv[i][c].y) + (wv[i][c].z + wv[i][c].w);
    if (__builtin_bit_cast(unsigned, s) == 0x7FC0DEADu) sink[threadIdx.x] = s;
}

}  // namespace leap
