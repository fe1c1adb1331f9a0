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
// One workgroup per CU: the fp32 input vector (and the rms weight) is read,
// normalised and quantized once per workgroup and shared through LDS, so that
// the int8 weights, which are a quarter of the fp32 bytes per row, are not
// outweighed by every workgroup re-reading 16-32 KiB of activations from L2.
// A row's int8 load is one contiguous E-byte access per thread (E = n/256; 1
// KiB per wave at n = 4096).
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

#include "decode_attention.hpp"  // raw buffer access helpers
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

// What the kernel's input vector is.
constexpr int kQ8InRms = 0;   // fp32 residual stream: rmsnorm with rms_w, then quantize
constexpr int kQ8InF32 = 1;   // fp32 vector (the attention output): quantize

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

// Group maximum over aligned groups of W lanes (W a power of two <= 64).
template <int W>
__device__ __forceinline__ float group_max_w(float v)
{
    if constexpr (W <= 16) {
        return group_max<W>(v);
    } else {
        v = group_max<16>(v);
        v = fmaxf(v, __shfl_xor(v, 16));
        if constexpr (W >= 64) v = fmaxf(v, __shfl_xor(v, 32));
        return v;
    }
}

// E int8 values per thread as E/4 packed words.
template <int E>
struct Q8Row {
    int v[E / 4];
};

// The same E bytes through a raw buffer load (non-temporal): `off` past the
// descriptor's range reads zeros without touching memory, which keeps the
// load unconditional for lanes that own no values.
template <int E>
__device__ __forceinline__ Q8Row<E> load_row_buf(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    Q8Row<E> w;
    if constexpr (E == 8) {
        const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kNt);
        w.v[0] = (int)a.x;
        w.v[1] = (int)a.y;
    } else {
#pragma unroll
        for (int c = 0; c < E / 16; c++) {
            const u32x4 a = __builtin_amdgcn_raw_buffer_load_b128(r, (int)(off + 16u * c), 0, kNt);
            w.v[4 * c] = (int)a.x;
            w.v[4 * c + 1] = (int)a.y;
            w.v[4 * c + 2] = (int)a.z;
            w.v[4 * c + 3] = (int)a.w;
        }
    }
    return w;
}

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

constexpr int kQ8Threads = 1024;  // one workgroup per CU: 16 waves
constexpr int kQ8Teams = kQ8Threads / kGemvThreads;
constexpr int kQ8Waves = kQ8Threads / 64;

// One workgroup of 1024 threads (16 waves, one per CU at the launch sizes
// used) owns rows [row0, row0 + 4*RPT): four teams of 256 threads, team k
// taking rows row0 + k*RPT + j, j < RPT.  In a team, thread t < ACT owns the
// E = n/ACT values [t*E, t*E + E) of each of its rows, so a group of gs values
// is L = gs/E adjacent lanes.  ACT is 256 when n is 256 times a power of two;
// for n = 3072 (ACT 192, E 16) and 5120 (ACT 160, E 32) the team's last
// threads own no values: their row loads read zeros past the range and they
// write nothing.  The input vector is read, normalised and quantized once per
// workgroup, each of the first 4*ACT threads taking E/4 consecutive values,
// and shared through LDS.
//
// Issue order: the input first, then the team's scales and weight rows
// (4*RPT*n bytes per workgroup, 96 KiB for Wq/Wk/Wv at Llama-3-8B), all before
// anything waits.  RPT is a compile-time count so that every load is
// unconditional: load waits count outstanding loads in issue order, and with a
// runtime row count the wait for the input had to assume the longest queue,
// which made the normalisation wait for every weight row (0.8 us at
// Llama-3-8B).  The input work now runs while the weights stream.
//
// Arguments: the input and weight pointers and the row count come first as
// scalars, which the dispatch preloads into scalar registers (the library is
// built with -mllvm -amdgpu-kernarg-preload-count=14), so that the first
// loads do not wait for a load of the arguments; the rest of Q8Args (the
// outputs) is read after the weight rows are issued (late_args).
constexpr unsigned kQ8ArgsOffset = 4 * sizeof(void *) + 8;  // Q8Args after the preloaded x, rms_w, w, ws, rows
static_assert(alignof(Q8Args) == 8, "argument layout");
#define LEAP_Q8_PRELOAD_PARAMS const float *pre_x, const float *pre_rms_w, const int8_t *pre_w, const float *pre_ws, int pre_rows
template <int E, int L, int RPT, int kIn, bool kResid, int ACT = kGemvThreads>
__global__ __launch_bounds__(kQ8Threads) void q8_gemv_kernel(LEAP_Q8_PRELOAD_PARAMS, Q8Args args)
{
    Q8Args a{};
    a.x = pre_x;
    a.rms_w = pre_rms_w;
    a.w = pre_w;
    a.ws = pre_ws;
    a.rows = pre_rows;
    constexpr int n = ACT * E;
    constexpr int NG = ACT / L;            // groups per row
    constexpr int VA = E / 4;              // input values per thread in the quantize step
    constexpr int QT = n / VA;             // threads of the quantize step (4 * ACT)
    constexpr int W = (L * E) / VA;        // threads per group in the quantize step (= 4 L)
    constexpr int SLOTS = kQ8Teams * RPT;
    static_assert(ACT <= kGemvThreads && ACT % L == 0 && ACT % 32 == 0 && NG % 4 == 0 && QT % W == 0,
                  "thread layout");
    __shared__ __align__(16) int8_t lds_xq[n];
    __shared__ float lds_xs[NG];
    // (float)idot and ws * sx of (row slot, group), [slot][group] with the
    // rows padded so that the chain lanes' 128-bit reads spread over the banks
    constexpr int NGP = NG + 4;
    __shared__ __align__(16) float lds_f[SLOTS * NGP];
    __shared__ __align__(16) float lds_c[SLOTS * NGP];
    __shared__ float ss_part[kQ8Waves];
    static_assert(2 * SLOTS * NGP * 4 + n + NG * 4 <= 64 * 1024, "LDS budget");
    constexpr int SCL = (RPT * NG / 4 + kGemvThreads - 1) / kGemvThreads;  // scale float4s per thread
    const int tid = threadIdx.x;
    const int team = tid / kGemvThreads, tt = tid % kGemvThreads;
    const int g = tt / L;  // this thread's group in the dot step
    const int row0 = blockIdx.x * SLOTS;
    const int rbase = row0 + team * RPT;

    // 1. the input: E/4 fp32 values (and rms weights) per thread
    float v[VA], gw[VA];
#pragma unroll
    for (int e = 0; e < VA; e++) v[e] = gw[e] = 0.f;
    if (QT < kQ8Threads && tid >= QT) {
        // owns no input values
    } else if constexpr (VA == 2) {
        const float2 t = reinterpret_cast<const float2 *>(a.x)[tid];
        v[0] = t.x;
        v[1] = t.y;
    } else {
#pragma unroll
        for (int c = 0; c < VA / 4; c++) {
            const float4 t = reinterpret_cast<const float4 *>(a.x + tid * VA)[c];
            v[4 * c] = t.x;
            v[4 * c + 1] = t.y;
            v[4 * c + 2] = t.z;
            v[4 * c + 3] = t.w;
        }
    }
    if constexpr (kIn == kQ8InRms) {
        if (QT < kQ8Threads && tid >= QT) {
        } else if constexpr (VA == 2) {
            const float2 t = reinterpret_cast<const float2 *>(a.rms_w)[tid];
            gw[0] = t.x;
            gw[1] = t.y;
        } else {
#pragma unroll
            for (int c = 0; c < VA / 4; c++) {
                const float4 t = reinterpret_cast<const float4 *>(a.rms_w + tid * VA)[c];
                gw[4 * c] = t.x;
                gw[4 * c + 1] = t.y;
                gw[4 * c + 2] = t.z;
                gw[4 * c + 3] = t.w;
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. this team's group scales (RPT * NG consecutive floats, as float4s),
    // then its weight rows
    gemv_f4 scv[SCL];
#pragma unroll
    for (int i = 0; i < SCL; i++) {
        const int e = 4 * (tt + i * kGemvThreads);  // scale index in the team's block
        const int r = min(rbase + e / NG, a.rows - 1);
        if (e < RPT * NG)
            scv[i] = __builtin_nontemporal_load(reinterpret_cast<const gemv_f4 *>(a.ws + (size_t)r * NG + e % NG));
    }
    Q8Row<E> wv[RPT];
    if constexpr (ACT == kGemvThreads) {
#pragma unroll
        for (int j = 0; j < RPT; j++) {
            const int r = min(rbase + j, a.rows - 1);
            wv[j] = load_row_nt<E>(a.w + (size_t)r * n + tt * E);
        }
    } else {
        const uint32_t w_bytes = (uint32_t)a.rows * (uint32_t)n;
        const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(a.w, w_bytes);
#pragma unroll
        for (int j = 0; j < RPT; j++) {
            const int r = min(rbase + j, a.rows - 1);
            wv[j] = load_row_buf<E>(w_rsrc, tt < ACT ? (uint32_t)r * (uint32_t)n + (uint32_t)(tt * E) : w_bytes);
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 3. the input normalised (if asked) and quantized into LDS: group max
    // over W lanes, scale, round half away from zero
    if constexpr (kIn == kQ8InRms) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < VA; e++) ss += v[e] * v[e];
        ss = wave_sum(ss);
        if (tid % 64 == 0) ss_part[tid / 64] = ss;
        __syncthreads();
        ss = 0.f;
#pragma unroll
        for (int w = 0; w < kQ8Waves; w++) ss += ss_part[w];
        const float scale = 1.0f / sqrtf(ss / (float)n + 1e-5f);
#pragma unroll
        for (int e = 0; e < VA; e++) v[e] = gw[e] * (scale * v[e]);
    }
    float m = 0.f;
#pragma unroll
    for (int e = 0; e < VA; e++) m = fmaxf(m, fabsf(v[e]));
    m = group_max_w<W>(m);
    const float sx = m * (1.0f / 127.0f);
    const float id = sx != 0.0f ? __frcp_rn(sx) : 0.0f;
    int8_t q[VA];
#pragma unroll
    for (int e = 0; e < VA; e++) q[e] = (int8_t)(int)roundf(v[e] * id);
    if (QT < kQ8Threads && tid >= QT) {
    } else if constexpr (VA == 2) {
        *reinterpret_cast<short *>(lds_xq + tid * 2) = (short)((q[0] & 0xFF) | ((q[1] & 0xFF) << 8));
    } else {
#pragma unroll
        for (int k = 0; k < VA / 4; k++)
            reinterpret_cast<int *>(lds_xq + tid * VA)[k] =
                (q[4 * k] & 0xFF) | ((q[4 * k + 1] & 0xFF) << 8) | ((q[4 * k + 2] & 0xFF) << 16) |
                ((q[4 * k + 3] & 0xFF) << 24);
    }
    if (tid % W == 0 && tid < QT) lds_xs[tid / W] = sx;
#pragma unroll
    for (int i = 0; i < SCL; i++) {
        const int e = 4 * (tt + i * kGemvThreads);
        if (e < RPT * NG) {
            float *dst = lds_c + (team * RPT + e / NG) * NGP + e % NG;
            dst[0] = scv[i].x;
            dst[1] = scv[i].y;
            dst[2] = scv[i].z;
            dst[3] = scv[i].w;
        }
    }
    __syncthreads();
    // The outputs, from here on: the barriers above wait for every scalar
    // load in flight, and these are needed only at the end.
    {
        const Q8Args late = late_args(args, kQ8ArgsOffset);
        a.out0 = late.out0;
        a.out1 = late.out1;
        a.out2 = late.out2;
        a.n0 = late.n0;
        a.n1 = late.n1;
        a.xq_out = late.xq_out;
        a.xs_out = late.xs_out;
    }
    if (blockIdx.x == 0 && a.xq_out) {  // the quantized input, for stage checks
        for (int i = tid; i < n / 4; i += kQ8Threads)
            reinterpret_cast<int *>(a.xq_out)[i] = reinterpret_cast<const int *>(lds_xq)[i];
        for (int i = tid; i < NG; i += kQ8Threads) a.xs_out[i] = lds_xs[i];
    }

    // 4. exact group dot products, one (float, scale product) pair per group
    const bool owns = ACT == kGemvThreads || tt < ACT;
    int xq[E / 4];
#pragma unroll
    for (int k = 0; k < E / 4; k++) xq[k] = owns ? reinterpret_cast<const int *>(lds_xq + tt * E)[k] : 0;
    const float sxg = owns ? lds_xs[g] : 0.f;
#pragma unroll
    for (int j = 0; j < RPT; j++) {
        int d = 0;
#pragma unroll
        for (int k = 0; k < E / 4; k++) d = __builtin_amdgcn_sdot4(xq[k], wv[j].v[k], d, false);
        d = group_sum_i32<L>(d);
        if (tt % L == 0 && owns) {
            const int at = (team * RPT + j) * NGP + g;
            lds_f[at] = (float)d;
            lds_c[at] = lds_c[at] * sxg;
        }
    }
    __syncthreads();

    // 5. the ordered accumulation, one lane per row
    if (tid < SLOTS) {
        float val = 0.f;
        const float4 *f4 = reinterpret_cast<const float4 *>(lds_f + tid * NGP);
        const float4 *c4 = reinterpret_cast<const float4 *>(lds_c + tid * NGP);
        // The wo product's chain reads all its LDS pairs ahead (0.24 us at
        // Llama-3-8B); the q/k/v product gains nothing and would spill.
        constexpr int kChainUnroll = kIn == kQ8InF32 ? NG / 4 : 4;
#pragma unroll kChainUnroll
        for (int j = 0; j < NG / 4; j++) {
            const float4 f = f4[j], c = c4[j];
            val = __builtin_fmaf(f.x, c.x, val);
            val = __builtin_fmaf(f.y, c.y, val);
            val = __builtin_fmaf(f.z, c.z, val);
            val = __builtin_fmaf(f.w, c.w, val);
        }
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

// The int8 weights alone (measurement only): the grid, block size, scale
// loads and row loads of q8_gemv_kernel<E, L, RPT, ..., ACT> over w [rows][n]
// and its scales ws [rows][n / gs], summed and kept only behind a test that
// real data never meets.  The launch plus the bare weight stream of one
// int8 projection.
template <int E, int L, int RPT, int ACT = kGemvThreads>
__global__ __launch_bounds__(kQ8Threads) void q8_floor_kernel(LEAP_Q8_PRELOAD_PARAMS, Q8Args a)
{
    (void)pre_x;
    (void)pre_rms_w;
    a.w = pre_w;
    a.ws = pre_ws;
    a.rows = pre_rows;
    constexpr int n = ACT * E;
    constexpr int NG = ACT / L;
    constexpr int SLOTS = kQ8Teams * RPT;
    constexpr int SCL = (RPT * NG / 4 + kGemvThreads - 1) / kGemvThreads;
    const int tid = threadIdx.x;
    const int team = tid / kGemvThreads, tt = tid % kGemvThreads;
    const int rbase = blockIdx.x * SLOTS + team * RPT;
    gemv_f4 scv[SCL];
#pragma unroll
    for (int i = 0; i < SCL; i++) {
        const int e = 4 * (tt + i * kGemvThreads);
        const int r = min(rbase + e / NG, a.rows - 1);
        scv[i] = e < RPT * NG ? __builtin_nontemporal_load(reinterpret_cast<const gemv_f4 *>(a.ws + (size_t)r * NG + e % NG))
                              : gemv_f4{0.f, 0.f, 0.f, 0.f};
    }
    Q8Row<E> wv[RPT];
    const uint32_t w_bytes = (uint32_t)a.rows * (uint32_t)n;
    const __amdgpu_buffer_rsrc_t w_rsrc = make_rsrc(a.w, w_bytes);
#pragma unroll
    for (int j = 0; j < RPT; j++) {
        const int r = min(rbase + j, a.rows - 1);
        if constexpr (ACT == kGemvThreads)
            wv[j] = load_row_nt<E>(a.w + (size_t)r * n + tt * E);
        else
            wv[j] = load_row_buf<E>(w_rsrc, tt < ACT ? (uint32_t)r * (uint32_t)n + (uint32_t)(tt * E) : w_bytes);
    }
    int acc = 0;
#pragma unroll
    for (int j = 0; j < RPT; j++)
#pragma unroll
        for (int k = 0; k < E / 4; k++) acc ^= wv[j].v[k];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < SCL; i++) s += (scv[i].x + scv[i].y) + (scv[i].z + scv[i].w);
    if (acc == 0x7EADBEEF && __builtin_bit_cast(unsigned, s) == 0x7FC0DEADu) a.out0[tid] = s;
}

}  // namespace leap
