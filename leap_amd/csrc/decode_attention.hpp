// Device code for LEAP decode attention on gfx950 (CDNA4, wave64).
//
// One launch performs the whole attention block of one layer step for one or
// more sequences (the reference's FloatTransformer.cpp:396-662):
//   - RoPE of q (every workgroup rotates the q heads of its KV group from the
//     fp32 table row `pos`, FloatTransformer.cpp:404-494),
//   - the KV append: the workgroup whose chunk holds `pos` rotates k_new,
//     stores k_new/v_new into cache[layer][pos] and uses them in registers,
//   - split-K flash decoding over the KV positions [0, pos]: each workgroup
//     owns one (sequence, KV head, chunk of positions), streams its K and V
//     rows straight into registers with 128-bit loads and serves all q heads
//     of the KV group from those registers (GQA score, :496-630), with an
//     online softmax (running max/sum, :216-238) and the weighted-V
//     accumulation (:634-661),
//   - the merge of the chunk partials, done by the last workgroup of each
//     (sequence, KV head) to finish (an atomic arrival counter it resets).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace leap {

constexpr int kWave = 64;
constexpr int kWaves = 4;                 // waves per workgroup
constexpr int kThreads = kWave * kWaves;  // 256
constexpr int kMaxChunks = 512;           // split-K chunks per (sequence, KV head)
// Positions one workgroup pass covers (kWaves sub-tiles of 2048/HD rows);
// chunk sizes are multiples of it.
__host__ __device__ constexpr int rows_per_pass(int hd) { return kWaves * (2048 / hd); }

struct StepArgs {
    const float *q;      // [n_seq][n_heads*HD], pre-RoPE
    const float *k_new;  // [n_seq][kv_dim], pre-RoPE
    const float *v_new;  // [n_seq][kv_dim]
    float *out;          // [n_seq][n_heads*HD]
    float *k_cache;      // slab base of sequence 0 at this layer
    float *v_cache;
    const float4 *rope;  // [seq_len][HD/4] of (cos_2i, sin_2i, cos_2i+1, sin_2i+1)
    const int *pos_dev;  // per-sequence positions, or nullptr -> pos_scalar
    float *ws_o;         // [n_seq][n_heads][kMaxChunks][HD] partial outputs
    float2 *ws_ml;       // [n_seq][n_heads][kMaxChunks] (max, sum) in log2 units
    int *counters;       // [n_seq][n_kv_heads] arrival counters, zero between launches
    long long seq_stride;// floats between sequence slabs
    int pos_scalar;
    int max_pos;         // launch was sized for positions <= max_pos
    int seq_len;
    int n_heads;
    int n_kv_heads;
    int chunk;           // positions per workgroup, multiple of rows_per_pass(HD)
    float scale_log2;    // log2(e) / sqrt(HD)
};

// ---- wave helpers ---------------------------------------------------------

template <int W>
__device__ __forceinline__ float xor_sum(float x)
{
#pragma unroll
    for (int o = 1; o < W; o <<= 1) x += __shfl_xor(x, o, kWave);
    return x;
}

// max over lanes that differ only in bits [log2(FROM), 6)
template <int FROM>
__device__ __forceinline__ float xor_max_above(float x)
{
#pragma unroll
    for (int o = FROM; o < kWave; o <<= 1) x = fmaxf(x, __shfl_xor(x, o, kWave));
    return x;
}

template <int FROM>
__device__ __forceinline__ float xor_sum_above(float x)
{
#pragma unroll
    for (int o = FROM; o < kWave; o <<= 1) x += __shfl_xor(x, o, kWave);
    return x;
}

__device__ __forceinline__ float dot4(float4 a, float4 b)
{
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// Interleaved-pair rotation of one float4 (two pairs) with table entry
// t = (cos_a, sin_a, cos_b, sin_b), products rounded separately as the
// reference's mul/mul/addsub body does (FloatTransformer.cpp:461-464).
__device__ __forceinline__ float4 rope4(float4 x, float4 t)
{
#pragma clang fp contract(off)
    float4 r;
    r.x = x.x * t.x - x.y * t.y;
    r.y = x.y * t.x + x.x * t.y;
    r.z = x.z * t.z - x.w * t.w;
    r.w = x.w * t.z + x.z * t.w;
    return r;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- the fused decode-attention kernel --------------------------------------

template <int HD, int G>
struct Shape {
    static constexpr int LPR = (HD * G >= 1024) ? 16 : 8;  // lanes per K row
    static constexpr int NF = HD / (4 * LPR);              // float4 per lane per K row
    static constexpr int RPK = kWave / LPR;                // K rows per load set
    static constexpr int R = 2048 / HD;                    // rows per wave sub-tile
    static constexpr int KS = R / RPK;                     // K load sets per sub-tile
    static constexpr int LPV = HD / 4;                     // lanes per V row
    static constexpr int RPV = kWave / LPV;                // V rows per load set
    static constexpr int VS = R / RPV;                     // V load sets per sub-tile
    static constexpr int ROWS = kWaves * R;                // positions per workgroup pass
    static_assert(HD % (4 * LPR) == 0, "head_dim vs lanes per row");
    static_assert(R % RPK == 0 && R % RPV == 0, "sub-tile shape");
    static_assert(G <= LPR, "group size vs lanes per row");
    static_assert(ROWS == rows_per_pass(HD), "pass shape");
};

template <int HD, int G>
__global__ __launch_bounds__(kThreads) void decode_attention_kernel(StepArgs a)
{
    using S = Shape<HD, G>;
    constexpr int LPR = S::LPR, NF = S::NF, RPK = S::RPK, R = S::R, KS = S::KS;
    constexpr int LPV = S::LPV, RPV = S::RPV, VS = S::VS;

    const int chunk_id = blockIdx.x;
    const int kvh = blockIdx.y;
    const int seq = blockIdx.z;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;

    const int pos = a.pos_dev ? a.pos_dev[seq] : a.pos_scalar;
    if (pos < 0 || pos >= a.seq_len || pos > a.max_pos) return;
    const int T = pos + 1;
    const int n_chunks = (T + a.chunk - 1) / a.chunk;
    if (chunk_id >= n_chunks) return;

    const int kv_dim = a.n_kv_heads * HD;
    const int q_dim = a.n_heads * HD;
    const size_t slab = (size_t)seq * (size_t)a.seq_stride;
    const float *kc = a.k_cache + slab + (size_t)kvh * HD;
    const float *vc = a.v_cache + slab + (size_t)kvh * HD;
    const float *qg = a.q + (size_t)seq * q_dim + (size_t)kvh * G * HD;
    const float4 *rope_row = a.rope + (size_t)pos * (HD / 4);

    __shared__ float p_lds[kWaves][R * G];
    __shared__ float comb_o[kWaves][G][HD];
    __shared__ float comb_ml[kWaves][G][2];
    __shared__ float merge_w[kWaves][kMaxChunks];
    __shared__ int s_last;

    // K layout: lane = kg*LPR + kj; lane holds dims 4*(f*LPR + kj) .. +3.
    const int kg = lane / LPR, kj = lane % LPR;
    // V layout: lane = vg*LPV + vj; lane holds dims 4*vj .. +3.
    const int vg = lane / LPV, vj = lane % LPV;

    // Rotated q for the G heads of this KV group, in the K layout.
    float4 qr[G][NF];
#pragma unroll
    for (int f = 0; f < NF; f++) {
        const int d4 = f * LPR + kj;
        const float4 tab = rope_row[d4];
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float4 x = *reinterpret_cast<const float4 *>(qg + (size_t)h * HD + 4 * d4);
            qr[h][f] = rope4(x, tab);
        }
    }

    const int chunk_begin = chunk_id * a.chunk;
    const int n_sub = a.chunk / S::ROWS;

    float m_run[G], l_run[G];
    float4 acc[G];
#pragma unroll
    for (int h = 0; h < G; h++) {
        m_run[h] = -INFINITY;
        l_run[h] = 0.0f;
        acc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    float4 kb[KS][NF], vb[VS];

    auto load_tile = [&](int sub, float4 (&kd)[KS][NF], float4 (&vd)[VS]) {
        const int base = chunk_begin + (sub * kWaves + wave) * R;
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int t = base + ks * RPK + kg;
            const float *row = (t == pos) ? a.k_new + (size_t)seq * kv_dim + (size_t)kvh * HD
                                          : kc + (size_t)t * kv_dim;
#pragma unroll
            for (int f = 0; f < NF; f++) {
                const int d4 = f * LPR + kj;
                kd[ks][f] = (t <= pos) ? *reinterpret_cast<const float4 *>(row + 4 * d4)
                                       : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
#pragma unroll
        for (int vs = 0; vs < VS; vs++) {
            const int t = base + vs * RPV + vg;
            const float *row = (t == pos) ? a.v_new + (size_t)seq * kv_dim + (size_t)kvh * HD
                                          : vc + (size_t)t * kv_dim;
            vd[vs] = (t <= pos) ? *reinterpret_cast<const float4 *>(row + 4 * vj)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };

    for (int sub = 0; sub < n_sub; sub++) {
        load_tile(sub, kb, vb);

        const int base = chunk_begin + (sub * kWaves + wave) * R;

        // The new token's row: rotate k, and append k and v to the cache.
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int t = base + ks * RPK + kg;
            if (t == pos) {
#pragma unroll
                for (int f = 0; f < NF; f++) {
                    const int d4 = f * LPR + kj;
                    kb[ks][f] = rope4(kb[ks][f], rope_row[d4]);
                    *reinterpret_cast<float4 *>(const_cast<float *>(kc) + (size_t)t * kv_dim + 4 * d4) =
                        kb[ks][f];
                }
            }
        }
#pragma unroll
        for (int vs = 0; vs < VS; vs++) {
            const int t = base + vs * RPV + vg;
            if (t == pos)
                *reinterpret_cast<float4 *>(const_cast<float *>(vc) + (size_t)t * kv_dim + 4 * vj) = vb[vs];
        }

        // Scores (log2 units) for the KS rows this lane group holds.
        float s[KS][G];
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const int t = base + ks * RPK + kg;
#pragma unroll
            for (int h = 0; h < G; h++) {
                float d = 0.f;
#pragma unroll
                for (int f = 0; f < NF; f++) d += dot4(qr[h][f], kb[ks][f]);
                d = xor_sum<LPR>(d) * a.scale_log2;
                s[ks][h] = (t <= pos) ? d : -INFINITY;
            }
        }

        // Online softmax update, per head, wave-wide.
        float alpha[G];
#pragma unroll
        for (int h = 0; h < G; h++) {
            float mt = s[0][h];
#pragma unroll
            for (int ks = 1; ks < KS; ks++) mt = fmaxf(mt, s[ks][h]);
            mt = xor_max_above<LPR>(mt);
            const float m_new = fmaxf(m_run[h], mt);
            // m_new == -inf only while every row seen so far is masked.
            alpha[h] = (m_new == -INFINITY) ? 1.0f : fast_exp2(m_run[h] - m_new);
#pragma unroll
            for (int ks = 0; ks < KS; ks++)
                s[ks][h] = (s[ks][h] == -INFINITY) ? 0.0f : fast_exp2(s[ks][h] - m_new);
            m_run[h] = m_new;
        }

        // Probabilities to LDS, [row][head].
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            float pv = s[ks][0];
#pragma unroll
            for (int h = 1; h < G; h++) pv = (kj == h) ? s[ks][h] : pv;
            if (kj < G) p_lds[wave][(ks * RPK + kg) * G + kj] = pv;
        }
        __builtin_amdgcn_wave_barrier();

#pragma unroll
        for (int h = 0; h < G; h++) {
            acc[h].x *= alpha[h];
            acc[h].y *= alpha[h];
            acc[h].z *= alpha[h];
            acc[h].w *= alpha[h];
            l_run[h] *= alpha[h];
        }

        // Weighted V.
#pragma unroll
        for (int vs = 0; vs < VS; vs++) {
            const int r = vs * RPV + vg;
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float p = p_lds[wave][r * G + h];
                acc[h].x += p * vb[vs].x;
                acc[h].y += p * vb[vs].y;
                acc[h].z += p * vb[vs].z;
                acc[h].w += p * vb[vs].w;
                l_run[h] += p;
            }
        }
        __builtin_amdgcn_wave_barrier();
    }

    // Fold the V row groups of the wave, then combine the waves in LDS.
#pragma unroll
    for (int h = 0; h < G; h++) {
        acc[h].x = xor_sum_above<LPV>(acc[h].x);
        acc[h].y = xor_sum_above<LPV>(acc[h].y);
        acc[h].z = xor_sum_above<LPV>(acc[h].z);
        acc[h].w = xor_sum_above<LPV>(acc[h].w);
        l_run[h] = xor_sum_above<LPV>(l_run[h]);
    }
    if (vg == 0) {
#pragma unroll
        for (int h = 0; h < G; h++)
            *reinterpret_cast<float4 *>(&comb_o[wave][h][4 * vj]) = acc[h];
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < G; h++) {
            comb_ml[wave][h][0] = m_run[h];
            comb_ml[wave][h][1] = l_run[h];
        }
    }
    __syncthreads();

    const bool single = (n_chunks == 1);
    for (int idx = tid; idx < G * HD; idx += kThreads) {
        const int h = idx / HD, d = idx % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; w++) M = fmaxf(M, comb_ml[w][h][0]);
        float o = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) {
            const float mw = comb_ml[w][h][0];
            const float sc = (mw == -INFINITY) ? 0.0f : fast_exp2(mw - M);
            o += sc * comb_o[w][h][d];
            L += sc * comb_ml[w][h][1];
        }
        const int qh = kvh * G + h;
        if (single) {
            a.out[(size_t)seq * q_dim + (size_t)qh * HD + d] = o / L;
        } else {
            const size_t row = ((size_t)seq * a.n_heads + qh) * kMaxChunks + chunk_id;
            a.ws_o[row * HD + d] = o;
            if (d == 0) a.ws_ml[row] = make_float2(M, L);
        }
    }
    if (single) return;

    // Arrival: the last chunk of this (sequence, KV head) merges.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        int *ctr = a.counters + (size_t)seq * a.n_kv_heads + kvh;
        const int prev = atomicAdd(ctr, 1);
        s_last = (prev == n_chunks - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();

    for (int h = wave; h < G; h += kWaves) {
        const int qh = kvh * G + h;
        const size_t row0 = ((size_t)seq * a.n_heads + qh) * kMaxChunks;
        const float2 *ml = a.ws_ml + row0;
        float M = -INFINITY;
        for (int c = lane; c < n_chunks; c += kWave) M = fmaxf(M, ml[c].x);
        M = xor_max_above<1>(M);
        float L = 0.f;
        for (int c = lane; c < n_chunks; c += kWave) {
            const float2 mlc = ml[c];
            const float mc = mlc.x, lc = mlc.y;
            const float w = fast_exp2(mc - M);
            merge_w[wave][c] = w;
            L += w * lc;
        }
        L = xor_sum_above<1>(L);
        __builtin_amdgcn_wave_barrier();
        const float inv_L = 1.0f / L;
        constexpr int DPL = HD / kWave;  // dims per lane
        float o[DPL];
#pragma unroll
        for (int i = 0; i < DPL; i++) o[i] = 0.f;
        const float *po = a.ws_o + row0 * HD;
        for (int c = 0; c < n_chunks; c++) {
            const float w = merge_w[wave][c];
#pragma unroll
            for (int i = 0; i < DPL; i++)
                o[i] += w * po[(size_t)c * HD + lane + i * kWave];
        }
#pragma unroll
        for (int i = 0; i < DPL; i++)
            a.out[(size_t)seq * q_dim + (size_t)qh * HD + lane + i * kWave] = o[i] * inv_L;
        __builtin_amdgcn_wave_barrier();
    }
    if (tid == 0) a.counters[(size_t)seq * a.n_kv_heads + kvh] = 0;
}

// ---- synthetic data ---------------------------------------------------------

__device__ __forceinline__ uint64_t splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Two N(0,1) values per counter (Box-Muller on two 24-bit uniforms).
__global__ void fill_normal_kernel(float *dst, size_t n, uint64_t seed, float scale)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x * 2;
    for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 2; i < n; i += stride) {
        const uint64_t r = splitmix64(seed ^ splitmix64(i));
        const float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
        const float u2 = (float)((r >> 16) & 0xFFFFFF) * (1.0f / 16777216.0f);
        const float rad = sqrtf(-2.0f * logf(u1)) * scale;
        float sn, cs;
        sincosf(6.28318530717958647692f * u2, &sn, &cs);
        dst[i] = rad * cs;
        if (i + 1 < n) dst[i + 1] = rad * sn;
    }
}

}  // namespace leap
