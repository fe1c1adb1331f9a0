/*
 * ORACLE — test infrastructure only.
 *
 * CPU restatement of LEAP's per-token decode-attention block (RoPE on q/k,
 * key/value cache append, GQA score pass, softmax, weighted-V accumulation).
 * Only the test suite, the smoke check and the CPU-baseline leg of the
 * benchmark load this library, always as the thing the HIP path is checked
 * against or compared with.  The product library never links or calls it.
 *
 * Every function follows the reference file:line it cites
 * (src/inference/FloatTransformer.cpp; the quantized engine repeats the same
 * fp32 block in src/inference/QuantizedTransformer.cpp:654-923).
 *
 * Deliberate differences from the reference, each one a parameter the
 * reference hard-codes or a range it cannot reach:
 *   - RoPE theta is an argument (the reference fixes 500000,
 *     FloatTransformer.cpp:65); with theta == 500000 the table expression is
 *     the reference's own constant-base expression.
 *   - cache offsets are 64-bit (the reference's int offsets,
 *     FloatTransformer.cpp:50 and :396, overflow at 2^31 elements).
 *   - one call covers one (sequence, layer, position); the caller passes the
 *     sequence's cache slab [n_layers][seq_len][kv_dim].
 *
 * Build flags are the reference's release flags (CMakeLists.txt:33):
 * -O3 -ffast-math -funroll-loops -fopenmp, with an AVX2+FMA target.
 *
 * How each function is pinned (checks live in tests/):
 *   oracle_rope_table     bitwise against the reference's own table
 *                         (oracle/_ref harness), cos=1/sin=0 at pos 0,
 *                         freq_0 = 1, cos^2+sin^2 = 1.
 *   oracle_rmsnorm,       bitwise against the reference's own rmsnorm and
 *   oracle_matmul         matmul (oracle/_ref harness, committed golden
 *                         fixtures); closed forms: a constant vector
 *                         normalises to w / sqrt(1 + 1e-5/c^2) * sign, an
 *                         identity matrix returns x, a one-hot x returns a
 *                         column of W, linearity in x.
 *   oracle_quantize,      bitwise against the reference's own quantize and
 *   oracle_matmul_q8      W8A8 matmul (oracle/_ref q8 harness, committed
 *                         golden fixtures); closed forms: the group maximum
 *                         maps to +-127, exact halves round away from zero,
 *                         an all-zero group has scale 0, dequantised values
 *                         lie within scale/2 of x; the matmul equals the
 *                         float64 sum of exact integer group dots times the
 *                         scales to within float rounding, one-hot x returns
 *                         a dequantised column.
 *   oracle_attention_step against the reference's run_layer (oracle/_ref
 *                         harness, committed golden fixtures), float64
 *                         brute force on tiny shapes, and closed forms
 *                         (T=1 returns v, equal keys give mean(V), a
 *                         dominant key returns its value row, position
 *                         permutation invariance, pos 0 RoPE identity).
 */
#include <immintrin.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <omp.h>

typedef float v8f __attribute__((vector_size(32), aligned(4)));

/* FloatTransformer.cpp:56-72 (QuantizedTransformer.cpp:65-81).
 * freq_i = 1 / theta^(i/head_size) for even i, angle = (float)pos * freq_i,
 * tables are [seq_len][head_size/2] fp32.  The 500000 branch keeps the base a
 * compile-time constant exactly as the reference writes it, so the compiler
 * folds the power the same way it does for the reference. */
void oracle_rope_table(int seq_len, int head_size, float theta, float *cos_tab, float *sin_tab)
{
    const int half = head_size / 2;
    for (int pos = 0; pos < seq_len; pos++) {
        for (int i = 0; i < head_size; i += 2) {
            float freq;
            if (theta == 500000.0f)
                freq = 1.0f / powf(500000.0f, (float)i / (float)head_size);
            else
                freq = 1.0f / powf(theta, (float)i / (float)head_size);
            const float val = (float)pos * freq;
            const size_t idx = (size_t)pos * half + (size_t)(i / 2);
            cos_tab[idx] = cosf(val);
            sin_tab[idx] = sinf(val);
        }
    }
}

/* One interleaved pair rotation, FloatTransformer.cpp:446-493.  The
 * reference's AVX2 body multiplies and then add/subtracts without fusing
 * (mul, mul, addsub at :461-464), so contraction is switched off here. */
__attribute__((optimize("fp-contract=off")))
static void rope_rotate(float *x, const float *c, const float *s, int head_size)
{
    for (int j = 0; j < head_size; j += 2) {
        const float fcr = c[j / 2];
        const float fci = s[j / 2];
        const float x0 = x[j];
        const float x1 = x[j + 1];
        const float a = x0 * fcr;
        const float b = x1 * fci;
        const float d = x1 * fcr;
        const float e = x0 * fci;
        x[j] = a - b;
        x[j + 1] = d + e;
    }
}

/* Horizontal sum in the reference's order (hsum lambda,
 * FloatTransformer.cpp:546-552): fold the upper four lanes onto the lower
 * four, then two pairwise adds. */
static inline float hsum8(v8f v)
{
    const float b0 = v[0] + v[4], b1 = v[1] + v[5], b2 = v[2] + v[6], b3 = v[3] + v[7];
    return (b0 + b1) + (b2 + b3);
}

/* a.b with one chain of eight-lane fused multiply-adds and the reference's
 * horizontal sum, then the scalar tail for lengths that are not a multiple of
 * 8 (the q.k dots of FloatTransformer.cpp:516-630 and every row of matmul,
 * :240-382).  Written with the reference's own intrinsics: a generic-vector
 * accumulator would let -ffast-math -funroll-loops split the chain into
 * several partial sums, which changes the rounding. */
static inline float dot_ref(const float *q, const float *k, int n)
{
    __m256 acc = _mm256_setzero_ps();
    int i = 0;
    for (; i <= n - 8; i += 8)
        acc = _mm256_fmadd_ps(_mm256_loadu_ps(q + i), _mm256_loadu_ps(k + i), acc);
    __m128 lo = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    lo = _mm_hadd_ps(lo, lo);
    lo = _mm_hadd_ps(lo, lo);
    float s = _mm_cvtss_f32(lo);
    for (; i < n; i++)
        s += q[i] * k[i];
    return s;
}

/* FloatTransformer.cpp:79-213 (the AVX2 path): ss = sum of x^2 with eight
 * lane FMA accumulators and the reference's horizontal sum, then the scalar
 * tail; ss = ss / size + 1e-5; the hardware reciprocal-square-root estimate
 * refined by one Newton step, (0.5 * est) * (3 - ss * est^2); o = w * (ss * x). */
void oracle_rmsnorm(float *o, const float *x, const float *w, int size)
{
    v8f acc = {0, 0, 0, 0, 0, 0, 0, 0};
    int j = 0;
    for (; j <= size - 8; j += 8) {
        v8f v;
        memcpy(&v, x + j, sizeof v);
        acc = v * v + acc;
    }
    float ss = hsum8(acc);
    for (; j < size; j++)
        ss += x[j] * x[j];
    ss /= (float)size;
    ss += 1e-5f;
    const __m128 sv = _mm_set_ss(ss);
    __m128 est = _mm_rsqrt_ss(sv);
    const __m128 term = _mm_sub_ss(_mm_set_ss(3.0f), _mm_mul_ss(sv, _mm_mul_ss(est, est)));
    est = _mm_mul_ss(_mm_mul_ss(_mm_set_ss(0.5f), est), term);
    ss = _mm_cvtss_f32(est);
    for (j = 0; j < size; j++)
        o[j] = w[j] * (ss * x[j]);
}

/* FloatTransformer.cpp:240-382: W (d,n) @ x (n,) -> xout (d,), row-major W.
 * Each row is a dot product with eight lane FMA accumulators, the reference's
 * horizontal sum and the scalar tail (its 8-row blocking changes no row's
 * sums); OpenMP over rows. */
void oracle_matmul(float *xout, const float *x, const float *w, int n, int d)
{
#pragma omp parallel for schedule(static)
    for (int i = 0; i < d; i++)
        xout[i] = dot_ref(w + (size_t)i * n, x, n);
}

/* QuantizedTransformer.cpp:338-357.  Per group of gs values (the last group
 * may be shorter): scale = max|x| / 127, id = 1 / scale (0 for an all-zero
 * group), q = round-half-away-from-zero(x * id).  The reference's release
 * flags (-ffast-math: reciprocal-math) turn the division by the constant 127
 * into a product with its float reciprocal; the restatement writes that
 * product out so that the scales agree bit for bit. */
void oracle_quantize(const float *x, int n, int gs, int8_t *q, float *s)
{
    for (int i = 0; i < n; i += gs) {
        const int cur = gs < n - i ? gs : n - i;
        float max_val = 0.0f;
        for (int j = 0; j < cur; j++) {
            const float a = fabsf(x[i + j]);
            if (a > max_val) max_val = a;
        }
        const float scale = max_val * (1.0f / 127.0f);
        const float id = scale != 0.0f ? 1.0f / scale : 0.0f;
        s[i / gs] = scale;
        for (int j = 0; j < cur; j++) q[i + j] = (int8_t)roundf(x[i + j] * id);
    }
}

/* QuantizedTransformer.cpp:359-652.  xout[i] = sum over the whole groups g of
 * row i, in order, of idot_g * (ws_g * sx_g): the int8 dot product of a
 * group is exact in int32 (the reference's madd/add tree or dot-product
 * instructions give the same integer), and the float accumulation is one
 * fused multiply-add per group, val = fma((float)idot, ws * sx, val).  That is
 * how the reference's release build evaluates `val += (float)ival * ws * sx`
 * (-ffast-math reassociates the product and contracts the sum; measured
 * bitwise against the compiled reference).  The weight scale of (row i,
 * column j) is ws[(i*n + j) / gs], elements past the last whole group of a
 * row are not used (the reference's loop bound j <= n - gs). */
void oracle_matmul_q8(float *xout, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws, int n,
                      int d, int gs)
{
#pragma omp parallel for schedule(static)
    for (int i = 0; i < d; i++) {
        const size_t in = (size_t)i * n;
        float val = 0.0f;
        for (int j = 0; j <= n - gs; j += gs) {
            int32_t ival = 0;
            for (int k = 0; k < gs; k++) ival += (int32_t)xq[j + k] * (int32_t)wq[in + j + k];
            val = fmaf((float)ival, ws[(in + j) / gs] * xs[j / gs], val);
        }
        xout[i] = val;
    }
}

/* FloatTransformer.cpp:216-238: max seeded with x[0], exp(x - max), sum,
 * multiply by the reciprocal of the sum. */
static void softmax_ref(float *x, int size)
{
    float max_val = x[0];
    for (int i = 1; i < size; i++)
        if (x[i] > max_val)
            max_val = x[i];
    float sum = 0.0f;
    for (int i = 0; i < size; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    const float inv_sum = 1.0f / sum;
    for (int i = 0; i < size; i++)
        x[i] *= inv_sum;
}

/*
 * One decode-attention step (FloatTransformer.cpp:396-662).
 *
 * key_cache / value_cache : this sequence's slab, [n_layers][seq_len][kv_dim]
 * cos_tab / sin_tab       : oracle_rope_table output, [seq_len][head_size/2]
 * q                       : in: pre-RoPE q [n_heads*head_size]; out: rotated
 * k_new / v_new           : pre-RoPE k, v [kv_dim] (the GEMV outputs the
 *                           reference writes straight into cache[l][pos])
 * att                     : scratch, at least n_heads*(pos+1) floats
 * out                     : [n_heads*head_size], the reference's s->xb
 * Returns 0, or -1 for arguments the reference would never pass.
 */
int oracle_attention_step(int n_heads, int n_kv_heads, int head_size, int seq_len,
                          int layer, int pos, float *key_cache, float *value_cache,
                          const float *cos_tab, const float *sin_tab, float *q,
                          const float *k_new, const float *v_new, float *att, float *out)
{
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_size <= 0 ||
        (head_size & 1) || pos < 0 || pos >= seq_len || layer < 0)
        return -1;
    const int kv_dim = n_kv_heads * head_size;
    const int kv_mul = n_heads / n_kv_heads;
    const int T = pos + 1;

    /* :396-402: the k and v GEMV outputs land in cache[l][pos]. */
    const size_t loff = (size_t)layer * (size_t)seq_len * (size_t)kv_dim;
    float *k = key_cache + loff + (size_t)pos * kv_dim;
    float *v = value_cache + loff + (size_t)pos * kv_dim;
    memcpy(k, k_new, sizeof(float) * (size_t)kv_dim);
    memcpy(v, v_new, sizeof(float) * (size_t)kv_dim);

    /* :404-494: rotate every q head, and the k heads (i < n_kv_heads) in the
     * cache slot, with table row pos. */
    const float *c = cos_tab + (size_t)pos * (head_size / 2);
    const float *s = sin_tab + (size_t)pos * (head_size / 2);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n_heads; i++) {
        rope_rotate(q + (size_t)i * head_size, c, s, head_size);
        if (i < n_kv_heads)
            rope_rotate(k + (size_t)i * head_size, c, s, head_size);
    }

    /* :497, scale applied after the dot. */
    const float att_scale = 1.0f / sqrtf((float)head_size);

    /* :499-662: per head, score over t = 0..pos, softmax, weighted V. */
#pragma omp parallel for schedule(static)
    for (int h = 0; h < n_heads; h++) {
        const float *qh = q + (size_t)h * head_size;
        float *a = att + (size_t)h * T;
        const size_t hoff = (size_t)(h / kv_mul) * head_size;
        for (int t = 0; t < T; t++) {
            const float *kt = key_cache + loff + (size_t)t * kv_dim + hoff;
            a[t] = dot_ref(qh, kt, head_size) * att_scale;
        }
        softmax_ref(a, T);
        float *xb = out + (size_t)h * head_size;
        memset(xb, 0, sizeof(float) * (size_t)head_size);
        for (int t = 0; t < T; t++) {
            const float *vt = value_cache + loff + (size_t)t * kv_dim + hoff;
            const float at = a[t];
            int i = 0;
            for (; i <= head_size - 8; i += 8) {
                v8f xv, vv;
                memcpy(&xv, xb + i, sizeof xv);
                memcpy(&vv, vt + i, sizeof vv);
                xv = at * vv + xv;
                memcpy(xb + i, &xv, sizeof xv);
            }
            for (; i < head_size; i++)
                xb[i] += at * vt[i];
        }
    }
    return 0;
}

/* FloatTransformer.cpp:74-77: zero both caches. */
void oracle_clear(float *key_cache, float *value_cache, size_t n_floats)
{
    memset(key_cache, 0, n_floats * sizeof(float));
    memset(value_cache, 0, n_floats * sizeof(float));
}

void oracle_set_threads(int n)
{
    if (n > 0)
        omp_set_num_threads(n);
}

int oracle_max_threads(void)
{
    return omp_get_max_threads();
}

/* Deliberately wrong variants, used only by the tests that show each pin
 * catches a plausible mistake.  mode 1: RoPE with (2j, 2j+1) sign swapped;
 * mode 2: GQA head map h % n_kv_heads instead of h / kv_mul; mode 3: score
 * scale dropped. */
int oracle_attention_step_mutant(int mode, int n_heads, int n_kv_heads, int head_size,
                                 int seq_len, int layer, int pos, float *key_cache,
                                 float *value_cache, const float *cos_tab,
                                 const float *sin_tab, float *q, const float *k_new,
                                 const float *v_new, float *att, float *out)
{
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads || head_size <= 0 ||
        (head_size & 1) || pos < 0 || pos >= seq_len || layer < 0)
        return -1;
    const int kv_dim = n_kv_heads * head_size;
    const int kv_mul = n_heads / n_kv_heads;
    const int T = pos + 1;
    const size_t loff = (size_t)layer * (size_t)seq_len * (size_t)kv_dim;
    float *k = key_cache + loff + (size_t)pos * kv_dim;
    float *v = value_cache + loff + (size_t)pos * kv_dim;
    memcpy(k, k_new, sizeof(float) * (size_t)kv_dim);
    memcpy(v, v_new, sizeof(float) * (size_t)kv_dim);
    const float *c = cos_tab + (size_t)pos * (head_size / 2);
    const float *s = sin_tab + (size_t)pos * (head_size / 2);
    for (int i = 0; i < n_heads; i++) {
        float *x = q + (size_t)i * head_size;
        for (int r = 0; r < (i < n_kv_heads ? 2 : 1); r++) {
            if (r == 1)
                x = k + (size_t)i * head_size;
            for (int j = 0; j < head_size; j += 2) {
                const float x0 = x[j], x1 = x[j + 1];
                const float cc = c[j / 2], ss = s[j / 2];
                if (mode == 1) {
                    x[j] = x0 * cc + x1 * ss;
                    x[j + 1] = x1 * cc - x0 * ss;
                } else {
                    x[j] = x0 * cc - x1 * ss;
                    x[j + 1] = x0 * ss + x1 * cc;
                }
            }
        }
    }
    const float att_scale = mode == 3 ? 1.0f : 1.0f / sqrtf((float)head_size);
    for (int h = 0; h < n_heads; h++) {
        const float *qh = q + (size_t)h * head_size;
        float *a = att + (size_t)h * T;
        const int kvh = mode == 2 ? h % n_kv_heads : h / kv_mul;
        const size_t hoff = (size_t)kvh * head_size;
        for (int t = 0; t < T; t++)
            a[t] = dot_ref(qh, key_cache + loff + (size_t)t * kv_dim + hoff, head_size) * att_scale;
        softmax_ref(a, T);
        float *xb = out + (size_t)h * head_size;
        memset(xb, 0, sizeof(float) * (size_t)head_size);
        for (int t = 0; t < T; t++) {
            const float *vt = value_cache + loff + (size_t)t * kv_dim + hoff;
            for (int i = 0; i < head_size; i++)
                xb[i] += a[t] * vt[i];
        }
    }
    return 0;
}
