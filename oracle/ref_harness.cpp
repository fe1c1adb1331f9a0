// ORACLE — test infrastructure only.
//
// A thin C driver around the reference's own FloatTransformer, compiled
// together with the reference source file where it lies (see
// oracle/Makefile); the product never links it.  It runs the reference's
// run_layer (src/inference/FloatTransformer.cpp:384-749) on synthetic state so
// the restatement in attn_oracle.c can be checked against the real code.
//
// How the attention block is isolated: the layer is given wo = identity,
// rms weights = 1 and zero FFN weights (hidden_dim may be tiny), so
//   s->xb2 = wo . xb = the attention output exactly (an identity GEMV adds
//            one product x*1 to zeros), and
//   cache[l][pos] holds the rotated k after the call.
// The pre-RoPE q, k, v are produced by the reference's own rmsnorm and matmul
// on the same inputs, computed here once before run_layer with the same
// deterministic functions (rmsnorm has no threading, matmul is a static
// OpenMP schedule with one owner per output row).
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <iostream>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>
#include <sys/mman.h>

// run_layer, rmsnorm, matmul and the run state are private members of the
// reference class; this test driver opens them up for itself only.
#include <chrono>

#define private public
#include "FloatTransformer.h"
#undef private

using Inference::Config;
using Inference::FloatTransformer;

namespace {

struct Weights {
    std::vector<float> buf;
};

// Lay out a weight blob in the order FloatTransformer::memory_map_weights
// carves it (FloatTransformer.cpp:947-978) for one layer, with wq/wk/wv given,
// rms_att and wo given or (nullptr) ones and the identity, rms_ffn 1 and zero
// FFN/embedding/classifier.
std::unique_ptr<FloatTransformer> make_engine(const Config &c, const float *wq, const float *wk,
                                              const float *wv, int layer, Weights &w,
                                              const float *rms_att = nullptr, const float *wo = nullptr)
{
    const size_t dim = c.dim, L = c.n_layers, hd = c.dim / c.n_heads;
    const size_t kv_dim = (size_t)c.n_kv_heads * hd;
    const size_t n_att = L * dim, n_ffn = L * dim, n_fin = dim, n_emb = (size_t)c.vocab_size * dim;
    const size_t n_wq = L * dim * dim, n_wk = L * dim * kv_dim, n_wv = n_wk, n_wo = L * dim * dim;
    const size_t n_w1 = L * dim * c.hidden_dim, n_w2 = n_w1, n_w3 = n_w1;
    w.buf.assign(n_att + n_ffn + n_fin + n_emb + n_wq + n_wk + n_wv + n_wo + n_w1 + n_w2 + n_w3, 0.0f);
    float *p = w.buf.data();
    std::fill(p, p + n_att + n_ffn + n_fin, 1.0f);
    float *pwq = p + n_att + n_ffn + n_fin + n_emb;
    float *pwk = pwq + n_wq;
    float *pwv = pwk + n_wk;
    float *pwo = pwv + n_wv;
    std::memcpy(pwq + (size_t)layer * dim * dim, wq, sizeof(float) * dim * dim);
    std::memcpy(pwk + (size_t)layer * dim * kv_dim, wk, sizeof(float) * dim * kv_dim);
    std::memcpy(pwv + (size_t)layer * dim * kv_dim, wv, sizeof(float) * dim * kv_dim);
    float *wo_l = pwo + (size_t)layer * dim * dim;
    if (wo)
        std::memcpy(wo_l, wo, sizeof(float) * dim * dim);
    else
        for (size_t i = 0; i < dim; i++) wo_l[i * dim + i] = 1.0f;
    if (rms_att) std::memcpy(p + (size_t)layer * dim, rms_att, sizeof(float) * dim);
    return std::make_unique<FloatTransformer>(c, -1, MAP_FAILED, 0, w.buf.data(), 1);
}

struct BlockTimer {
    Weights w;
    std::unique_ptr<FloatTransformer> eng;
    int n_layers = 1, next = 0;
};

Config make_config(int dim, int n_heads, int n_kv_heads, int n_layers, int seq_len)
{
    Config c{};
    c.dim = dim;
    c.hidden_dim = 8;
    c.n_layers = n_layers;
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv_heads;
    c.vocab_size = 1;
    c.seq_len = seq_len;
    return c;
}

}  // namespace

extern "C" {

// The reference's RoPE tables (precompute_freqs, FloatTransformer.cpp:56-72).
int leapref_rope_table(int dim, int n_heads, int seq_len, float *cos_out, float *sin_out)
{
    try {
        Config c = make_config(dim, n_heads, n_heads, 1, seq_len);
        const size_t hd = dim / n_heads;
        std::vector<float> wq((size_t)dim * dim), wk((size_t)dim * dim), wv((size_t)dim * dim);
        Weights w;
        auto eng = make_engine(c, wq.data(), wk.data(), wv.data(), 0, w);
        std::memcpy(cos_out, eng->rope_cos.data(), sizeof(float) * (size_t)seq_len * (hd / 2));
        std::memcpy(sin_out, eng->rope_sin.data(), sizeof(float) * (size_t)seq_len * (hd / 2));
        return 0;
    } catch (const std::exception &e) {
        std::cerr << "leapref_rope_table: " << e.what() << "\n";
        return -1;
    }
}

// Run the reference run_layer(layer, pos, x) once.
//   key_cache/value_cache: [n_layers][seq_len][kv_dim], in: prior state,
//                          out: the reference's state after the call
//   q_pre/k_pre/v_pre:     out, the pre-RoPE projections run_layer computes
//   q_rot:                 out, s->q after the call (rotated q)
//   att_out:               out, s->xb (head-major attention output)
int leapref_run_layer(int dim, int n_heads, int n_kv_heads, int n_layers, int seq_len, int layer,
                      int pos, const float *x_in, const float *wq, const float *wk, const float *wv,
                      float *key_cache, float *value_cache, float *q_pre, float *k_pre,
                      float *v_pre, float *q_rot, float *att_out)
{
    try {
        Config c = make_config(dim, n_heads, n_kv_heads, n_layers, seq_len);
        const size_t hd = dim / n_heads, kv_dim = (size_t)n_kv_heads * hd;
        const size_t cache_n = (size_t)n_layers * seq_len * kv_dim;
        Weights w;
        auto eng = make_engine(c, wq, wk, wv, layer, w);
        if (eng->state.key_cache.size() != cache_n) throw std::runtime_error("cache size");
        std::memcpy(eng->state.key_cache.data(), key_cache, sizeof(float) * cache_n);
        std::memcpy(eng->state.value_cache.data(), value_cache, sizeof(float) * cache_n);

        std::vector<float> x(x_in, x_in + dim), xb(dim);
        FloatTransformer::rmsnorm(xb.data(), x.data(), eng->weights.rms_att_weight + (size_t)layer * dim, dim);
        FloatTransformer::matmul(q_pre, xb.data(), eng->weights.wq + (size_t)layer * dim * dim, dim, dim);
        FloatTransformer::matmul(k_pre, xb.data(), eng->weights.wk + (size_t)layer * dim * kv_dim, dim, (int)kv_dim);
        FloatTransformer::matmul(v_pre, xb.data(), eng->weights.wv + (size_t)layer * dim * kv_dim, dim, (int)kv_dim);

        eng->run_layer(layer, pos, x.data());

        std::memcpy(key_cache, eng->state.key_cache.data(), sizeof(float) * cache_n);
        std::memcpy(value_cache, eng->state.value_cache.data(), sizeof(float) * cache_n);
        std::memcpy(q_rot, eng->state.q.data(), sizeof(float) * dim);
        std::memcpy(att_out, eng->state.xb2.data(), sizeof(float) * dim);
        return 0;
    } catch (const std::exception &e) {
        std::cerr << "leapref_run_layer: " << e.what() << "\n";
        return -1;
    }
}

// The reference's rmsnorm (FloatTransformer.cpp:79-213) and matmul (:240-382).
int leapref_rmsnorm(float *o, const float *x, const float *weight, int size)
{
    FloatTransformer::rmsnorm(o, x, weight, size);
    return 0;
}

int leapref_matmul(float *xout, const float *x, const float *w, int n, int d)
{
    FloatTransformer::matmul(xout, x, w, n, d);
    return 0;
}

// run_layer(layer, pos, x) with the given rms_att, wq, wk, wv and wo of the
// layer and a zero FFN, so that x afterwards is x + wo . attention(...): the
// attention sub-block with its residual (FloatTransformer.cpp:394-683; the
// FFN adds w2 . (silu(w1 . xb) * (w3 . xb)) = 0).  key_cache/value_cache as
// in leapref_run_layer; x is updated in place.
int leapref_block(int dim, int n_heads, int n_kv_heads, int n_layers, int seq_len, int layer, int pos,
                  const float *rms_att, const float *wq, const float *wk, const float *wv, const float *wo,
                  float *key_cache, float *value_cache, float *x)
{
    try {
        Config c = make_config(dim, n_heads, n_kv_heads, n_layers, seq_len);
        const size_t hd = dim / n_heads, kv_dim = (size_t)n_kv_heads * hd;
        const size_t cache_n = (size_t)n_layers * seq_len * kv_dim;
        Weights w;
        auto eng = make_engine(c, wq, wk, wv, layer, w, rms_att, wo);
        if (eng->state.key_cache.size() != cache_n) throw std::runtime_error("cache size");
        std::memcpy(eng->state.key_cache.data(), key_cache, sizeof(float) * cache_n);
        std::memcpy(eng->state.value_cache.data(), value_cache, sizeof(float) * cache_n);
        eng->run_layer(layer, pos, x);
        std::memcpy(key_cache, eng->state.key_cache.data(), sizeof(float) * cache_n);
        std::memcpy(value_cache, eng->state.value_cache.data(), sizeof(float) * cache_n);
        return 0;
    } catch (const std::exception &e) {
        std::cerr << "leapref_block: " << e.what() << "\n";
        return -1;
    }
}

// For timing the reference's sub-block on the host: an engine of n_layers
// layers, each holding the given rms_att, wq, wk, wv, wo (copies at their own
// addresses, so that cycling through the layers streams the weights from
// memory as a real engine does rather than from the CPU caches), a zero FFN
// of hidden size 8 (negligible next to the attention weights), and cache
// rows [0, rows) set from key_rows/value_rows ([rows][kv_dim]).  NULL on
// failure.
void *leapref_block_timer_create(int dim, int n_heads, int n_kv_heads, int seq_len, int n_layers,
                                 const float *rms_att, const float *wq, const float *wk, const float *wv,
                                 const float *wo, const float *key_rows, const float *value_rows, int rows)
{
    try {
        Config c = make_config(dim, n_heads, n_kv_heads, n_layers, seq_len);
        auto t = std::make_unique<BlockTimer>();
        t->eng = make_engine(c, wq, wk, wv, 0, t->w, rms_att, wo);
        const size_t d = dim, kv = (size_t)n_kv_heads * (dim / n_heads);
        auto &W = t->eng->weights;
        for (int l = 1; l < n_layers; l++) {  // the blob is ours: copy layer 0's slices
            std::memcpy(const_cast<float *>(W.rms_att_weight) + l * d, W.rms_att_weight, sizeof(float) * d);
            std::memcpy(const_cast<float *>(W.wq) + l * d * d, W.wq, sizeof(float) * d * d);
            std::memcpy(const_cast<float *>(W.wk) + l * d * kv, W.wk, sizeof(float) * d * kv);
            std::memcpy(const_cast<float *>(W.wv) + l * d * kv, W.wv, sizeof(float) * d * kv);
            std::memcpy(const_cast<float *>(W.wo) + l * d * d, W.wo, sizeof(float) * d * d);
        }
        for (int l = 0; l < n_layers; l++) {
            const size_t off = (size_t)l * seq_len * kv;
            std::memcpy(t->eng->state.key_cache.data() + off, key_rows, sizeof(float) * rows * kv);
            std::memcpy(t->eng->state.value_cache.data() + off, value_rows, sizeof(float) * rows * kv);
        }
        t->n_layers = n_layers;
        return t.release();
    } catch (const std::exception &e) {
        std::cerr << "leapref_block_timer_create: " << e.what() << "\n";
        return nullptr;
    }
}

// run_layer(l, pos, x) `iters` times, l cycling through the layers (x
// updated in place each time); returns the mean seconds per call.
double leapref_block_timer_run(void *timer, int pos, float *x, int iters)
{
    auto *t = static_cast<BlockTimer *>(timer);
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < iters; i++) {
        t->eng->run_layer(t->next, pos, x);
        t->next = (t->next + 1) % t->n_layers;
    }
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() / iters;
}

void leapref_block_timer_destroy(void *timer) { delete static_cast<BlockTimer *>(timer); }

// clear_kv_cache (FloatTransformer.cpp:74-77) on a filled engine; returns the
// number of nonzero floats left in either cache (0 expected).
long leapref_clear_check(int dim, int n_heads, int n_kv_heads, int n_layers, int seq_len)
{
    Config c = make_config(dim, n_heads, n_kv_heads, n_layers, seq_len);
    std::vector<float> wq((size_t)dim * dim), wk((size_t)dim * dim), wv((size_t)dim * dim);
    Weights w;
    auto eng = make_engine(c, wq.data(), wk.data(), wv.data(), 0, w);
    std::fill(eng->state.key_cache.begin(), eng->state.key_cache.end(), 1.0f);
    std::fill(eng->state.value_cache.begin(), eng->state.value_cache.end(), 2.0f);
    eng->clear_kv_cache();
    long nz = 0;
    for (float f : eng->state.key_cache) nz += f != 0.0f;
    for (float f : eng->state.value_cache) nz += f != 0.0f;
    return nz;
}

}  // extern "C"
