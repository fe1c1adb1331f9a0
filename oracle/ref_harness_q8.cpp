// ORACLE — test infrastructure only.
//
// A thin C driver around the reference's own QuantizedTransformer, compiled
// together with the reference source file where it lies (see
// oracle/Makefile); the product never links it.  It exposes the reference's
// activation quantizer and W8A8 matmul (src/inference/QuantizedTransformer.cpp:
// 338-357 and :359-652) and runs its run_layer (:654-...) on synthetic state,
// so that the restatement in attn_oracle.c can be checked against the real
// code.
//
// The layer is given its rms_att, wq, wk, wv and wo (int8 values plus one
// float scale per group, the reference's QuantizedTensor) and an all-zero FFN
// (int8 values and scales 0): the FFN then adds exactly 0 to x, so x after
// run_layer is x + wo . attention(...), the quantized engine's attention
// sub-block with its residual.
#include <cstdint>
#include <cstring>
#include <iostream>
#include <memory>
#include <chrono>
#include <stdexcept>
#include <vector>
#include <sys/mman.h>

// quantize, matmul, run_layer and the run state are private members of the
// reference class; this test driver opens them up for itself only.
#define private public
#include "QuantizedTransformer.h"
#undef private

using Inference::Config;
using Inference::QuantizedTensor;
using Inference::QuantizedTransformer;

namespace {

struct Blob {
    std::vector<uint8_t> buf;
    size_t at = 0;
    float *f32(size_t n)
    {
        float *p = reinterpret_cast<float *>(buf.data() + at);
        at += 4 * n;
        return p;
    }
    int8_t *i8(size_t n)
    {
        int8_t *p = reinterpret_cast<int8_t *>(buf.data() + at);
        at += n;
        return p;
    }
};

struct LayerQ8 {  // one layer's attention weights, int8 values + per-group scales
    const float *rms_att;
    const int8_t *wq_q, *wk_q, *wv_q, *wo_q;
    const float *wq_s, *wk_s, *wv_s, *wo_s;
};

Config make_config(int dim, int n_heads, int n_kv_heads, int n_layers, int seq_len, int gs)
{
    Config c{};
    c.dim = dim;
    c.hidden_dim = gs;  // the smallest FFN the matmul's group loop covers
    c.n_layers = n_layers;
    c.n_heads = n_heads;
    c.n_kv_heads = n_kv_heads;
    c.vocab_size = 1;
    c.seq_len = seq_len;
    return c;
}

// Lay out a weight blob in the order QuantizedTransformer::memory_map_weights
// carves it (QuantizedTransformer.cpp:102-134, each tensor's int8 values
// followed by its scales, init_quantized_tensors :88-100), with a shared
// classifier, unit rms weights, and zeros elsewhere; `lw` (if given) fills
// layer `layer`'s rms_att and attention weights.
std::unique_ptr<QuantizedTransformer> make_engine(const Config &c, int gs, Blob &b, int layer = -1,
                                                  const LayerQ8 *lw = nullptr)
{
    const size_t dim = c.dim, L = c.n_layers, hd = c.dim / c.n_heads;
    const size_t kv_dim = (size_t)c.n_kv_heads * hd, hid = c.hidden_dim;
    const size_t per[7] = {dim * dim, dim * kv_dim, dim * kv_dim, dim * dim, dim * hid, hid * dim, dim * hid};
    size_t attn_bytes = 0, ffn_bytes = 0;
    for (size_t t = 0; t < 7; t++) (t < 4 ? attn_bytes : ffn_bytes) += L * (per[t] + 4 * (per[t] / gs));
    const size_t head_bytes = 4 * (2 * L * dim + dim) + (size_t)c.vocab_size * dim + 4 * (c.vocab_size * dim / gs);
    b.buf.assign(head_bytes + attn_bytes + ffn_bytes, 0);  // the FFN stays all zero
    b.at = 0;
    float *rms = b.f32(2 * L * dim + dim);
    for (size_t i = 0; i < 2 * L * dim + dim; i++) rms[i] = 1.0f;
    if (lw) std::memcpy(rms + (size_t)layer * dim, lw->rms_att, 4 * dim);
    b.i8((size_t)c.vocab_size * dim);
    b.f32((size_t)c.vocab_size * dim / gs);
    const int8_t *src_q[4] = {lw ? lw->wq_q : nullptr, lw ? lw->wk_q : nullptr, lw ? lw->wv_q : nullptr,
                              lw ? lw->wo_q : nullptr};
    const float *src_s[4] = {lw ? lw->wq_s : nullptr, lw ? lw->wk_s : nullptr, lw ? lw->wv_s : nullptr,
                             lw ? lw->wo_s : nullptr};
    for (size_t t = 0; t < 4; t++) {
        for (size_t l = 0; l < L; l++) {
            int8_t *q = b.i8(per[t]);
            float *s = b.f32(per[t] / gs);
            if (lw && (int)l == layer) {
                std::memcpy(q, src_q[t], per[t]);
                std::memcpy(s, src_s[t], 4 * (per[t] / gs));
            }
        }
    }
    if (b.at != head_bytes + attn_bytes) throw std::runtime_error("blob layout");
    return std::make_unique<QuantizedTransformer>(c, -1, MAP_FAILED, 0, b.buf.data(), 1, gs);
}

struct BlockTimer {
    Blob b;
    std::unique_ptr<QuantizedTransformer> eng;
    int n_layers = 1, next = 0;
};

}  // namespace

extern "C" {

// The reference's activation quantizer (QuantizedTransformer.cpp:338-357):
// q[n] int8 values, s[ceil(n/gs)] scales.
int leapref_q8_quantize(const float *x, int n, int gs, int8_t *q, float *s)
{
    try {
        Blob b;
        auto eng = make_engine(make_config(gs, 1, 1, 1, 1, gs), gs, b);
        QuantizedTensor t{q, s};
        eng->quantize(&t, x, n);
        return 0;
    } catch (const std::exception &e) {
        std::cerr << "leapref_q8_quantize: " << e.what() << "\n";
        return -1;
    }
}

// The reference's W8A8 matmul (QuantizedTransformer.cpp:359-652):
// xout[d] = W (d x n, int8 + per-group scales) . x (int8 + per-group scales).
int leapref_q8_matmul(float *xout, const int8_t *xq, const float *xs, const int8_t *wq, const float *ws, int n,
                      int d, int gs)
{
    try {
        Blob b;
        auto eng = make_engine(make_config(gs, 1, 1, 1, 1, gs), gs, b);
        const QuantizedTensor x{const_cast<int8_t *>(xq), const_cast<float *>(xs)};
        const QuantizedTensor w{const_cast<int8_t *>(wq), const_cast<float *>(ws)};
        eng->matmul(xout, &x, &w, n, d);
        return 0;
    } catch (const std::exception &e) {
        std::cerr << "leapref_q8_matmul: " << e.what() << "\n";
        return -1;
    }
}

// run_layer(layer, pos, x) of the quantized engine with the given attention
// weights and a zero FFN: x is updated in place to x + wo . attention(...).
// key_cache/value_cache [n_layers][seq_len][kv_dim]: in, the prior state;
// out, the reference's state after the call.
int leapref_q8_block(int dim, int n_heads, int n_kv_heads, int n_layers, int seq_len, int gs, int layer, int pos,
                     const float *rms_att, const int8_t *wq_q, const float *wq_s, const int8_t *wk_q,
                     const float *wk_s, const int8_t *wv_q, const float *wv_s, const int8_t *wo_q,
                     const float *wo_s, float *key_cache, float *value_cache, float *x)
{
    try {
        const Config c = make_config(dim, n_heads, n_kv_heads, n_layers, seq_len, gs);
        const size_t kv_dim = (size_t)n_kv_heads * (dim / n_heads);
        const size_t cache_n = (size_t)n_layers * seq_len * kv_dim;
        const LayerQ8 lw{rms_att, wq_q, wk_q, wv_q, wo_q, wq_s, wk_s, wv_s, wo_s};
        Blob b;
        auto eng = make_engine(c, gs, b, layer, &lw);
        if (eng->state.key_cache.size() != cache_n) throw std::runtime_error("cache size");
        std::memcpy(eng->state.key_cache.data(), key_cache, sizeof(float) * cache_n);
        std::memcpy(eng->state.value_cache.data(), value_cache, sizeof(float) * cache_n);
        eng->run_layer(layer, pos, x);
        std::memcpy(key_cache, eng->state.key_cache.data(), sizeof(float) * cache_n);
        std::memcpy(value_cache, eng->state.value_cache.data(), sizeof(float) * cache_n);
        return 0;
    } catch (const std::exception &e) {
        std::cerr << "leapref_q8_block: " << e.what() << "\n";
        return -1;
    }
}

// For timing the reference's int8 sub-block on the host: an engine of
// n_layers layers, each holding copies of the given weights at its own
// addresses (cycling through them streams the weights from memory, as a real
// engine does), a zero FFN of hidden size gs, and cache rows [0, rows) set
// from key_rows/value_rows ([rows][kv_dim]).  NULL on failure.
void *leapref_q8_block_timer_create(int dim, int n_heads, int n_kv_heads, int seq_len, int n_layers, int gs,
                                    const float *rms_att, const int8_t *wq_q, const float *wq_s, const int8_t *wk_q,
                                    const float *wk_s, const int8_t *wv_q, const float *wv_s, const int8_t *wo_q,
                                    const float *wo_s, const float *key_rows, const float *value_rows, int rows)
{
    try {
        const Config c = make_config(dim, n_heads, n_kv_heads, n_layers, seq_len, gs);
        const LayerQ8 lw{rms_att, wq_q, wk_q, wv_q, wo_q, wq_s, wk_s, wv_s, wo_s};
        auto t = std::make_unique<BlockTimer>();
        t->eng = make_engine(c, gs, t->b, 0, &lw);
        const size_t d = dim, kv = (size_t)n_kv_heads * (dim / n_heads);
        auto &W = t->eng->weights;
        const size_t per[4] = {d * d, kv * d, kv * d, d * d};
        std::vector<QuantizedTensor> *ts[4] = {&W.wq, &W.wk, &W.wv, &W.wo};
        for (int l = 1; l < n_layers; l++) {  // the blob is ours: copy layer 0's tensors
            std::memcpy(W.rms_att_weight + l * d, W.rms_att_weight, sizeof(float) * d);
            for (int k = 0; k < 4; k++) {
                std::memcpy((*ts[k])[l].q, (*ts[k])[0].q, per[k]);
                std::memcpy((*ts[k])[l].s, (*ts[k])[0].s, sizeof(float) * (per[k] / gs));
            }
        }
        for (int l = 0; l < n_layers; l++) {
            const size_t off = (size_t)l * seq_len * kv;
            std::memcpy(t->eng->state.key_cache.data() + off, key_rows, sizeof(float) * rows * kv);
            std::memcpy(t->eng->state.value_cache.data() + off, value_rows, sizeof(float) * rows * kv);
        }
        t->n_layers = n_layers;
        return t.release();
    } catch (const std::exception &e) {
        std::cerr << "leapref_q8_block_timer_create: " << e.what() << "\n";
        return nullptr;
    }
}

// run_layer(l, pos, x) `iters` times, l cycling through the layers; the mean
// seconds per call.
double leapref_q8_block_timer_run(void *timer, int pos, float *x, int iters)
{
    auto *t = static_cast<BlockTimer *>(timer);
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < iters; i++) {
        t->eng->run_layer(t->next, pos, x);
        t->next = (t->next + 1) % t->n_layers;
    }
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() / iters;
}

void leapref_q8_block_timer_destroy(void *timer) { delete static_cast<BlockTimer *>(timer); }

}  // extern "C"
