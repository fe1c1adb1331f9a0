// ORACLE — test infrastructure only.
//
// A thin C driver around the reference's own checkpoint loader, compiled
// together with the reference sources where they lie (see oracle/Makefile);
// the product never links it.  It builds the engine from a .bin file with
// Transformer::create (src/inference/TransformerFactory.cpp:59-135, which
// memory-maps the weights in memory_map_weights' order) and runs one
// run_layer on given cache state, so that checkpoint files written by the
// tests can be shown to carry their tensors where the reference reads them.
#include <cstring>
#include <iostream>
#include <memory>
#include <stdexcept>

// run_layer and the run state are private members of the reference classes;
// this test driver opens them up for itself only.
#define private public
#include "FloatTransformer.h"
#include "QuantizedTransformer.h"
#include "Transformer.h"
#undef private

namespace {

template <class T>
void run(T *t, int layer, int pos, float *x, float *key_cache, float *value_cache)
{
    const size_t n = t->state.key_cache.size();
    std::memcpy(t->state.key_cache.data(), key_cache, sizeof(float) * n);
    std::memcpy(t->state.value_cache.data(), value_cache, sizeof(float) * n);
    t->run_layer(layer, pos, x);
    std::memcpy(key_cache, t->state.key_cache.data(), sizeof(float) * n);
    std::memcpy(value_cache, t->state.value_cache.data(), sizeof(float) * n);
}

}  // namespace

extern "C" {

// run_layer(layer, pos, x) of the engine Transformer::create builds from
// `path`; key_cache/value_cache are [n_layers][seq_len][kv_dim] of the file's
// Config, in: the prior state, out: the state after the call.  Returns 1 for
// an fp32 engine, 2 for an int8 engine, -1 on failure.
int leapref_ckpt_run_layer(const char *path, int layer, int pos, float *x, float *key_cache, float *value_cache)
{
    try {
        auto t = Inference::Transformer::create(path);
        if (auto *f = dynamic_cast<Inference::FloatTransformer *>(t.get())) {
            run(f, layer, pos, x, key_cache, value_cache);
            return 1;
        }
        if (auto *q = dynamic_cast<Inference::QuantizedTransformer *>(t.get())) {
            run(q, layer, pos, x, key_cache, value_cache);
            return 2;
        }
        return -1;
    } catch (const std::exception &e) {
        std::cerr << "leapref_ckpt_run_layer: " << e.what() << "\n";
        return -1;
    }
}

}  // extern "C"
