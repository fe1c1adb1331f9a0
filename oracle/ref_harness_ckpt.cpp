// ORACLE — test infrastructure only.
//
// A thin C driver around the reference's own checkpoint loader, compiled
// together with the reference sources where they lie (see oracle/Makefile);
// the product never links it.  It builds the engine from a .bin file with
// Transformer::create (src/inference/TransformerFactory.cpp:59-135, which
// memory-maps the weights in memory_map_weights' order) and runs one
// run_layer on given cache state, so that checkpoint files written by the
// tests can be shown to carry their tensors where the reference reads them.
// It also runs the engine's pipeline roles, forward() as the master
// (FloatTransformer.cpp:751-797) and worker_loop() (:799-945), over a
// transport that records what they send and replays given packets, so that
// the wire format and the forward-or-drop rule of the stage hand-off can be
// read off the reference itself.
#include <cstring>
#include <deque>
#include <iostream>
#include <memory>
#include <stdexcept>
#include <vector>

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

// A transport that keeps what is sent and hands out queued packets; when
// the queue is empty recv throws, which ends worker_loop (its catch breaks
// out of the loop, FloatTransformer.cpp:940-943).
struct Recorder : Inference::Transport {
    std::vector<unsigned char> sent;
    size_t sends = 0;
    std::deque<std::vector<unsigned char>> inbox;
    void initialize() override {}
    void send(const void *data, size_t size) override
    {
        const auto *b = static_cast<const unsigned char *>(data);
        sent.insert(sent.end(), b, b + size);
        sends++;
    }
    void recv(void *data, size_t size) override
    {
        if (inbox.empty()) throw std::runtime_error("no more packets");
        if (inbox.front().size() != size) throw std::runtime_error("packet size");
        std::memcpy(data, inbox.front().data(), size);
        inbox.pop_front();
    }
};

void queue(Recorder &r, const unsigned char *packets, int n, size_t bytes)
{
    for (int i = 0; i < n; i++) r.inbox.emplace_back(packets + i * bytes, packets + (i + 1) * bytes);
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

// forward(tokens[i], pos[i], flags[i]) for i < n on the engine built from
// `path`, as the master of a pipeline that runs layers [0, split) itself.
// The packets it sends are written to `sent` (n packets of 8 + 4*dim bytes);
// the forwards that ask for a reply take theirs, in order, from `replies`.
// Returns the number of packets sent, or -1 on failure.
int leapref_ckpt_master(const char *path, int split, int n, const int *tokens, const int *pos, const int *flags,
                        const unsigned char *replies, int n_replies, unsigned char *sent)
{
    try {
        auto t = Inference::Transformer::create(path);
        const size_t bytes = sizeof(Inference::PacketHeader) + sizeof(float) * t->config.dim;
        Recorder r;
        queue(r, replies, n_replies, bytes);
        Inference::DistributedConfig d;
        d.mode = Inference::DistributedMode::Master;
        d.split_layer = split;
        d.transport = &r;
        t->set_distributed_config(d);
        for (int i = 0; i < n; i++) t->forward(tokens[i], pos[i], flags[i]);
        std::memcpy(sent, r.sent.data(), r.sent.size());
        return (int)r.sends;
    } catch (const std::exception &e) {
        std::cerr << "leapref_ckpt_master: " << e.what() << "\n";
        return -1;
    }
}

// worker_loop() of the engine built from `path` for layers [split, end),
// fed the n packets of `in`; what it forwards is written to `out`.  Returns
// the number of packets forwarded, or -1 on failure.
int leapref_ckpt_worker(const char *path, int split, int end, int is_tail, int n, const unsigned char *in,
                        unsigned char *out)
{
    try {
        auto t = Inference::Transformer::create(path);
        const size_t bytes = sizeof(Inference::PacketHeader) + sizeof(float) * t->config.dim;
        Recorder r;
        queue(r, in, n, bytes);
        Inference::DistributedConfig d;
        d.mode = Inference::DistributedMode::Worker;
        d.split_layer = split;
        d.end_layer = end;
        d.is_tail = is_tail != 0;
        d.transport = &r;
        t->set_distributed_config(d);
        t->worker_loop();
        std::memcpy(out, r.sent.data(), r.sent.size());
        return (int)r.sends;
    } catch (const std::exception &e) {
        std::cerr << "leapref_ckpt_worker: " << e.what() << "\n";
        return -1;
    }
}

}  // extern "C"
