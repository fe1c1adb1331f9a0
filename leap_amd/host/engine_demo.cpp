// Minimal engine loop that keeps LEAP's structure around the attention shim.
//
// The reference decodes one token at a time: forward(token, pos) runs
// run_layer(l, pos, x) for every layer (FloatTransformer.cpp:751-770), and
// run_layer projects q/k/v (:394-402), runs the attention block (:404-662) and
// continues with wo and the FFN (:664-748).  This program keeps that loop and
// its RunState-style buffers (q, k, v, xb per FloatTransformer.h:24-37), feeds
// synthetic q/k/v in place of the projections (the GEMVs are outside the
// path) and calls the shim for the attention block of every layer.
//
//   engine_demo n_layers n_heads n_kv_heads head_dim seq_len n_tokens out_dir [block | ckpt PATH]
//
// writes, per (token, layer) in decode order, q|k|v|xb as raw fp32 to
// out_dir/trace.bin so a checker can replay the same steps on a CPU
// implementation.  With `block`, the shim runs run_layer from its start to the
// attention residual (:394-683) instead: the program generates each layer's
// rms_att, wq, wk, wv, wo (written to out_dir/weights.bin in that order, per
// layer), feeds the residual stream x from layer to layer and token to token,
// and writes x before and after every (token, layer) to trace.bin.  With
// `ckpt PATH` the weights come from a LEAP checkpoint file instead (fp32 or
// int8, through the shim's loader; the file's Config must match the
// arguments), and the same trace is written.
// Exit status: 0 success, 2 bad usage, 3 shim error.
#include <cstdio>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <exception>
#include <string>
#include <vector>

#include "hip_attention.hpp"

namespace {

// SplitMix64 -> uniform in [-1, 1) scaled by 1/sqrt(head_dim): stand-in for
// the projection outputs.
struct Rng {
    uint64_t s;
    float next(float scale)
    {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        z ^= z >> 31;
        return ((float)(z >> 40) * (1.0f / 8388608.0f) - 1.0f) * scale;
    }
};

struct RunState {  // the attention-facing part of FloatRunState
    std::vector<float> q, k, v, xb;
};

}  // namespace

int main(int argc, char **argv)
{
    const bool block = argc == 9 && std::string(argv[8]) == "block";
    const bool ckpt = argc == 10 && std::string(argv[8]) == "ckpt";
    if (argc != 8 && !block && !ckpt) {
        std::fprintf(stderr,
                     "usage: %s n_layers n_heads n_kv_heads head_dim seq_len n_tokens out_dir [block | ckpt PATH]\n",
                     argv[0]);
        return 2;
    }
    const int n_layers = std::atoi(argv[1]), n_heads = std::atoi(argv[2]), n_kv = std::atoi(argv[3]);
    const int head_dim = std::atoi(argv[4]), seq_len = std::atoi(argv[5]), n_tokens = std::atoi(argv[6]);
    const std::string out_dir = argv[7];
    if (n_tokens <= 0 || n_tokens > seq_len) {
        std::fprintf(stderr, "n_tokens must be in [1, seq_len]\n");
        return 2;
    }
    try {
        leap::HipAttention attn({n_layers, 0, n_layers, n_heads, n_kv, head_dim, seq_len});
        RunState s;
        const int dim = n_heads * head_dim, kv_dim = n_kv * head_dim;
        s.q.resize(dim);
        s.k.resize(kv_dim);
        s.v.resize(kv_dim);
        s.xb.resize(dim);
        Rng rng{0x4C454150};
        const float scale = 1.0f / std::sqrt((float)head_dim);
        std::FILE *f = std::fopen((out_dir + "/trace.bin").c_str(), "wb");
        if (!f) {
            std::fprintf(stderr, "cannot write %s/trace.bin\n", out_dir.c_str());
            return 2;
        }
        if (ckpt) {  // the weights of every layer from a checkpoint file
            const auto info = leap::HipAttention::checkpoint_read(argv[9]);
            std::printf("engine_demo: checkpoint version %d, %d layers, dim %d\n", info.version, info.n_layers,
                        info.dim);
            attn.load_checkpoint(argv[9]);
            std::vector<float> x(dim);
            for (float &e : x) e = rng.next(1.0f);
            for (int pos = 0; pos < n_tokens; pos++) {
                for (int l = 0; l < n_layers; l++) {
                    std::fwrite(x.data(), 4, x.size(), f);
                    attn.block(l, pos, x);
                    std::fwrite(x.data(), 4, x.size(), f);
                }
            }
            std::fclose(f);
            std::printf("engine_demo: %d tokens x %d layers done (checkpoint)\n", n_tokens, n_layers);
            return 0;
        }
        if (block) {
            std::FILE *wf = std::fopen((out_dir + "/weights.bin").c_str(), "wb");
            if (!wf) {
                std::fclose(f);
                std::fprintf(stderr, "cannot write %s/weights.bin\n", out_dir.c_str());
                return 2;
            }
            const float wscale = 1.0f / std::sqrt((float)dim);
            std::vector<float> rms(dim), wq((size_t)dim * dim), wk((size_t)kv_dim * dim),
                wv((size_t)kv_dim * dim), wo((size_t)dim * dim);
            for (int l = 0; l < n_layers; l++) {  // the layer slices of FloatTransformerWeights
                for (float &w : rms) w = 1.0f + rng.next(0.1f);
                for (auto *m : {&wq, &wk, &wv, &wo})
                    for (float &w : *m) w = rng.next(wscale);
                attn.set_layer_weights(l, rms, wq, wk, wv, wo);
                for (auto *m : {&rms, &wq, &wk, &wv, &wo}) std::fwrite(m->data(), 4, m->size(), wf);
            }
            std::fclose(wf);
            std::vector<float> x(dim);
            for (float &e : x) e = rng.next(1.0f);  // the token embedding row
            for (int pos = 0; pos < n_tokens; pos++) {
                for (int l = 0; l < n_layers; l++) {
                    std::fwrite(x.data(), 4, x.size(), f);
                    attn.block(l, pos, x);  // run_layer :394-683
                    std::fwrite(x.data(), 4, x.size(), f);
                }
            }
            std::fclose(f);
            std::printf("engine_demo: %d tokens x %d layers done (sub-block)\n", n_tokens, n_layers);
            return 0;
        }
        for (int pos = 0; pos < n_tokens; pos++) {      // generate(): one token per step
            for (int l = 0; l < n_layers; l++) {        // forward(): the layer loop
                for (float &x : s.q) x = rng.next(scale);   // stand-ins for the q/k/v GEMVs
                for (float &x : s.k) x = rng.next(scale);
                for (float &x : s.v) x = rng.next(scale);
                attn.step(l, pos, s.q, s.k, s.v, s.xb);  // the attention block of run_layer
                std::fwrite(s.q.data(), 4, s.q.size(), f);
                std::fwrite(s.k.data(), 4, s.k.size(), f);
                std::fwrite(s.v.data(), 4, s.v.size(), f);
                std::fwrite(s.xb.data(), 4, s.xb.size(), f);
            }
        }
        std::fclose(f);
        std::printf("engine_demo: %d tokens x %d layers done\n", n_tokens, n_layers);
        return 0;
    } catch (const std::exception &e) {
        std::fprintf(stderr, "%s\n", e.what());
        return 3;
    }
}
