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
//
//   engine_demo ... out_dir pipeline PATH SPLIT
//
// runs the same checkpoint as a two-node pipeline in one process: a master
// handle holds layers [0, SPLIT) and a tail worker handle [SPLIT, n_layers),
// each keeping its residual stream in device memory.  Per token the master
// runs its layers and sends the packet {pos, flags} + x (FloatTransformer.cpp:
// 775-778); the worker receives it (:925-926), runs its layers and forwards
// it back only when a reply is wanted (:937-939), and the master takes x
// from the reply (:785-788).  Every third token is sent without asking for a
// reply, as a prompt token is.  Per token the trace holds x before the
// master's layers, the packet sent, an int32 that says whether the worker
// forwarded, the packet it forwarded and the master's x after the reply
// (zeros where nothing was forwarded).
// Exit status: 0 success, 2 bad usage, 3 shim error.
#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdio>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <algorithm>
#include <exception>
#include <stdexcept>
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

// Device memory the engine owns for its residual stream.
struct DeviceFloats {
    float *p = nullptr;
    explicit DeviceFloats(size_t n)
    {
        if (hipMalloc((void **)&p, n * sizeof(float)) != hipSuccess) throw std::runtime_error("hipMalloc failed");
    }
    ~DeviceFloats() { (void)hipFree(p); }
    DeviceFloats(const DeviceFloats &) = delete;
    DeviceFloats &operator=(const DeviceFloats &) = delete;
};

void hip_ok(hipError_t e, const char *what)
{
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// The two-node pipeline of the checkpoint at `path` (see the header).
int run_pipeline(int n_layers, int n_heads, int n_kv, int head_dim, int seq_len, int n_tokens, const std::string &path,
                 int split, std::FILE *f)
{
    leap::HipAttention master({n_layers, 0, split, n_heads, n_kv, head_dim, seq_len});
    leap::HipAttention worker({n_layers, split, n_layers, n_heads, n_kv, head_dim, seq_len});
    master.load_checkpoint(path);
    worker.load_checkpoint(path);
    const int dim = n_heads * head_dim;
    DeviceFloats xm(dim), xw(dim);
    hipStream_t s;
    hip_ok(hipStreamCreate(&s), "hipStreamCreate");
    std::vector<std::byte> sent(master.packet_bytes()), reply(master.packet_bytes());
    std::vector<float> x(dim), back(dim);
    Rng rng{0x4C454150};
    for (float &e : x) e = rng.next(1.0f);
    for (int pos = 0; pos < n_tokens; pos++) {
        const int flags = pos % 3 == 2 ? LEAP_HIP_ATTENTION_FLAG_NO_REPLY : LEAP_HIP_ATTENTION_FLAG_NEED_REPLY;
        std::fwrite(x.data(), 4, x.size(), f);
        hip_ok(hipMemcpyAsync(xm.p, x.data(), dim * sizeof(float), hipMemcpyHostToDevice, s), "copy x");
        for (int l = 0; l < split; l++) master.block_async(l, pos, xm.p, s);  // forward :768-770
        master.download_packet(xm.p, {pos, flags}, sent, s);
        hip_ok(hipStreamSynchronize(s), "sync");  // the transport sends the packet
        std::fwrite(sent.data(), 1, sent.size(), f);
        // the worker (worker_loop :869-939)
        const auto hd = worker.upload_packet(sent, xw.p, s);
        if (!hd) throw std::runtime_error("a data packet was read as a control packet");
        for (int l = split; l < n_layers; l++) worker.block_async(l, hd->pos, xw.p, s);
        const int32_t fwd = leap::HipAttention::forwards(true, hd->flags) ? 1 : 0;
        std::fill(reply.begin(), reply.end(), std::byte{0});
        std::fill(back.begin(), back.end(), 0.0f);
        if (fwd) {
            worker.download_packet(xw.p, *hd, reply, s);
            hip_ok(hipStreamSynchronize(s), "sync");
            // the master receives the reply and takes its x (:785-788)
            if (!master.upload_packet(reply, xm.p, s)) throw std::runtime_error("reply read as a control packet");
            hip_ok(hipMemcpyAsync(back.data(), xm.p, dim * sizeof(float), hipMemcpyDeviceToHost, s), "copy x");
        }
        hip_ok(hipStreamSynchronize(s), "sync");
        std::fwrite(&fwd, 4, 1, f);
        std::fwrite(reply.data(), 1, reply.size(), f);
        std::fwrite(back.data(), 4, back.size(), f);
        for (float &e : x) e = rng.next(1.0f);  // the next token's embedding row
    }
    hip_ok(hipStreamDestroy(s), "hipStreamDestroy");
    std::printf("engine_demo: %d tokens through a %d + %d layer pipeline\n", n_tokens, split, n_layers - split);
    return 0;
}

}  // namespace

int main(int argc, char **argv)
{
    const bool block = argc == 9 && std::string(argv[8]) == "block";
    const bool ckpt = argc == 10 && std::string(argv[8]) == "ckpt";
    const bool pipeline = argc == 11 && std::string(argv[8]) == "pipeline";
    if (argc != 8 && !block && !ckpt && !pipeline) {
        std::fprintf(stderr,
                     "usage: %s n_layers n_heads n_kv_heads head_dim seq_len n_tokens out_dir "
                     "[block | ckpt PATH | pipeline PATH SPLIT]\n",
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
        if (pipeline) {
            const int split = std::atoi(argv[10]);
            if (split <= 0 || split >= n_layers) {
                std::fprintf(stderr, "SPLIT must be in [1, n_layers)\n");
                return 2;
            }
            std::FILE *f = std::fopen((out_dir + "/trace.bin").c_str(), "wb");
            if (!f) {
                std::fprintf(stderr, "cannot write %s/trace.bin\n", out_dir.c_str());
                return 2;
            }
            const int rc = run_pipeline(n_layers, n_heads, n_kv, head_dim, seq_len, n_tokens, argv[9], split, f);
            std::fclose(f);
            return rc;
        }
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
