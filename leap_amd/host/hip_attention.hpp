// C++20 engine-side wrapper of the leap_hip_attention C ABI.
//
// This is the thin layer a LEAP engine (src/inference/FloatTransformer.cpp or
// QuantizedTransformer.cpp) keeps around the shim: it owns one handle, turns
// negative status codes into std::runtime_error the way the engine reports
// its own failures (TransformerFactory.cpp:59-135 throws runtime_error), and
// exposes the attention block of run_layer (FloatTransformer.cpp:396-662) as
// one call.
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <utility>

#include "leap_hip_attention.h"

namespace leap {

class HipAttention {
public:
    struct Dims {
        int n_layers, layer_begin, layer_end, n_heads, n_kv_heads, head_dim, seq_len;
        float rope_theta = 500000.0f;  // FloatTransformer.cpp:65
        int max_batch = 1;
        int device = 0;
    };

    explicit HipAttention(const Dims &d)
    {
        const leap_hip_attention_config c{d.n_layers, d.layer_begin, d.layer_end, d.n_heads,
                                          d.n_kv_heads, d.head_dim,    d.seq_len,   d.rope_theta,
                                          d.max_batch,  d.device};
        check(leap_hip_attention_create(&c, &h_), nullptr);
        q_dim_ = d.n_heads * d.head_dim;
        kv_dim_ = d.n_kv_heads * d.head_dim;
    }
    HipAttention(const HipAttention &) = delete;
    HipAttention &operator=(const HipAttention &) = delete;
    HipAttention(HipAttention &&o) noexcept : h_(std::exchange(o.h_, nullptr)), q_dim_(o.q_dim_), kv_dim_(o.kv_dim_) {}
    ~HipAttention() { leap_hip_attention_destroy(h_); }

    // The attention block of run_layer(l, pos, x): q is s->q (pre-RoPE),
    // k_new / v_new the k and v GEMV outputs, out receives s->xb.
    void step(int layer, int pos, std::span<const float> q, std::span<const float> k_new,
              std::span<const float> v_new, std::span<float> out)
    {
        if ((int)q.size() != q_dim_ || (int)out.size() != q_dim_ || (int)k_new.size() != kv_dim_ ||
            (int)v_new.size() != kv_dim_)
            throw std::invalid_argument("HipAttention::step: buffer sizes do not match the model");
        check(leap_hip_attention_step(h_, layer, pos, q.data(), k_new.data(), v_new.data(), out.data()), h_);
    }

    // Weights of one held layer for block(): the layer's slices of
    // FloatTransformerWeights (FloatTransformer.h:9-22), row-major.
    void set_layer_weights(int layer, std::span<const float> rms_att, std::span<const float> wq,
                           std::span<const float> wk, std::span<const float> wv, std::span<const float> wo)
    {
        const size_t dim = (size_t)q_dim_, kv = (size_t)kv_dim_;
        if (rms_att.size() != dim || wq.size() != dim * dim || wk.size() != kv * dim || wv.size() != kv * dim ||
            wo.size() != dim * dim)
            throw std::invalid_argument("HipAttention::set_layer_weights: weight sizes do not match the model");
        check(leap_hip_attention_set_layer_weights(h_, layer, rms_att.data(), wq.data(), wk.data(), wv.data(),
                                                   wo.data()),
              h_);
    }

    // The int8 engine's weights of one held layer: each projection as the
    // reference's QuantizedTensor (QuantizedTransformer.h:9-12), int8 values
    // [d][n] and one scale per group of group_size values.
    struct QTensor {
        std::span<const int8_t> q;
        std::span<const float> s;
    };
    void set_layer_weights_q8(int layer, int group_size, std::span<const float> rms_att, QTensor wq, QTensor wk,
                              QTensor wv, QTensor wo)
    {
        const size_t dim = (size_t)q_dim_, kv = (size_t)kv_dim_;
        const auto ok = [&](const QTensor &t, size_t rows) {
            return group_size > 0 && t.q.size() == rows * dim && t.s.size() == rows * dim / (size_t)group_size;
        };
        if (rms_att.size() != dim || !ok(wq, dim) || !ok(wk, kv) || !ok(wv, kv) || !ok(wo, dim))
            throw std::invalid_argument("HipAttention::set_layer_weights_q8: weight sizes do not match the model");
        check(leap_hip_attention_set_layer_weights_q8(h_, layer, group_size, rms_att.data(), wq.q.data(),
                                                      wq.s.data(), wk.q.data(), wk.s.data(), wv.q.data(),
                                                      wv.s.data(), wo.q.data(), wo.s.data()),
              h_);
    }

    // run_layer(l, pos, x) from its start to the attention residual
    // (FloatTransformer.cpp:394-683): x += Wo . attention(Wq/Wk/Wv . rmsnorm(x)).
    void block(int layer, int pos, std::span<float> x)
    {
        if ((int)x.size() != q_dim_)
            throw std::invalid_argument("HipAttention::block: x must hold dim floats");
        check(leap_hip_attention_block(h_, layer, pos, x.data()), h_);
    }

    // The same with x in device memory (16-byte aligned), enqueued on `stream`.
    void block_async(int layer, int pos, float *x_dev, void *stream)
    {
        check(leap_hip_attention_block_async(h_, layer, pos, x_dev, stream), h_);
    }

    // ---- the stage hand-off of a pipeline (FloatTransformer.cpp:775-788, 925-939)

    // PacketHeader (Transformer.h:25-28).
    struct PacketHeader {
        int pos, flags;
    };
    size_t packet_bytes() const { return LEAP_HIP_ATTENTION_PACKET_HEADER_BYTES + sizeof(float) * (size_t)q_dim_; }

    // A received packet's x into the device residual stream x_dev; its header,
    // or nothing for a control packet (the transport's business).  Enqueued on
    // `stream`; a null stream waits for the copy.
    std::optional<PacketHeader> upload_packet(std::span<const std::byte> packet, float *x_dev, void *stream = nullptr)
    {
        PacketHeader hd{};
        const int rc = leap_hip_attention_packet_upload(h_, packet.data(), packet.size(), x_dev, &hd.pos, &hd.flags,
                                                        stream);
        if (rc == 1) return std::nullopt;
        check(rc, h_);
        return hd;
    }

    // The packet {header, x_dev} for the next stage; its values are in place
    // once `stream` has passed the copy (at return for a null stream).
    void download_packet(const float *x_dev, PacketHeader hd, std::span<std::byte> packet, void *stream = nullptr)
    {
        check(leap_hip_attention_packet_download(h_, x_dev, hd.pos, hd.flags, packet.data(), packet.size(), stream),
              h_);
    }

    // worker_loop forwards after its layers unless it is the tail and no
    // reply is wanted (FloatTransformer.cpp:937).
    static bool forwards(bool is_tail, int flags) { return !is_tail || flags == LEAP_HIP_ATTENTION_FLAG_NEED_REPLY; }

    // Every held layer's attention weights from a checkpoint file
    // (Transformer::create's format, TransformerFactory.cpp:59-135).
    void load_checkpoint(const std::string &path) { check(leap_hip_attention_load_checkpoint(h_, path.c_str()), h_); }

    // The header of a checkpoint file.
    static leap_hip_attention_checkpoint checkpoint_read(const std::string &path)
    {
        leap_hip_attention_checkpoint c{};
        if (int rc = leap_hip_attention_checkpoint_read(path.c_str(), &c))
            throw std::runtime_error("leap_hip_attention: cannot read checkpoint " + path + " (status " +
                                     std::to_string(rc) + ")");
        return c;
    }

    // clear_kv_cache (FloatTransformer.cpp:74-77).
    void clear_kv_cache() { check(leap_hip_attention_clear(h_), h_); }

    void kv_download(int seq, int layer, int pos_begin, int pos_end, float *k, float *v)
    {
        check(leap_hip_attention_kv_download(h_, seq, layer, pos_begin, pos_end, k, v), h_);
    }

    leap_hip_attention *handle() const { return h_; }

private:
    static void check(int rc, const leap_hip_attention *h)
    {
        if (rc != 0)
            throw std::runtime_error(std::string("leap_hip_attention: ") + leap_hip_attention_last_error(h) +
                                     " (status " + std::to_string(rc) + ")");
    }

    leap_hip_attention *h_ = nullptr;
    int q_dim_ = 0, kv_dim_ = 0;
};

}  // namespace leap
