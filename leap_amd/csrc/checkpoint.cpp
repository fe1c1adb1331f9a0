// Checkpoint (.bin) header parsing and tensor layout, host C++.
//
// The header follows Transformer::create (TransformerFactory.cpp:59-115):
//   - magic 0x616B3432, then version 1 (fp32) or 2 (int8), then the Config
//     (Config.h:5-13, seven int32), for version 2 a shared-classifier byte and
//     the int32 group size; the weights start at byte 256;
//   - no magic: the legacy fp32 layout, the Config at byte 0 and the weights
//     right after it (byte 28).
// For the fp32 versions the classifier is taken as shared when vocab_size > 0
// and vocab_size is made positive, as the reference does (the byte that the
// version-1 writer puts after the Config is not read, TransformerFactory.cpp:
// 80-84 and 110-113).  The tensor order is memory_map_weights'
// (FloatTransformer.cpp:947-978; QuantizedTransformer.cpp:102-134).
#include "checkpoint.hpp"

#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sys/stat.h>

namespace leap {

namespace {

constexpr int32_t kMagic = 0x616B3432;
constexpr size_t kHeaderBytes = 256;

// a += b * c with overflow checks
bool mac(size_t &a, size_t b, size_t c)
{
    size_t p;
    if (__builtin_mul_overflow(b, c, &p) || __builtin_add_overflow(a, p, &a)) return false;
    return true;
}

}  // namespace

bool ckpt_layer(const leap_hip_attention_checkpoint &c, int layer, CkptLayer *out, size_t *needed)
{
    const size_t L = (size_t)c.n_layers, dim = (size_t)c.dim, hd = dim / (size_t)c.n_heads;
    const size_t kv = (size_t)c.n_kv_heads * hd, vocab = (size_t)c.vocab_size, l = (size_t)layer;
    size_t at = (size_t)c.header_bytes;
    CkptLayer o{};
    if (c.version != 2) {
        // rms_att [L][dim], rms_ffn [L][dim], rms_final [dim], embeddings
        // [vocab][dim], wq [L][dim][dim], wk [L][kv][dim], wv, wo [L][dim][dim]
        o.rms_att = at + 4 * l * dim;
        if (!mac(at, 4 * (2 * L + 1), dim) || !mac(at, 4 * vocab, dim)) return false;
        o.wq = at + 4 * l * dim * dim;
        if (!mac(at, 4 * L, dim * dim)) return false;
        o.wk = at + 4 * l * kv * dim;
        if (!mac(at, 4 * L, kv * dim)) return false;
        o.wv = at + 4 * l * kv * dim;
        if (!mac(at, 4 * L, kv * dim)) return false;
        o.wo = at + 4 * l * dim * dim;
        if (!mac(at, 4 * L, dim * dim)) return false;
    } else {
        // rms weights as above, then the quantized tensors, each one
        // tensor's values then its scales: embeddings, wq[0..L), wk, wv, wo
        const size_t gs = (size_t)c.group_size;
        o.rms_att = at + 4 * l * dim;
        if (!mac(at, 4 * (2 * L + 1), dim) || !mac(at, vocab, dim) || !mac(at, 4, vocab * dim / gs)) return false;
        const size_t sizes[4] = {dim * dim, kv * dim, kv * dim, dim * dim};
        size_t *vals[4] = {&o.wq, &o.wk, &o.wv, &o.wo};
        size_t *scales[4] = {&o.wq_s, &o.wk_s, &o.wv_s, &o.wo_s};
        for (int t = 0; t < 4; t++) {
            const size_t per = sizes[t] + 4 * (sizes[t] / gs);  // one layer's tensor
            *vals[t] = at + l * per;
            *scales[t] = *vals[t] + sizes[t];
            if (!mac(at, L, per)) return false;
        }
    }
    *out = o;
    *needed = at;
    return true;
}

}  // namespace leap

extern "C" int leap_hip_attention_checkpoint_read(const char *path, leap_hip_attention_checkpoint *out)
{
    if (!path || !out) return -EINVAL;
    std::FILE *f = std::fopen(path, "rb");
    if (!f) return -EIO;
    struct stat st {};
    if (fstat(fileno(f), &st) != 0) {
        std::fclose(f);
        return -EIO;
    }
    unsigned char head[64] = {};
    const size_t got = std::fread(head, 1, sizeof head, f);
    std::fclose(f);
    int32_t w[10];
    std::memcpy(w, head, sizeof w);
    leap_hip_attention_checkpoint c{};
    c.file_bytes = (long long)st.st_size;
    const int32_t *cfg;
    if (w[0] == leap::kMagic) {
        if (got < 8 + 28) return -EINVAL;
        c.version = w[1];
        if (c.version != 1 && c.version != 2) return -EINVAL;
        cfg = w + 2;
        c.header_bytes = (long long)leap::kHeaderBytes;
        if (c.version == 2) {
            if (got < 8 + 28 + 1 + 4) return -EINVAL;
            c.shared_classifier = head[36];
            int32_t gs;
            std::memcpy(&gs, head + 37, 4);
            c.group_size = gs;
        }
    } else {
        if (got < 28) return -EINVAL;
        c.version = 0;
        cfg = w;
        c.header_bytes = 28;
    }
    c.dim = cfg[0];
    c.hidden_dim = cfg[1];
    c.n_layers = cfg[2];
    c.n_heads = cfg[3];
    c.n_kv_heads = cfg[4];
    c.vocab_size = cfg[5];
    c.seq_len = cfg[6];
    if (c.version != 2) {
        // (the most negative int has no magnitude in int: not a vocabulary size)
        if (c.vocab_size == INT32_MIN) return -EINVAL;
        c.shared_classifier = c.vocab_size > 0 ? 1 : 0;
        c.vocab_size = std::abs(c.vocab_size);
    }
    if (c.dim <= 0 || c.n_layers <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.dim % c.n_heads ||
        c.n_heads % c.n_kv_heads || c.vocab_size < 0 || c.hidden_dim < 0 || c.seq_len <= 0)
        return -EINVAL;
    if (c.version == 2 && (c.group_size <= 0 || c.dim % c.group_size)) return -EINVAL;
    leap::CkptLayer lay;
    size_t needed;
    if (!leap::ckpt_layer(c, 0, &lay, &needed)) return -EINVAL;
    // reported as a signed count: larger than any file can be is not a model
    if (needed > (size_t)INT64_MAX) return -EINVAL;
    c.attention_bytes = (long long)needed;
    *out = c;
    return 0;
}
