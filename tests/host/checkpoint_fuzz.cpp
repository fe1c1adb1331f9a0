// Header fuzz of the checkpoint reader and bounds checks of the host-side
// tensor layout and RoPE table, for an AddressSanitizer + UBSan build
// (tests/test_host_sanitizers.py compiles and runs it; no GPU involved).
//
// Every file the reader accepts must describe tensors that all lie inside
// the attention_bytes it reports, since the upload reads
// [offset, offset + size) of the mapped file for every held layer.
#include <cerrno>
#include <climits>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "checkpoint.hpp"
#include "leap_hip_attention.h"

extern "C" void leap_rope_table_host(int seq_len, int head_size, float theta, float *cos_tab, float *sin_tab);

namespace {

int g_fail = 0;
#define CHECK(cond, ...)                                          \
    do {                                                          \
        if (!(cond)) {                                            \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);                    \
            std::fprintf(stderr, "\n");                           \
            g_fail++;                                             \
        }                                                         \
    } while (0)

std::string g_path;

int read_bytes(const std::vector<unsigned char> &bytes, leap_hip_attention_checkpoint *c)
{
    std::FILE *f = std::fopen(g_path.c_str(), "wb");
    if (!f) return -1000;
    if (!bytes.empty()) std::fwrite(bytes.data(), 1, bytes.size(), f);
    std::fclose(f);
    return leap_hip_attention_checkpoint_read(g_path.c_str(), c);
}

// Every tensor of every layer inside [header_bytes, needed).
void check_layout(const leap_hip_attention_checkpoint &c)
{
    const size_t dim = (size_t)c.dim, hd = dim / (size_t)c.n_heads, kv = (size_t)c.n_kv_heads * hd;
    for (int layer : {0, c.n_layers / 2, c.n_layers - 1}) {
        leap::CkptLayer o;
        size_t needed = 0;
        const bool ok = leap::ckpt_layer(c, layer, &o, &needed);
        CHECK(ok, "accepted header whose layout overflows");
        if (!ok) return;
        CHECK(needed == (size_t)c.attention_bytes, "needed %zu != attention_bytes %lld", needed, c.attention_bytes);
        auto inside = [&](size_t off, size_t n, const char *what) {
            CHECK(off >= (size_t)c.header_bytes && off <= needed && n <= needed - off,
                  "%s [%zu, +%zu) of layer %d outside [%lld, %zu)", what, off, n, layer, c.header_bytes, needed);
        };
        inside(o.rms_att, 4 * dim, "rms_att");
        if (c.version != 2) {
            inside(o.wq, 4 * dim * dim, "wq");
            inside(o.wk, 4 * kv * dim, "wk");
            inside(o.wv, 4 * kv * dim, "wv");
            inside(o.wo, 4 * dim * dim, "wo");
        } else {
            const size_t gs = (size_t)c.group_size;
            inside(o.wq, dim * dim, "wq");
            inside(o.wq_s, 4 * (dim * dim / gs), "wq_s");
            inside(o.wk, kv * dim, "wk");
            inside(o.wk_s, 4 * (kv * dim / gs), "wk_s");
            inside(o.wv, kv * dim, "wv");
            inside(o.wv_s, 4 * (kv * dim / gs), "wv_s");
            inside(o.wo, dim * dim, "wo");
            inside(o.wo_s, 4 * (dim * dim / gs), "wo_s");
        }
    }
}

void check_accepted(int rc, const leap_hip_attention_checkpoint &c)
{
    CHECK(rc == 0 || rc == -EINVAL, "rc %d", rc);
    if (rc != 0) return;
    CHECK(c.version >= 0 && c.version <= 2, "version %d", c.version);
    CHECK(c.dim > 0 && c.n_layers > 0 && c.n_heads > 0 && c.n_kv_heads > 0 && c.seq_len > 0, "config");
    CHECK(c.dim % c.n_heads == 0 && c.n_heads % c.n_kv_heads == 0, "head split");
    CHECK(c.vocab_size >= 0 && c.hidden_dim >= 0, "sizes");
    CHECK(c.attention_bytes >= c.header_bytes, "attention bytes");
    check_layout(c);
}

void put32(std::vector<unsigned char> &b, size_t at, int32_t v)
{
    if (b.size() < at + 4) b.resize(at + 4);
    std::memcpy(b.data() + at, &v, 4);
}

std::vector<unsigned char> header(int version, const int32_t cfg[7], int shared, int32_t gs)
{
    std::vector<unsigned char> b;
    if (version == 0) {
        for (int i = 0; i < 7; i++) put32(b, 4 * i, cfg[i]);
    } else {
        put32(b, 0, 0x616B3432);
        put32(b, 4, version);
        for (int i = 0; i < 7; i++) put32(b, 8 + 4 * i, cfg[i]);
        b.resize(37);
        b[36] = (unsigned char)shared;
        put32(b, 37, gs);
        b.resize(256, 0);
    }
    return b;
}

}  // namespace

int main(int argc, char **argv)
{
    g_path = argc > 1 ? argv[1] : "/tmp/leap_ckpt_fuzz.bin";
    leap_hip_attention_checkpoint c;

    // arguments and missing files
    CHECK(leap_hip_attention_checkpoint_read(nullptr, &c) == -EINVAL, "NULL path");
    CHECK(leap_hip_attention_checkpoint_read(g_path.c_str(), nullptr) == -EINVAL, "NULL out");
    CHECK(leap_hip_attention_checkpoint_read("/nonexistent/leap.bin", &c) == -EIO, "missing file");

    // every truncation of valid headers of each version
    const int32_t good[7] = {256, 64, 2, 4, 2, 8, 16};
    for (int version = 0; version <= 2; version++) {
        const auto full = header(version, good, 1, 64);
        for (size_t n = 0; n <= full.size(); n++) {
            std::vector<unsigned char> cut(full.begin(), full.begin() + n);
            const int rc = read_bytes(cut, &c);
            check_accepted(rc, c);
            const size_t need = version == 0 ? 28 : version == 1 ? 36 : 41;
            if (n < need) CHECK(rc == -EINVAL, "version %d cut at %zu accepted", version, n);
        }
    }

    // extreme and random Config values
    const int32_t extremes[] = {INT_MIN, INT_MIN + 1, -65536, -2, -1, 0, 1, 2, 3, 4, 7, 8, 31, 32, 64, 128,
                                4096, 65536, 1 << 20, 1 << 28, INT_MAX - 1, INT_MAX};
    std::mt19937_64 rng(0x4C454150);
    auto pick = [&]() -> int32_t {
        const unsigned r = (unsigned)(rng() % 4);
        if (r < 3) return extremes[rng() % (sizeof extremes / sizeof extremes[0])];
        return (int32_t)(uint32_t)rng();
    };
    for (int it = 0; it < 20000; it++) {
        int32_t cfg[7];
        for (int &v : cfg) v = pick();
        if (it % 3 == 0) {  // mostly consistent head shapes, extreme elsewhere
            cfg[3] = 1 << (rng() % 7);
            cfg[4] = cfg[3] >> (rng() % 3);
            if (cfg[4] <= 0) cfg[4] = 1;
            cfg[0] = cfg[3] * (int32_t)(1 + rng() % 128);
        }
        const int version = (int)(rng() % 4);  // 3: a bad version number after the magic
        auto b = header(version == 3 ? 1 : version, cfg, (int)(rng() % 256), pick());
        if (version == 3) put32(b, 4, pick());
        if (rng() % 4 == 0) b.resize(rng() % (b.size() + 1));
        check_accepted(read_bytes(b, &c), c);
    }

    // garbage files
    for (int it = 0; it < 2000; it++) {
        std::vector<unsigned char> b(rng() % 300);
        for (auto &x : b) x = (unsigned char)rng();
        if (b.size() >= 4 && it % 2) put32(b, 0, 0x616B3432);
        check_accepted(read_bytes(b, &c), c);
    }

    // the RoPE table at the shapes a handle can ask for, and a few odd ones
    for (int hs : {2, 4, 6, 8, 20, 64, 128, 7, 1}) {
        for (int sl : {1, 3, 17}) {
            const size_t n = (size_t)sl * (size_t)(hs / 2);
            std::vector<float> cs(n + 1, -7.0f), sn(n + 1, -7.0f);
            leap_rope_table_host(sl, hs, 500000.0f, cs.data(), sn.data());
            CHECK(cs[n] == -7.0f && sn[n] == -7.0f, "rope table wrote past %zu entries (head size %d)", n, hs);
            if (n) CHECK(cs[0] == 1.0f && sn[0] == 0.0f, "pos 0 is not the identity");
        }
    }

    std::remove(g_path.c_str());
    std::printf("%s: %d failures\n", g_fail ? "FAIL" : "ok", g_fail);
    return g_fail ? 1 : 0;
}
