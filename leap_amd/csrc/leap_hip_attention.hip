// C-ABI of the MI355X decode-attention library (include/leap_hip_attention.h).
//
// Host side: argument checks, device allocations in the reference's cache
// layout, the RoPE table upload, launch sizing for the split-K kernel, and the
// host<->device copies of the synchronous entry points.  Device side:
// decode_attention.hpp.
#include "leap_hip_attention.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <new>
#include <string>
#include <utility>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#include "aux_kernels.hpp"
#include "checkpoint.hpp"
#include "kernels.hpp"

extern "C" void leap_rope_table_host(int seq_len, int head_size, float theta, float *cos_tab,
                                     float *sin_tab);

struct leap_hip_attention {
    leap_hip_attention_config cfg{};
    int n_local = 0;          // layers held
    int kv_dim = 0, q_dim = 0, group = 0;
    size_t layer_floats = 0;  // seq_len * kv_dim
    size_t slab_floats = 0;   // n_local * layer_floats, one sequence
    float *k_cache = nullptr, *v_cache = nullptr;
    float4 *rope = nullptr;
    float *ws_o = nullptr;
    float2 *ws_ml = nullptr;
    int *counters = nullptr;
    float *ws_po = nullptr;    // part records of spread launches: [kXcds][group][head_dim]
    float2 *ws_pml = nullptr;  // [kXcds][group]
    size_t counter_bytes = 0;
    // The host-pointer entry points stage their inputs through one pinned
    // host buffer and one device region (q rows | k rows | v rows | pos, packed
    // for the call's n_seq), so that each call makes one DMA in and one out.
    char *in_dev = nullptr;
    char *in_host = nullptr;  // pinned, the same size
    float *out_host = nullptr;// pinned, max_batch * q_dim
    size_t in_bytes = 0;
    float *out_dev = nullptr;
    // attention sub-block: per-layer weights (allocated on the first
    // set_layer_weights) and the block's own q, k, v, attention-out buffers
    float *w_qkv = nullptr;   // [n_local][dim + 2*kv_dim][dim]
    float *w_o = nullptr;     // [n_local][dim][dim]
    float *w_rms = nullptr;   // [n_local][dim]
    std::vector<char> w_set;  // per held layer: weights uploaded
    float *blk = nullptr;     // q [dim] | k [kv_dim] | v [kv_dim] | xb [dim] | x staging [dim]
    // int8 weights of the quantized engine (one format per handle: the first
    // set_layer_weights* call fixes it) with one float scale per group of gs
    int w_fmt = 0;            // 0 none yet, 1 fp32, 2 int8
    int gs = 0;
    int8_t *w8_qkv = nullptr; // [n_local][dim + 2*kv_dim][dim]
    float *s8_qkv = nullptr;  // [n_local][dim + 2*kv_dim][dim / gs]
    int8_t *w8_o = nullptr;   // [n_local][dim][dim]
    float *s8_o = nullptr;    // [n_local][dim][dim / gs]
    int8_t *q8_act = nullptr; // xq [dim] | aq [dim]: the quantized projection inputs of the last block
    float *q8_act_s = nullptr;// xs [dim / gs] | as [dim / gs]: their group scales
    hipStream_t stream = nullptr;
    int split = 0;
    int n_cu = 256;  // compute units of the device
    int max_chunks = 1;  // chunks per sequence the workspace holds records for
    bool valu = false;   // score and weighted-V products on the VALU (measurement knob)
    int fold_helper = 1; // 1: two workgroups share a one-level merge's final fold; 0: the last alone; 2: test of the fallback
    std::string err;
};

using namespace leap_kernels;

namespace {

// The message of the last failure of a call made without a handle (create,
// the placement map) on this thread: a fixed buffer, so that recording it
// allocates nothing.
thread_local char g_create_error[512];

int set_err(leap_hip_attention *h, int code, const char *fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (h)
        h->err = buf;
    else
        std::memcpy(g_create_error, buf, sizeof buf);
    return code;
}

// A failed HIP call also leaves its code as the thread's sticky "last
// error"; it is read (cleared) here so that it cannot be reported again by a
// later, unrelated query.
#define HIP_TRY(h, call)                                                                       \
    do {                                                                                       \
        hipError_t e_ = (call);                                                                \
        if (e_ != hipSuccess) {                                                                \
            (void)hipGetLastError();                                                           \
            return set_err((h), e_ == hipErrorOutOfMemory ? -ENOMEM : -EIO, "%s: %s", #call,  \
                           hipGetErrorString(e_));                                             \
        }                                                                                      \
    } while (0)

template <typename T>
struct same_type {
    using type = T;
};

// Enqueue fn<<<grid, block, 0, stream>>>(args...) and return that launch's
// own status (not the thread's sticky last error, which may be older).
template <typename... P>
hipError_t launch_k(void (*fn)(P...), dim3 grid, dim3 block, hipStream_t stream, typename same_type<P>::type... args)
{
    void *kargs[] = {static_cast<void *>(&args)...};
    return hipLaunchKernel(reinterpret_cast<const void *>(fn), grid, block, kargs, 0, stream);
}

// How launches see a head shape: 16 q heads per KV head run as two groups
// of 8 per cache head (the decode kernel's kv_split), so that no kernel
// instance holds more than 8 heads' accumulators; other shapes as they are.
struct KvView {
    int group;       // q heads per launch group
    int n_kv_heads;  // launch groups per sequence
    int kv_split;
};
KvView kv_view(int group, int n_kv_heads)
{
    return group == 16 ? KvView{8, 2 * n_kv_heads, 1} : KvView{group, n_kv_heads, 0};
}
bool shape_supported(int head_dim, int group)
{
    const KvView v = kv_view(group, 1);
    return pick_kernel(head_dim, v.group, kDecode, false, false, v.kv_split) != nullptr;
}

int check_layer(leap_hip_attention *h, int layer)
{
    if (layer < h->cfg.layer_begin || layer >= h->cfg.layer_end)
        return set_err(h, -EINVAL, "layer %d outside the held range [%d, %d)", layer,
                       h->cfg.layer_begin, h->cfg.layer_end);
    return 0;
}

int round_up(int x, int q) { return (x + q - 1) / q * q; }

// What sizes and places one decode-attention launch: the head shape, the
// device's compute units, a forced chunk size (0 = automatic) and the most
// chunks per sequence the workspace holds records for.
struct LaunchShape {
    int head_dim, group, n_heads, n_kv_heads, seq_len;
    int n_cu;
    int split;
    int max_chunks;
    bool valu = false;  // products as VALU FMAs instead of MFMAs (the A/B knob)
    bool ws_parts = true;  // the buffers hold part records and kXcds part-groups' records
    int fold_helper = 1;   // leap_hip_attention_set_fold_helper
    int kv_split = 0;      // 2^kv_split launch groups per cache head (kv_view's, launch_view's)
};

// The device buffers of one launch (one layer): the cache slabs of sequence
// 0 at this layer and the distance between sequences, the RoPE table, and
// the split-K workspace (records_per_head(grid) records per head and
// sequence, counters zero between launches).
struct LaunchBuffers {
    float *k_cache, *v_cache;
    long long seq_stride;
    const float4 *rope;
    float *ws_o;
    float2 *ws_ml;
    int *counters;
    float *ws_po;    // spread launches: kXcds part records of G heads x head_dim
    float2 *ws_pml;  // and their (max, sum)
};

LaunchShape shape_of(const leap_hip_attention *h)
{
    const KvView v = kv_view(h->group, h->cfg.n_kv_heads);
    LaunchShape s{h->cfg.head_dim, v.group, h->cfg.n_heads, v.n_kv_heads, h->cfg.seq_len,
                  h->n_cu, h->split, h->max_chunks, h->valu};
    s.fold_helper = h->fold_helper;
    s.kv_split = v.kv_split;
    return s;
}

// Small launches of 4 or 8 q heads per KV head, over at most kXcds
// (sequence, KV head) groups, run as two launch groups of 2 or 4 q heads per
// cache head (kv_split 1, instances of their own): each workgroup reads its
// chunk's rows for half the heads, so the launch has twice the workgroups,
// each with half the score, softmax, combine and fold work.  Same process,
// both orders, graph replay, µs per layer-step, 8 q heads per KV head (up to
// 24 MiB of K/V rows): TinyLlama ctx 1 4.33 -> 3.62, 256 5.51 -> 4.95, 1024
// 6.14 -> 5.53, 4096 8.41 -> 7.75, 8192 11.73 -> 10.50; the 70B heads ctx
// 512 7.11 -> 5.57, 1024 7.43 -> 6.19, 2048 8.84 -> 8.40, 3072 10.50 ->
// 10.38; 4 KV heads of 8 at head_dim 128 ctx 4096 11.27 -> 9.57; one KV head
// ctx 4096 11.61 -> 8.85.  4 q heads per KV head (up to 8 MiB): Llama-3-8B
// heads ctx 1 3.82 -> 3.51, 256 5.32-5.38 -> 4.95, 512 5.46 -> 5.11, 1024
// 6.05 -> 5.83.  Reading every row twice loses once the launch streams: the
// 70B heads at ctx 4096 (32 MiB) 11.67 -> 12.30, TinyLlama at 32768 23.1 ->
// 26.1, one KV head at 32768 16.8 -> 18.3, Llama-3-8B heads at ctx 2048 (16
// MiB) 6.81 -> 8.09.
// The smallest launches of 8 q heads per KV head over four (sequence, KV
// head) groups (up to 2 MiB) go one step further, four launch groups of 2 q
// heads per cache head (sixteen groups, two per XCD), against twins:
// TinyLlama ctx 1 3.57 -> 3.21, 64 3.64 -> 3.33, 256 4.86-4.99 -> 4.69-4.74,
// 512 5.06-5.10 -> 4.76-4.82, 1024 (2 MiB) 5.49-5.52 either way; 4 KV heads
// of 8 at head_dim 128 ctx 512 5.62 -> 5.22, 1024 (4 MiB) 6.12 -> 5.89, but
// TinyLlama ctx 2048 (4 MiB) 6.06 -> 7.03.  With one group (one KV head)
// they lost: ctx 2048 (2 MiB) 6.31 -> 6.92, 4096 9.03 -> 9.47.
long long twin_bytes(int group)
{
    return group == 8 ? 24ll << 20 : group == 4 ? 8ll << 20 : -1;
}
constexpr long long kQuarterBytes = 2ll << 20;
LaunchShape launch_view(const LaunchShape &s, int n_seq, long long total_rows)
{
    LaunchShape v = s;
    const long long bytes = total_rows * s.n_kv_heads * s.head_dim * 8ll;
    if (s.group == 8 && s.kv_split == 0 && !s.valu && (long long)n_seq * s.n_kv_heads == leap::kXcds / 2 &&
        bytes <= kQuarterBytes) {
        v.group = 2;
        v.n_kv_heads = 4 * s.n_kv_heads;
        v.kv_split = 2;
        return v;
    }
    if (s.kv_split == 0 && !s.valu && (long long)n_seq * s.n_kv_heads <= leap::kXcds &&
        bytes <= twin_bytes(s.group)) {
        v.group = s.group / 2;
        v.n_kv_heads = 2 * s.n_kv_heads;
        v.kv_split = 1;
    }
    return v;
}

// Positions per workgroup (chunk), from the size and shape of the launch:
//   - small launches (K/V bytes up to kLatencyBytes) are latency-bound: two
//     workgroups per CU, all resident at once, each one pass of its waves;
//   - large launches of equal-length sequences stream best with one
//     workgroup per CU walking a long contiguous run of rows;
//   - large ragged batches (mean length under 3/4 of the longest) take
//     about 12 workgroups per CU over the launch, so that the last ones to
//     start are short.
// The sequence length (the mean one when ragged) is cut into equal chunks,
// rounded up to whole passes; at most s.max_chunks chunks per sequence.
// Equal-length sequences in the latency regime are cut into near-equal
// chunks instead when that keeps every CU busy (even_chunks_for).
constexpr long long kLatencyBytes = 128ll << 20;
constexpr int kSplitRows = 8;  // granularity of any chunk (one MFMA row set)

// A launch of fewer (sequence, KV head) groups than XCDs leaves XCDs idle
// (a group's chunks share one L2).  When the groups stream at least
// kSpreadBytes of K/V rows each, each group's chunks are cut into 2, 4 or 8
// parts, one per XCD, and a second, small launch merges the parts' records
// across the L2s.  One CU takes in about 30-40 GB/s, so a group's 32 CUs
// stream 4 MiB in about 3-4 us, and the merge launch costs about 2 us:
// below that size the launch on fewer XCDs is faster (measured at 1, 2 and
// 4 KV heads, contexts 512-4096).
constexpr long long kSpreadBytes = 4ll << 20;  // per group

// Whether a decode launch spreads its groups over the XCDs (see
// launch_attention; it also needs two chunks or more).
bool spreads(const LaunchShape &s, int n_seq, long long total_rows)
{
    const long long n_groups = (long long)n_seq * s.n_kv_heads;
    const long long bytes = total_rows * (long long)s.n_kv_heads * s.head_dim * 8ll;
    return s.ws_parts && n_groups < leap::kXcds && bytes >= n_groups * kSpreadBytes;
}

// CUs a launch's workgroups can run on: a (sequence, KV head) group's chunks
// share one XCD, so a launch of fewer groups than XCDs that does not spread
// runs on that many XCDs only.  (TinyLlama's four KV heads at ctx 5120-6144
// were split for all 256 CUs, four workgroups per CU on four XCDs: 17.0-17.2
// us per layer-step, against 12.0-12.3 us split for their 128 CUs.)
long long launch_cus(const LaunchShape &s, int n_seq, long long total_rows)
{
    const long long n_groups = (long long)n_seq * s.n_kv_heads;
    if (n_groups >= leap::kXcds || spreads(s, n_seq, total_rows)) return s.n_cu;
    return std::max<long long>(1, s.n_cu * n_groups / leap::kXcds);
}

// Workgroups per CU in the latency regime: two, except
//   - in a launch of equal lengths with at least two (sequence, KV head)
//     groups per XCD (counting the two launch groups of a cache head with
//     sixteen q heads per KV head), which takes one per CU, with chunks twice
//     as long.  Forced chunk lengths put the best there every time, and the
//     rule measured 1.0-2.1 us faster at the Llama-3.1-405B stage's
//     128/8/128 at ctx 2048-8192 (ctx 4096 17.7 -> 16.0 us), 0.75-0.97 us at
//     32 KV heads of one q head (ctx 2048-4096), and 0.24-1.39 us for
//     batches of 2-4 Llama-3-8B, 64/8/128 and TinyLlama sequences at ctx
//     2048-4096.  With fewer groups (batch 1 at 8 KV heads; two KV heads at
//     head_dim 64 with sixteen q heads each, 0.5-0.7 us slower) two per CU
//     stays faster;
//   - in a launch that spreads its groups over the XCDs, when one per CU
//     gives chunks of two passes or more.  There one per CU measured 3.4-3.8
//     us faster than one-pass chunks two per CU (one, two and four KV heads
//     at ctx 32768, 16384 and 8192) and was no slower at the other sizes
//     measured.
int latency_per_cu(const LaunchShape &s, int n_seq, long long total_rows, int max_T)
{
    const long long n_groups = (long long)n_seq * s.n_kv_heads;
    if (!spreads(s, n_seq, total_rows)) {
        const bool ragged = total_rows * 4 < 3ll * n_seq * max_T;
        return (n_groups >= 2 * leap::kXcds && !ragged) ? 1 : 2;
    }
    const long long per_seq = std::max<long long>(1, (s.n_cu + n_groups / 2) / n_groups);
    const int pass = leap::rows_per_pass(s.head_dim, s.group, kWaves);
    return (max_T + per_seq - 1) / per_seq >= 2 * pass ? 1 : 2;
}

int choose_chunk(const LaunchShape &s, int n_seq, long long total_rows, int max_T)
{
    const int quantum = leap::rows_per_pass(s.head_dim, s.group, kWaves);
    const int floor_chunk = round_up((max_T + s.max_chunks - 1) / s.max_chunks, kSplitRows);
    const long long kv_dim = (long long)s.n_kv_heads * s.head_dim;
    int c;
    if (s.split > 0) {
        c = round_up(s.split, kSplitRows);
    } else {
        const long long bytes = total_rows * kv_dim * 8ll;
        const bool ragged = total_rows * 4 < 3ll * n_seq * max_T;
        const long long per_cu = bytes <= kLatencyBytes ? latency_per_cu(s, n_seq, total_rows, max_T) : ragged ? 12 : 1;
        const long long n_groups = (long long)n_seq * s.n_kv_heads;
        const long long want_wgs = std::max<long long>(1, per_cu * launch_cus(s, n_seq, total_rows));
        const long long per_seq = std::max<long long>(1, (want_wgs + n_groups / 2) / n_groups);
        const long long len = ragged ? (total_rows + n_seq - 1) / n_seq : max_T;
        c = round_up((int)std::min<long long>((len + per_seq - 1) / per_seq, 1 << 20), quantum);
        c = std::min(c, round_up(max_T, quantum));
        // Short contexts: 2-4 one-pass chunks per group (2-8 with at most 4 q
        // heads per KV head at head_dim 128) leave most CUs idle, and each CU
        // takes in its chunk at the rate one CU reads.  Half-pass chunks put
        // twice the CUs on the stream for twice the records in the one-level
        // merge (Llama-3-8B ctx 128 6.48 -> 6.11, 256 6.49 -> 6.16, 512 6.54
        // -> 6.27 us; 64 q heads at ctx 256 7.60 -> 7.21 us).  At 12 or more
        // chunks, or once the halved launch would fill more than half the
        // CUs, they measured slower.  Shapes with 2-wave instances
        // (launch_attention) run half-pass chunks without masked waves,
        // which pays from up to 8 one-pass chunks and up to one half-pass
        // workgroup per CU (graph replay: TinyLlama ctx 320 5.73 -> 5.52,
        // 512 6.13 -> 5.64; 16/16/64 ctx 512 5.28 -> 4.72; 32 KV heads of
        // one q head at ctx 256 5.82 -> 5.25; 16 of two at ctx 512 5.75 ->
        // 5.27 us); two per CU made 32 KV heads at ctx 512 slower (6.46 ->
        // 8.37 us), and 10-16 chunks stayed slower (Llama-3-8B heads ctx
        // 640-1024 +0.4-0.5 us).
        const long long n_chunks = (max_T + quantum - 1) / quantum;
        const bool two_waves = short_waves_shape(s.head_dim, s.group) && !s.valu && (s.kv_split == 0 || s.group <= 4);
        const bool few = two_waves ? n_chunks <= 8
                                   : n_chunks <= 4 || (n_chunks <= 8 && s.group <= 4 && s.head_dim == 128);
        if (bytes <= kLatencyBytes && !ragged && c == quantum && n_chunks >= 2 && few &&
            (two_waves ? 2 : 4) * n_chunks * n_groups <= launch_cus(s, n_seq, total_rows))
            c = quantum / 2;
    }
    return std::max(c, std::max(floor_chunk, kSplitRows));
}

// The latency regime's split of equal-length sequences into exactly per_seq
// chunks of near-equal length (0: use choose_chunk), when each chunk then
// holds more than kEvenMinRows rows.  Chunks of whole passes leave
// ceil(T / chunk) chunks per sequence, and for most contexts that is not a
// whole number of workgroups per CU: at Llama-3-8B, ctx 2304-3584 put a
// second chunk on some CUs only (10.4-10.8 us against 8.1 at 2048), and ctx
// 4608-7168 ran 288-448 workgroups of two passes (17.4-19.5 us against
// 10.3 at 4096).  The even split keeps two workgroups on every CU, with the
// asymmetric merge while a chunk is one pass (9.0-10.0 us at 2304-3584;
// 14.3-15.9 us at 4608-7168, where 128 one-pass chunks were slower still).
// Shorter chunks than kEvenMinRows were slower than 64-row chunks on fewer
// CUs (ctx 2048: 8.7 against 8.1 us).
constexpr int kEvenMinRows = 32;

int even_chunks_for(const LaunchShape &s, int n_seq, long long total_rows, int max_T)
{
    if (s.split > 0) return 0;
    const int pass = leap::rows_per_pass(s.head_dim, s.group, kWaves);
    const long long bytes = total_rows * (long long)s.n_kv_heads * s.head_dim * 8ll;
    const bool ragged = total_rows * 4 < 3ll * n_seq * max_T;
    if (bytes > kLatencyBytes || ragged) return 0;
    const long long n_groups = (long long)n_seq * s.n_kv_heads;
    const long long per_cu = latency_per_cu(s, n_seq, total_rows, max_T);
    const long long per_seq =
        std::max<long long>(1, (per_cu * launch_cus(s, n_seq, total_rows) + n_groups / 2) / n_groups);
    if (per_seq < 2 || per_seq > s.max_chunks) return 0;
    if (max_T <= kEvenMinRows * per_seq) return 0;
    // whole passes per chunk: fixed-size chunks cut the same rows
    if (max_T % (pass * per_seq) == 0) return 0;
    return (int)per_seq;
}

// Most chunks per sequence any launch of a handle can make, for sizing its
// workspace: a pass of rows per chunk; the even split of one sequence
// (even_chunks_for: up to 2 * n_cu / n_kv_heads chunks of more than
// kEvenMinRows rows); forced splits down to kSplitRows rows, up to 64
// chunks.
int max_chunks_for(int seq_len, int head_dim, int group, int n_kv_heads, int n_cu, int cap)
{
    const int quantum = leap::rows_per_pass(head_dim, group, kWaves);
    const int by_pass = (seq_len + quantum - 1) / quantum;
    const int even = std::min((2 * n_cu + n_kv_heads / 2) / n_kv_heads, seq_len / kEvenMinRows);
    const int by_rows = std::min(64, (seq_len + kSplitRows - 1) / kSplitRows);
    return std::max(1, std::min(cap, std::max(by_pass, std::max(even, by_rows))));
}

#ifdef LEAP_TIMELINE
// The timeline build's ring of per-launch stamps ([kTlSlots][kTlMaxWgs]
// [kTlPoints] words), allocated by the first create on the device, and the
// number of decode launches enqueued so far (launch i uses slot i %
// kTlSlots).
unsigned long long *g_tl_ring = nullptr;
long long g_tl_launches = 0;
constexpr size_t kTlRingWords = (size_t)leap::kTlSlots * leap::kTlMaxWgs * leap::kTlPoints;
#endif

// Enqueue one decode-attention launch.  Returns 0, or a HIP error code
// (hipErrorInvalidValue for a shape without a kernel or a launch too large).
hipError_t launch_attention(const LaunchShape &shape, const LaunchBuffers &b, int n_seq, const int *pos_dev,
                            int pos_scalar, int max_pos, long long total_rows, const float *q, const float *k,
                            const float *v, float *out, hipStream_t stream, int kind = kDecode)
{
    const LaunchShape s = launch_view(shape, n_seq, total_rows);
    const int hd = s.head_dim;
    const int even = even_chunks_for(s, n_seq, total_rows, max_pos + 1);
    const int chunk = even ? (max_pos + even) / even : choose_chunk(s, n_seq, total_rows, max_pos + 1);
    // Chunks of at most half a pass (the short contexts' half-pass chunks,
    // and contexts of up to 32 positions) run 2-wave workgroups, whose one
    // pass is the chunk: a 4-wave workgroup gave them two waves of masked
    // rows, whose empty loads and products still held up the combine.  Same
    // process, graph replay, µs per layer-step: TinyLlama ctx 256 5.75 ->
    // 5.34, ctx 130 5.48 -> 5.11, ctx 1 4.54 -> 4.33; Llama-3-8B heads ctx
    // 256 5.71 -> 5.32, ctx 512 5.77 -> 5.44, ctx 1-32 4.00-4.17 ->
    // 3.76-3.90.  Forced 32-row chunks at ctx 768-2048 stay slower than the
    // automatic choice either way, so forced splits keep 4 waves.
    const int waves = (short_waves_shape(hd, s.group) && !s.valu && (s.kv_split == 0 || s.group <= 4) &&
                       s.split == 0 && !even &&
                       std::min(chunk, max_pos + 1) <= leap::rows_per_pass(hd, s.group, kWavesShort))
                          ? kWavesShort
                          : kWaves;
    // The PART instance: chunks that are not whole passes, and chunks of 2-8
    // passes, whose pass order it rotates (the 2-wave instances are all PART).
    const bool part =
        waves == kWavesShort || leap::part_launch(even, chunk, leap::rows_per_pass(hd, s.group, kWaves));
    KernelFn fn = pick_kernel(hd, s.group, kind, s.valu, part, s.kv_split, waves);
    if (!fn) return hipErrorInvalidValue;
    const int n_chunk_max = even ? std::min(even, max_pos + 1) : (max_pos + 1 + chunk - 1) / chunk;  // chunks of the longest sequence
    if (n_chunk_max > s.max_chunks || s.n_kv_heads >= 65536) return hipErrorInvalidValue;  // (leap::Preload::w0)
    const long long n_groups = (long long)n_seq * s.n_kv_heads;
    int spread_log2 = 0;
    if (kind == kDecode && spreads(s, n_seq, total_rows))
        while (n_groups << (spread_log2 + 1) <= leap::kXcds && n_chunk_max >= (2 << spread_log2)) spread_log2++;
    const int grid_x = (n_chunk_max + (1 << spread_log2) - 1) >> spread_log2;  // chunks per part

    leap::StepArgs a{};
    a.q = q;
    a.k_new = k;
    a.v_new = v;
    a.out = out;
    a.k_cache = b.k_cache;
    a.v_cache = b.v_cache;
    a.rope = b.rope;
    a.pos_dev = pos_dev;
    a.ws_o = b.ws_o;
    a.ws_ml = b.ws_ml;
    a.counters = b.counters;
    a.seq_stride = b.seq_stride;
    a.pos_scalar = pos_scalar;
    a.max_pos = max_pos;
    a.seq_len = s.seq_len;
    a.n_heads = s.n_heads;
    a.n_kv_heads = s.n_kv_heads;
    a.chunk = chunk;
    a.even_chunks = even;
    a.grid_chunks = grid_x;
    a.n_groups = n_seq * s.n_kv_heads;
    a.scale_log2 = (float)(1.4426950408889634 / std::sqrt((double)hd));

    a.spread_log2 = spread_log2;
    a.by_grid_chunks = leap::make_fastdiv((uint32_t)grid_x);
    a.by_kv_heads = leap::make_fastdiv((uint32_t)s.n_kv_heads);
    a.by_chunk = leap::make_fastdiv((uint32_t)chunk);
    a.by_even = leap::make_fastdiv(even > 0 ? (uint32_t)even : 1u);
    a.kv_split = s.kv_split;
#ifdef LEAP_TIMELINE
    a.tl = (g_tl_ring && kind == kDecode)
               ? g_tl_ring + (size_t)(g_tl_launches++ % leap::kTlSlots) * leap::kTlMaxWgs * leap::kTlPoints
               : nullptr;
#endif
    a.ws_po = b.ws_po;
    a.ws_pml = b.ws_pml;

    // Workgroup id = ((pg / 8) * grid_x + chunk) * 8 + pg % 8, with the
    // part-group pg = (seq * n_kv_heads + kv_head) * 2^spread_log2 + part:
    // a part-group's chunks share one XCD.
    const long long n_pgroups = n_groups << spread_log2;
    const long long n_wg = (n_pgroups + leap::kXcds - 1) / leap::kXcds * leap::kXcds * grid_x;
    if (n_wg > 0x7fffffffLL) return hipErrorInvalidValue;
    // At least two workgroups per CU of the XCDs the launch runs on, each of
    // at most 8 passes: a CU's second workgroup receives its rows after its
    // first (with several passes, each of its passes after the first's), so
    // each group's first-dispatched half of chunks can fold while the rest
    // streams.  Chunks of 2-8 passes at Llama-3-8B, against the two-level
    // tree: ctx 4608 13.48 -> 12.78 us, 8192 16.41 -> 15.86, 16384 25.57 ->
    // 25.04 us.
    const int asym = (chunk <= 8 * leap::rows_per_pass(hd, s.group, kWaves) &&
                      n_pgroups * grid_x >= 2LL * launch_cus(s, n_seq, total_rows)) ? 1 : 0;
    a.merge_asym = asym | (s.fold_helper << 1);
    // The prologue's words, preloaded into scalar registers (leap::Preload).
    const leap::Preload p = leap::make_preload(a, n_seq == 1);
    hipError_t e = launch_k(fn, dim3((unsigned)n_wg), dim3((unsigned)(waves * leap::kWave)), stream, p.q, p.k_new,
                            p.k_cache, p.v_cache, p.rope, p.m_gc, p.w0, p.w1, p.w2, a);
    if (e != hipSuccess || spread_log2 == 0) return e;
    MergeFn mf = pick_merge(hd, s.group);
    if (!mf) return hipErrorInvalidValue;
    return launch_k(mf, dim3((unsigned)n_groups), dim3((unsigned)(s.group * hd / 4)), stream, a);
}

int launch(leap_hip_attention *h, int layer, int n_seq, const int *pos_dev, int pos_scalar,
           int max_pos, long long total_rows, const float *q, const float *k, const float *v,
           float *out, hipStream_t stream, int kind = kDecode)
{
    if (!shape_supported(h->cfg.head_dim, h->group))
        return set_err(h, -EINVAL, "unsupported head_dim %d / group %d", h->cfg.head_dim, h->group);
    const size_t loff = (size_t)(layer - h->cfg.layer_begin) * h->layer_floats;
    const LaunchBuffers b{h->k_cache + loff, h->v_cache + loff, (long long)h->slab_floats, h->rope,
                          h->ws_o,           h->ws_ml,          h->counters,          h->ws_po, h->ws_pml};
    HIP_TRY(h, launch_attention(shape_of(h), b, n_seq, pos_dev, pos_scalar, max_pos, total_rows, q, k, v, out,
                                stream, kind));
    return 0;
}

// Allocate every (pointer, bytes) pair or none of them: on a failure the
// ones already made are freed and the pointers stay null, so a later call
// starts over instead of finding half a set.
int alloc_all(leap_hip_attention *h, std::initializer_list<std::pair<void **, size_t>> bufs)
{
    std::vector<void *> made;
    for (const auto &b : bufs) {
        void *p = nullptr;
        const hipError_t e = hipMalloc(&p, b.second);
        if (e != hipSuccess) {
            (void)hipGetLastError();
            for (void *q : made) (void)hipFree(q);
            return set_err(h, e == hipErrorOutOfMemory ? -ENOMEM : -EIO, "hipMalloc(%zu bytes): %s", b.second,
                           hipGetErrorString(e));
        }
        made.push_back(p);
    }
    size_t i = 0;
    for (const auto &b : bufs) *b.first = made[i++];
    return 0;
}

int launch_block_q8(leap_hip_attention *h, int li, int layer, int pos, float *x, float *x_res, hipStream_t stream)
{
    const int dim = h->q_dim, kv = h->kv_dim, gs = h->gs;
    float *q = h->blk, *k = q + dim, *v = k + kv, *xb = v + kv;
    const size_t rows_qkv = (size_t)(dim + 2 * kv);
    leap::Q8Args qa{};
    qa.x = x;
    qa.rms_w = h->w_rms + (size_t)li * dim;
    qa.w = h->w8_qkv + (size_t)li * rows_qkv * dim;
    qa.ws = h->s8_qkv + (size_t)li * rows_qkv * (dim / gs);
    qa.out0 = q;
    qa.out1 = k;
    qa.out2 = v;
    qa.rows = (int)rows_qkv;
    qa.n0 = dim;
    qa.n1 = kv;
    qa.xq_out = h->q8_act;
    qa.xs_out = h->q8_act_s;
    int rpt = 0;
    Q8Fn fn = pick_q8(dim, gs, leap::kQ8InRms, (int)rows_qkv, h->n_cu, &rpt);
    if (!fn) return set_err(h, -EINVAL, "dim %d with group size %d has no int8 projection kernel", dim, gs);
    int per_wg = leap::kQ8Teams * rpt;
    HIP_TRY(h, launch_k(fn, dim3((unsigned)((rows_qkv + per_wg - 1) / per_wg)), dim3(leap::kQ8Threads), stream, qa.x,
                        qa.rms_w, qa.w, qa.ws, qa.rows, qa));
    int8_t *aq = h->q8_act + dim;
    float *as = h->q8_act_s + dim / gs;
    if (int rc = launch(h, layer, 1, nullptr, pos, pos, pos + 1, q, k, v, xb, stream)) return rc;
    leap::Q8Args pa{};
    pa.x = xb;
    pa.w = h->w8_o + (size_t)li * dim * dim;
    pa.ws = h->s8_o + (size_t)li * dim * (dim / gs);
    pa.out0 = x_res;
    pa.rows = dim;
    pa.n0 = dim;
    pa.xq_out = aq;
    pa.xs_out = as;
    fn = pick_q8(dim, gs, leap::kQ8InF32, dim, h->n_cu, &rpt);
    if (!fn) return set_err(h, -EINVAL, "dim %d with group size %d has no int8 projection kernel", dim, gs);
    per_wg = leap::kQ8Teams * rpt;
    HIP_TRY(h, launch_k(fn, dim3((unsigned)((dim + per_wg - 1) / per_wg)), dim3(leap::kQ8Threads), stream, pa.x,
                        pa.rms_w, pa.w, pa.ws, pa.rows, pa));
    return 0;
}

// The floor of the sub-block (measurement only; leap_hip_attention_floor_async
// kind 3): the q/k/v projection's and the wo projection's grids streaming
// their weights alone, around the attention's bare K/V stream floor (kind 2),
// at one sequence and position pos.
constexpr int kFloorBlock = 3;
int launch_block_floor(leap_hip_attention *h, int layer, int pos, hipStream_t stream)
{
    const int li = layer - h->cfg.layer_begin;
    if (h->w_fmt == 0 || !h->w_set[li]) return set_err(h, -EINVAL, "no weights set for layer %d", layer);
    const int dim = h->q_dim, kv = h->kv_dim;
    const int rows_qkv = dim + 2 * kv;
    float *sink = h->out_dev;
    if (h->w_fmt == 2) {
        const int gs = h->gs;
        for (int pass = 0; pass < 2; pass++) {
            if (pass == 1)
                if (int rc = launch(h, layer, 1, nullptr, pos, pos, pos + 1, nullptr, nullptr, nullptr, sink, stream,
                                    kFloorStream))
                    return rc;
            const int rows = pass == 0 ? rows_qkv : dim;
            int rpt = 0;
            Q8Fn floor = nullptr;
            if (!pick_q8(dim, gs, pass == 0 ? leap::kQ8InRms : leap::kQ8InF32, rows, h->n_cu, &rpt, &floor) || !floor)
                return set_err(h, -EINVAL, "dim %d with group size %d has no int8 projection kernel", dim, gs);
            leap::Q8Args qa{};
            qa.w = pass == 0 ? h->w8_qkv + (size_t)li * rows_qkv * dim : h->w8_o + (size_t)li * dim * dim;
            qa.ws = pass == 0 ? h->s8_qkv + (size_t)li * rows_qkv * (dim / gs) : h->s8_o + (size_t)li * dim * (dim / gs);
            qa.rows = rows;
            qa.out0 = sink;
            const int per_wg = leap::kQ8Teams * rpt;
            HIP_TRY(h, launch_k(floor, dim3((unsigned)((rows + per_wg - 1) / per_wg)), dim3(leap::kQ8Threads), stream,
                                qa.x, qa.rms_w, qa.w, qa.ws, qa.rows, qa));
        }
        return 0;
    }
    QkvFn qkv;
    ProjFn proj;
    GemvFloorFn floor = nullptr;
    int rb;
    if (!pick_proj(dim, &qkv, &proj, &rb, &floor))
        return set_err(h, -EINVAL, "dim %d: the projections need dim in {2048, 3072, 4096, 5120, 8192}", dim);
    HIP_TRY(h, launch_k(floor, dim3((unsigned)((rows_qkv + rb - 1) / rb)), dim3(leap::kGemvThreads), stream,
                        (const float *)(h->w_qkv + (size_t)li * rows_qkv * dim), rows_qkv, sink));
    if (int rc = launch(h, layer, 1, nullptr, pos, pos, pos + 1, nullptr, nullptr, nullptr, sink, stream, kFloorStream))
        return rc;
    HIP_TRY(h, launch_k(floor, dim3((unsigned)((dim + rb - 1) / rb)), dim3(leap::kGemvThreads), stream,
                        (const float *)(h->w_o + (size_t)li * dim * dim), dim, sink));
    return 0;
}

// x: the residual stream the q/k/v projection normalises; x_res: where the
// wo product is added (x itself, or a device-accessible host copy of it).
int launch_block(leap_hip_attention *h, int layer, int pos, float *x, float *x_res, hipStream_t stream)
{
    const int li = layer - h->cfg.layer_begin;
    if (h->w_fmt == 0 || !h->w_set[li]) return set_err(h, -EINVAL, "no weights set for layer %d", layer);
    if (h->w_fmt == 2) return launch_block_q8(h, li, layer, pos, x, x_res, stream);
    QkvFn qkv;
    ProjFn proj;
    int rb;
    const int dim = h->q_dim, kv = h->kv_dim;
    if (!pick_proj(dim, &qkv, &proj, &rb))
        return set_err(h, -EINVAL, "dim %d: the projections need dim in {2048, 3072, 4096, 5120, 8192}", dim);
    float *q = h->blk, *k = q + dim, *v = k + kv, *xb = v + kv;
    leap::QkvArgs qa{};
    qa.x = x;
    qa.rms_w = h->w_rms + (size_t)li * dim;
    qa.w = h->w_qkv + (size_t)li * (dim + 2 * kv) * dim;
    qa.q = q;
    qa.k = k;
    qa.v = v;
    qa.dim = dim;
    qa.kv_dim = kv;
    HIP_TRY(h, launch_k(qkv, dim3((unsigned)((dim + 2 * kv + rb - 1) / rb)), dim3(leap::kGemvThreads), stream, qa.x,
                        qa.rms_w, qa.w, qa.q, qa.k, qa.v, qa.dim, qa.kv_dim));
    if (int rc = launch(h, layer, 1, nullptr, pos, pos, pos + 1, q, k, v, xb, stream)) return rc;
    leap::ProjArgs pa{};
    pa.xb = xb;
    pa.w = h->w_o + (size_t)li * dim * dim;
    pa.x = x_res;
    pa.d = dim;
    HIP_TRY(h, launch_k(proj, dim3((unsigned)((dim + rb - 1) / rb)), dim3(leap::kGemvThreads), stream, pa.xb, pa.w,
                        pa.x, pa.d));
    return 0;
}

// The kernel tables are compiled in translation units of their own, each
// with its own code object, which the runtime would load onto a device at the
// first launch of one of its kernels, allocating device memory then.  Asking
// for one kernel's attributes in each loads them all at once, at create and
// at the allocation-free step's set-up, so that no later launch allocates.
hipError_t load_kernel_tables()
{
    int rpt = 0;
    const void *fns[] = {
        reinterpret_cast<const void *>(pick_kernel(64, 4, kDecode, false, false, false)),
        reinterpret_cast<const void *>(pick_kernel(64, 4, kDecode, false, true, false)),
        reinterpret_cast<const void *>(pick_kernel(128, 4, kDecode, false, false, false)),
        reinterpret_cast<const void *>(pick_kernel(128, 4, kDecode, false, true, false)),
        reinterpret_cast<const void *>(pick_kernel(128, 4, kFloorLaunch, false, false, false)),
        reinterpret_cast<const void *>(pick_q8(4096, 64, leap::kQ8InRms, 6144, 256, &rpt)),
    };
    QkvFn qkv = nullptr;
    ProjFn proj = nullptr;
    int rb = 0;
    pick_proj(4096, &qkv, &proj, &rb);
    for (const void *f : fns) {
        hipFuncAttributes attr;
        if (!f) return hipErrorInvalidValue;
        if (hipError_t e = hipFuncGetAttributes(&attr, f); e != hipSuccess) return e;
    }
    hipFuncAttributes attr;
    return hipFuncGetAttributes(&attr, reinterpret_cast<const void *>(qkv));
}

// Run the XCC probe over n_wg workgroups of the decode kernel's block size
// on `device` and copy the XCC id of each to xcc_host[n_wg].
int xcc_map(leap_hip_attention *h, int device, int n_wg, int *xcc_host)
{
    HIP_TRY(h, hipSetDevice(device));
    int *d = nullptr;
    HIP_TRY(h, hipMalloc(&d, (size_t)n_wg * sizeof(int)));
    hipError_t e = launch_k(leap::xcc_probe_kernel, dim3((unsigned)n_wg), dim3(kThreads), nullptr, d);
    if (e == hipSuccess) e = hipMemcpy(xcc_host, d, (size_t)n_wg * sizeof(int), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_err(h, -EIO, "XCC probe: %s", hipGetErrorString(e));
    }
    return 0;
}

// The decode kernel's merge needs every workgroup whose id is equal modulo
// kXcds on one XCD (one L2).  Check it on a launch of n_wg workgroups:
// -ENOTSUP, with a message, when the device deals workgroups otherwise.
int check_placement(leap_hip_attention *h, int device, int n_wg)
{
    std::vector<int> xcc((size_t)n_wg);
    if (int rc = xcc_map(h, device, n_wg, xcc.data())) return rc;
    for (int i = leap::kXcds; i < n_wg; i++)
        if (xcc[i] != xcc[i % leap::kXcds])
            return set_err(h, -ENOTSUP,
                           "device %d placed workgroup %d on XCD %d and workgroup %d on XCD %d: the split-K "
                           "merge needs workgroup ids equal modulo %d on one XCD",
                           device, i, xcc[i], i % leap::kXcds, xcc[i % leap::kXcds], leap::kXcds);
    return 0;
}

}  // namespace

extern "C" {

int leap_hip_attention_xcc_map(int device, int n_wg, int *xcc_out)
{
    if (!xcc_out || n_wg <= 0 || n_wg > (1 << 20)) return set_err(nullptr, -EINVAL, "bad probe arguments");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return set_err(nullptr, -ENODEV, "no HIP device");
    if (device < 0 || device >= ndev) return set_err(nullptr, -EINVAL, "device %d of %d", device, ndev);
    return xcc_map(nullptr, device, n_wg, xcc_out);
}

int leap_hip_attention_create(const leap_hip_attention_config *cfg, leap_hip_attention **out)
{
    if (!out) return set_err(nullptr, -EINVAL, "out is NULL");
    *out = nullptr;
    if (!cfg) return set_err(nullptr, -EINVAL, "cfg is NULL");
    const leap_hip_attention_config c = *cfg;
    if (c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads != 0)
        return set_err(nullptr, -EINVAL, "n_heads %d must be a positive multiple of n_kv_heads %d",
                       c.n_heads, c.n_kv_heads);
    if (!shape_supported(c.head_dim, c.n_heads / c.n_kv_heads))
        return set_err(nullptr, -EINVAL, "unsupported head_dim %d with %d q heads per kv head",
                       c.head_dim, c.n_heads / c.n_kv_heads);
    if (c.seq_len <= 0 || c.n_layers <= 0 || c.layer_begin < 0 || c.layer_end > c.n_layers ||
        c.layer_begin >= c.layer_end)
        return set_err(nullptr, -EINVAL, "bad layer range [%d, %d) of %d or seq_len %d",
                       c.layer_begin, c.layer_end, c.n_layers, c.seq_len);
    // K/V rows are addressed with 32-bit byte offsets inside one (sequence,
    // layer) slab, with one chunk of slack past seq_len.
    const unsigned long long slab_bytes =
        ((unsigned long long)c.seq_len + leap::rows_per_pass(c.head_dim, 1, kWaves)) *
        (unsigned long long)c.n_kv_heads * c.head_dim * sizeof(float);
    if (slab_bytes >= (1ull << 32))
        return set_err(nullptr, -EINVAL, "seq_len %d: one layer's cache rows exceed 4 GiB", c.seq_len);
    if (c.max_batch <= 0 || c.max_batch > 65535)
        return set_err(nullptr, -EINVAL, "max_batch %d out of range", c.max_batch);
    if (!(c.rope_theta <= 0.0f || std::isfinite(c.rope_theta)))
        return set_err(nullptr, -EINVAL, "rope_theta must be finite");

    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0)
        return set_err(nullptr, -ENODEV, "no HIP device");
    if (c.device < 0 || c.device >= ndev)
        return set_err(nullptr, -EINVAL, "device %d of %d", c.device, ndev);

    leap_hip_attention *h = new (std::nothrow) leap_hip_attention;
    if (!h) return set_err(nullptr, -ENOMEM, "host allocation failed");
    h->cfg = c;
    if (h->cfg.rope_theta <= 0.0f) h->cfg.rope_theta = 500000.0f;
    h->n_local = c.layer_end - c.layer_begin;
    h->kv_dim = c.n_kv_heads * c.head_dim;
    h->q_dim = c.n_heads * c.head_dim;
    h->group = c.n_heads / c.n_kv_heads;
    h->layer_floats = (size_t)c.seq_len * h->kv_dim;
    h->slab_floats = (size_t)h->n_local * h->layer_floats;

    auto fail = [&](int rc) {
        std::snprintf(g_create_error, sizeof g_create_error, "%s", h->err.c_str());
        leap_hip_attention_destroy(h);
        return rc;
    };
    int rc;
#define CREATE_TRY(call)                                   \
    do {                                                   \
        if ((rc = [&]() -> int { HIP_TRY(h, call); return 0; }()) != 0) return fail(rc); \
    } while (0)

    CREATE_TRY(hipSetDevice(c.device));
    CREATE_TRY(hipDeviceGetAttribute(&h->n_cu, hipDeviceAttributeMultiprocessorCount, c.device));
    // The handle's own stream (host-pointer calls, clear, transfers) is a
    // blocking stream: it is ordered with work the caller enqueues on the
    // legacy default stream (stream 0); other caller streams must be
    // synchronised by the caller first.
    CREATE_TRY(hipStreamCreate(&h->stream));
    CREATE_TRY(load_kernel_tables());
    if (int prc = check_placement(h, c.device, 2 * h->n_cu)) return fail(prc);
    const size_t cache_bytes = (size_t)c.max_batch * h->slab_floats * sizeof(float);
    CREATE_TRY(hipMalloc(&h->k_cache, cache_bytes));
    CREATE_TRY(hipMalloc(&h->v_cache, cache_bytes));
    CREATE_TRY(hipMemsetAsync(h->k_cache, 0, cache_bytes, h->stream));
    CREATE_TRY(hipMemsetAsync(h->v_cache, 0, cache_bytes, h->stream));

    const size_t rope_n = (size_t)c.seq_len * (c.head_dim / 2);
    std::vector<float> cs(rope_n), sn(rope_n);
    leap_rope_table_host(c.seq_len, c.head_dim, h->cfg.rope_theta, cs.data(), sn.data());
    std::vector<float> packed(2 * rope_n);  // (cos, sin) per pair
    for (size_t i = 0; i < rope_n; i++) {
        packed[2 * i] = cs[i];
        packed[2 * i + 1] = sn[i];
    }
    CREATE_TRY(hipMalloc(&h->rope, packed.size() * sizeof(float)));
    CREATE_TRY(hipMemcpyAsync(h->rope, packed.data(), packed.size() * sizeof(float),
                              hipMemcpyHostToDevice, h->stream));

    // launch groups (kv_view), their records and counters: for max_batch *
    // n_kv_heads groups, or for kXcds part-groups when a launch spreads fewer
    // groups over the XCDs
    const KvView kvv = kv_view(h->group, c.n_kv_heads);
    h->max_chunks = max_chunks_for(c.seq_len, c.head_dim, kvv.group, kvv.n_kv_heads, h->n_cu, leap::kMaxChunks);
    const size_t n_pg = std::max<size_t>((size_t)c.max_batch * kvv.n_kv_heads, leap::kXcds);
    const size_t ws_rows = n_pg * kvv.group * leap::records_per_head(h->max_chunks);
    CREATE_TRY(hipMalloc(&h->ws_o, ws_rows * c.head_dim * sizeof(float)));
    CREATE_TRY(hipMalloc(&h->ws_ml, ws_rows * sizeof(float2)));
    // (launch_view's two groups of 2 or 4 q heads per cache head, or four of
    // 2: up to 2 kXcds groups, whose records fit in those of kXcds groups of
    // 4 or 8)
    const bool twins = (kvv.group == 8 || kvv.group == 4) && kvv.kv_split == 0;
    const size_t n_ctr = std::max<size_t>(n_pg, twins ? 2 * leap::kXcds : 0);
    h->counter_bytes = n_ctr * leap::counters_per_group(h->max_chunks) * sizeof(int);
    CREATE_TRY(hipMalloc(&h->ws_po, (size_t)leap::kXcds * h->group * c.head_dim * sizeof(float)));
    CREATE_TRY(hipMalloc(&h->ws_pml, (size_t)leap::kXcds * h->group * sizeof(float2)));
    CREATE_TRY(hipMalloc(&h->counters, h->counter_bytes));
    CREATE_TRY(hipMemsetAsync(h->counters, 0, h->counter_bytes, h->stream));
    // rounded up to 16 bytes: the inputs are staged in as 16-byte words
    h->in_bytes = ((size_t)c.max_batch * ((h->q_dim + 2 * h->kv_dim) * sizeof(float) + sizeof(int)) + 15) / 16 * 16;
    CREATE_TRY(hipMalloc(&h->in_dev, h->in_bytes));
    CREATE_TRY(hipHostMalloc((void **)&h->in_host, h->in_bytes, hipHostMallocDefault));
    CREATE_TRY(hipHostMalloc((void **)&h->out_host, (size_t)c.max_batch * h->q_dim * sizeof(float),
                             hipHostMallocDefault));
    CREATE_TRY(hipMalloc(&h->out_dev, (size_t)c.max_batch * h->q_dim * sizeof(float)));
    CREATE_TRY(hipMalloc(&h->blk, (size_t)(3 * h->q_dim + 2 * h->kv_dim) * sizeof(float)));
    h->w_set.assign(h->n_local, 0);
#ifdef LEAP_TIMELINE
    if (!g_tl_ring) {
        CREATE_TRY(hipMalloc(&g_tl_ring, kTlRingWords * sizeof(unsigned long long)));
        CREATE_TRY(hipMemsetAsync(g_tl_ring, 0, kTlRingWords * sizeof(unsigned long long), h->stream));
    }
#endif
    CREATE_TRY(hipStreamSynchronize(h->stream));
#undef CREATE_TRY
    *out = h;
    return 0;
}

int leap_hip_attention_destroy(leap_hip_attention *h)
{
    if (!h) return 0;
    (void)hipSetDevice(h->cfg.device);  // the handle's device, as for every other call
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    void *bufs[] = {h->ws_po,   h->ws_pml,
                    h->k_cache, h->v_cache, h->rope,  h->ws_o,  h->ws_ml, h->counters, h->in_dev,
                    h->out_dev, h->blk,     h->w_qkv, h->w_o,   h->w_rms, h->w8_qkv,   h->s8_qkv,
                    h->w8_o,    h->s8_o,    h->q8_act, h->q8_act_s};
    for (void *p : bufs)
        if (p) (void)hipFree(p);
    for (void *p : {(void *)h->in_host, (void *)h->out_host})
        if (p) (void)hipHostFree(p);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
    return 0;
}

const char *leap_hip_attention_last_error(const leap_hip_attention *h)
{
    return h ? h->err.c_str() : g_create_error;
}

// The kernel reads q, k_new and v_new and writes out with 8- and 16-byte
// vector accesses.
static inline bool aligned16(const void *p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int leap_hip_attention_step_async(leap_hip_attention *h, int layer, int pos, const float *q,
                                  const float *k_new, const float *v_new, float *out,
                                  void *stream)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (pos < 0 || pos >= h->cfg.seq_len)
        return set_err(h, -EINVAL, "pos %d outside [0, %d)", pos, h->cfg.seq_len);
    if (!q || !k_new || !v_new || !out) return set_err(h, -EINVAL, "NULL buffer");
    if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new) || !aligned16(out))
        return set_err(h, -EINVAL, "q, k_new, v_new and out must be 16-byte aligned");
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    return launch(h, layer, 1, nullptr, pos, pos, pos + 1, q, k_new, v_new, out,
                  (hipStream_t)stream);
}

// ---- the step on caller-owned buffers, allocating nothing ----------------
//
// Its split-K workspace (arrival counters, partial (max, sum) records and
// partial outputs) is this file-scope device array, one copy per device,
// held until the process ends.  Host code uses the address that
// hipGetSymbolAddress returns on each device, never the array's name.

}  // extern "C"

namespace {

constexpr size_t kScratchBytes = 4u << 20;
constexpr int kScratchChunks = 64;  // chunks per launch at most: records_per_head(64) = 72
constexpr int kScratchDevices = 64;
constexpr int kScratchMaxKvHeads = 128;
// The arrival counters sit at the start of the array, in a region of the
// same size for every shape: the records of one shape must never overlap
// the counters of another, which have to stay zero between calls.  Then the
// part records of spread launches (kXcds part-groups of up to 8 heads of
// 128), then a shape's chunk records.
constexpr size_t kScratchCounterBytes =
    (size_t)kScratchMaxKvHeads * leap::counters_per_group(kScratchChunks) * sizeof(int);
constexpr size_t kScratchPartOBytes = (size_t)leap::kXcds * 8 * 128 * sizeof(float);
constexpr size_t kScratchPartMlBytes = (size_t)leap::kXcds * 8 * sizeof(float2);

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchDevice {
    std::once_flag once;
    int rc = 0;
    unsigned char *ptr = nullptr;  // this device's copy of `scratch`
    int n_cu = 0;
    char msg[256] = {};
};
ScratchDevice g_scratch[kScratchDevices];

size_t align256(size_t x) { return (x + 255) / 256 * 256; }

// Bytes of scratch a shape needs: the counter region (fixed), then its
// (max, sum) records, then its partial outputs, each 256-byte aligned.
void scratch_layout(const leap_hip_attention_config &c, size_t *ml_off, size_t *o_off, size_t *total)
{
    // records for the launch groups (kv_view), or for kXcds part-groups of a
    // spread launch
    const KvView v = kv_view(c.n_heads / c.n_kv_heads, c.n_kv_heads);
    const size_t n_pg = std::max<size_t>((size_t)v.n_kv_heads, leap::kXcds);
    const size_t rec = n_pg * (size_t)v.group * leap::records_per_head(kScratchChunks);
    *ml_off = align256(kScratchCounterBytes) + align256(kScratchPartOBytes) + align256(kScratchPartMlBytes);
    *o_off = *ml_off + align256(rec * sizeof(float2));
    *total = *o_off + rec * (size_t)c.head_dim * sizeof(float);
}

// Zero n ints on the device (a kernel rather than a memset, so that a
// caller may capture the first call into a graph).
__global__ void zero_ints_kernel(int *p, size_t n)
{
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

}  // namespace

extern "C" {

int leap_hip_attention_step_noalloc(const leap_hip_attention_config *cfg, int pos, const float *rope,
                                    float *k_cache, float *v_cache, const float *q, const float *k_new,
                                    const float *v_new, float *out, void *stream)
{
    if (!cfg) return set_err(nullptr, -EINVAL, "cfg is NULL");
    const leap_hip_attention_config c = *cfg;
    if (c.n_heads <= 0 || c.n_kv_heads <= 0 || c.n_heads % c.n_kv_heads != 0)
        return set_err(nullptr, -EINVAL, "n_heads %d must be a positive multiple of n_kv_heads %d", c.n_heads,
                       c.n_kv_heads);
    const int group = c.n_heads / c.n_kv_heads;
    if (!shape_supported(c.head_dim, group))
        return set_err(nullptr, -EINVAL, "unsupported head_dim %d with %d q heads per kv head", c.head_dim, group);
    const KvView kvv = kv_view(group, c.n_kv_heads);
    if (c.seq_len <= 0) return set_err(nullptr, -EINVAL, "seq_len %d", c.seq_len);
    if (kvv.n_kv_heads > kScratchMaxKvHeads)
        return set_err(nullptr, -EINVAL,
                       "%d launch groups (%d kv heads of %d q heads): the static workspace holds counters for %d",
                       kvv.n_kv_heads, c.n_kv_heads, group, kScratchMaxKvHeads);
    const unsigned long long slab_bytes = ((unsigned long long)c.seq_len + leap::rows_per_pass(c.head_dim, 1, kWaves)) *
                                          (unsigned long long)c.n_kv_heads * c.head_dim * sizeof(float);
    if (slab_bytes >= (1ull << 32))
        return set_err(nullptr, -EINVAL, "seq_len %d: one layer's cache rows exceed 4 GiB", c.seq_len);
    if (pos < 0 || pos >= c.seq_len) return set_err(nullptr, -EINVAL, "pos %d outside [0, %d)", pos, c.seq_len);
    if (!rope || !k_cache || !v_cache || !q || !k_new || !v_new || !out)
        return set_err(nullptr, -EINVAL, "NULL buffer");
    if (!aligned16(rope) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(q) || !aligned16(k_new) ||
        !aligned16(v_new) || !aligned16(out))
        return set_err(nullptr, -EINVAL, "rope, the caches, q, k_new, v_new and out must be 16-byte aligned");
    size_t ml_off, o_off, need;
    scratch_layout(c, &ml_off, &o_off, &need);
    if (need > kScratchBytes)
        return set_err(nullptr, -EINVAL,
                       "%d heads of %d (%d kv heads) need %zu bytes of workspace; the static workspace holds %zu",
                       c.n_heads, c.head_dim, c.n_kv_heads, need, kScratchBytes);
    if (c.device < 0 || c.device >= kScratchDevices)
        return set_err(nullptr, -EINVAL, "device %d outside [0, %d)", c.device, kScratchDevices);
    if (hipSetDevice(c.device) != hipSuccess) return set_err(nullptr, -ENODEV, "device %d unavailable", c.device);
    ScratchDevice &d = g_scratch[c.device];
    std::call_once(d.once, [&]() {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e == hipSuccess) e = hipDeviceGetAttribute(&d.n_cu, hipDeviceAttributeMultiprocessorCount, c.device);
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (e == hipSuccess) e = hipStreamIsCapturing((hipStream_t)stream, &cap);
        if (e == hipSuccess && cap == hipStreamCaptureStatusNone) e = load_kernel_tables();
        if (e == hipSuccess && cap == hipStreamCaptureStatusNone) {
            // The arrival counters must start at zero (every launch leaves
            // them at zero, and no shape's records overlap them).  The array
            // is zero when the code object loads (it has no initialiser);
            // it is also cleared once, on the first call's stream, ahead of
            // its launch, unless that call is being captured: a clear
            // recorded into the caller's graph would run again at every
            // replay, under the feet of calls on other streams.
            e = launch_k(zero_ints_kernel, dim3(256), dim3(256), (hipStream_t)stream, static_cast<int *>(p),
                         kScratchBytes / sizeof(int));
        }
        if (e != hipSuccess) {
            d.rc = -EIO;
            std::snprintf(d.msg, sizeof d.msg, "static workspace on device %d: %s", c.device, hipGetErrorString(e));
            return;
        }
        d.ptr = static_cast<unsigned char *>(p);
    });
    if (d.rc) return set_err(nullptr, d.rc, "%s", d.msg);
    LaunchShape shape{c.head_dim, kvv.group, c.n_heads, kvv.n_kv_heads, c.seq_len, d.n_cu, 0, kScratchChunks};
    shape.kv_split = kvv.kv_split;
    const size_t po_off = align256(kScratchCounterBytes), pml_off = po_off + align256(kScratchPartOBytes);
    const LaunchBuffers b{k_cache,
                          v_cache,
                          0,
                          reinterpret_cast<const float4 *>(rope),
                          reinterpret_cast<float *>(d.ptr + o_off),
                          reinterpret_cast<float2 *>(d.ptr + ml_off),
                          reinterpret_cast<int *>(d.ptr),
                          reinterpret_cast<float *>(d.ptr + po_off),
                          reinterpret_cast<float2 *>(d.ptr + pml_off)};
    const hipError_t e = launch_attention(shape, b, 1, nullptr, pos, pos, pos + 1, q, k_new, v_new, out,
                                          (hipStream_t)stream);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_err(nullptr, -EIO, "launch: %s", hipGetErrorString(e));
    }
    return 0;
}

int leap_hip_attention_step(leap_hip_attention *h, int layer, int pos, const float *q,
                            const float *k_new, const float *v_new, float *out)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (pos < 0 || pos >= h->cfg.seq_len)
        return set_err(h, -EINVAL, "pos %d outside [0, %d)", pos, h->cfg.seq_len);
    if (!q || !k_new || !v_new || !out) return set_err(h, -EINVAL, "NULL buffer");
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    hipStream_t s = h->stream;
    const size_t qb = h->q_dim * sizeof(float), kb = h->kv_dim * sizeof(float);
    std::memcpy(h->in_host, q, qb);
    std::memcpy(h->in_host + qb, k_new, kb);
    std::memcpy(h->in_host + qb + kb, v_new, kb);
    const int n16 = (int)((qb + 2 * kb) / 16);
    HIP_TRY(h, launch_k(leap::stage_in_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), s,
                        reinterpret_cast<float4 *>(h->in_dev), reinterpret_cast<const float4 *>(h->in_host), n16));
    const float *qd = reinterpret_cast<const float *>(h->in_dev);
    // The output goes straight to the pinned buffer (device-accessible host
    // memory): the kernel's final stores cross PCIe, with no copy after it.
    if (int rc = launch(h, layer, 1, nullptr, pos, pos, pos + 1, qd, qd + h->q_dim, qd + h->q_dim + h->kv_dim,
                        h->out_host, s))
        return rc;
    HIP_TRY(h, hipStreamSynchronize(s));
    std::memcpy(out, h->out_host, qb);
    return 0;
}

int leap_hip_attention_step_batched_async(leap_hip_attention *h, int layer, int n_seq,
                                          const int *pos, int max_pos, long long total_rows,
                                          const float *q, const float *k_new, const float *v_new,
                                          float *out, void *stream)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (n_seq <= 0 || n_seq > h->cfg.max_batch)
        return set_err(h, -EINVAL, "n_seq %d outside [1, %d]", n_seq, h->cfg.max_batch);
    if (max_pos < 0 || max_pos >= h->cfg.seq_len)
        return set_err(h, -EINVAL, "max_pos %d outside [0, %d)", max_pos, h->cfg.seq_len);
    if (!pos || !q || !k_new || !v_new || !out) return set_err(h, -EINVAL, "NULL buffer");
    if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new) || !aligned16(out) ||
        reinterpret_cast<uintptr_t>(pos) % 4)
        return set_err(h, -EINVAL, "q, k_new, v_new and out must be 16-byte aligned, pos 4-byte aligned");
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    if (total_rows < 0 || total_rows > (long long)n_seq * (max_pos + 1))
        return set_err(h, -EINVAL, "total_rows %lld outside [0, %lld]", total_rows,
                       (long long)n_seq * (max_pos + 1));
    // Without the host's row count, size the chunks as if the lengths were
    // spread evenly up to the longest.
    const long long rows = total_rows > 0 ? total_rows : (long long)n_seq * (max_pos + 1) / 2 + 1;
    return launch(h, layer, n_seq, pos, 0, max_pos, rows, q, k_new, v_new, out,
                  (hipStream_t)stream);
}

int leap_hip_attention_step_batched(leap_hip_attention *h, int layer, int n_seq, const int *pos,
                                    const float *q, const float *k_new, const float *v_new,
                                    float *out)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (n_seq <= 0 || n_seq > h->cfg.max_batch)
        return set_err(h, -EINVAL, "n_seq %d outside [1, %d]", n_seq, h->cfg.max_batch);
    if (!pos || !q || !k_new || !v_new || !out) return set_err(h, -EINVAL, "NULL buffer");
    int max_pos = 0;
    long long rows = 0;
    for (int i = 0; i < n_seq; i++) {
        if (pos[i] < 0 || pos[i] >= h->cfg.seq_len)
            return set_err(h, -EINVAL, "pos[%d] = %d outside [0, %d)", i, pos[i], h->cfg.seq_len);
        max_pos = std::max(max_pos, pos[i]);
        rows += pos[i] + 1;
    }
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    hipStream_t s = h->stream;
    // packed for n_seq: q rows | k rows | v rows | pos (every offset a multiple of 256 bytes but pos's)
    const size_t qb = (size_t)n_seq * h->q_dim * sizeof(float), kb = (size_t)n_seq * h->kv_dim * sizeof(float);
    std::memcpy(h->in_host, q, qb);
    std::memcpy(h->in_host + qb, k_new, kb);
    std::memcpy(h->in_host + qb + kb, v_new, kb);
    std::memcpy(h->in_host + qb + 2 * kb, pos, n_seq * sizeof(int));
    const int n16 = (int)((qb + 2 * kb + n_seq * sizeof(int) + 15) / 16);  // in_bytes is a multiple of 16
    HIP_TRY(h, launch_k(leap::stage_in_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), s,
                        reinterpret_cast<float4 *>(h->in_dev), reinterpret_cast<const float4 *>(h->in_host), n16));
    const float *qd = reinterpret_cast<const float *>(h->in_dev);
    const float *kd = qd + (size_t)n_seq * h->q_dim, *vd = kd + (size_t)n_seq * h->kv_dim;
    const int *pd = reinterpret_cast<const int *>(h->in_dev + qb + 2 * kb);
    if (int rc = launch(h, layer, n_seq, pd, 0, max_pos, rows, qd, kd, vd, h->out_host, s)) return rc;
    HIP_TRY(h, hipStreamSynchronize(s));
    std::memcpy(out, h->out_host, qb);
    return 0;
}

int leap_hip_attention_set_layer_weights(leap_hip_attention *h, int layer, const float *rms_att,
                                         const float *wq, const float *wk, const float *wv,
                                         const float *wo)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (!rms_att || !wq || !wk || !wv || !wo) return set_err(h, -EINVAL, "NULL weight");
    QkvFn qkv;
    ProjFn proj;
    int rb;
    const int dim = h->q_dim, kv = h->kv_dim;
    if (!pick_proj(dim, &qkv, &proj, &rb))
        return set_err(h, -EINVAL, "dim %d: the projections need dim in {2048, 3072, 4096, 5120, 8192}", dim);
    if (h->w_fmt == 2) return set_err(h, -EINVAL, "this handle holds int8 weights");
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    const size_t n_qkv = (size_t)(dim + 2 * kv) * dim, n_o = (size_t)dim * dim;
    if (!h->w_qkv) {
        if (int rc = alloc_all(h, {{(void **)&h->w_qkv, (size_t)h->n_local * n_qkv * sizeof(float)},
                                   {(void **)&h->w_o, (size_t)h->n_local * n_o * sizeof(float)},
                                   {(void **)&h->w_rms, (size_t)h->n_local * dim * sizeof(float)}}))
            return rc;
        h->w_fmt = 1;
    }
    const int li = layer - h->cfg.layer_begin;
    float *dq = h->w_qkv + (size_t)li * n_qkv;
    hipStream_t s = h->stream;
    HIP_TRY(h, hipMemcpyAsync(dq, wq, (size_t)dim * dim * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(dq + (size_t)dim * dim, wk, (size_t)kv * dim * sizeof(float),
                              hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(dq + (size_t)(dim + kv) * dim, wv, (size_t)kv * dim * sizeof(float),
                              hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(h->w_o + (size_t)li * n_o, wo, n_o * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(h->w_rms + (size_t)li * dim, rms_att, (size_t)dim * sizeof(float),
                              hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    h->w_set[li] = 1;
    return 0;
}

int leap_hip_attention_set_layer_weights_q8(leap_hip_attention *h, int layer, int group_size,
                                            const float *rms_att, const int8_t *wq, const float *wq_s,
                                            const int8_t *wk, const float *wk_s, const int8_t *wv,
                                            const float *wv_s, const int8_t *wo, const float *wo_s)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (!rms_att || !wq || !wq_s || !wk || !wk_s || !wv || !wv_s || !wo || !wo_s)
        return set_err(h, -EINVAL, "NULL weight");
    const int dim = h->q_dim, kv = h->kv_dim, gs = group_size;
    if (!q8_supported(dim, gs))
        return set_err(h, -EINVAL,
                       "dim %d with group size %d: the int8 projections need dim and group size 2048 with "
                       "32-128, 3072 with 32-128, 4096 with 32-256, 5120 with 64-128 or 8192 with 64-256",
                       dim, gs);
    if (h->w_fmt == 1) return set_err(h, -EINVAL, "this handle holds fp32 weights");
    if (h->w_fmt == 2 && gs != h->gs)
        return set_err(h, -EINVAL, "group size %d differs from the handle's %d", gs, h->gs);
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    const size_t rows_qkv = (size_t)(dim + 2 * kv), ng = (size_t)(dim / gs);
    if (!h->w8_qkv) {
        if (int rc = alloc_all(h, {{(void **)&h->w8_qkv, (size_t)h->n_local * rows_qkv * dim},
                                   {(void **)&h->s8_qkv, (size_t)h->n_local * rows_qkv * ng * sizeof(float)},
                                   {(void **)&h->w8_o, (size_t)h->n_local * dim * dim},
                                   {(void **)&h->s8_o, (size_t)h->n_local * dim * ng * sizeof(float)},
                                   {(void **)&h->w_rms, (size_t)h->n_local * dim * sizeof(float)},
                                   {(void **)&h->q8_act, (size_t)2 * dim},
                                   {(void **)&h->q8_act_s, 2 * ng * sizeof(float)}}))
            return rc;
        h->gs = gs;
        h->w_fmt = 2;
    }
    const int li = layer - h->cfg.layer_begin;
    int8_t *dq = h->w8_qkv + (size_t)li * rows_qkv * dim;
    float *ds = h->s8_qkv + (size_t)li * rows_qkv * ng;
    hipStream_t s = h->stream;
    const size_t nq = (size_t)dim * dim, nk = (size_t)kv * dim;
    HIP_TRY(h, hipMemcpyAsync(dq, wq, nq, hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(dq + nq, wk, nk, hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(dq + nq + nk, wv, nk, hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(ds, wq_s, nq / gs * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(ds + nq / gs, wk_s, nk / gs * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(ds + (nq + nk) / gs, wv_s, nk / gs * sizeof(float), hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(h->w8_o + (size_t)li * nq, wo, nq, hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(h->s8_o + (size_t)li * nq / gs, wo_s, nq / gs * sizeof(float),
                              hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipMemcpyAsync(h->w_rms + (size_t)li * dim, rms_att, (size_t)dim * sizeof(float),
                              hipMemcpyHostToDevice, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    h->w_set[li] = 1;
    return 0;
}

int leap_hip_attention_block_views_get(leap_hip_attention *h, leap_hip_attention_block_views *out)
{
    if (!h) return -EINVAL;
    if (!out) return set_err(h, -EINVAL, "NULL output");
    const int dim = h->q_dim, kv = h->kv_dim;
    out->q = h->blk;
    out->k = h->blk + dim;
    out->v = h->blk + dim + kv;
    out->att = h->blk + dim + 2 * kv;
    out->xq = h->q8_act;
    out->xs = h->q8_act_s;
    out->aq = h->q8_act ? h->q8_act + dim : nullptr;
    out->as = h->q8_act_s ? h->q8_act_s + dim / h->gs : nullptr;
    return 0;
}

int leap_hip_attention_block_async(leap_hip_attention *h, int layer, int pos, float *x, void *stream)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (pos < 0 || pos >= h->cfg.seq_len)
        return set_err(h, -EINVAL, "pos %d outside [0, %d)", pos, h->cfg.seq_len);
    if (!x) return set_err(h, -EINVAL, "NULL buffer");
    if (reinterpret_cast<uintptr_t>(x) % 16) return set_err(h, -EINVAL, "x must be 16-byte aligned");
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    return launch_block(h, layer, pos, x, x, (hipStream_t)stream);
}

int leap_hip_attention_block(leap_hip_attention *h, int layer, int pos, float *x)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (pos < 0 || pos >= h->cfg.seq_len)
        return set_err(h, -EINVAL, "pos %d outside [0, %d)", pos, h->cfg.seq_len);
    if (!x) return set_err(h, -EINVAL, "NULL buffer");
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    hipStream_t s = h->stream;
    float *xd = h->blk + 2 * h->q_dim + 2 * h->kv_dim;
    const size_t xb = (size_t)h->q_dim * sizeof(float);
    std::memcpy(h->out_host, x, xb);  // through pinned memory: staged in by a kernel, one DMA out
    HIP_TRY(h, launch_k(leap::stage_in_kernel, dim3((unsigned)((xb / 16 + 255) / 256)), dim3(256), s,
                        reinterpret_cast<float4 *>(xd), reinterpret_cast<const float4 *>(h->out_host), (int)(xb / 16)));
    if (int rc = launch_block(h, layer, pos, xd, xd, s)) return rc;
    // (adding the wo product straight into the pinned copy measured slower:
    // the residual reads cross PCIe on the wo kernel's critical path)
    HIP_TRY(h, hipMemcpyAsync(h->out_host, xd, xb, hipMemcpyDeviceToHost, s));
    HIP_TRY(h, hipStreamSynchronize(s));
    std::memcpy(x, h->out_host, xb);
    return 0;
}

// ---- stage hand-off -------------------------------------------------------

int leap_hip_attention_packet_header(const void *packet, size_t bytes, int dim, int *pos, int *flags)
{
    constexpr size_t kHead = LEAP_HIP_ATTENTION_PACKET_HEADER_BYTES;
    if (!packet || dim <= 0 || bytes != kHead + sizeof(float) * (size_t)dim) return -EINVAL;
    uint16_t magic;
    std::memcpy(&magic, packet, sizeof magic);
    if (magic == LEAP_HIP_ATTENTION_CONTROL_MAGIC) return 1;
    int32_t head[2];
    std::memcpy(head, packet, sizeof head);
    if (pos) *pos = head[0];
    if (flags) *flags = head[1];
    return 0;
}

int leap_hip_attention_packet_upload(leap_hip_attention *h, const void *packet, size_t bytes, float *x,
                                     int *pos, int *flags, void *stream)
{
    if (!h) return -EINVAL;
    if (!packet || !x || !pos || !flags) return set_err(h, -EINVAL, "NULL buffer");
    int p, f;
    const int rc = leap_hip_attention_packet_header(packet, bytes, h->q_dim, &p, &f);
    if (rc < 0) return set_err(h, rc, "packet of %zu bytes, expected %zu", bytes,
                               LEAP_HIP_ATTENTION_PACKET_HEADER_BYTES + sizeof(float) * (size_t)h->q_dim);
    if (rc == 1) return 1;
    if (p < 0 || p >= h->cfg.seq_len) return set_err(h, -EINVAL, "packet pos %d outside [0, %d)", p, h->cfg.seq_len);
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    const char *src = static_cast<const char *>(packet) + LEAP_HIP_ATTENTION_PACKET_HEADER_BYTES;
    HIP_TRY(h, hipMemcpyAsync(x, src, sizeof(float) * (size_t)h->q_dim, hipMemcpyHostToDevice, s));
    if (!stream) HIP_TRY(h, hipStreamSynchronize(s));
    *pos = p;
    *flags = f;
    return 0;
}

int leap_hip_attention_packet_download(leap_hip_attention *h, const float *x, int pos, int flags, void *packet,
                                       size_t bytes, void *stream)
{
    if (!h) return -EINVAL;
    if (!packet || !x) return set_err(h, -EINVAL, "NULL buffer");
    constexpr size_t kHead = LEAP_HIP_ATTENTION_PACKET_HEADER_BYTES;
    if (bytes != kHead + sizeof(float) * (size_t)h->q_dim)
        return set_err(h, -EINVAL, "packet of %zu bytes, expected %zu", bytes, kHead + sizeof(float) * (size_t)h->q_dim);
    if (pos < 0 || pos >= h->cfg.seq_len) return set_err(h, -EINVAL, "pos %d outside [0, %d)", pos, h->cfg.seq_len);
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    hipStream_t s = stream ? (hipStream_t)stream : h->stream;
    const int32_t head[2] = {pos, flags};
    std::memcpy(packet, head, sizeof head);
    HIP_TRY(h, hipMemcpyAsync(static_cast<char *>(packet) + kHead, x, sizeof(float) * (size_t)h->q_dim,
                              hipMemcpyDeviceToHost, s));
    if (!stream) HIP_TRY(h, hipStreamSynchronize(s));
    return 0;
}

int leap_hip_attention_clear(leap_hip_attention *h)
{
    if (!h) return -EINVAL;
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    const size_t bytes = (size_t)h->cfg.max_batch * h->slab_floats * sizeof(float);
    HIP_TRY(h, hipMemsetAsync(h->k_cache, 0, bytes, h->stream));
    HIP_TRY(h, hipMemsetAsync(h->v_cache, 0, bytes, h->stream));
    // The merge's arrival counters too: they are zero between launches, and
    // clearing them lets a handle recover after launches that overlapped on
    // two streams.
    HIP_TRY(h, hipMemsetAsync(h->counters, 0, h->counter_bytes, h->stream));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    return 0;
}

static int kv_range(leap_hip_attention *h, int seq, int layer, int pos_begin, int pos_end,
                    size_t *off, size_t *n)
{
    if (!h) return -EINVAL;
    if (int rc = check_layer(h, layer)) return rc;
    if (seq < 0 || seq >= h->cfg.max_batch)
        return set_err(h, -EINVAL, "seq %d outside [0, %d)", seq, h->cfg.max_batch);
    if (pos_begin < 0 || pos_end > h->cfg.seq_len || pos_begin > pos_end)
        return set_err(h, -EINVAL, "position range [%d, %d) outside [0, %d)", pos_begin, pos_end,
                       h->cfg.seq_len);
    *off = (size_t)seq * h->slab_floats + (size_t)(layer - h->cfg.layer_begin) * h->layer_floats +
           (size_t)pos_begin * h->kv_dim;
    *n = (size_t)(pos_end - pos_begin) * h->kv_dim;
    return 0;
}

int leap_hip_attention_kv_upload(leap_hip_attention *h, int seq, int layer, int pos_begin,
                                 int pos_end, const float *k, const float *v)
{
    size_t off, n;
    if (int rc = kv_range(h, seq, layer, pos_begin, pos_end, &off, &n)) return rc;
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    if (n == 0) return 0;
    if (k) HIP_TRY(h, hipMemcpyAsync(h->k_cache + off, k, n * sizeof(float), hipMemcpyHostToDevice, h->stream));
    if (v) HIP_TRY(h, hipMemcpyAsync(h->v_cache + off, v, n * sizeof(float), hipMemcpyHostToDevice, h->stream));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    return 0;
}

int leap_hip_attention_kv_download(leap_hip_attention *h, int seq, int layer, int pos_begin,
                                   int pos_end, float *k, float *v)
{
    size_t off, n;
    if (int rc = kv_range(h, seq, layer, pos_begin, pos_end, &off, &n)) return rc;
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    if (n == 0) return 0;
    if (k) HIP_TRY(h, hipMemcpyAsync(k, h->k_cache + off, n * sizeof(float), hipMemcpyDeviceToHost, h->stream));
    if (v) HIP_TRY(h, hipMemcpyAsync(v, h->v_cache + off, n * sizeof(float), hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    return 0;
}

int leap_hip_attention_kv_fill_normal(leap_hip_attention *h, uint64_t seed, float scale)
{
    if (!h) return -EINVAL;
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    const size_t n = (size_t)h->cfg.max_batch * h->slab_floats;
    const int blocks = 256 * 16;
    HIP_TRY(h, launch_k(leap::fill_normal_kernel, dim3(blocks), dim3(256), h->stream, h->k_cache, n, seed, scale));
    HIP_TRY(h, launch_k(leap::fill_normal_kernel, dim3(blocks), dim3(256), h->stream, h->v_cache, n,
                        seed ^ 0x5DEECE66DA3B9F21ull, scale));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    return 0;
}

int leap_hip_attention_rope_download(leap_hip_attention *h, int pos_begin, int pos_end,
                                     float *cos_out, float *sin_out)
{
    if (!h) return -EINVAL;
    if (pos_begin < 0 || pos_end > h->cfg.seq_len || pos_begin > pos_end)
        return set_err(h, -EINVAL, "position range [%d, %d) outside [0, %d)", pos_begin, pos_end,
                       h->cfg.seq_len);
    if (!cos_out || !sin_out) return set_err(h, -EINVAL, "NULL buffer");
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    const size_t half = h->cfg.head_dim / 2;
    const size_t n = (size_t)(pos_end - pos_begin) * half;
    if (n == 0) return 0;
    std::vector<float> packed(2 * n);
    HIP_TRY(h, hipMemcpyAsync(packed.data(),
                              reinterpret_cast<float *>(h->rope) + 2 * (size_t)pos_begin * half,
                              packed.size() * sizeof(float), hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(h, hipStreamSynchronize(h->stream));
    for (size_t i = 0; i < n; i++) {
        cos_out[i] = packed[2 * i];
        sin_out[i] = packed[2 * i + 1];
    }
    return 0;
}

int leap_hip_attention_floor_async(leap_hip_attention *h, int kind, int layer, int n_seq, const int *pos,
                                   int max_pos, long long total_rows, void *stream)
{
    if (!h) return -EINVAL;
    if (kind != kFloorLaunch && kind != kFloorStream && kind != kFloorBlock)
        return set_err(h, -EINVAL, "floor kind %d is not 1, 2 or 3", kind);
    if (int rc = check_layer(h, layer)) return rc;
    if (n_seq <= 0 || n_seq > h->cfg.max_batch)
        return set_err(h, -EINVAL, "n_seq %d outside [1, %d]", n_seq, h->cfg.max_batch);
    if (max_pos < 0 || max_pos >= h->cfg.seq_len)
        return set_err(h, -EINVAL, "max_pos %d outside [0, %d)", max_pos, h->cfg.seq_len);
    if (total_rows <= 0 || total_rows > (long long)n_seq * (max_pos + 1))
        return set_err(h, -EINVAL, "total_rows %lld outside [1, %lld]", total_rows, (long long)n_seq * (max_pos + 1));
    if (reinterpret_cast<uintptr_t>(pos) % 4) return set_err(h, -EINVAL, "pos must be 4-byte aligned");
    if (kind == kFloorBlock) {
        if (n_seq != 1 || pos || total_rows != (long long)max_pos + 1)
            return set_err(h, -EINVAL, "the sub-block floor takes one sequence at max_pos (pos NULL)");
        HIP_TRY(h, hipSetDevice(h->cfg.device));
        return launch_block_floor(h, layer, max_pos, (hipStream_t)stream);
    }
    if (spreads(launch_view(shape_of(h), n_seq, total_rows), n_seq, total_rows))
        return set_err(h, -EINVAL,
                       "%d sequences of %d KV heads and %lld rows spread over the XCDs in the step; the floor "
                       "kernels have no spread grid",
                       n_seq, h->cfg.n_kv_heads, total_rows);
    HIP_TRY(h, hipSetDevice(h->cfg.device));
    // with pos NULL, every sequence at max_pos
    return launch(h, layer, n_seq, pos, max_pos, max_pos, total_rows, nullptr, nullptr, nullptr, h->out_dev,
                  (hipStream_t)stream, kind);
}

int leap_hip_attention_set_products(leap_hip_attention *h, int valu)
{
    if (!h) return -EINVAL;
    if (valu != 0 && valu != 1) return set_err(h, -EINVAL, "products mode %d is not 0 (MFMA) or 1 (VALU)", valu);
    h->valu = valu == 1;
    return 0;
}

int leap_hip_attention_set_fold_helper(leap_hip_attention *h, int mode)
{
    if (!h) return -EINVAL;
    if (mode < 0 || mode > 2) return set_err(h, -EINVAL, "fold helper mode %d is not 0, 1 or 2", mode);
    h->fold_helper = mode;
    return 0;
}

int leap_hip_attention_set_split(leap_hip_attention *h, int chunk_positions)
{
    if (!h) return -EINVAL;
    if (chunk_positions < 0 || chunk_positions % 8 != 0)
        return set_err(h, -EINVAL, "chunk %d is not a non-negative multiple of 8",
                       chunk_positions);
    h->split = chunk_positions;
    return 0;
}

int leap_hip_attention_load_checkpoint(leap_hip_attention *h, const char *path)
{
    if (!h) return -EINVAL;
    if (!path) return set_err(h, -EINVAL, "NULL path");
    leap_hip_attention_checkpoint c;
    if (int rc = leap_hip_attention_checkpoint_read(path, &c))
        return set_err(h, rc, "%s: %s", path, rc == -EIO ? "cannot read" : "not a LEAP checkpoint");
    const leap_hip_attention_config &hc = h->cfg;
    if (c.n_layers != hc.n_layers || c.n_heads != hc.n_heads || c.n_kv_heads != hc.n_kv_heads ||
        c.dim != hc.n_heads * hc.head_dim)
        return set_err(h, -EINVAL, "%s: model %d layers, %d/%d heads, dim %d; the handle holds %d layers, %d/%d heads of %d",
                       path, c.n_layers, c.n_heads, c.n_kv_heads, c.dim, hc.n_layers, hc.n_heads, hc.n_kv_heads,
                       hc.head_dim);
    if (c.attention_bytes < c.header_bytes || c.file_bytes < c.attention_bytes)
        return set_err(h, -EINVAL, "%s: %lld bytes, the attention weights need %lld", path, c.file_bytes,
                       c.attention_bytes);
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return set_err(h, -EIO, "%s: cannot open", path);
    void *map = mmap(nullptr, (size_t)c.file_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return set_err(h, -EIO, "%s: cannot map", path);
    const char *base = static_cast<const char *>(map);
    int rc = 0;
    for (int layer = hc.layer_begin; layer < hc.layer_end && rc == 0; layer++) {
        leap::CkptLayer o;
        size_t needed;
        if (!leap::ckpt_layer(c, layer, &o, &needed)) {
            rc = set_err(h, -EINVAL, "%s: tensor sizes overflow", path);
            break;
        }
        const auto f32 = [&](size_t off) { return reinterpret_cast<const float *>(base + off); };
        const auto i8 = [&](size_t off) { return reinterpret_cast<const int8_t *>(base + off); };
        if (c.version == 2)
            rc = leap_hip_attention_set_layer_weights_q8(h, layer, c.group_size, f32(o.rms_att), i8(o.wq), f32(o.wq_s),
                                                         i8(o.wk), f32(o.wk_s), i8(o.wv), f32(o.wv_s), i8(o.wo),
                                                         f32(o.wo_s));
        else
            rc = leap_hip_attention_set_layer_weights(h, layer, f32(o.rms_att), f32(o.wq), f32(o.wk), f32(o.wv),
                                                      f32(o.wo));
    }
    munmap(map, (size_t)c.file_bytes);
    return rc;
}

int leap_hip_attention_timeline(void *dst, size_t bytes, long long *launches)
{
#ifdef LEAP_TIMELINE
    if (!dst || !launches) return set_err(nullptr, -EINVAL, "NULL buffer");
    if (bytes < kTlRingWords * sizeof(unsigned long long))
        return set_err(nullptr, -EINVAL, "the timeline ring is %zu bytes", kTlRingWords * sizeof(unsigned long long));
    if (!g_tl_ring) return set_err(nullptr, -EINVAL, "no handle has been created");
    const hipError_t e = hipMemcpy(dst, g_tl_ring, kTlRingWords * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return set_err(nullptr, -EIO, "timeline copy: %s", hipGetErrorString(e));
    }
    *launches = g_tl_launches;
    return 0;
#else
    (void)dst;
    (void)bytes;
    (void)launches;
    return set_err(nullptr, -ENOTSUP, "this library has no timeline: load libleap_hip_attention_tl.so");
#endif
}

int leap_hip_attention_kv_device_ptr(leap_hip_attention *h, int seq, int layer, float **k,
                                     float **v)
{
    size_t off, n;
    if (int rc = kv_range(h, seq, layer, 0, 0, &off, &n)) return rc;
    if (k) *k = h->k_cache + off;
    if (v) *v = h->v_cache + off;
    return 0;
}

}  // extern "C"
