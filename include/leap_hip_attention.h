/*
 * leap_hip_attention — MI355X (gfx950) decode attention for the LEAP engine.
 *
 * Replaces the per-token attention block of the reference engine's layer
 * step: RoPE on q and k, the key/value cache write, the GQA score pass,
 * softmax and the weighted-V accumulation.  In the reference that block is
 * inline code between the v projection and the wo projection:
 *   src/inference/FloatTransformer.cpp:396-662   (fp32 engine)
 *   src/inference/QuantizedTransformer.cpp:670-923 (int8 engine, same fp32 block)
 * Entry state: the un-rotated q, k, v of one token for one layer.
 * Exit state:  the head-major attention output (the reference's s->xb) and the
 *              rotated k / plain v stored in cache[layer][pos].
 *
 * The key/value caches live in device memory with the reference's layout,
 * one slab per sequence: [layer][pos][n_kv_heads*head_dim] fp32 (the
 * reference's RunState key_cache/value_cache, FloatTransformer.cpp:50-51,
 * offset l*seq_len*kv_dim + pos*kv_dim, :396-398), with 64-bit offsets.
 *
 * Conventions
 *   - Every entry point returns 0 on success or a negative errno value:
 *     -EINVAL bad argument, -ENOMEM allocation failure, -ENODEV no usable
 *     GPU, -ENOTSUP a device that does not place workgroups the way the
 *     kernel's merge needs (checked at create), -EIO a HIP runtime error.
 *     The message of the last failure on a handle is kept for
 *     leap_hip_attention_last_error.  Nothing throws across this boundary.
 *   - A handle is used by one host thread at a time; distinct handles are
 *     independent.  Device work is ordered on a stream: the host-pointer
 *     entry points use the handle's own stream and return when results are
 *     in host memory; the _async entry points take device pointers and a
 *     hipStream_t (0 = the legacy default stream) and return after
 *     enqueueing.
 *   - Every launch of a handle shares its caches, its split-K workspace and
 *     its arrival counters, so launches of one handle must not overlap.  The
 *     handle's own stream is ordered with the legacy default stream; after
 *     _async calls on any other stream, synchronise that stream (or make the
 *     next stream wait for it) before a host-pointer call, clear, a
 *     kv_upload/kv_download, set_layer_weights*, load_checkpoint or
 *     destroy, and before _async calls on a different stream.  Launches that
 *     overlapped leave the counters inconsistent and later outputs wrong;
 *     leap_hip_attention_clear resets them.
 *   - `layer` is the model's global layer index, as in the reference's layer
 *     loop (FloatTransformer.cpp:768-770); a handle holds the layers
 *     [layer_begin, layer_end).
 */
#ifndef LEAP_HIP_ATTENTION_H
#define LEAP_HIP_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct leap_hip_attention leap_hip_attention;

/* Model dimensions (the reference's Config, Config.h:5-13, restricted to what
 * attention needs) plus the RoPE base, which the reference fixes at 500000
 * (FloatTransformer.cpp:65) and its file header does not carry. */
typedef struct leap_hip_attention_config {
    int n_layers;    /* model layers (range check for `layer`)                 */
    int layer_begin; /* first layer held by this handle                        */
    int layer_end;   /* one past the last layer held                           */
    int n_heads;     /* query heads                                            */
    int n_kv_heads;  /* key/value heads; n_heads / n_kv_heads in {1,2,3,4,8,16} */
    int head_dim;    /* dim / n_heads: 64 or 128                               */
    int seq_len;     /* cache rows per layer (Config.seq_len)                  */
    float rope_theta;/* 500000 in the reference; <= 0 selects 500000           */
    int max_batch;   /* sequences (cache slabs) held; 1 for the engine         */
    int device;      /* HIP device ordinal                                     */
} leap_hip_attention_config;

/* Allocates both caches (zeroed, as the reference's std::vector resize),
 * builds the fp32 RoPE table on the host with the reference's formula
 * (FloatTransformer.cpp:56-72) and uploads it, and allocates the split-K
 * workspace.  Replaces init_run_state / precompute_freqs
 * (FloatTransformer.cpp:39-72) for the attention state. */
int leap_hip_attention_create(const leap_hip_attention_config *cfg, leap_hip_attention **out);

/* Frees everything the handle owns.  NULL is accepted. */
int leap_hip_attention_destroy(leap_hip_attention *h);

/* Message of the last failure on `h` ("" if none); with h == NULL, the last
 * failure on this thread of a call made without a handle
 * (leap_hip_attention_create, leap_hip_attention_step_noalloc,
 * leap_hip_attention_xcc_map). */
const char *leap_hip_attention_last_error(const leap_hip_attention *h);

/* One token, one layer, sequence 0 (FloatTransformer.cpp:396-662).
 *   q     [n_heads*head_dim]   pre-RoPE query (the reference's s->q)
 *   k_new [kv_dim]             pre-RoPE key of this token
 *   v_new [kv_dim]             value of this token
 *   out   [n_heads*head_dim]   attention output (the reference's s->xb)
 * Host pointers; returns when `out` is written.  0 <= pos < seq_len. */
int leap_hip_attention_step(leap_hip_attention *h, int layer, int pos, const float *q,
                            const float *k_new, const float *v_new, float *out);

/* As leap_hip_attention_step, with device pointers, enqueued on `stream`.
 * q, k_new, v_new and out must be 16-byte aligned (-EINVAL otherwise). */
int leap_hip_attention_step_async(leap_hip_attention *h, int layer, int pos, const float *q,
                                  const float *k_new, const float *v_new, float *out,
                                  void *stream);

/* n_seq independent sequences (slabs 0..n_seq-1) at one layer, each at its
 * own position pos[i] (ragged contexts).  Rows are [n_seq][...] with the
 * per-sequence sizes of leap_hip_attention_step.  Host pointers.  The
 * reference runs one sequence per engine; this is that step applied to a
 * batch of engines' states. */
int leap_hip_attention_step_batched(leap_hip_attention *h, int layer, int n_seq, const int *pos,
                                    const float *q, const float *k_new, const float *v_new,
                                    float *out);

/* As leap_hip_attention_step_batched with device pointers (pos included),
 * enqueued on `stream`.  max_pos is a host-side upper bound of pos[] used to
 * size the launch; a sequence whose pos lies outside [0, max_pos] or at or
 * beyond seq_len is skipped: its cache rows are neither read nor written,
 * and its output row is filled with NaN so that a caller's bad position
 * cannot pass for attention output.  total_rows is the
 * host's sum of pos[i] + 1 when it has one (it only steers the split of the
 * positions over workgroups), or 0 when it does not: the launch is then
 * sized as if the sequences were spread evenly up to max_pos.  q, k_new,
 * v_new and out must be 16-byte aligned and pos 4-byte aligned (-EINVAL
 * otherwise). */
int leap_hip_attention_step_batched_async(leap_hip_attention *h, int layer, int n_seq,
                                          const int *pos, int max_pos, long long total_rows,
                                          const float *q, const float *k_new, const float *v_new,
                                          float *out, void *stream);

/* clear_kv_cache (FloatTransformer.cpp:74-77): zero both caches (and the
 * split-K merge's arrival counters). */
int leap_hip_attention_clear(leap_hip_attention *h);

/* Copy cache rows [pos_begin, pos_end) of (seq, layer) between host memory
 * and the device cache, in the reference's row layout ([pos][kv_dim]).
 * Either k or v may be NULL to skip it.  Used for checkpoints, tests and to
 * hand the same bytes to a CPU path. */
int leap_hip_attention_kv_upload(leap_hip_attention *h, int seq, int layer, int pos_begin,
                                 int pos_end, const float *k, const float *v);
int leap_hip_attention_kv_download(leap_hip_attention *h, int seq, int layer, int pos_begin,
                                   int pos_end, float *k, float *v);

/* The attention step of leap_hip_attention_step_async for one sequence on
 * caller-owned device buffers, allocating nothing: no handle, no hipMalloc,
 * no allocating library call.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  The split-K workspace is
 * a 4 MiB static device array, one per device (held until the process ends):
 * a fixed 144 KiB region of arrival counters for at most 128 launch groups
 * (128 KV heads, or 64 with 16 q heads per KV head, whose heads run as two
 * groups each; small launches of 4 or 8 q heads per KV head run as up to 16
 * groups of 2 or 4 q heads) and 33 KiB of part records, then n_heads x 72 partial
 * records of (head_dim + 2) floats (for at least 8 KV heads' worth of q
 * heads), at most 64 split-K chunks per call (up to 107 heads of 128 or 211
 * heads of 64; Llama-3-8B uses 1.38 MB, Llama-3-70B 2.58 MB); larger shapes
 * return -EINVAL.  Every call on one device shares that array: launches
 * leave the counters at zero, and the array is zero from the start (the
 * first call on a device that is not under stream capture also clears it
 * on its stream, ahead of its launch), so calls that overlap on one GPU,
 * on any streams, race.
 *   cfg      n_heads, n_kv_heads, head_dim, seq_len and device are read
 *   rope     [seq_len][head_dim/2] (cos, sin) pairs of fp32: row p holds
 *            cos(p * f_i), sin(p * f_i) for f_i = theta^(-2i/head_dim),
 *            i < head_dim/2, each pair adjacent
 *   k_cache, v_cache  this layer's cache rows of the sequence,
 *            [seq_len][kv_dim] row-major, kv_dim = n_kv_heads * head_dim;
 *            row pos is written (rotated k, v)
 *   q, k_new, v_new, out   as leap_hip_attention_step_async
 * Device pointers, all 16-byte aligned; enqueued on `stream`.  Failures
 * are reported by leap_hip_attention_last_error(NULL). */
int leap_hip_attention_step_noalloc(const leap_hip_attention_config *cfg, int pos, const float *rope,
                                    float *k_cache, float *v_cache, const float *q, const float *k_new,
                                    const float *v_new, float *out, void *stream);

/* ---- The attention sub-block of run_layer on the device ----------------- */

/* Weights of one held layer for leap_hip_attention_block, copied from host
 * memory in the reference's layout (FloatTransformerWeights,
 * FloatTransformer.h:9-22; the layer's slices start at l*dim, l*dim*dim and
 * l*dim*kv_dim as run_layer reads them, FloatTransformer.cpp:394-402, 664):
 * rms_att [dim], wq [dim][dim], wk [kv_dim][dim], wv [kv_dim][dim],
 * wo [dim][dim], row-major, dim = n_heads * head_dim.  The projections need
 * dim in {2048, 3072, 4096, 5120, 8192}; other sizes return -EINVAL.  Device memory for
 * every held layer is allocated on the first call. */
int leap_hip_attention_set_layer_weights(leap_hip_attention *h, int layer, const float *rms_att,
                                         const float *wq, const float *wk, const float *wv,
                                         const float *wo);

/* run_layer from its start to the attention residual
 * (FloatTransformer.cpp:394-683): xb = rmsnorm(x, rms_att) (:394, rmsnorm
 * :88-213), q, k, v = Wq, Wk, Wv . xb (:400-402, matmul :240-382), the
 * attention block of leap_hip_attention_step (k and v appended to
 * cache[layer][pos]), then x += Wo . out (:664-683).  x is the dim-float
 * residual stream, updated in place: a device pointer, 16-byte aligned,
 * enqueued on `stream`. */
int leap_hip_attention_block_async(leap_hip_attention *h, int layer, int pos, float *x,
                                   void *stream);

/* As leap_hip_attention_block_async with a host pointer, synchronous. */
int leap_hip_attention_block(leap_hip_attention *h, int layer, int pos, float *x);

/* The quantized engine's weights of one held layer, for the same block calls:
 * each projection is the reference's QuantizedTensor (QuantizedTransformer.h:
 * 9-12; carved by init_quantized_tensors, QuantizedTransformer.cpp:88-100),
 * int8 values [d][n] row-major plus one float scale per group of group_size
 * consecutive values, [d*n/group_size]: wq/wo [dim][dim], wk/wv
 * [kv_dim][dim]; rms_att [dim] fp32.  With these weights a block call runs
 * QuantizedTransformer::run_layer from its start to the attention residual
 * (QuantizedTransformer.cpp:654-945): xb = rmsnorm(x); quantize(xb) (:338-357);
 * q, k, v = W8A8 matmul (:359-652); the fp32 attention step; quantize(out);
 * x += Wo . out.  A handle holds either fp32 or int8 weights, fixed by its
 * first set call, and one group size.  dim and group_size (a power of two)
 * must be 2048 with [32, 128], 3072 with [32, 128], 4096 with [32, 256],
 * 5120 with [64, 128] or 8192 with [64, 256]; others return -EINVAL. */
int leap_hip_attention_set_layer_weights_q8(leap_hip_attention *h, int layer, int group_size,
                                            const float *rms_att, const int8_t *wq, const float *wq_s,
                                            const int8_t *wk, const float *wk_s, const int8_t *wv,
                                            const float *wv_s, const int8_t *wo, const float *wo_s);

/* ---- Checkpoints ---------------------------------------------------------- */

/* A LEAP checkpoint's header as Transformer::create reads it
 * (TransformerFactory.cpp:59-115): magic 0x616B3432 with version 1 (fp32) or
 * 2 (int8: shared-classifier byte and group size after the Config), weights
 * from byte 256; or no magic (version 0, legacy fp32), the Config at byte 0
 * and the weights from byte 28.  For fp32 files shared_classifier is
 * vocab_size > 0 and vocab_size is made positive, as the reference does. */
typedef struct leap_hip_attention_checkpoint {
    int version;            /* 0, 1 or 2                                            */
    int dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len; /* Config.h */
    int shared_classifier;
    int group_size;         /* version 2                                            */
    long long header_bytes; /* where the weights start                              */
    long long attention_bytes; /* the file must hold this many bytes for every
                                  layer's rms_att, wq, wk, wv and wo               */
    long long file_bytes;
} leap_hip_attention_checkpoint;

/* Parse the header of the checkpoint at `path` (host only, no GPU needed).
 * -EIO if the file cannot be read, -EINVAL if it is not a checkpoint. */
int leap_hip_attention_checkpoint_read(const char *path, leap_hip_attention_checkpoint *out);

/* Upload, from the checkpoint at `path`, the attention weights (rms_att, wq,
 * wk, wv, wo) of every layer the handle holds: memory-mapped, in the tensor
 * order of memory_map_weights (FloatTransformer.cpp:947-978 for versions 0
 * and 1, QuantizedTransformer.cpp:102-134 for version 2), through
 * leap_hip_attention_set_layer_weights or _q8.  The checkpoint's n_layers,
 * n_heads, n_kv_heads and head size must be the handle's (-EINVAL
 * otherwise, and for a file shorter than attention_bytes).  This replaces the
 * attention part of the engine's construction from a file. */
int leap_hip_attention_load_checkpoint(leap_hip_attention *h, const char *path);

/* ---- Stage hand-off (pipeline across nodes) -------------------------------- */

/* A pipeline packet is the reference's PacketHeader {int32 pos; int32 flags}
 * (Transformer.h:25-31) followed by the dim fp32 values of the residual
 * stream x, dim = n_heads * head_dim: the master sends it after its layers
 * (FloatTransformer.cpp:775-788) and each worker reads it, runs its layers
 * and forwards it (:925-939).  A packet that starts with the uint16
 * CONTROL_MAGIC 0xC0DE is a control message of the same size (Transport.h:
 * 41-47, worker_loop :871-923); control messages belong to the transport's
 * control plane and are not handled here. */
#define LEAP_HIP_ATTENTION_PACKET_HEADER_BYTES 8
#define LEAP_HIP_ATTENTION_FLAG_NO_REPLY 0
#define LEAP_HIP_ATTENTION_FLAG_NEED_REPLY 1
#define LEAP_HIP_ATTENTION_CONTROL_MAGIC 0xC0DE

/* Read a packet's header (host only, no GPU): returns 0 for a data packet
 * with *pos and *flags set, 1 for a control packet, -EINVAL when `bytes` is
 * not 8 + 4*dim. */
int leap_hip_attention_packet_header(const void *packet, size_t bytes, int dim, int *pos,
                                     int *flags);

/* worker_loop's receive side (FloatTransformer.cpp:925-926): copy a data
 * packet's dim floats into the device residual stream `x` and return its
 * header in *pos and *flags, ready for leap_hip_attention_block_async(h,
 * layer, *pos, x, stream) over the held layers.  Returns 1, copying
 * nothing, for a control packet; -EINVAL for a wrong size or a pos outside
 * [0, seq_len).  With a NULL stream the copy runs on the handle's own
 * stream and has finished when the call returns; that stream does not wait
 * for work the caller enqueued on other streams, so x must not be in use
 * there.  Otherwise the copy is enqueued on `stream` and `packet` must stay
 * unchanged until the stream has passed it (pinned host memory makes it a
 * DMA; the reference's worker receives into a std::vector, which is
 * pageable). */
int leap_hip_attention_packet_upload(leap_hip_attention *h, const void *packet, size_t bytes,
                                     float *x, int *pos, int *flags, void *stream);

/* The send side (FloatTransformer.cpp:775-778 and 937-938): write the header
 * {pos, flags} and copy the device residual stream `x` after it, into the
 * host buffer `packet` of 8 + 4*dim bytes.  With a NULL stream the packet is
 * complete when the call returns (the copy runs on the handle's own stream:
 * finish the work that writes x on other streams first); otherwise its
 * values are, once `stream` has passed the copy.  A worker forwards the packet unless it is the tail
 * and flags is not FLAG_NEED_REPLY (:937). */
int leap_hip_attention_packet_download(leap_hip_attention *h, const float *x, int pos, int flags,
                                       void *packet, size_t bytes, void *stream);

/* ---- Extras with no counterpart in the reference ---------------------- */

/* Fill every cache row of every held sequence and layer with seeded
 * N(0,1)*scale values (SplitMix64 counter hash -> Box-Muller), on the device.
 * Synthetic data for benchmarks and large tests. */
int leap_hip_attention_kv_fill_normal(leap_hip_attention *h, uint64_t seed, float scale);

/* Copy RoPE table rows [pos_begin, pos_end) to host memory as the reference
 * holds them: cos and sin, each [pos][head_dim/2]. */
int leap_hip_attention_rope_download(leap_hip_attention *h, int pos_begin, int pos_end,
                                     float *cos_out, float *sin_out);

/* Positions per split-K chunk for later steps: 0 restores the automatic
 * choice; otherwise a multiple of 8 (a chunk that is not a whole number of
 * 64-row passes masks the rows past its end).  A tuning and test knob. */
int leap_hip_attention_set_split(leap_hip_attention *h, int chunk_positions);

/* Where later steps compute the score (q . K) and weighted-V products: 0 on
 * the matrix cores (4x4x1 f32 MFMAs, the default), 1 as per-lane VALU FMAs
 * with the same cross-lane sums.  Both give results within the same bar of
 * the reference; a measurement knob for the A/B of the matrix-core choice. */
int leap_hip_attention_set_products(leap_hip_attention *h, int valu);

/* How later steps finish a one-level split-K merge of 32 or more records
 * (no counterpart in the reference: a device-side scheduling choice).
 * 1 (the default): the second-to-last workgroup to count in waits for the
 * last, polling its counter a bounded number of times, and the two fold
 * half of the q heads each; 0: the last workgroup folds every head alone;
 * 2: the waiting workgroup gives up at once, which exercises the fallback
 * where the last folds every head.  All three give identical results.
 * -EINVAL for other modes. */
int leap_hip_attention_set_fold_helper(leap_hip_attention *h, int mode);

/* Device addresses of the (seq, layer) cache slabs, for callers that keep
 * their own device-side views of the cache. */
int leap_hip_attention_kv_device_ptr(leap_hip_attention *h, int seq, int layer, float **k,
                                     float **v);

/* Device addresses of the sub-block's intermediate vectors as the last block
 * call left them (valid until destroy; overwritten by the next call): the
 * pre-RoPE q [dim], k and v [kv_dim] of the projections, the attention
 * output att [dim] (the reference's s->xb before wo), and with int8 weights
 * the quantized projection inputs xq/xs (rmsnorm output) and aq/as (the
 * attention output): int8 [dim] and one scale per group (NULL with fp32
 * weights).  For checking each stage of the block on its own. */
typedef struct leap_hip_attention_block_views {
    const float *q, *k, *v, *att;
    const int8_t *xq;
    const float *xs;
    const int8_t *aq;
    const float *as;
} leap_hip_attention_block_views;
int leap_hip_attention_block_views_get(leap_hip_attention *h, leap_hip_attention_block_views *out);

/* Measurement floors of a step's launch shape (no counterpart in the
 * reference): enqueue on `stream` one launch with the grid, block size and
 * argument block that leap_hip_attention_step_batched_async(h, layer,
 * n_seq, pos, max_pos, total_rows, ...) would make, running kind 1: a
 * kernel that reads its arguments and exits (the launch floor), or kind 2:
 * a kernel that streams the same K and V rows ([0, pos[i]] of each
 * sequence) with the same loads and only sums them (the launch plus
 * bare-stream floor).  pos is device memory as in step_batched_async, or
 * NULL for every sequence at max_pos.  Neither kind writes memory or
 * changes the cache.  n_seq = 1, pos = NULL, max_pos = the position,
 * total_rows = position + 1 is the single-sequence step.  Kind 3, for a
 * layer with weights set (one sequence, pos NULL, total_rows = max_pos +
 * 1): the floor of leap_hip_attention_block_async, three launches with the
 * grids, block sizes and weight loads of its q/k/v and wo projections
 * streaming their weights (and int8 scales) alone, around the kind 2 launch
 * of its attention step.  -EINVAL for a
 * launch whose step spreads its (sequence, KV head) groups over the XCDs
 * (fewer than 8 groups of at least 4 MiB of rows each): the floor kernels
 * have no spread grid. */
int leap_hip_attention_floor_async(leap_hip_attention *h, int kind, int layer, int n_seq, const int *pos,
                                   int max_pos, long long total_rows, void *stream);

/* Placement diagnostic: launch n_wg workgroups of the decode kernel's size on
 * `device` and write the XCD (XCC_ID) each ran on to xcc_out[n_wg].  The
 * decode kernel's merge needs xcc_out[i] == xcc_out[i % 8] for every i;
 * leap_hip_attention_create checks that and returns -ENOTSUP otherwise. */
int leap_hip_attention_xcc_map(int device, int n_wg, int *xcc_out);

/* Per-workgroup timeline of the decode launches (measurement only; no
 * counterpart in the reference).  Only the timeline build of the library,
 * libleap_hip_attention_tl.so (compiled with LEAP_TIMELINE), records it; this
 * library returns -ENOTSUP.  There, every decode launch since the first
 * create stores, for each of its first 2048 workgroups, 16 64-bit words: the
 * 100 MHz device clock (s_memrealtime) at fixed points of the kernel (entry,
 * prologue, first scores, main loop end, wave combine, record or output
 * stored, record drained, arrival counted, fold loads issued, fold pairs
 * shared, fold stored, sub-group counted, sub-group stored, exit; 0 where a
 * workgroup did not pass), its role bits (1 output written alone, 2 final
 * fold, 4 fold helper, 8 sub-group fold) with its arrival count << 8, and
 * XCC_ID << 32 | HW_ID.  Launch i writes slot i % 64 of a ring of
 * 64 x 2048 x 16 words.  Copies the ring to dst (at least 16 MiB) and the
 * number of launches so far to *launches; the caller synchronises its
 * streams first. */
int leap_hip_attention_timeline(void *dst, size_t bytes, long long *launches);

#ifdef __cplusplus
}
#endif

#endif /* LEAP_HIP_ATTENTION_H */
