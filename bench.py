#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X.

Default workload: Llama-3-8B-shaped decode attention, batch 1, context 4096
cached positions (pos = 4095), all 32 layers stepped in sequence; n_heads 32,
n_kv_heads 8, head_dim 128, RoPE theta 500000; fp32 KV cache (1 GiB) and fp32
q/k/v filled with seeded N(0,1)/sqrt(128) values on the device.

One step = one token through the attention block of every layer of the
workload, back to back on one stream with q/k/v/out resident in HBM (one
kernel launch per layer-step).  Reported value: algorithmic HBM GB/s over the
timed region, with B(T) = 8*T*kv_dim + 8*dim + 16*kv_dim + 4*head_dim bytes
per layer-step and sequence; microseconds per layer-step and the fraction of
the 8 TB/s HBM peak alongside.

The CPU baseline is the reference's own code (oracle/_ref, built from its
sources with its release flags) timed on the host cores on a bounded sample of
the same workload, with sequence 0's device cache bytes downloaded.  The
reference keeps its attention inline in run_layer, between the projections:
for the attention workloads, calls at the workload's position and at position
0 alternate, and the difference of their medians is the attention; for the
sub-block workloads, run_layer itself is timed (zero FFN).  Without that
library (or for a RoPE base other than the reference's fixed 500000), the
oracle, the restated reference (OpenMP over heads, AVX2), is timed instead.

The `*-block-*` workloads time the whole attention sub-block of the layer step
instead (rmsnorm, q/k/v projections, attention, wo projection and residual;
three launches per layer-step), with synthetic N(0,1)/sqrt(dim) weights: one
random set uploaded into every layer's own slot, so each layer streams its own
copy from HBM.  Their bytes add the weights (Wq, Wk, Wv, Wo, rms) and the
residual stream to B(T).  The `*-q8-block-*` workloads run the quantized
engine's sub-block: int8 weights with one float scale per group of 64 values
(the reference exporter's default), the activations quantized per group on the
device; their bytes count the int8 weights and their scales.

For the batch-1 workloads the line also carries `host_pointer`: the same bytes
per layer-step over the time of the synchronous host-pointer entry point
(`leap_hip_attention_step`, or `leap_hip_attention_block`), which copies its
inputs and result over PCIe and waits for them in every call.  It is reported
beside `value`, never as `value`.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--workload NAME] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "attn decode µs/layer-step + HBM GB/s (% of peak), Llama-3-8B shape ctx 4096"
HBM_PEAK_GBS = 8000.0
KERNEL = "decode_attention_kernel"
BLOCK_METRIC = "attn sub-block (rmsnorm, qkv, attention, wo, residual) µs/layer-step + HBM GB/s, Llama-3-8B ctx 4096"
BLOCK_KERNELS = "qkv_kernel + decode_attention_kernel + proj_residual_kernel"
Q8_METRIC = ("attn sub-block, int8 weights (rmsnorm, quantize, W8A8 qkv, attention, quantize, W8A8 wo, residual) "
             "µs/layer-step + HBM GB/s, Llama-3-8B ctx 4096")
Q8_KERNELS = "q8_gemv_kernel (qkv) + decode_attention_kernel + q8_gemv_kernel (wo)"
Q8_GROUP = 64
SEED = 0x4C454150

# name -> (layers, n_heads, n_kv_heads, head_dim, theta, batch, context, seed index)
# context: an int, or ("ragged", lo, hi) drawn uniformly per sequence.
WORKLOADS = {
    "llama3-8b-ctx4096": (32, 32, 8, 128, 500000.0, 1, 4096, 1),
    "tinyllama-ctx256": (1, 32, 4, 64, 10000.0, 1, 256, 0),
    "llama3-8b-batch64-ragged": (32, 32, 8, 128, 500000.0, 64, ("ragged", 512, 8192), 2),
    "llama3-70b-stage20-batch16": (20, 64, 8, 128, 500000.0, 16, 8192, 3),
    "llama3.1-8b-ctx131072": (32, 32, 8, 128, 500000.0, 1, 131072, 4),
    "llama3-8b-block-ctx4096": (32, 32, 8, 128, 500000.0, 1, 4096, 5),
    "llama3-8b-q8-block-ctx4096": (32, 32, 8, 128, 500000.0, 1, 4096, 6),
    "llama3.2-3b-ctx4096": (28, 24, 8, 128, 500000.0, 1, 4096, 7),
}
BLOCK_WORKLOADS = {"llama3-8b-block-ctx4096", "llama3-8b-q8-block-ctx4096"}
Q8_WORKLOADS = {"llama3-8b-q8-block-ctx4096"}
DEFAULT_STEPS = {"llama3-8b-ctx4096": 100, "tinyllama-ctx256": 2000,
                 "llama3-8b-batch64-ragged": 10, "llama3-70b-stage20-batch16": 10,
                 "llama3.1-8b-ctx131072": 10, "llama3-8b-block-ctx4096": 30,
                 "llama3-8b-q8-block-ctx4096": 50, "llama3.2-3b-ctx4096": 100}


def algorithmic_bytes(T: int, n_heads: int, n_kv: int, hd: int) -> int:
    """Bytes one layer-step must move for one sequence: the K and V rows
    [0, T), q in and out, new k and v in and their cache rows out, and the
    RoPE table row."""
    kv_dim, dim = n_kv * hd, n_heads * hd
    return 8 * T * kv_dim + 8 * dim + 16 * kv_dim + 4 * hd


def block_bytes(T: int, n_heads: int, n_kv: int, hd: int) -> int:
    """Bytes of one attention sub-block layer-step: the attention's B(T), the
    weights Wq, Wk, Wv, Wo and rms_att, and the residual stream read twice and
    written once."""
    dim, kv_dim = n_heads * hd, n_kv * hd
    return algorithmic_bytes(T, n_heads, n_kv, hd) + 4 * ((dim + 2 * kv_dim) * dim + dim * dim + dim) + 12 * dim


def q8_block_bytes(T: int, n_heads: int, n_kv: int, hd: int, gs: int = Q8_GROUP) -> int:
    """Bytes of one layer-step of the quantized engine's sub-block: the
    attention's B(T), the int8 weights Wq, Wk, Wv, Wo with one 4-byte scale per
    group of gs, rms_att, and the residual stream read twice and written once."""
    dim, kv_dim = n_heads * hd, n_kv * hd
    w = (dim + 2 * kv_dim) * dim + dim * dim
    return algorithmic_bytes(T, n_heads, n_kv, hd) + w + 4 * (w // gs) + 4 * dim + 12 * dim


def quantize_groups(w: np.ndarray, gs: int):
    """Synthetic int8 weights in the quantized engine's format: int8 values
    [d][n] and one float scale per group of gs values of a row (max|w| / 127,
    values rounded to nearest)."""
    g = w.reshape(-1, gs)
    sc = (np.abs(g).max(axis=1) / 127.0).astype(np.float32)
    q = np.rint(g / np.where(sc > 0, sc, 1.0)[:, None]).clip(-127, 127).astype(np.int8)
    return q.reshape(w.shape), sc


def hip_graph_us(one_step, stream, steps: int, n_layers: int) -> float:
    """Microseconds per layer-step of one_step captured once into a HIP graph
    (its launches only: the entry points enqueue kernels and nothing else)
    and replayed `steps` times on `stream`."""
    import torch
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        one_step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(2):
            graph.replay()
        e0.record(stream)
        for _ in range(steps):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (steps * n_layers)


def traffic_from_profiles(workload: str):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE runs
    (scaled by a copy kernel's counters), recorded in profiles/."""
    path = os.path.join(ROOT, "profiles", f"decode_attention_{workload}_traffic.txt")
    if not os.path.isfile(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def contexts(workload: str):
    L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[workload]
    if isinstance(ctx, tuple):
        rng = np.random.default_rng(SEED + sidx)
        return rng.integers(ctx[1], ctx[2] + 1, size=batch).astype(np.int64)
    return np.full(batch, ctx, np.int64)


def cpu_baseline_block(att, workload, Ts, n_layers_sample: int, budget_s: float, weights, q8: bool = False):
    """The sub-block on the host cores, on the device cache bytes of layer 0
    (downloaded).  When oracle/_ref is present: the reference's own run_layer
    (compiled from its sources with its release flags, OpenMP as it ships) on
    an engine whose layers each hold these weights and a zero FFN of
    negligible size, cycled so that the weights come from memory.  Otherwise:
    the oracle's chain (rmsnorm, matmul, attention, matmul, residual) on layers
    [0, n_layers_sample)."""
    from oracle import oracle as O
    L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[workload]
    T = int(Ts[0])
    x0 = np.random.default_rng(SEED + sidx).standard_normal(nh * hd).astype(np.float32)
    nbytes = (q8_block_bytes if q8 else block_bytes)(T, nh, nkv, hd)
    if (O.ref_q8_available() if q8 else O.ref_available()) and theta == 500000.0:
        k, v = att.kv_download(0, 0, 0, T - 1)
        # enough layers (each its own copy of the weights and cache rows) that
        # the CPU caches cannot hold them: about 1.6 GB
        n_l = max(4, -(-1_600_000_000 // nbytes))
        timer = O.RefBlockTimer(nh * hd, nh, nkv, T, *weights, k, v, gs=Q8_GROUP if q8 else None, n_layers=n_l)
        try:
            x = x0.copy()
            timer.run(T - 1, x, 1)  # the OpenMP pool starts
            times = []
            t_end = time.perf_counter() + budget_s
            while time.perf_counter() < t_end or len(times) < 3:
                x[:] = x0
                times.append(timer.run(T - 1, x, 1))
        finally:
            timer.close()
        us = float(np.median(times)) * 1e6
        threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count() or 1
        return {
            "value": round(nbytes / (us * 1e-6) / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
            "us_per_layer_step": round(us, 2),
            "sample": f"{len(times)} calls of the reference's {'QuantizedTransformer' if q8 else 'FloatTransformer'}"
                      f"::run_layer at pos {T - 1}, cycling through an engine of {n_l} layers that each hold "
                      f"the workload's weights (zero FFN of hidden size {Q8_GROUP if q8 else 8}) and layer 0's "
                      f"device cache rows; median per call; the reference's own OpenMP",
        }
    if not os.path.isfile(O.ORACLE_SO):
        O.build(ref=False)
    env_threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(env_threads or os.cpu_count() or 1, 16)
    O.lib().oracle_set_threads(threads)
    n_l = min(n_layers_sample, L)
    orc = O.Oracle(n_l, nh, nkv, hd, T, theta=theta)
    for l in range(n_l):
        k, v = att.kv_download(0, l, 0, T)
        orc.key_cache[l] = k
        orc.value_cache[l] = v
    x = x0
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        for l in range(n_l):
            if q8:
                orc.block_q8(l, T - 1, x, *weights, Q8_GROUP)
            else:
                orc.block(l, T - 1, x, *weights)
        times.append((time.perf_counter() - t0) / n_l)
    us = float(np.median(times)) * 1e6
    return {
        "value": round(nbytes / (us * 1e-6) / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "us_per_layer_step": round(us, 2),
        "sample": f"{len(times)} sweeps of the sub-block over layers 0..{n_l - 1} of the same workload "
                  f"(context {T}), device cache bytes downloaded; median per layer-step; OpenMP over "
                  f"rows and heads",
    }


def cpu_baseline_reference(att, workload, T: int, budget_s: float):
    """The reference's own attention on the host cores, timed through its
    run_layer (oracle/_ref), which holds the attention inline between the
    projections: calls at pos T-1 and at pos 0 alternate on an engine of
    several layers (each its own copy of synthetic weights and of sequence
    0's first T-1 device cache rows, cycled so that nothing stays in the CPU
    caches), and the difference of their medians is the attention over T
    rows; the projections, the residual and the zero FFN are the same work
    in both."""
    from oracle import oracle as O
    L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[workload]
    dim, kvd = nh * hd, nkv * hd
    wrng = np.random.default_rng(SEED + sidx)
    w = [(1.0 + 0.1 * wrng.standard_normal(dim)).astype(np.float32)] + [
        (wrng.standard_normal(shape) / np.sqrt(dim)).astype(np.float32)
        for shape in ((dim, dim), (kvd, dim), (kvd, dim), (dim, dim))]
    k, v = att.kv_download(0, 0, 0, T - 1)
    per_layer = 4 * (2 * dim * dim + 2 * kvd * dim) + 8 * T * kvd
    n_l = max(4, -(-1_600_000_000 // per_layer))
    timer = O.RefBlockTimer(dim, nh, nkv, T, *w, k, v, n_layers=n_l)
    x0 = wrng.standard_normal(dim).astype(np.float32)
    x = x0.copy()
    long_t, short_t = [], []
    try:
        timer.run(T - 1, x, n_l)  # the OpenMP pool starts, every layer touched once
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(long_t) < 5:
            x[:] = x0
            long_t.append(timer.run(T - 1, x, 1))
            x[:] = x0
            short_t.append(timer.run(0, x, 1))
    finally:
        timer.close()
    us = (float(np.median(long_t)) - float(np.median(short_t))) * 1e6
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count() or 1
    return {
        "value": round(algorithmic_bytes(T, nh, nkv, hd) / (us * 1e-6) / 1e9, 3), "unit": "GB/s",
        "cores": threads, "kind": "reference", "us_per_layer_step": round(us, 2),
        "sample": f"the reference's FloatTransformer::run_layer, {len(long_t)} calls each at pos {T - 1} and pos 0 "
                  f"alternating over an engine of {n_l} layers (synthetic weights, sequence 0's device cache "
                  f"rows); attention = difference of the medians ({float(np.median(long_t)) * 1e6:.1f} - "
                  f"{float(np.median(short_t)) * 1e6:.1f} us); the reference's own OpenMP",
    }


def cpu_baseline(att, workload, Ts, n_layers_sample: int, budget_s: float):
    """The reference's attention through its run_layer when oracle/_ref is
    present and the workload uses the reference's fixed RoPE base; otherwise
    the oracle on the host on layers [0, n_layers_sample) of sequence 0 of
    the device cache (downloaded bytes), repeating sweeps for about budget_s
    seconds."""
    from oracle import oracle as O
    L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[workload]
    if O.ref_available() and theta == 500000.0:
        return cpu_baseline_reference(att, workload, int(Ts[0]), budget_s)
    if not os.path.isfile(O.ORACLE_SO):
        O.build(ref=False)
    env_threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(nh, env_threads or os.cpu_count() or 1, 16)
    O.lib().oracle_set_threads(threads)
    T = int(Ts[0])
    n_l = min(n_layers_sample, L)
    rng = np.random.default_rng(SEED + sidx)
    orc = O.Oracle(n_l, nh, nkv, hd, T, theta=theta)
    for l in range(n_l):
        k, v = att.kv_download(0, l, 0, T)
        orc.key_cache[l] = k
        orc.value_cache[l] = v
    qs = [(rng.standard_normal(nh * hd) / np.sqrt(hd)).astype(np.float32) for _ in range(n_l)]
    ks = [(rng.standard_normal(nkv * hd) / np.sqrt(hd)).astype(np.float32) for _ in range(n_l)]
    vs = [(rng.standard_normal(nkv * hd) / np.sqrt(hd)).astype(np.float32) for _ in range(n_l)]
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        for l in range(n_l):
            orc.step(l, T - 1, qs[l], ks[l], vs[l])
        times.append((time.perf_counter() - t0) / n_l)
    us = float(np.median(times)) * 1e6
    gbs = algorithmic_bytes(T, nh, nkv, hd) / (us * 1e-6) / 1e9
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "us_per_layer_step": round(us, 2),
        "sample": f"{len(times)} sweeps of layers 0..{n_l - 1} of sequence 0 (context {T}) of the "
                  f"same workload, device cache bytes downloaded; median per layer-step; "
                  f"OpenMP over heads",
    }


def host_pointer_rate(att, L, pos, bytes_layer, is_block, sweeps):
    """The synchronous host-pointer entry point the engine calls, timed on the host clock.

    Each call copies its inputs from pageable host memory, runs the launches
    and copies the result back before it returns, as `leap_hip_attention_step`
    (or `leap_hip_attention_block`) does for an engine whose buffers live in
    std::vector.  Buffers are allocated once; the call is made through ctypes
    without the binding's per-call copies.
    """
    from leap_amd.attention import _fp
    rng = np.random.default_rng(SEED)
    lib, h = att.lib, att.h
    if is_block:
        x = (rng.standard_normal(att.q_dim) * 0.1).astype(np.float32)
        xp = _fp(x)

        def sweep():
            for l in range(L):
                rc = lib.leap_hip_attention_block(h, l, pos, xp)
                if rc:
                    raise RuntimeError(f"leap_hip_attention_block returned {rc}")
        entry, host_bytes = "leap_hip_attention_block", 8 * att.q_dim
    else:
        bufs = [(rng.standard_normal(n) / np.sqrt(att.head_dim)).astype(np.float32)
                for n in (att.q_dim, att.kv_dim, att.kv_dim)]
        out = np.empty(att.q_dim, np.float32)
        ptrs = [_fp(b) for b in bufs] + [_fp(out)]

        def sweep():
            for l in range(L):
                rc = lib.leap_hip_attention_step(h, l, pos, *ptrs)
                if rc:
                    raise RuntimeError(f"leap_hip_attention_step returned {rc}")
        entry, host_bytes = "leap_hip_attention_step", 4 * (2 * att.q_dim + 2 * att.kv_dim)
    sweep()
    t0 = time.perf_counter()
    for _ in range(sweeps):
        sweep()
    us = (time.perf_counter() - t0) * 1e6 / (sweeps * L)
    return {"entry": entry, "value": round(bytes_layer / (us * 1e-6) / 1e9, 2), "unit": "GB/s",
            "us_per_layer_step": round(us, 3), "host_bytes_per_layer_step": host_bytes,
            "sweeps": sweeps,
            "note": "pageable host buffers: copies in, launches, copy out and a stream "
                    "synchronisation in every call (PCIe-inclusive; not the device-resident value)"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="llama3-8b-ctx4096", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-host-pointer", action="store_true",
                    help="skip the host-pointer (PCIe-inclusive) leg, e.g. under a profiler")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-layers", type=int, default=4)
    ap.add_argument("--split", type=int, default=0, help="positions per split-K chunk (0 = auto)")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP graph replay timing")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 10 plain device copies of MIB MiB (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()
    if args.copy_probe:
        import torch
        n = args.copy_probe * (1 << 20) // 4
        src = torch.ones(n, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n * 4, "copies": 10}))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the attention step shards by sequence or KV head with no exchange; "
              "run --gpus 1).", file=sys.stderr)
        sys.exit(2)
    steps = args.steps or DEFAULT_STEPS[args.workload]

    import torch
    from leap_amd.attention import HipAttention

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[args.workload]
    Ts = contexts(args.workload)
    seq_len = int(Ts.max())
    att = HipAttention(nh, nkv, hd, seq_len, n_layers=L, rope_theta=theta, max_batch=batch)
    if args.split:
        att.set_split(args.split)
    att.kv_fill_normal(SEED + sidx, 1.0 / np.sqrt(hd))

    g = torch.Generator(device=dev)
    g.manual_seed(SEED + sidx)
    scale = 1.0 / np.sqrt(hd)
    q = torch.randn(L, batch, nh * hd, device=dev, generator=g) * scale
    k = torch.randn(L, batch, nkv * hd, device=dev, generator=g) * scale
    v = torch.randn(L, batch, nkv * hd, device=dev, generator=g) * scale
    out = torch.empty(L, batch, nh * hd, device=dev)
    pos_dev = torch.tensor(Ts - 1, dtype=torch.int32, device=dev)
    max_pos = int(Ts.max()) - 1
    stream = torch.cuda.Stream(device=dev)
    sp = stream.cuda_stream
    ptrs = [(q[l].data_ptr(), k[l].data_ptr(), v[l].data_ptr(), out[l].data_ptr()) for l in range(L)]

    is_block = args.workload in BLOCK_WORKLOADS
    weights = None
    if is_block:
        dim, kvd = nh * hd, nkv * hd
        wrng = np.random.default_rng(SEED + sidx)
        weights = (
            (1.0 + 0.1 * wrng.standard_normal(dim)).astype(np.float32),
            (wrng.standard_normal((dim, dim)) / np.sqrt(dim)).astype(np.float32),
            (wrng.standard_normal((kvd, dim)) / np.sqrt(dim)).astype(np.float32),
            (wrng.standard_normal((kvd, dim)) / np.sqrt(dim)).astype(np.float32),
            (wrng.standard_normal((dim, dim)) / np.sqrt(dim)).astype(np.float32),
        )
        if args.workload in Q8_WORKLOADS:
            weights = (weights[0],) + tuple(quantize_groups(w, Q8_GROUP) for w in weights[1:])
            for l in range(L):
                att.set_layer_weights_q8(l, Q8_GROUP, *weights)
        else:
            for l in range(L):
                att.set_layer_weights(l, *weights)
        x_res = torch.randn(dim, device=dev, generator=g)
        xp = x_res.data_ptr()
        pos = int(Ts[0]) - 1

        def one_step():
            for l in range(L):
                att.block_async(l, pos, xp, sp)
    elif batch == 1:
        pos = int(Ts[0]) - 1

        def one_step():
            for l in range(L):
                qp, kp, vp, op = ptrs[l]
                att.step_async(l, pos, qp, kp, vp, op, sp)
    else:
        pp = pos_dev.data_ptr()
        total_rows = int(np.sum(Ts))

        def one_step():
            for l in range(L):
                qp, kp, vp, op = ptrs[l]
                att.step_batched_async(l, batch, pp, max_pos, qp, kp, vp, op, sp, total_rows)

    torch.cuda.synchronize()
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()

    # The timed region, cut into up to 10 segments by events on the same
    # stream (for the spread); the total runs from the first event to the last.
    n_seg = min(10, steps)
    bounds = [round(i * steps / n_seg) for i in range(n_seg + 1)]
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n_seg + 1)]
    torch.cuda.synchronize()
    evs[0].record(stream)
    t0 = time.perf_counter()
    for i in range(n_seg):
        for _ in range(bounds[i + 1] - bounds[i]):
            one_step()
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = evs[0].elapsed_time(evs[-1])
    seg_us = np.array([evs[i].elapsed_time(evs[i + 1]) * 1e3 / ((bounds[i + 1] - bounds[i]) * L)
                       for i in range(n_seg)])

    launches = steps * L
    us_layer = ms_total * 1e3 / launches
    graph_us = None if args.no_graph else hip_graph_us(one_step, stream, steps, L)
    is_q8 = args.workload in Q8_WORKLOADS
    per_seq = q8_block_bytes if is_q8 else block_bytes if is_block else algorithmic_bytes
    bytes_layer = int(sum(per_seq(int(T), nh, nkv, hd) for T in Ts))
    gbs = bytes_layer / (us_layer * 1e-6) / 1e9
    if not np.isfinite((x_res if is_block else out).float().sum().item()):
        print("non-finite output", file=sys.stderr)
        sys.exit(1)

    result = {
        "metric": Q8_METRIC if is_q8 else BLOCK_METRIC if is_block else METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_total / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8+f32" if is_q8 else "f32",
        "data": (f"synthetic (seeded N(0,1)/sqrt({hd}) KV cache generated on the device; "
                 f"N(0,1)/sqrt(dim) weights{f', int8 with one scale per {Q8_GROUP} values' if is_q8 else ''}, "
                 f"one set uploaded into every layer)") if is_block else
                f"synthetic (seeded N(0,1)/sqrt({hd}) KV cache and q/k/v, generated on the device)",
        "config": {
            "workload": args.workload, "n_layers": L, "n_heads": nh, "n_kv_heads": nkv,
            "head_dim": hd, "batch": batch, "rope_theta": theta,
            "context": int(Ts[0]) if batch == 1 else
            {"min": int(Ts.min()), "max": int(Ts.max()), "sum": int(Ts.sum())},
        },
        "us_per_layer_step": round(us_layer, 3),
        "us_per_layer_step_spread": {"segments": n_seg, "median": round(float(np.median(seg_us)), 3),
                                     "p10": round(float(np.percentile(seg_us, 10)), 3),
                                     "p90": round(float(np.percentile(seg_us, 90)), 3)},
        "pct_of_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "tokens_layers_per_s": round(batch * 1e6 / us_layer, 1),
        "host_wall_s": round(wall, 4),
        "roofline": {
            "kernel": Q8_KERNELS if is_q8 else BLOCK_KERNELS if is_block else KERNEL,
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles(args.workload),
            "bytes_per_launch": bytes_layer,
            "launch_us": round(us_layer, 3),
        },
        "cpu_baseline": None,
    }
    if graph_us is not None:
        result["hip_graph"] = {
            "us_per_layer_step": round(graph_us, 3),
            "value": round(bytes_layer / (graph_us * 1e-6) / 1e9, 2),
            "unit": "GB/s",
            "note": "the same step captured once into a HIP graph and replayed; `value` above is eager launches",
        }
    if batch == 1 and not args.no_host_pointer:
        result["host_pointer"] = host_pointer_rate(att, L, pos, bytes_layer, is_block,
                                                   sweeps=max(1, min(steps, 20)))
    if not args.no_cpu:
        try:
            if is_block:
                result["cpu_baseline"] = cpu_baseline_block(att, args.workload, Ts, args.cpu_layers,
                                                            args.cpu_seconds, weights, q8=is_q8)
            else:
                result["cpu_baseline"] = cpu_baseline(att, args.workload, Ts, args.cpu_layers,
                                                      args.cpu_seconds)
        except Exception as e:  # the GPU line still stands; say why the CPU leg is missing
            result["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    att.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
