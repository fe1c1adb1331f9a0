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

The default run's line also carries, for the same build and box:
  - `floor`: the same launch shape (grid, block, argument block) running a
    kernel that only reads its arguments, and one that only streams the same
    K/V rows with the same loads; the per-launch cost any one-launch design
    pays at this shape;
  - `workloads`: the other configurations, each allocated, filled, timed
    (events over >= 10 steps) and freed in turn, each with its same-grid
    stream floor: TinyLlama ctx 256, a batch of 64 Llama-3-8B sequences with
    ragged contexts in [512, 8192], a Llama-3-70B pipeline stage (20 layers,
    batch 16, ctx 8192), Llama-3.1-8B at ctx 131072, and the Llama-3-8B
    attention sub-block at ctx 4096 with fp32 and with int8 weights;
  - `t_sweep`: microseconds per layer-step over contexts 1 .. 16384 at the
    Llama-3-8B and TinyLlama head shapes, eager and replayed from a HIP graph
    (every decode walks these contexts from position 0), and a generation's
    mean over T = 1 .. 4096 at Llama-3-8B from every 32nd context
    (`mean_us_per_layer_step_T1_4096`);
  - `cpu_baseline`: the reference's own code (oracle/_ref, built from its
    sources with its release flags) on the host cores, in a child process
    pinned as the reference's README says (OMP_PROC_BIND=close,
    OMP_PLACES=cores), at min(n_heads, physical cores) threads and at every
    usable logical CPU, on a bounded sample of the same workload with
    sequence 0's device cache bytes downloaded.  The reference keeps its
    attention inline in run_layer, between the projections: for the
    attention workloads, calls at the workload's position and at position 0
    alternate, and the difference of their medians is the attention; for the
    sub-block workloads, run_layer itself is timed (zero FFN).  Without that
    library (or for a RoPE base other than the reference's fixed 500000), the
    oracle, the restated reference (OpenMP over heads, AVX2), is timed
    instead.

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
                    [--no-extra] [--no-host-pointer] [--no-graph]
    python bench.py --timeline [--workload NAME] [--split N] [--fold-helper M]

`--timeline` runs the workload on the library's timeline build instead and
prints where each launch's time goes: per-workgroup device-clock stamps at the
kernel's phase boundaries (see timeline_report).
"""
from __future__ import annotations

import argparse
import json
import os
import re
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HEADLINE_METRIC = "attn decode µs/layer-step + HBM GB/s (% of peak), Llama-3-8B shape ctx 4096"
HBM_PEAK_GBS = 8000.0
KERNEL = "decode_attention_kernel"
BLOCK_KERNELS = "qkv_kernel + decode_attention_kernel + proj_residual_kernel"
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
    # a pipeline stage of Llama-3.1-405B (16 of its 126 layers): 16 q heads per KV head
    "llama3.1-405b-stage16-ctx4096": (16, 128, 8, 128, 500000.0, 1, 4096, 8),
}
SHAPE_NAMES = {
    "llama3-8b-ctx4096": "Llama-3-8B shape ctx 4096",
    "tinyllama-ctx256": "TinyLlama-1.1B shape (32/4/64) ctx 256, one layer",
    "llama3-8b-batch64-ragged": "Llama-3-8B shape, 64 sequences, ctx U[512, 8192]",
    "llama3-70b-stage20-batch16": "Llama-3-70B stage (64/8/128, 20 layers), 16 sequences, ctx 8192",
    "llama3.1-8b-ctx131072": "Llama-3.1-8B shape ctx 131072",
    "llama3-8b-block-ctx4096": "Llama-3-8B ctx 4096",
    "llama3-8b-q8-block-ctx4096": "Llama-3-8B ctx 4096",
    "llama3.2-3b-ctx4096": "Llama-3.2-3B shape (24/8/128) ctx 4096",
    "llama3.1-405b-stage16-ctx4096": "Llama-3.1-405B stage (128/8/128, 16 layers) ctx 4096",
}
BLOCK_WORKLOADS = {"llama3-8b-block-ctx4096", "llama3-8b-q8-block-ctx4096"}
Q8_WORKLOADS = {"llama3-8b-q8-block-ctx4096"}
DEFAULT_STEPS = {"llama3-8b-ctx4096": 100, "tinyllama-ctx256": 2000,
                 "llama3-8b-batch64-ragged": 10, "llama3-70b-stage20-batch16": 10,
                 "llama3.1-8b-ctx131072": 10, "llama3-8b-block-ctx4096": 30,
                 "llama3-8b-q8-block-ctx4096": 50, "llama3.2-3b-ctx4096": 100,
                 "llama3.1-405b-stage16-ctx4096": 100}
# the configurations timed beside the headline in the default run
EXTRA_WORKLOADS = ("tinyllama-ctx256", "llama3-8b-batch64-ragged", "llama3-70b-stage20-batch16",
                   "llama3.1-8b-ctx131072", "llama3-8b-block-ctx4096", "llama3-8b-q8-block-ctx4096")
SWEEP_T = (1, 16, 64, 256, 512, 1024, 2048, 2304, 3072, 4096, 6144, 8192, 16384)
SWEEP_SHAPES = {"llama3-8b": (32, 32, 8, 128, 500000.0), "tinyllama": (22, 32, 4, 64, 10000.0)}


def metric_for(workload: str) -> str:
    if workload == "llama3-8b-ctx4096":
        return HEADLINE_METRIC
    if workload in Q8_WORKLOADS:
        return ("attn sub-block, int8 weights (rmsnorm, quantize, W8A8 qkv, attention, quantize, W8A8 wo, "
                f"residual) µs/layer-step + HBM GB/s, {SHAPE_NAMES[workload]}")
    if workload in BLOCK_WORKLOADS:
        return (f"attn sub-block (rmsnorm, qkv, attention, wo, residual) µs/layer-step + HBM GB/s, "
                f"{SHAPE_NAMES[workload]}")
    return f"attn decode µs/layer-step + HBM GB/s (% of peak), {SHAPE_NAMES[workload]}"


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


def contexts(workload: str):
    L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[workload]
    if isinstance(ctx, tuple):
        rng = np.random.default_rng(SEED + sidx)
        return rng.integers(ctx[1], ctx[2] + 1, size=batch).astype(np.int64)
    return np.full(batch, ctx, np.int64)


def traffic_from_profiles(workload: str):
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE runs
    (scaled by a copy kernel's counters), recorded in profiles/."""
    path = os.path.join(ROOT, "profiles", f"decode_attention_{workload}_traffic.txt")
    if not os.path.isfile(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


# ---- timing helpers -------------------------------------------------------------

def timed_steps(one_step, stream, steps: int, warmup: int, n_layers: int):
    """Run `warmup` untimed steps, then exactly `steps` steps bracketed by a
    device synchronisation on both sides, cut into up to 10 segments by
    events on `stream`.  Returns (total ms, per-segment us per layer-step,
    host wall seconds)."""
    import torch
    torch.cuda.synchronize()
    for _ in range(warmup):
        one_step()
    torch.cuda.synchronize()
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
    seg_us = np.array([evs[i].elapsed_time(evs[i + 1]) * 1e3 / ((bounds[i + 1] - bounds[i]) * n_layers)
                       for i in range(n_seg)])
    return ms_total, seg_us, wall


def hip_graph_us(one_step, stream, steps: int, n_layers: int) -> float:
    """Microseconds per layer-step of one_step captured into a HIP graph (its
    launches only: the entry points enqueue kernels and nothing else) and
    replayed on `stream`.  A graph holds enough steps for at least 32
    launches (replaying a graph has a fixed cost of its own), and is
    replayed until at least `steps` steps have run."""
    import torch
    per_graph = max(1, -(-32 // n_layers))
    replays = max(2, -(-steps // per_graph))
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(per_graph):
            one_step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for _ in range(2):
            graph.replay()
        e0.record(stream)
        for _ in range(replays):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (replays * per_graph * n_layers)
    del graph
    return us


class Workload:
    """One configuration on the device: the handle, its filled cache, the
    step's inputs, and one_step() running the layer sweep on `stream`."""

    def __init__(self, workload: str, split: int = 0, valu: bool = False, lib=None):
        import torch
        from leap_amd.attention import HipAttention
        self.name = workload
        L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[workload]
        self.L, self.nh, self.nkv, self.hd, self.theta, self.batch, self.sidx = L, nh, nkv, hd, theta, batch, sidx
        self.Ts = contexts(workload)
        self.is_block = workload in BLOCK_WORKLOADS
        self.is_q8 = workload in Q8_WORKLOADS
        dev = torch.device("cuda:0")
        self.att = att = HipAttention(nh, nkv, hd, int(self.Ts.max()), n_layers=L, rope_theta=theta,
                                      max_batch=batch, lib=lib)
        if split:
            att.set_split(split)
        if valu:
            att.set_products(True)
        att.kv_fill_normal(SEED + sidx, 1.0 / np.sqrt(hd))
        g = torch.Generator(device=dev)
        g.manual_seed(SEED + sidx)
        scale = 1.0 / np.sqrt(hd)
        self.q = torch.randn(L, batch, nh * hd, device=dev, generator=g) * scale
        self.k = torch.randn(L, batch, nkv * hd, device=dev, generator=g) * scale
        self.v = torch.randn(L, batch, nkv * hd, device=dev, generator=g) * scale
        self.out = torch.empty(L, batch, nh * hd, device=dev)
        self.pos_dev = torch.tensor(self.Ts - 1, dtype=torch.int32, device=dev)
        self.max_pos = int(self.Ts.max()) - 1
        self.total_rows = int(np.sum(self.Ts))
        self.stream = torch.cuda.Stream(device=dev)
        sp = self.stream.cuda_stream
        ptrs = [(self.q[l].data_ptr(), self.k[l].data_ptr(), self.v[l].data_ptr(), self.out[l].data_ptr())
                for l in range(L)]
        self.weights = None
        if self.is_block:
            dim, kvd = nh * hd, nkv * hd
            wrng = np.random.default_rng(SEED + sidx)
            w = (
                (1.0 + 0.1 * wrng.standard_normal(dim)).astype(np.float32),
                (wrng.standard_normal((dim, dim)) / np.sqrt(dim)).astype(np.float32),
                (wrng.standard_normal((kvd, dim)) / np.sqrt(dim)).astype(np.float32),
                (wrng.standard_normal((kvd, dim)) / np.sqrt(dim)).astype(np.float32),
                (wrng.standard_normal((dim, dim)) / np.sqrt(dim)).astype(np.float32),
            )
            if self.is_q8:
                w = (w[0],) + tuple(quantize_groups(x, Q8_GROUP) for x in w[1:])
                for l in range(L):
                    att.set_layer_weights_q8(l, Q8_GROUP, *w)
            else:
                for l in range(L):
                    att.set_layer_weights(l, *w)
            self.weights = w
            self.x_res = torch.randn(dim, device=dev, generator=g)
            xp = self.x_res.data_ptr()
            pos = int(self.Ts[0]) - 1

            def one_step():
                for l in range(L):
                    att.block_async(l, pos, xp, sp)
        elif batch == 1:
            pos = int(self.Ts[0]) - 1

            def one_step():
                for l in range(L):
                    qp, kp, vp, op = ptrs[l]
                    att.step_async(l, pos, qp, kp, vp, op, sp)
        else:
            pp = self.pos_dev.data_ptr()
            max_pos, total_rows = self.max_pos, self.total_rows

            def one_step():
                for l in range(L):
                    qp, kp, vp, op = ptrs[l]
                    att.step_batched_async(l, batch, pp, max_pos, qp, kp, vp, op, sp, total_rows)
        self.one_step = one_step
        per_seq = q8_block_bytes if self.is_q8 else block_bytes if self.is_block else algorithmic_bytes
        self.bytes_layer = int(sum(per_seq(int(T), nh, nkv, hd) for T in self.Ts))

    def finite(self) -> bool:
        return bool(np.isfinite((self.x_res if self.is_block else self.out).float().sum().item()))

    def floor_us(self, kind: int, steps: int, warmup: int) -> float:
        """Microseconds per layer-step of the floor launches (kind 1: the
        launch alone, kind 2: the bare K/V stream; kind 3, sub-block
        workloads: both projections streaming their weights alone around the
        bare K/V stream) with this step's shape."""
        att, sp, L = self.att, self.stream.cuda_stream, self.L
        n, mp, tr = self.batch, self.max_pos, (self.total_rows if self.batch > 1 else self.max_pos + 1)
        pp = self.pos_dev.data_ptr() if self.batch > 1 else None

        def one():
            for l in range(L):
                att.floor_async(kind, l, n, mp, tr, sp, pos_ptr=pp)
        ms, _, _ = timed_steps(one, self.stream, steps, warmup, L)
        return ms * 1e3 / (steps * L)

    def close(self):
        self.att.close()
        for name in ("q", "k", "v", "out", "pos_dev", "x_res"):
            if hasattr(self, name):
                delattr(self, name)


def measure(w: Workload, steps: int, warmup: int, graph: bool = True):
    ms_total, seg_us, wall = timed_steps(w.one_step, w.stream, steps, warmup, w.L)
    us_layer = ms_total * 1e3 / (steps * w.L)
    r = {
        "us_per_layer_step": round(us_layer, 3),
        "value": round(w.bytes_layer / (us_layer * 1e-6) / 1e9, 2),
        "unit": "GB/s",
        "frac": round(w.bytes_layer / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        "bytes_per_launch": w.bytes_layer,
        "steps": steps, "warmup": warmup, "ms_total": ms_total, "wall": wall,
        "spread": {"segments": len(seg_us), "median": round(float(np.median(seg_us)), 3),
                   "p10": round(float(np.percentile(seg_us, 10)), 3),
                   "p90": round(float(np.percentile(seg_us, 90)), 3)},
    }
    if graph:
        gus = hip_graph_us(w.one_step, w.stream, steps, w.L)
        r["hip_graph_us"] = round(gus, 3)
    return r


def extra_workload(name: str):
    """One of the other configurations: allocated, filled, timed and freed."""
    import torch
    steps = max(10, min(DEFAULT_STEPS[name], 200))
    w = Workload(name)
    try:
        r = measure(w, steps, 3)
        ok = w.finite()
        floor = w.floor_us(3 if w.is_block else 2, steps, 3)
    finally:
        w.close()
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    L, nh, nkv, hd, theta, batch, ctx, sidx = WORKLOADS[name]
    Ts = contexts(name)
    return {
        "metric": metric_for(name), "us_per_layer_step": r["us_per_layer_step"], "value": r["value"],
        "unit": "GB/s", "frac": r["frac"], "hip_graph_us_per_layer_step": r["hip_graph_us"],
        "bytes_per_launch": r["bytes_per_launch"], "steps": steps,
        "tokens_layers_per_s": round(batch * 1e6 / r["us_per_layer_step"], 1),
        "config": {"n_layers": L, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd, "batch": batch,
                   "rope_theta": theta,
                   "context": int(Ts[0]) if batch == 1 else {"min": int(Ts.min()), "max": int(Ts.max()),
                                                             "sum": int(Ts.sum())}},
        "stream_floor_us_per_layer_step": round(floor, 3) if floor else None,
        "stream_floor_frac": round(r["bytes_per_launch"] / (floor * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) if floor else None,
        "stream_floor_note": ("three launches per layer-step: the q/k/v and wo projections' grids streaming their "
                              "weights alone around the attention's bare K/V stream") if w.is_block else
                             "the step's grid streaming its K/V rows alone",
        "finite": ok,
    }


def t_sweep():
    """Microseconds per layer-step over short to long contexts (eager launches
    and HIP graph replay) at two head shapes; each layer its own cache rows."""
    import torch
    from leap_amd.attention import HipAttention
    dev = torch.device("cuda:0")
    res = {}
    for name, (L, nh, nkv, hd, th) in SWEEP_SHAPES.items():
        att = HipAttention(nh, nkv, hd, max(SWEEP_T), n_layers=L, rope_theta=th)
        try:
            att.kv_fill_normal(SEED + 11, 1 / np.sqrt(hd))
            q = torch.randn(L, nh * hd, device=dev) / np.sqrt(hd)
            k = torch.randn(L, nkv * hd, device=dev) / np.sqrt(hd)
            v = torch.randn(L, nkv * hd, device=dev) / np.sqrt(hd)
            out = torch.empty(L, nh * hd, device=dev)
            s = torch.cuda.Stream()
            sp = s.cuda_stream
            ptrs = [(q[l].data_ptr(), k[l].data_ptr(), v[l].data_ptr(), out[l].data_ptr()) for l in range(L)]
            rows = {}
            for T in SWEEP_T:
                def one_step():
                    for l in range(L):
                        att.step_async(l, T - 1, *ptrs[l], sp)
                ms, _, _ = timed_steps(one_step, s, 100, 10, L)
                eager = ms * 1e3 / (100 * L)
                gus = hip_graph_us(one_step, s, 100, L)
                rows[str(T)] = {"eager_us": round(eager, 3), "graph_us": round(gus, 3),
                                "graph_GBps": round(algorithmic_bytes(T, nh, nkv, hd) / (gus * 1e-6) / 1e9, 1)}
            res[name] = {"n_layers": L, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd, "T": rows}
        finally:
            att.close()
    res["note"] = ("eager: one Python ctypes call per launch (the launch floor of about 3-4 us per launch from "
                   "Python), so the shortest contexts are host-bound there; graph: the same launches replayed "
                   "from a HIP graph")
    gen = generation_sweep()
    res["generation_llama3-8b"] = gen
    res["mean_us_per_layer_step_T1_4096"] = gen["mean_us_per_layer_step_T1_4096"]
    res["mean_graph_us_per_layer_step_T1_4096"] = gen["mean_graph_us_per_layer_step_T1_4096"]
    return res


GEN_T = (1, 2, 4, 8, 16) + tuple(range(32, 4097, 32))


def generation_sweep(steps: int = 20):
    """A generation's decode steps at the Llama-3-8B head shape (32 layers):
    the reference's generate loop walks T = pos + 1 from 1 to the context
    (main.cpp:77-82).  Microseconds per layer-step at every 32nd context
    (and 1-16), eager and replayed from a HIP graph, and their mean over T =
    1..4096 with the samples joined linearly (one value per T)."""
    import torch
    from leap_amd.attention import HipAttention
    L, nh, nkv, hd, th = SWEEP_SHAPES["llama3-8b"]
    dev = torch.device("cuda:0")
    att = HipAttention(nh, nkv, hd, max(GEN_T), n_layers=L, rope_theta=th)
    eager, graph = [], []
    try:
        att.kv_fill_normal(SEED + 12, 1 / np.sqrt(hd))
        q = torch.randn(L, nh * hd, device=dev) / np.sqrt(hd)
        k = torch.randn(L, nkv * hd, device=dev) / np.sqrt(hd)
        v = torch.randn(L, nkv * hd, device=dev) / np.sqrt(hd)
        out = torch.empty(L, nh * hd, device=dev)
        s = torch.cuda.Stream()
        sp = s.cuda_stream
        ptrs = [(q[l].data_ptr(), k[l].data_ptr(), v[l].data_ptr(), out[l].data_ptr()) for l in range(L)]
        for T in GEN_T:
            def one_step():
                for l in range(L):
                    att.step_async(l, T - 1, *ptrs[l], sp)
            ms, _, _ = timed_steps(one_step, s, steps, 3, L)
            eager.append(ms * 1e3 / (steps * L))
            graph.append(hip_graph_us(one_step, s, steps, L))
    finally:
        att.close()
    allT = np.arange(1, 4097)
    return {
        "n_layers": L, "n_heads": nh, "n_kv_heads": nkv, "head_dim": hd,
        "T": list(GEN_T), "eager_us": [round(x, 3) for x in eager], "graph_us": [round(x, 3) for x in graph],
        "mean_us_per_layer_step_T1_4096": round(float(np.interp(allT, GEN_T, eager).mean()), 3),
        "mean_graph_us_per_layer_step_T1_4096": round(float(np.interp(allT, GEN_T, graph).mean()), 3),
    }


# ---- timeline (the library's timeline build) ---------------------------------------

TL_POINTS = ("start", "prologue", "scored", "loop_end", "combined", "stored", "drained", "counted",
             "fold_issued", "fold_loaded", "folded", "sub_counted", "sub_folded", "end")
TL_ROLE, TL_HW, TL_WORDS, TL_SLOTS, TL_WGS = 14, 15, 16, 64, 2048
TL_SINGLE, TL_FINAL, TL_HELPER, TL_SUB = 1, 2, 4, 8


def timeline_report(workload: str, steps: int, warmup: int, split: int = 0, fold_helper: int = 1):
    """Per-workgroup device-clock stamps of the workload's decode launches,
    from the timeline build of the library (libleap_hip_attention_tl.so,
    the same sources with LEAP_TIMELINE; see leap_hip_attention_timeline).
    Over the last launches the ring holds (up to 64), each launch's stamps
    are taken relative to its first workgroup's entry, in microseconds; the
    report gives, per point, the median over launches of the median and of
    the last workgroup to pass it, the final folder's and the fold helper's
    own points, the launch end (the last workgroup's exit) and the gap to the
    next launch's first workgroup."""
    import ctypes
    import torch
    from leap_amd import attention as A
    lib = A.load_timeline_library()
    w = Workload(workload, split=split, lib=lib)
    if fold_helper != 1:
        w.att.set_fold_helper(fold_helper)
    try:
        for _ in range(warmup):
            w.one_step()
        n_steps = max(steps, -(-TL_SLOTS // w.L))
        for _ in range(n_steps):
            w.one_step()
        torch.cuda.synchronize()
        ring = np.zeros(TL_SLOTS * TL_WGS * TL_WORDS, np.uint64)
        launches = ctypes.c_longlong(0)
        rc = lib.leap_hip_attention_timeline(ring.ctypes.data, ring.nbytes, ctypes.byref(launches))
        if rc != 0:
            raise RuntimeError(f"leap_hip_attention_timeline returned {rc}")
    finally:
        w.close()
    ring = ring.reshape(TL_SLOTS, TL_WGS, TL_WORDS)
    n = min(TL_SLOTS, launches.value, n_steps * w.L)
    order = [(launches.value - n + i) % TL_SLOTS for i in range(n)]
    per = []
    for j, slot in enumerate(order):
        t = ring[slot].astype(np.int64)
        st = t[:, 0]
        live = st > 0
        anchor = np.median(st[live])
        wg = live & (np.abs(st - anchor) < 10_000)  # this launch's workgroups (100 us window)
        t0 = st[wg].min()
        rel = np.where(t[wg, :14] > 0, (t[wg, :14] - t0) / 100.0, np.nan)  # ticks of 10 ns -> us
        role = t[wg, TL_ROLE]
        r = {"n_wg": int(wg.sum()), "end": float(np.nanmax(rel[:, 13]))}
        for k, name in enumerate(TL_POINTS[1:13], start=1):
            col = rel[:, k]
            if np.isfinite(col).any():
                r[name] = (float(np.nanmedian(col)), float(np.nanmax(col)))
        for tag, bit in (("final", TL_FINAL), ("helper", TL_HELPER)):
            sel = (role & bit) != 0
            if sel.any():
                sub = rel[sel]
                r[tag] = {name: float(np.nanmedian(sub[:, k])) for k, name in enumerate(TL_POINTS)
                          if k > 0 and np.isfinite(sub[:, k]).any()}
        if j + 1 < n:
            nxt = ring[order[j + 1]].astype(np.int64)[:, 0]
            nl = nxt > 0
            nwin = nl & (np.abs(nxt - np.median(nxt[nl])) < 10_000)
            r["gap_to_next"] = (nxt[nwin].min() - t0) / 100.0 - r["end"]
        per.append(r)

    def med(vals):
        vals = [v for v in vals if v is not None]
        return round(float(np.median(vals)), 3) if vals else None
    out = {"workload": workload, "launches": n, "n_wg": int(np.median([r["n_wg"] for r in per])),
           "launch_end_us": med([r["end"] for r in per]),
           "gap_to_next_us": med([r.get("gap_to_next") for r in per]), "points_us": {}}
    for name in TL_POINTS[1:13]:
        have = [r[name] for r in per if name in r]
        if have:
            out["points_us"][name] = {"median_wg": med([h[0] for h in have]), "last_wg": med([h[1] for h in have])}
    for tag in ("final", "helper"):
        have = [r[tag] for r in per if tag in r]
        if have:
            out[tag + "_us"] = {name: med([h.get(name) for h in have]) for name in TL_POINTS[1:]
                                if any(name in h for h in have)}
    out["note"] = ("device clock (s_memrealtime, 100 MHz) per workgroup from libleap_hip_attention_tl.so, "
                   "relative to each launch's first workgroup entry; medians over the launches; the stamps "
                   "themselves cost a little (wave 0 keeps them in registers and stores them at exit)")
    return out


# ---- CPU baseline (the reference's own code, or the oracle) ------------------------

def host_cpu():
    """CPU model, usable logical CPUs, physical cores among them, AVX-512F."""
    model, flags = "unknown", ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name") and model == "unknown":
                model = line.split(":", 1)[1].strip()
            elif line.startswith("flags") and not flags:
                flags = line.split(":", 1)[1]
    except OSError:
        pass
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        try:
            core = open(f"/sys/devices/system/cpu/cpu{c}/topology/core_id").read().strip()
            pkg = open(f"/sys/devices/system/cpu/cpu{c}/topology/physical_package_id").read().strip()
            cores.add((pkg, core))
        except OSError:
            cores.add(("?", str(c)))
    return {"model": model, "logical_cpus": len(cpus), "physical_cores": len(cores),
            "avx512f": " avx512f " in f" {flags} "}


def cpu_leg_child(spec_path: str):
    """The CPU leg proper, in a child process whose OpenMP settings the parent
    fixed (no GPU, no torch): prints one JSON object."""
    from oracle import oracle as O
    spec = json.load(open(spec_path))
    data = np.load(spec["data"])
    T, budget, kind = spec["T"], spec["budget_s"], spec["kind"]
    dim, nh, nkv = spec["dim"], spec["n_heads"], spec["n_kv"]
    if kind in ("attention", "block", "block_q8"):
        if kind == "attention":
            w = [data["rms"], data["wq"], data["wk"], data["wv"], data["wo"]]
            gs = None
        elif kind == "block":
            w = [data["rms"], data["wq"], data["wk"], data["wv"], data["wo"]]
            gs = None
        else:
            w = [data["rms"]] + [(data[f"{n}_q"], data[f"{n}_s"]) for n in ("wq", "wk", "wv", "wo")]
            gs = Q8_GROUP
        timer = O.RefBlockTimer(dim, nh, nkv, T, *w, data["k"], data["v"], gs=gs, n_layers=spec["n_layers"])
        x0 = data["x"]
        x = x0.copy()
        long_t, short_t = [], []
        try:
            timer.run(T - 1, x, spec["n_layers"])  # the OpenMP pool starts, every layer touched once
            t_end = time.perf_counter() + budget
            while time.perf_counter() < t_end or len(long_t) < 5:
                x[:] = x0
                long_t.append(timer.run(T - 1, x, 1))
                if kind == "attention":
                    x[:] = x0
                    short_t.append(timer.run(0, x, 1))
        finally:
            timer.close()
        us = float(np.median(long_t)) * 1e6
        res = {"calls": len(long_t), "long_us": us}
        if kind == "attention":
            res["short_us"] = float(np.median(short_t)) * 1e6
            us -= res["short_us"]
        res["us"] = us
    else:  # the oracle restatement of the attention step
        O.lib().oracle_set_threads(spec["threads"])
        n_l = data["k"].shape[0]
        hd = dim // nh
        orc = O.Oracle(n_l, nh, nkv, hd, T, theta=spec["theta"])
        for l in range(n_l):
            orc.key_cache[l, :T - 1] = data["k"][l]
            orc.value_cache[l, :T - 1] = data["v"][l]
        rng = np.random.default_rng(SEED)
        qs = [(rng.standard_normal(dim) / np.sqrt(hd)).astype(np.float32) for _ in range(n_l)]
        ks = [(rng.standard_normal(nkv * hd) / np.sqrt(hd)).astype(np.float32) for _ in range(n_l)]
        vs = [(rng.standard_normal(nkv * hd) / np.sqrt(hd)).astype(np.float32) for _ in range(n_l)]
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            for l in range(n_l):
                orc.step(l, T - 1, qs[l], ks[l], vs[l])
            times.append((time.perf_counter() - t0) / n_l)
        res = {"calls": len(times), "us": float(np.median(times)) * 1e6}
    print(json.dumps(res), flush=True)


def cpu_baseline(w: Workload, budget_s: float, cpu_layers: int):
    """The CPU baseline of workload `w` on the host cores at min(n_heads,
    physical cores) threads and at every usable logical CPU, each in a child
    process with OMP_PROC_BIND=close OMP_PLACES=cores (the reference README's
    pinning).  The data (sequence 0's first T-1 device cache rows, synthetic
    weights) is written to a temporary file the child reads."""
    from oracle import oracle as O
    cpu = host_cpu()
    T = int(w.Ts[0])
    nh, nkv, hd = w.nh, w.nkv, w.hd
    dim, kvd = nh * hd, nkv * hd
    variant = "v4" if cpu["avx512f"] else "v3"
    env_base = dict(os.environ, OMP_PROC_BIND="close", OMP_PLACES="cores", LEAP_REF_VARIANT=variant)
    if dim > 8192:
        # the reference's run_layer at this width holds 2 GiB of weights per
        # layer, and the timed engine cycles several such layers
        raise RuntimeError(f"no CPU leg at dim {dim}: the reference engine would hold "
                           f"{4 * (2 * dim * dim + 2 * kvd * dim) / 2**30:.1f} GiB of weights per layer")
    ref_ok = (O.ref_q8_available() if w.is_q8 else O.ref_available()) and w.theta == 500000.0
    if ref_ok:
        kind = "block_q8" if w.is_q8 else "block" if w.is_block else "attention"
        if w.is_block:
            nbytes = w.bytes_layer
            arrays = {"rms": w.weights[0]}
            if w.is_q8:
                for n, (q, sc) in zip(("wq", "wk", "wv", "wo"), w.weights[1:]):
                    arrays[f"{n}_q"], arrays[f"{n}_s"] = q, sc
            else:
                arrays.update(zip(("wq", "wk", "wv", "wo"), w.weights[1:]))
            per_layer = nbytes
        else:
            nbytes = algorithmic_bytes(T, nh, nkv, hd)
            wrng = np.random.default_rng(SEED + w.sidx)
            arrays = {"rms": (1.0 + 0.1 * wrng.standard_normal(dim)).astype(np.float32)}
            for n, shape in (("wq", (dim, dim)), ("wk", (kvd, dim)), ("wv", (kvd, dim)), ("wo", (dim, dim))):
                arrays[n] = (wrng.standard_normal(shape) / np.sqrt(dim)).astype(np.float32)
            per_layer = 4 * (2 * dim * dim + 2 * kvd * dim) + 8 * T * kvd
        arrays["k"], arrays["v"] = w.att.kv_download(0, 0, 0, T - 1)
        arrays["x"] = np.random.default_rng(SEED + w.sidx + 100).standard_normal(dim).astype(np.float32)
        # enough layers (each its own copy of the weights and cache rows) that the
        # host's caches cannot hold them: about 1.6 GB
        n_layers = max(4, -(-1_600_000_000 // per_layer))
    else:
        kind = "oracle"
        nbytes = algorithmic_bytes(T, nh, nkv, hd)
        n_layers = min(cpu_layers, w.L)
        ks, vs = zip(*[w.att.kv_download(0, l, 0, T - 1) for l in range(n_layers)])
        arrays = {"k": np.stack(ks), "v": np.stack(vs)}
        if not os.path.isfile(O.ORACLE_SO):
            O.build(ref=False)
    counts = sorted({min(nh, cpu["physical_cores"]), cpu["logical_cpus"]})
    runs = {}
    with tempfile.TemporaryDirectory(prefix="leap_cpu_leg_") as tmp:
        data_path = os.path.join(tmp, "data.npz")
        np.savez(data_path, **arrays)
        for threads in counts:
            spec = {"data": data_path, "T": T, "budget_s": budget_s / len(counts), "kind": kind, "dim": dim,
                    "n_heads": nh, "n_kv": nkv, "n_layers": n_layers, "threads": threads, "theta": w.theta}
            spec_path = os.path.join(tmp, f"spec{threads}.json")
            json.dump(spec, open(spec_path, "w"))
            env = dict(env_base, OMP_NUM_THREADS=str(threads))
            r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-leg", spec_path], env=env,
                               capture_output=True, text=True, timeout=budget_s * 4 + 120)
            if r.returncode != 0:
                raise RuntimeError(f"CPU leg with {threads} threads failed: {r.stderr[-400:]}")
            runs[threads] = json.loads(r.stdout.strip().splitlines()[-1])
    best_t = min(runs, key=lambda t: runs[t]["us"])
    us = runs[best_t]["us"]
    lib_name = ("QuantizedTransformer" if w.is_q8 else "FloatTransformer")
    if kind == "attention":
        r0 = runs[best_t]
        sample = (f"the reference's FloatTransformer::run_layer, {r0['calls']} calls each at pos {T - 1} and pos 0 "
                  f"alternating over an engine of {n_layers} layers (synthetic weights, sequence 0's device cache "
                  f"rows); attention = difference of the medians ({r0['long_us']:.1f} - {r0['short_us']:.1f} us)")
    elif kind in ("block", "block_q8"):
        sample = (f"{runs[best_t]['calls']} calls of the reference's {lib_name}::run_layer at pos {T - 1}, cycling "
                  f"through an engine of {n_layers} layers that each hold the workload's weights (zero FFN) and "
                  f"layer 0's device cache rows; median per call")
    else:
        sample = (f"{runs[best_t]['calls']} sweeps of the oracle (the restated reference, OpenMP over heads, AVX2) "
                  f"over layers 0..{n_layers - 1} of sequence 0 (context {T}), device cache bytes downloaded; "
                  f"median per layer-step")
    return {
        "value": round(nbytes / (us * 1e-6) / 1e9, 3), "unit": "GB/s", "cores": best_t,
        "kind": "reference" if ref_ok else "port", "us_per_layer_step": round(us, 2),
        "by_threads": {str(t): {"us_per_layer_step": round(r["us"], 2),
                                "value": round(nbytes / (r["us"] * 1e-6) / 1e9, 3)} for t, r in runs.items()},
        "threads_note": f"min(n_heads, physical cores) = {min(nh, cpu['physical_cores'])}, "
                        f"all usable logical CPUs = {cpu['logical_cpus']}; `value` is the faster",
        "cpu": cpu, "omp": "OMP_PROC_BIND=close OMP_PLACES=cores (the reference README's pinning)",
        "march": (f"x86-64-{variant} with the reference's other release flags (-O3 -ffast-math -funroll-loops "
                  f"-fomit-frame-pointer -fopenmp); its CMakeLists.txt:33 says -march=native, which needs the "
                  f"sources on the host that runs it; the reference has only NEON and AVX2 paths, so both take "
                  f"its __AVX2__ code"),
        "sample": sample,
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
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the floor, the other workloads and the context sweep")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--cpu-layers", type=int, default=4)
    ap.add_argument("--split", type=int, default=0, help="positions per split-K chunk (0 = auto)")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP graph replay timing")
    ap.add_argument("--products", choices=("mfma", "valu"), default="mfma",
                    help="score and weighted-V products on the matrix cores (default) or the VALU")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run 10 plain device copies of MIB MiB (the reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    ap.add_argument("--timeline", action="store_true",
                    help="only run the workload on the library's timeline build and print the per-phase "
                         "device-clock medians of its launches")
    ap.add_argument("--fold-helper", type=int, default=1, choices=(0, 1, 2),
                    help="the fold-helper mode of the timeline run (leap_hip_attention_set_fold_helper)")
    ap.add_argument("--cpu-leg", default=None, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_leg:
        cpu_leg_child(args.cpu_leg)
        return
    if args.timeline:
        print(json.dumps(timeline_report(args.workload, args.steps or 8, args.warmup, args.split,
                                         args.fold_helper)), flush=True)
        return
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
    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        sys.exit(1)

    w = Workload(args.workload, split=args.split, valu=args.products == "valu")
    r = measure(w, steps, args.warmup, graph=not args.no_graph)
    if not w.finite():
        print("non-finite output", file=sys.stderr)
        sys.exit(1)
    us_layer, gbs = r["us_per_layer_step"], r["value"]
    L, nh, nkv, hd, theta, batch = w.L, w.nh, w.nkv, w.hd, w.theta, w.batch
    Ts = w.Ts
    result = {
        "metric": metric_for(args.workload),
        "value": gbs,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms_total"] / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8+f32" if w.is_q8 else "f32",
        "products": args.products,
        "data": (f"synthetic (seeded N(0,1)/sqrt({hd}) KV cache generated on the device; "
                 f"N(0,1)/sqrt(dim) weights{f', int8 with one scale per {Q8_GROUP} values' if w.is_q8 else ''}, "
                 f"one set uploaded into every layer)") if w.is_block else
                f"synthetic (seeded N(0,1)/sqrt({hd}) KV cache and q/k/v, generated on the device)",
        "config": {
            "workload": args.workload, "n_layers": L, "n_heads": nh, "n_kv_heads": nkv,
            "head_dim": hd, "batch": batch, "rope_theta": theta,
            "context": int(Ts[0]) if batch == 1 else
            {"min": int(Ts.min()), "max": int(Ts.max()), "sum": int(Ts.sum())},
        },
        "us_per_layer_step": us_layer,
        "us_per_layer_step_spread": r["spread"],
        "pct_of_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "tokens_layers_per_s": round(batch * 1e6 / us_layer, 1),
        "host_wall_s": round(r["wall"], 4),
        "roofline": {
            "kernel": Q8_KERNELS if w.is_q8 else BLOCK_KERNELS if w.is_block else KERNEL,
            "bound": "hbm",
            "achieved": gbs,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": r["frac"],
            "traffic": traffic_from_profiles(args.workload),
            "traffic_source": f"profiles/decode_attention_{args.workload}_traffic.txt (rocprofv3 FETCH_SIZE and "
                              "WRITE_SIZE of the same kernels, copy-scaled; counters need a run of their own)",
            "bytes_per_launch": w.bytes_layer,
            "launch_us": us_layer,
        },
        "cpu_baseline": None,
    }
    if "hip_graph_us" in r:
        gus = r["hip_graph_us"]
        result["hip_graph"] = {
            "us_per_layer_step": gus,
            "value": round(w.bytes_layer / (gus * 1e-6) / 1e9, 2),
            "unit": "GB/s",
            "note": "the same steps captured into a HIP graph (at least 32 launches per graph) and replayed; "
                    "`value` above is eager launches",
        }
    if not args.no_extra and not w.is_block:
        fl = w.floor_us(1, steps, args.warmup)
        fs = w.floor_us(2, steps, args.warmup)
        kv_bytes = int(sum(8 * (int(T) - 1) * nkv * hd for T in Ts))
        result["floor"] = {
            "launch_us_per_layer_step": round(fl, 3),
            "stream_us_per_layer_step": round(fs, 3),
            "stream_GBps": round(kv_bytes / (fs * 1e-6) / 1e9, 1),
            "kernel_over_stream_floor_us": round(us_layer - fs, 3),
            "note": "the same grid, block and argument block as the step: a kernel that only reads its "
                    "arguments (launch floor), and one that only streams the same K/V rows with the same "
                    "loads and sums them (launch + bare stream); eager launches, events over the same steps",
        }
    if not args.no_extra and not w.is_block:
        # the A/B of the matrix-core choice: the same launches with the products on the VALU
        w.att.set_products(args.products == "mfma")
        rv = measure(w, steps, args.warmup, graph=False)
        w.att.set_products(args.products == "valu")
        other = "valu" if args.products == "mfma" else "mfma"
        result["products_ab"] = {
            f"{args.products}_us_per_layer_step": us_layer, f"{other}_us_per_layer_step": rv["us_per_layer_step"],
            "note": "score (q.K) and weighted-V products on the matrix cores (4x4x1 f32 MFMA) or as per-lane "
                    "VALU FMAs with the same cross-lane sums; same launches, same events",
        }
    if batch == 1 and not args.no_host_pointer:
        pos = int(Ts[0]) - 1
        result["host_pointer"] = host_pointer_rate(w.att, L, pos, w.bytes_layer, w.is_block,
                                                   sweeps=max(1, min(steps, 20)))
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds, args.cpu_layers)
        except Exception as e:  # the GPU line still stands; say why the CPU leg is missing
            result["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    w.close()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    if not args.no_extra and args.workload == "llama3-8b-ctx4096":
        result["workloads"] = {}
        for name in EXTRA_WORKLOADS:
            try:
                result["workloads"][name] = extra_workload(name)
            except Exception as e:
                result["workloads"][name] = {"error": f"{type(e).__name__}: {e}"}
            print(f"[bench] {name}: {result['workloads'][name].get('us_per_layer_step')} us/layer-step",
                  file=sys.stderr, flush=True)
        result["t_sweep"] = t_sweep()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
