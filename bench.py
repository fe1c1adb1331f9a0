#!/usr/bin/env python3
"""Decode-attention benchmark on one MI355X.

Workload: Llama-3-8B-shaped decode attention, batch 1, context 4096 cached
positions (pos = 4095), all 32 layers stepped in sequence; n_heads 32,
n_kv_heads 8, head_dim 128, RoPE theta 500000; fp32 KV cache (1 GiB) and fp32
q/k/v filled with seeded N(0,1)/sqrt(128) values on the device.

One step = one token through the attention block of all 32 layers: 32
launches of the fused decode-attention kernel, back to back on one stream,
with q/k/v/out resident in HBM.  Reported value: algorithmic HBM GB/s over the
timed region, B(T) = 8*T*kv_dim + 8*dim + 16*kv_dim + 4*head_dim bytes per
layer-step, with microseconds per layer-step and the fraction of the 8 TB/s
HBM peak alongside.

The CPU baseline is the oracle (the restated reference attention, OpenMP over
heads, AVX2) timed on the host cores on a bounded sample of the same
workload: the same device bytes of a few layers, downloaded.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
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

N_LAYERS, N_HEADS, N_KV, HD, CTX, THETA = 32, 32, 8, 128, 4096, 500000.0
SEED = 0x4C454150 + 1


def algorithmic_bytes(T: int, n_heads=N_HEADS, n_kv=N_KV, hd=HD) -> int:
    """Bytes one layer-step must move for one sequence: the K and V rows
    [0, T), q in and out, new k and v in and their cache rows out, and the
    RoPE table row."""
    kv_dim, dim = n_kv * hd, n_heads * hd
    return 8 * T * kv_dim + 8 * dim + 16 * kv_dim + 4 * hd


def traffic_from_profiles():
    """HBM bytes per launch measured by rocprofv3 FETCH_SIZE/WRITE_SIZE runs
    (scaled by a copy kernel's counters), recorded in profiles/."""
    path = os.path.join(ROOT, "profiles", "decode_attention_llama3_8b_ctx4096_traffic.txt")
    if not os.path.isfile(path):
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", open(path).read(), re.M)
    return float(m.group(1)) if m else None


def cpu_baseline(att, n_layers_sample: int, budget_s: float):
    """Time the oracle on the host on layers [0, n_layers_sample) of the
    device cache (downloaded bytes), repeating sweeps for about budget_s."""
    from oracle import oracle as O
    if not os.path.isfile(O.ORACLE_SO):
        O.build(ref=False)
    threads = min(N_HEADS, int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count() or 1, 16)
    O.lib().oracle_set_threads(threads)
    pos = CTX - 1
    rng = np.random.default_rng(SEED)
    orc = O.Oracle(n_layers_sample, N_HEADS, N_KV, HD, CTX, theta=THETA)
    for l in range(n_layers_sample):
        k, v = att.kv_download(0, l, 0, CTX)
        orc.key_cache[l] = k
        orc.value_cache[l] = v
    qs = [(rng.standard_normal(N_HEADS * HD) / np.sqrt(HD)).astype(np.float32) for _ in range(n_layers_sample)]
    ks = [(rng.standard_normal(N_KV * HD) / np.sqrt(HD)).astype(np.float32) for _ in range(n_layers_sample)]
    vs = [(rng.standard_normal(N_KV * HD) / np.sqrt(HD)).astype(np.float32) for _ in range(n_layers_sample)]
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        for l in range(n_layers_sample):
            orc.step(l, pos, qs[l], ks[l], vs[l])
        times.append((time.perf_counter() - t0) / n_layers_sample)
    us = float(np.median(times)) * 1e6
    gbs = algorithmic_bytes(CTX) / (us * 1e-6) / 1e9
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "us_per_layer_step": round(us, 2),
        "sample": f"{len(times)} sweeps of layers 0..{n_layers_sample - 1} of the same workload "
                  f"(device cache bytes downloaded), median per layer-step, OpenMP over heads",
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-layers", type=int, default=4)
    ap.add_argument("--split", type=int, default=0, help="positions per split-K chunk (0 = auto)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the attention step shards by sequence or KV head with no exchange; "
              "run --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch
    from leap_amd.attention import HipAttention

    if not torch.cuda.is_available():
        print("no HIP device", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    att = HipAttention(N_HEADS, N_KV, HD, CTX, n_layers=N_LAYERS, rope_theta=THETA)
    if args.split:
        att.set_split(args.split)
    att.kv_fill_normal(SEED, 1.0 / np.sqrt(HD))

    g = torch.Generator(device=dev)
    g.manual_seed(SEED)
    scale = 1.0 / np.sqrt(HD)
    q = torch.randn(N_LAYERS, N_HEADS * HD, device=dev, generator=g) * scale
    k = torch.randn(N_LAYERS, N_KV * HD, device=dev, generator=g) * scale
    v = torch.randn(N_LAYERS, N_KV * HD, device=dev, generator=g) * scale
    out = torch.empty(N_LAYERS, N_HEADS * HD, device=dev)
    stream = torch.cuda.Stream(device=dev)
    sp = stream.cuda_stream
    pos = CTX - 1
    ptrs = [(q[l].data_ptr(), k[l].data_ptr(), v[l].data_ptr(), out[l].data_ptr()) for l in range(N_LAYERS)]

    def one_step():
        for l in range(N_LAYERS):
            qp, kp, vp, op = ptrs[l]
            att.step_async(l, pos, qp, kp, vp, op, sp)

    torch.cuda.synchronize()
    for _ in range(args.warmup):
        one_step()
    torch.cuda.synchronize()

    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        one_step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = ev0.elapsed_time(ev1)

    launches = args.steps * N_LAYERS
    us_layer = ms_total * 1e3 / launches
    bytes_layer = algorithmic_bytes(CTX)
    gbs = bytes_layer / (us_layer * 1e-6) / 1e9
    if not np.isfinite(out.float().sum().item()):
        print("non-finite attention output", file=sys.stderr)
        sys.exit(1)

    traffic = traffic_from_profiles()
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_total / args.steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1)/sqrt(128) KV cache and q/k/v, generated on the device)",
        "config": {
            "workload": "llama3-8b decode attention, batch 1, ctx 4096, 32 layers per step",
            "n_layers": N_LAYERS, "n_heads": N_HEADS, "n_kv_heads": N_KV, "head_dim": HD,
            "context": CTX, "batch": 1, "rope_theta": THETA,
        },
        "us_per_layer_step": round(us_layer, 3),
        "pct_of_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "tokens_layers_per_s": round(1e6 / us_layer, 1),
        "host_wall_s": round(wall, 4),
        "roofline": {
            "kernel": KERNEL,
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": bytes_layer,
            "launch_us": round(us_layer, 3),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        try:
            result["cpu_baseline"] = cpu_baseline(att, args.cpu_layers, args.cpu_seconds)
        except Exception as e:  # the GPU line still stands; say why the CPU leg is missing
            result["cpu_baseline"] = {"error": f"{type(e).__name__}: {e}"}
    att.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
