"""Write the golden fixtures of tests/golden/ from the reference's own code.

Runs the reference's FloatTransformer::run_layer and precompute_freqs through
the test driver oracle/_ref (built by `make -C oracle ref` from the reference
sources), on seeded synthetic inputs, and stores inputs and outputs as .npz:

  run_layer_<name>.npz : config, layer, pos, the pre-RoPE q/k/v the reference
                         computed, the cache rows [0, pos] of that layer before
                         the call, and after it: the rotated q, the cache rows
                         at pos (rotated k, v) and the attention output s->xb.
  rope_<name>.npz      : sampled rows of the reference's rope_cos/rope_sin.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import oracle as O  # noqa: E402

CASES = [
    # name, dim, n_heads, n_kv_heads, n_layers, seq_len, layer, pos
    ("tinyllama_pos255", 2048, 32, 4, 2, 256, 1, 255),
    ("tinyllama_pos0", 2048, 32, 4, 2, 256, 0, 0),
    ("llama3_8b_pos69", 4096, 32, 8, 1, 128, 0, 69),
    ("mha_hd128_pos40", 1024, 8, 8, 1, 64, 0, 40),
    ("gqa8_hd128_pos33", 2048, 16, 2, 2, 48, 1, 33),
]

ROPE = [
    # name, dim, n_heads, seq_len, rows sampled
    ("hd64_256", 2048, 32, 256, list(range(256))),
    ("hd128_131072", 4096, 32, 131072,
     [0, 1, 2, 3, 255, 256, 4095, 4096, 8191, 65535, 100000, 131070, 131071]),
]


def main():
    if not O.ref_available():
        O.build(ref=True)
    for name, dim, nh, nkv, L, sl, layer, pos in CASES:
        rng = np.random.default_rng(np.random.SeedSequence([0x4C454150, len(name), dim, pos]))
        hd = dim // nh
        kvd = nkv * hd
        x = rng.standard_normal(dim).astype(np.float32)
        wq = (rng.standard_normal((dim, dim)) / np.sqrt(dim)).astype(np.float32)
        wk = (rng.standard_normal((kvd, dim)) / np.sqrt(dim)).astype(np.float32)
        wv = (rng.standard_normal((kvd, dim)) / np.sqrt(dim)).astype(np.float32)
        kc = np.zeros((L, sl, kvd), np.float32)
        vc = np.zeros_like(kc)
        kc[layer, :pos] = rng.standard_normal((pos, kvd)) / np.sqrt(hd)
        vc[layer, :pos] = rng.standard_normal((pos, kvd)) / np.sqrt(hd)
        r = O.ref_run_layer(dim, nh, nkv, L, sl, layer, pos, x, wq, wk, wv, kc, vc)
        np.savez(os.path.join(HERE, f"run_layer_{name}.npz"),
                 dims=np.array([dim, nh, nkv, L, sl, layer, pos], np.int32),
                 q_pre=r["q_pre"], k_pre=r["k_pre"], v_pre=r["v_pre"],
                 k_rows=kc[layer, :pos], v_rows=vc[layer, :pos],
                 q_rot=r["q_rot"], k_slot=r["key_cache"][layer, pos],
                 v_slot=r["value_cache"][layer, pos], out=r["out"])
    for name, dim, nh, sl, rows in ROPE:
        c, s = O.ref_rope_table(dim, nh, sl)
        rows = np.array(rows, np.int64)
        np.savez(os.path.join(HERE, f"rope_{name}.npz"),
                 dims=np.array([dim, nh, sl], np.int64), rows=rows, cos=c[rows], sin=s[rows])
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
