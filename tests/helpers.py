"""Shared test helpers: seeded inputs, a float64 textbook attention, tolerance."""
from __future__ import annotations

import numpy as np

# Parity bar for the attention output: max |delta| <= REL_TOL * max |reference|
# (fp32 reductions in a different order from the reference's).
REL_TOL = 1e-4


def rng_for(*key) -> np.random.Generator:
    return np.random.default_rng(np.random.SeedSequence([0x4C454150, *key]))


def normal(rng, shape, head_dim):
    return (rng.standard_normal(shape) / np.sqrt(head_dim)).astype(np.float32)


def rel_err(got, want) -> float:
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    return float(np.abs(got - want).max() / scale)


def assert_close(got, want, rel=REL_TOL, what="output"):
    e = rel_err(got, want)
    assert e <= rel, f"{what}: max|delta|/Linf = {e:.3e} > {rel:.1e}"
    return e


def rope_f32(x, cos_row, sin_row):
    """Interleaved-pair rotation with fp32 table rows, products rounded
    separately (the reference's RoPE rule, FloatTransformer.cpp:478-493)."""
    x = np.asarray(x, np.float32).reshape(-1, cos_row.size * 2)
    x0, x1 = x[:, 0::2], x[:, 1::2]
    c, s = cos_row[None, :], sin_row[None, :]
    y = np.empty_like(x)
    y[:, 0::2] = (x0 * c).astype(np.float32) - (x1 * s).astype(np.float32)
    y[:, 1::2] = (x1 * c).astype(np.float32) + (x0 * s).astype(np.float32)
    return y.reshape(-1)


def attention_f64(q_rot, k_rows, v_rows, n_heads, n_kv_heads, head_dim):
    """Textbook softmax(q.K^T / sqrt(d)) V in float64 for every head.
    q_rot: [n_heads*hd]; k_rows, v_rows: [T, n_kv_heads*hd] (k already rotated)."""
    kv_mul = n_heads // n_kv_heads
    q = np.asarray(q_rot, np.float64).reshape(n_heads, head_dim)
    K = np.asarray(k_rows, np.float64).reshape(-1, n_kv_heads, head_dim)
    V = np.asarray(v_rows, np.float64).reshape(-1, n_kv_heads, head_dim)
    out = np.empty((n_heads, head_dim))
    for h in range(n_heads):
        g = h // kv_mul
        s = K[:, g, :] @ q[h] / np.sqrt(head_dim)
        s -= s.max()
        p = np.exp(s)
        p /= p.sum()
        out[h] = p @ V[:, g, :]
    return out.reshape(-1)


def block_inputs(rng, dim, n_kv_dim):
    """Seeded inputs of the attention sub-block: the residual stream x, the
    rms_att weight (around 1) and the projections Wq [dim][dim],
    Wk/Wv [kv_dim][dim], Wo [dim][dim] scaled by 1/sqrt(dim)."""
    x = rng.standard_normal(dim).astype(np.float32)
    rms = (1.0 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    wq = normal(rng, (dim, dim), dim)
    wk = normal(rng, (n_kv_dim, dim), dim)
    wv = normal(rng, (n_kv_dim, dim), dim)
    wo = normal(rng, (dim, dim), dim)
    return x, rms, wq, wk, wv, wo


def write_checkpoint(path, version, dim, hidden_dim, n_heads, n_kv_heads, vocab_size, seq_len, layers,
                     shared=True, group_size=64, rms_ffn=None, rms_final=None, emb=None, ffn=None, wcls=None):
    """Write a LEAP checkpoint in the layout the reference's exporters write
    and Transformer::create reads (Export.cpp:17-90 and :95-274,
    TransformerFactory.cpp:59-135, memory_map_weights): `layers` is one
    (rms_att, wq, wk, wv, wo) per layer, fp32 arrays for versions 0/1 and
    (int8 values, scales) pairs for the projections in version 2.  The FFN,
    embeddings and classifier default to zeros (the FFN then adds exactly 0
    in run_layer).  Version 0 (legacy) stores vocab_size negated when the
    classifier is not shared."""
    import struct
    L = len(layers)
    hd = dim // n_heads
    kv = n_kv_heads * hd
    f32 = lambda a: np.ascontiguousarray(a, np.float32).tobytes()  # noqa: E731
    out = bytearray()
    cfg = [dim, hidden_dim, L, n_heads, n_kv_heads, vocab_size, seq_len]
    if version == 0:
        cfg[5] = vocab_size if shared else -vocab_size
        out += struct.pack("<7i", *cfg)
    else:
        out += struct.pack("<Ii", 0x616B3432, version) + struct.pack("<7i", *cfg)
        out += struct.pack("<B", 1 if shared else 0)
        if version == 2:
            out += struct.pack("<i", group_size)
        out += bytes(256 - len(out))
    z = lambda *shape: np.zeros(shape, np.float32)  # noqa: E731
    rms_ffn = z(L, dim) + 1 if rms_ffn is None else rms_ffn
    rms_final = z(dim) + 1 if rms_final is None else rms_final
    emb = z(vocab_size, dim) if emb is None else emb
    out += b"".join(f32(l[0]) for l in layers) + f32(rms_ffn) + f32(rms_final)
    if version != 2:
        out += f32(emb)
        for t in range(1, 5):
            out += b"".join(f32(l[t]) for l in layers)
        if ffn is None:
            out += bytes(4 * L * 3 * dim * hidden_dim)
        else:
            out += b"".join(f32(w) for w in ffn)
        if not shared:
            out += f32(z(vocab_size, dim) if wcls is None else wcls)
    else:
        def q8(q, sc):
            return np.ascontiguousarray(q, np.int8).tobytes() + f32(sc)
        out += q8(np.zeros(vocab_size * dim, np.int8), z(vocab_size * dim // group_size))
        for t in range(1, 5):
            out += b"".join(q8(*l[t]) for l in layers)
        for n in (dim * hidden_dim,) * 3:  # w1, w2, w3: zero values and scales
            out += L * (bytes(n) + bytes(4 * (n // group_size)))
        if not shared:
            out += q8(np.zeros(vocab_size * dim, np.int8), z(vocab_size * dim // group_size))
    with open(path, "wb") as f:
        f.write(out)
    return len(out)
