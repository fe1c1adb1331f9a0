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
