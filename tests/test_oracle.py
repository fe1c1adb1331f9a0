"""Pins for the oracle (CPU restatement of the reference's attention block).

Each check is chosen so that a plausible slip fails it: the reference's own
outputs (golden fixtures written by tests/golden/make_golden.py from
oracle/_ref, and the live reference driver when it is built), a float64
textbook attention on tiny shapes, closed forms, and deliberately wrong
variants of the oracle that must fail those pins.
"""
import glob
import os

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import assert_close, attention_f64, block_inputs, normal, rel_err, rng_for, rope_f32

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module", autouse=True)
def _built():
    if not os.path.isfile(O.ORACLE_SO):
        O.build(ref=False)


def _load(path):
    with np.load(path, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _run_fixture(fx, mutant=0):
    dim, nh, nkv, L, sl, layer, pos = (int(v) for v in fx["dims"])
    hd = dim // nh
    orc = O.Oracle(L, nh, nkv, hd, sl)
    orc.key_cache[layer, :pos] = fx["k_rows"]
    orc.value_cache[layer, :pos] = fx["v_rows"]
    out, q_rot = orc.step(layer, pos, fx["q_pre"], fx["k_pre"], fx["v_pre"], mutant=mutant)
    return out, q_rot, orc.key_cache[layer, pos], orc.value_cache[layer, pos]


# ---- RoPE table (FloatTransformer.cpp:56-72) ---------------------------------

@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "rope_*.npz"))))
def test_rope_table_bitwise_reference_golden(path):
    fx = _load(path)
    dim, nh, sl = (int(v) for v in fx["dims"])
    c, s = O.rope_table(sl, dim // nh, 500000.0)
    rows = fx["rows"]
    assert np.array_equal(c[rows], fx["cos"])
    assert np.array_equal(s[rows], fx["sin"])


def test_rope_table_closed_forms():
    for theta in (500000.0, 10000.0):
        c, s = O.rope_table(4096, 128, theta)
        assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)  # pos 0: identity
        # freq_0 = 1: column 0 is cos/sin of the integer position itself.
        pos = np.arange(4096)
        assert np.abs(c[:, 0] - np.cos(pos)).max() < 2e-6
        assert np.abs(s[:, 0] - np.sin(pos)).max() < 2e-6
        assert np.abs(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2 - 1).max() < 1e-6
        # column i follows theta^(-2i/hd) (float64 textbook, fp32-angle tolerance)
        i = np.arange(64)
        ang = 1000.0 * theta ** (-(2.0 * i) / 128.0)
        assert np.abs(c[1000] - np.cos(ang)).max() < 1e-3
        assert np.abs(s[1000] - np.sin(ang)).max() < 1e-3
    # different theta -> different table (the parameter is used)
    assert not np.array_equal(O.rope_table(64, 64, 10000.0)[0], O.rope_table(64, 64, 500000.0)[0])


def test_rope_table_bitwise_live_reference():
    if not O.ref_available():
        pytest.skip("reference driver not built (reference sources absent)")
    for dim, nh, sl in [(2048, 32, 300), (4096, 32, 5000), (1024, 4, 64)]:
        rc, rs = O.ref_rope_table(dim, nh, sl)
        oc, os_ = O.rope_table(sl, dim // nh, 500000.0)
        assert np.array_equal(rc, oc) and np.array_equal(rs, os_)


# ---- the attention step against the reference ----------------------------------

@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "run_layer_*.npz"))))
def test_step_reference_golden(path):
    fx = _load(path)
    out, q_rot, k_slot, v_slot = _run_fixture(fx)
    assert np.array_equal(q_rot, fx["q_rot"]), "rotated q differs from the reference"
    assert np.array_equal(k_slot, fx["k_slot"]), "rotated k in the cache differs"
    assert np.array_equal(v_slot, fx["v_slot"]), "v in the cache differs"
    assert np.array_equal(out, fx["out"]), f"output differs: {rel_err(out, fx['out']):.2e}"



@pytest.mark.parametrize("dim,nh,nkv,L,sl,layer,pos", [
    (512, 8, 2, 3, 100, 2, 99),
    (1024, 16, 16, 1, 37, 0, 36),
    (2048, 16, 2, 2, 20, 0, 7),
    (768, 6, 2, 2, 40, 1, 39),  # three q heads per KV head
])
def test_step_live_reference(dim, nh, nkv, L, sl, layer, pos):
    if not O.ref_available():
        pytest.skip("reference driver not built (reference sources absent)")
    rng = rng_for(dim, pos, 11)
    hd, kvd = dim // nh, nkv * (dim // nh)
    x = rng.standard_normal(dim).astype(np.float32)
    wq = normal(rng, (dim, dim), dim)
    wk = normal(rng, (kvd, dim), dim)
    wv = normal(rng, (kvd, dim), dim)
    kc = normal(rng, (L, sl, kvd), hd)
    vc = normal(rng, (L, sl, kvd), hd)
    r = O.ref_run_layer(dim, nh, nkv, L, sl, layer, pos, x, wq, wk, wv, kc, vc)
    orc = O.Oracle(L, nh, nkv, hd, sl)
    orc.key_cache[:] = kc
    orc.value_cache[:] = vc
    out, q_rot = orc.step(layer, pos, r["q_pre"], r["k_pre"], r["v_pre"])
    assert np.array_equal(q_rot, r["q_rot"])
    assert np.array_equal(orc.key_cache, r["key_cache"])
    assert np.array_equal(orc.value_cache, r["value_cache"])
    assert np.array_equal(out, r["out"]), f"output differs: {rel_err(out, r['out']):.2e}"


def test_clear_matches_reference():
    orc = O.Oracle(2, 4, 2, 8, 16)
    orc.key_cache[:] = 1
    orc.value_cache[:] = 2
    orc.clear()
    assert not orc.key_cache.any() and not orc.value_cache.any()
    if O.ref_available():
        assert O.ref().leapref_clear_check(32, 4, 2, 2, 16) == 0


# ---- independent pins: float64 brute force and closed forms --------------------

def _tiny(seed, nh=4, nkv=2, hd=8, T=64, theta=10000.0, sl=80):
    rng = rng_for(seed, nh, nkv, hd, T)
    orc = O.Oracle(1, nh, nkv, hd, sl, theta=theta)
    pos = T - 1
    orc.key_cache[0, :pos] = normal(rng, (pos, nkv * hd), hd)
    orc.value_cache[0, :pos] = normal(rng, (pos, nkv * hd), hd)
    q = normal(rng, nh * hd, hd)
    k = normal(rng, nkv * hd, hd)
    v = normal(rng, nkv * hd, hd)
    return orc, pos, q, k, v


def _bruteforce(orc, pos, q, k, v):
    c, s = orc.cos[pos], orc.sin[pos]
    K = orc.key_cache[0, :pos + 1].copy()
    V = orc.value_cache[0, :pos + 1].copy()
    K[pos] = rope_f32(k, c, s)
    V[pos] = v
    return attention_f64(rope_f32(q, c, s), K, V, orc.n_heads, orc.n_kv_heads, orc.head_dim)


@pytest.mark.parametrize("nh,nkv,hd,T", [(4, 2, 8, 64), (4, 4, 8, 1), (8, 2, 16, 33),
                                         (6, 3, 10, 17), (4, 1, 64, 50), (6, 2, 16, 29)])
def test_step_float64_bruteforce(nh, nkv, hd, T):
    orc, pos, q, k, v = _tiny(1, nh, nkv, hd, T)
    want = _bruteforce(orc, pos, q, k, v)
    out, _ = orc.step(0, pos, q, k, v)
    assert_close(out, want, rel=1e-5)


def test_first_position_returns_v():
    orc, _, q, k, v = _tiny(2, T=1)
    out, _ = orc.step(0, 0, q, k, v)
    kv_mul = orc.n_heads // orc.n_kv_heads
    want = np.concatenate([v.reshape(orc.n_kv_heads, -1)[h // kv_mul] for h in range(orc.n_heads)])
    assert np.array_equal(out, want)
    assert np.array_equal(orc.key_cache[0, 0], k)  # pos 0 rotation is the identity


def test_identical_keys_give_mean_of_values():
    orc, pos, q, k, v = _tiny(3, T=40)
    c, s = orc.cos[pos], orc.sin[pos]
    krot = rope_f32(k, c, s)
    orc.key_cache[0, :pos] = krot  # every row equals the new (rotated) key
    out, _ = orc.step(0, pos, q, k, v)
    V = orc.value_cache[0, :pos + 1].astype(np.float64).reshape(pos + 1, orc.n_kv_heads, -1)
    kv_mul = orc.n_heads // orc.n_kv_heads
    want = np.concatenate([V[:, h // kv_mul].mean(0) for h in range(orc.n_heads)])
    assert_close(out, want, rel=1e-5)


def test_dominant_key_returns_its_value():
    orc, pos, q, k, v = _tiny(4, nh=2, nkv=1, hd=8, T=30)
    c, s = orc.cos[pos], orc.sin[pos]
    qr = rope_f32(q, c, s).reshape(2, 8)
    planted = 7
    orc.key_cache[0, planted] = (qr[0] / np.linalg.norm(qr[0]) * 400.0).astype(np.float32)
    out, _ = orc.step(0, pos, q, k, v)
    # head 0 sees a score gap of ~400*|q|/sqrt(8) >> 104: every other weight underflows
    assert np.array_equal(out[:8], orc.value_cache[0, planted])


def test_permuting_positions_leaves_output_unchanged():
    orc, pos, q, k, v = _tiny(5, T=48)
    out1, _ = orc.step(0, pos, q, k, v)
    perm = rng_for(5, 99).permutation(pos)
    orc2, _, _, _, _ = _tiny(5, T=48)
    orc2.key_cache[0, :pos] = orc2.key_cache[0, perm]
    orc2.value_cache[0, :pos] = orc2.value_cache[0, perm]
    out2, _ = orc2.step(0, pos, q, k, v)
    assert_close(out2, out1, rel=1e-6)


def test_gqa_heads_with_equal_q_agree():
    orc, pos, q, k, v = _tiny(6, nh=8, nkv=2, hd=8, T=20)
    qh = q.reshape(8, 8)
    qh[1:4] = qh[0]  # heads 0..3 share KV head 0
    out, _ = orc.step(0, pos, qh.reshape(-1), k, v)
    o = out.reshape(8, 8)
    for h in (1, 2, 3):
        assert np.array_equal(o[h], o[0])


def test_relative_position_property():
    # score(q at m, k at n) depends on m - n only (rotation group), up to table rounding
    hd = 16
    orc = O.Oracle(1, 1, 1, hd, 64, theta=10000.0)
    rng = rng_for(7)
    q, k = normal(rng, hd, hd), normal(rng, hd, hd)

    def score(m, n):
        return float(np.dot(rope_f32(q, orc.cos[m], orc.sin[m]).astype(np.float64),
                            rope_f32(k, orc.cos[n], orc.sin[n]).astype(np.float64)))
    for d in (0, 3, 11):
        ref = score(d, 0)
        for m in (d + 5, d + 20, 60):
            assert abs(score(m, m - d) - ref) < 1e-5


# ---- rmsnorm, matmul and the attention sub-block ---------------------------------

def _block_fixture(path):
    fx = _load(path)
    dim, nh, nkv, L, sl, layer, pos = (int(v) for v in fx["dims"])
    hd = dim // nh
    x, rms, wq, wk, wv, wo = block_inputs(rng_for(*(int(k) for k in fx["key"])), dim, nkv * hd)
    return fx, (dim, nh, nkv, L, sl, layer, pos), (x, rms, wq, wk, wv, wo)


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "block_*.npz"))))
def test_block_reference_golden(path):
    fx, (dim, nh, nkv, L, sl, layer, pos), (x, rms, wq, wk, wv, wo) = _block_fixture(path)
    xb = O.rmsnorm(x, rms)
    assert np.array_equal(xb, fx["xb"]), "rmsnorm differs from the reference"
    for w, key in ((wq, "q_pre"), (wk, "k_pre"), (wv, "v_pre")):
        assert np.array_equal(O.matmul(w, xb), fx[key]), f"matmul ({key}) differs from the reference"
    orc = O.Oracle(L, nh, nkv, dim // nh, sl)
    orc.key_cache[layer, :pos] = fx["k_rows"]
    orc.value_cache[layer, :pos] = fx["v_rows"]
    got = orc.block(layer, pos, x, rms, wq, wk, wv, wo)
    if (dim // nh) % 8 == 0:
        assert np.array_equal(got, fx["x_out"]), f"block output differs: {rel_err(got, fx['x_out']):.2e}"
        assert np.array_equal(orc.key_cache[layer, pos], fx["k_slot"])
    else:
        # head sizes off the 8-wide vectors leave scalar tails in the score,
        # RoPE and weighted-V loops, whose -ffast-math vectorisation differs
        # between the two builds in the last bit
        assert_close(got, fx["x_out"], rel=1e-6)
        assert_close(orc.key_cache[layer, pos], fx["k_slot"], rel=1e-6)
    assert np.array_equal(orc.value_cache[layer, pos], fx["v_slot"])


@pytest.mark.parametrize("n,d", [(8, 3), (7, 9), (100, 20), (2048, 64), (4096, 48)])
def test_rmsnorm_matmul_live_reference(n, d):
    if not O.ref_available():
        pytest.skip("reference driver not built (reference sources absent)")
    rng = rng_for(n, d, 5)
    x = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    assert np.array_equal(O.rmsnorm(x, w), O.ref_rmsnorm(x, w))
    W = normal(rng, (d, n), n)
    assert np.array_equal(O.matmul(W, x), O.ref_matmul(W, x))


@pytest.mark.parametrize("dim,nh,nkv,L,sl,layer,pos", [(512, 4, 2, 2, 50, 1, 49), (256, 8, 8, 1, 9, 0, 5)])
def test_block_live_reference(dim, nh, nkv, L, sl, layer, pos):
    if not O.ref_available():
        pytest.skip("reference driver not built (reference sources absent)")
    hd = dim // nh
    x, rms, wq, wk, wv, wo = block_inputs(rng_for(dim, pos, 3), dim, nkv * hd)
    rng = rng_for(dim, pos, 4)
    kc = normal(rng, (L, sl, nkv * hd), hd)
    vc = normal(rng, (L, sl, nkv * hd), hd)
    xr, kr, vr = O.ref_block(dim, nh, nkv, L, sl, layer, pos, x, rms, wq, wk, wv, wo, kc, vc)
    orc = O.Oracle(L, nh, nkv, hd, sl)
    orc.key_cache[:] = kc
    orc.value_cache[:] = vc
    assert np.array_equal(orc.block(layer, pos, x, rms, wq, wk, wv, wo), xr)
    assert np.array_equal(orc.key_cache, kr) and np.array_equal(orc.value_cache, vr)


def test_rmsnorm_closed_forms():
    n = 64
    for c in (1e-3, 0.5, 3.0, -7.0):
        x = np.full(n, c, np.float32)
        w = np.linspace(0.5, 2.0, n).astype(np.float32)
        want = w.astype(np.float64) * c / np.sqrt(c * c + 1e-5)
        assert rel_err(O.rmsnorm(x, w), want) < 1e-6
    rng = rng_for(64, 1)
    x = rng.standard_normal(n).astype(np.float32)
    w = np.ones(n, np.float32)
    # the float64 formula at two scales (the epsilon matters at the smaller
    # one only), and mean(o^2) = m / (m + 1e-5) for unit weights
    for a in (1.0, 1000.0):
        xa = (a * x).astype(np.float32)
        m = float(np.mean(xa.astype(np.float64) ** 2))
        assert rel_err(O.rmsnorm(xa, w), xa.astype(np.float64) / np.sqrt(m + 1e-5)) < 1e-6
        assert abs(float(np.mean(O.rmsnorm(xa, w).astype(np.float64) ** 2)) - m / (m + 1e-5)) < 1e-6


def test_matmul_closed_forms():
    rng = rng_for(77)
    for n, d in ((16, 16), (100, 100), (37, 19)):
        W = normal(rng, (d, n), n)
        x = rng.standard_normal(n).astype(np.float32)
        if n == d:
            assert np.array_equal(O.matmul(np.eye(n, dtype=np.float32), x), x)
        for j in (0, n // 2, n - 1):
            e = np.zeros(n, np.float32)
            e[j] = 1.0
            assert np.array_equal(O.matmul(W, e), W[:, j])
        assert rel_err(O.matmul(W, x), W.astype(np.float64) @ x) < 1e-6
        y = rng.standard_normal(n).astype(np.float32)
        assert rel_err(O.matmul(W, x + y), O.matmul(W, x).astype(np.float64) + O.matmul(W, y)) < 1e-5


def test_projection_pins_catch_mistakes():
    # a transposed weight, a dropped epsilon, a sum in place of the mean, a
    # dropped residual: each fails at least one of the pins above
    rng = rng_for(78)
    n = 37
    W = normal(rng, (n, n), n)
    e = np.zeros(n, np.float32)
    e[5] = 1.0
    assert not np.array_equal(W.T @ e, O.matmul(W, e))
    x = np.full(64, 1e-3, np.float32)
    w = np.ones(64, np.float32)
    good = O.rmsnorm(x, w)
    assert rel_err(x / np.sqrt(np.mean(x ** 2)), good) > 1e-3          # no epsilon
    assert rel_err(x / np.sqrt(np.sum(x ** 2) + 1e-5), good) > 1e-3    # sum, not mean
    path = sorted(glob.glob(os.path.join(GOLDEN, "block_*.npz")))[0]
    fx, (dim, nh, nkv, L, sl, layer, pos), (x, rms, wq, wk, wv, wo) = _block_fixture(path)
    orc = O.Oracle(L, nh, nkv, dim // nh, sl)
    orc.key_cache[layer, :pos] = fx["k_rows"]
    orc.value_cache[layer, :pos] = fx["v_rows"]
    no_residual = orc.block(layer, pos, x, rms, wq, wk, wv, wo) - x
    assert rel_err(no_residual, fx["x_out"]) > 1e-2


# ---- the quantized engine: quantize, W8A8 matmul, its sub-block ------------------

def _q8_fixture(path):
    fx = _load(path)
    dim, nh, nkv, L, sl, layer, pos, gs = (int(v) for v in fx["dims"])
    hd = dim // nh
    x, rms, *wf = block_inputs(rng_for(*(int(k) for k in fx["key"])), dim, nkv * hd)
    return fx, (dim, nh, nkv, L, sl, layer, pos, gs), x, rms, wf


def test_q8_quantize_golden():
    fx = _load(os.path.join(GOLDEN, "q8_quantize.npz"))
    q, sc = O.quantize(fx["x"], int(fx["gs"]))
    assert np.array_equal(q, fx["q"]) and np.array_equal(sc, fx["s"])
    # exact halves at scale 1 round away from zero; the zero group has scale 0
    assert list(q[:8]) == [127, 3, -3, 1, -1, 2, 127, -127] and sc[0] == 1.0 and sc[2] == 0.0


@pytest.mark.parametrize("path", sorted(glob.glob(os.path.join(GOLDEN, "q8block_*.npz"))))
def test_q8_block_reference_golden(path):
    fx, (dim, nh, nkv, L, sl, layer, pos, gs), x, rms, wf = _q8_fixture(path)
    w8 = [O.quantize_weight(w, gs) for w in wf]
    assert np.array_equal(np.concatenate([w[1] for w in w8]), fx["w_scales"]), "weight quantization differs"
    xq, xs = O.quantize(O.rmsnorm(x, rms), gs)
    assert np.array_equal(xq, fx["xq"]) and np.array_equal(xs, fx["xs"])
    for w, key in zip(w8[:3], ("q_pre", "k_pre", "v_pre")):
        assert np.array_equal(O.matmul_q8(*w, xq, xs, gs), fx[key]), f"W8A8 matmul ({key}) differs"
    orc = O.Oracle(L, nh, nkv, dim // nh, sl)
    orc.key_cache[layer, :pos] = fx["k_rows"]
    orc.value_cache[layer, :pos] = fx["v_rows"]
    got = orc.block_q8(layer, pos, x, rms, *w8, gs)
    assert np.array_equal(got, fx["x_out"]), f"q8 block output differs: {rel_err(got, fx['x_out']):.2e}"
    assert np.array_equal(orc.key_cache[layer, pos], fx["k_slot"])
    assert np.array_equal(orc.value_cache[layer, pos], fx["v_slot"])


@pytest.mark.parametrize("n,d,gs", [(64, 4, 64), (256, 7, 32), (200, 9, 64), (4096, 40, 64), (1024, 13, 128),
                                   (3072, 11, 64), (5120, 5, 128)])
def test_q8_quantize_matmul_live_reference(n, d, gs):
    if not O.ref_q8_available():
        pytest.skip("quantized reference driver not built (reference sources absent)")
    rng = rng_for(n, d, gs, 6)
    for scale in (1e-3, 1.0, 50.0):
        x = (scale * rng.standard_normal(n)).astype(np.float32)
        a, b = O.quantize(x, gs), O.ref_q8_quantize(x, gs)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # n = 200 leaves a partial group that the matmul's loop bound skips; d = 7,
    # 9, 13 exercise the reference's row tail after its blocks of 4 rows
    wq = rng.integers(-127, 128, (d, n), dtype=np.int8)
    ws = (rng.random(d * n // gs) * 0.02).astype(np.float32)
    xq, xs = O.quantize(rng.standard_normal(n), gs)
    assert np.array_equal(O.matmul_q8(wq, ws, xq, xs, gs), O.ref_q8_matmul(wq, ws, xq, xs, gs))


@pytest.mark.parametrize("dim,nh,nkv,L,sl,layer,pos,gs",
                         [(512, 4, 2, 2, 50, 1, 49, 64), (256, 8, 8, 1, 9, 0, 5, 32), (1024, 8, 2, 1, 30, 0, 29, 128)])
def test_q8_block_live_reference(dim, nh, nkv, L, sl, layer, pos, gs):
    if not O.ref_q8_available():
        pytest.skip("quantized reference driver not built (reference sources absent)")
    hd = dim // nh
    x, rms, *wf = block_inputs(rng_for(dim, pos, gs, 3), dim, nkv * hd)
    w8 = [O.quantize_weight(w, gs) for w in wf]
    rng = rng_for(dim, pos, gs, 4)
    kc = normal(rng, (L, sl, nkv * hd), hd)
    vc = normal(rng, (L, sl, nkv * hd), hd)
    xr, kr, vr = O.ref_q8_block(dim, nh, nkv, L, sl, gs, layer, pos, x, rms, *w8, kc, vc)
    orc = O.Oracle(L, nh, nkv, hd, sl)
    orc.key_cache[:] = kc
    orc.value_cache[:] = vc
    assert np.array_equal(orc.block_q8(layer, pos, x, rms, *w8, gs), xr)
    assert np.array_equal(orc.key_cache, kr) and np.array_equal(orc.value_cache, vr)


def test_q8_closed_forms():
    rng = rng_for(79)
    gs = 64
    x = (rng.standard_normal(gs * 8) * rng.uniform(0.01, 100, gs * 8)).astype(np.float32)
    q, sc = O.quantize(x, gs)
    g = x.reshape(-1, gs)
    # the group's largest |x| maps to +-127 and sets the scale
    assert np.all(np.abs(q.reshape(-1, gs)).max(axis=1) == 127)
    assert np.all(np.abs(sc - np.abs(g).max(axis=1) / 127.0) <= 1e-7 * np.abs(g).max(axis=1))
    # dequantised values lie within half a step of x
    deq = q.reshape(-1, gs).astype(np.float64) * sc[:, None]
    assert np.all(np.abs(deq - g) <= sc[:, None] * (0.5 + 1e-5))
    # the matmul is the exact integer group dot products times both scales
    d, n = 11, gs * 8
    wq = rng.integers(-127, 128, (d, n), dtype=np.int8)
    ws = (rng.random(d * n // gs) * 0.01).astype(np.float32)
    idot = (wq.reshape(d, -1, gs).astype(np.int64) * q.reshape(1, -1, gs)).sum(axis=2)
    want = (idot * ws.reshape(d, -1).astype(np.float64) * sc[None, :].astype(np.float64)).sum(axis=1)
    assert rel_err(O.matmul_q8(wq, ws, q, sc, gs), want) < 1e-6
    # a one-hot x quantizes to 127 at its index with scale 1/127: the
    # product returns that column of W dequantised
    j = 77
    e = np.zeros(n, np.float32)
    e[j] = 1.0
    eq, es = O.quantize(e, gs)
    col = wq[:, j].astype(np.float64) * ws.reshape(d, -1)[:, j // gs]
    assert rel_err(O.matmul_q8(wq, ws, eq, es, gs), col) < 1e-6


def test_q8_pins_catch_mistakes():
    # ties to even in place of half away from zero, a transposed scale index
    # and a dropped activation scale each fail a pin above
    fx = _load(os.path.join(GOLDEN, "q8_quantize.npz"))
    assert not np.array_equal(np.rint(fx["x"][:8] * 1.0).astype(np.int8), fx["q"][:8])
    rng = rng_for(80)
    gs, d, n = 64, 8, 256
    wq = rng.integers(-127, 128, (d, n), dtype=np.int8)
    ws = (rng.random(d * n // gs) * 0.01).astype(np.float32)
    xq, xs = O.quantize(rng.standard_normal(n) * 5, gs)
    good = O.matmul_q8(wq, ws, xq, xs, gs)
    ws_t = np.ascontiguousarray(ws.reshape(d, -1).T).reshape(-1)
    assert rel_err(O.matmul_q8(wq, ws_t, xq, xs, gs), good) > 1e-3
    assert rel_err(O.matmul_q8(wq, ws, xq, np.ones_like(xs), gs), good) > 1e-3


# ---- the pins catch plausible mistakes -------------------------------------------

@pytest.mark.parametrize("mutant", [1, 2, 3])
def test_mutants_fail_the_pins(mutant):
    failed = []
    for path in sorted(glob.glob(os.path.join(GOLDEN, "run_layer_*.npz"))):
        fx = _load(path)
        out, q_rot, k_slot, _ = _run_fixture(fx, mutant=mutant)
        failed.append(rel_err(out, fx["out"]) > 1e-4 or not np.array_equal(k_slot, fx["k_slot"]))
    orc, pos, q, k, v = _tiny(8, nh=8, nkv=2, hd=8, T=40)
    want = _bruteforce(orc, pos, q, k, v)
    out, _ = orc.step(0, pos, q, k, v, mutant=mutant)
    failed.append(rel_err(out, want) > 1e-5)
    assert any(failed), f"mutant {mutant} passed every pin"


def test_rejects_bad_arguments():
    orc = O.Oracle(1, 4, 3, 8, 16)  # 4 % 3 != 0
    with pytest.raises(ValueError):
        orc.step(0, 0, np.zeros(32, np.float32), np.zeros(24, np.float32), np.zeros(24, np.float32))
    orc = O.Oracle(1, 4, 2, 8, 16)
    with pytest.raises(ValueError):
        orc.step(0, 16, np.zeros(32, np.float32), np.zeros(16, np.float32), np.zeros(16, np.float32))


@pytest.mark.parametrize("gs", [None, 64])
def test_reference_block_timer_runs_the_reference(gs):
    """The CPU-baseline timer (the reference's run_layer on a one-layer
    engine) computes what the oracle's chain computes, bit for bit."""
    if not (O.ref_q8_available() if gs else O.ref_available()):
        pytest.skip("reference driver not built (reference sources absent)")
    dim, nh, nkv, T = 512, 8, 2, 70
    hd, kv = dim // nh, nkv * (dim // nh)
    x0, rms, *wf = block_inputs(rng_for(dim, T, 81), dim, kv)
    w = [O.quantize_weight(m, gs) for m in wf] if gs else wf
    rng = rng_for(dim, T, 82)
    k, v = normal(rng, (T, kv), hd), normal(rng, (T, kv), hd)
    orc = O.Oracle(1, nh, nkv, hd, T + 1)
    orc.key_cache[0, :T] = k
    orc.value_cache[0, :T] = v
    want = orc.block_q8(0, T, x0, rms, *w, gs) if gs else orc.block(0, T, x0, rms, *w)
    timer = O.RefBlockTimer(dim, nh, nkv, T + 1, rms, *w, k, v, gs=gs, n_layers=3)
    try:
        for layer in range(3):  # each call runs the next layer, all holding the same weights and rows
            x = x0.copy()
            assert timer.run(T, x, 1) > 0
            assert np.array_equal(x, want), f"layer {layer}"
    finally:
        timer.close()
