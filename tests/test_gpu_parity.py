"""HIP path vs the oracle, through the C-ABI, on seeded inputs.

Bar: max |delta| <= 1e-4 * max |oracle output| for the attention output
(fp32 reductions reordered); bit-exact for the RoPE table, the rotated k and
the v written into cache[layer][pos], and every other cache row.
"""
import numpy as np
import pytest

from oracle import oracle as O
from leap_amd.attention import HipAttention, LeapError
from tests.helpers import REL_TOL, assert_close, normal, rng_for, rope_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _needs_gpu(hip_device):
    return hip_device


def _oracle_for(att: HipAttention, layer_rows_k, layer_rows_v, theta):
    orc = O.Oracle(1, att.n_heads, att.n_kv_heads, att.head_dim, att.seq_len, theta=theta)
    n = layer_rows_k.shape[0]
    orc.key_cache[0, :n] = layer_rows_k
    orc.value_cache[0, :n] = layer_rows_v
    return orc


def _step_and_check(att, seq_layer, pos, q, k, v, theta, layer_index=0, seq=0, out=None,
                    rel=REL_TOL):
    """Run the oracle on the device cache rows [0, pos) of (seq, layer) and
    compare with `out` (the HIP result) and with the cache row at pos."""
    kr, vr = att.kv_download(seq, seq_layer, 0, pos + 1)
    orc = _oracle_for(att, kr[:pos], vr[:pos], theta)
    want, _ = orc.step(0, pos, q, k, v)
    err = assert_close(out, want, rel=rel)
    assert np.array_equal(kr[pos], orc.key_cache[0, pos]), "rotated k row differs"
    assert np.array_equal(vr[pos], orc.value_cache[0, pos]), "v row differs"
    return err


# ---- RoPE table --------------------------------------------------------------------

@pytest.mark.parametrize("theta,hd,seq_len", [(500000.0, 128, 131072), (10000.0, 64, 256),
                                              (500000.0, 64, 4096)])
def test_rope_table_bitwise(theta, hd, seq_len):
    with HipAttention(4, 4, hd, seq_len, rope_theta=theta) as att:
        c, s = att.rope_download()
    oc, os_ = O.rope_table(seq_len, hd, theta)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)


# ---- golden fixtures from the reference ------------------------------------------

def test_reference_golden_fixtures():
    import glob
    import os
    gold = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    for path in sorted(glob.glob(os.path.join(gold, "run_layer_*.npz"))):
        with np.load(path, allow_pickle=False) as z:
            fx = {k: z[k] for k in z.files}
        dim, nh, nkv, L, sl, layer, pos = (int(v) for v in fx["dims"])
        hd = dim // nh
        with HipAttention(nh, nkv, hd, sl, n_layers=L) as att:
            if pos:
                att.kv_upload(0, layer, 0, fx["k_rows"], fx["v_rows"])
            out = att.step(layer, pos, fx["q_pre"], fx["k_pre"], fx["v_pre"])
            kr, vr = att.kv_download(0, layer, pos, pos + 1)
        assert_close(out, fx["out"], what=os.path.basename(path))
        assert np.array_equal(kr[0], fx["k_slot"]) and np.array_equal(vr[0], fx["v_slot"])


# ---- single sequence, many shapes, forced split-K chunkings -----------------------

SHAPES = [  # n_heads, n_kv_heads, head_dim
    (32, 4, 64), (32, 8, 128), (64, 8, 128), (8, 8, 128), (16, 2, 128), (8, 4, 64), (4, 4, 64),
    (16, 16, 64), (8, 2, 64), (24, 8, 128), (12, 4, 64),  # kv_mul 3: Llama-3.2-3B's 24/8 at head_dim 128
    (128, 8, 128), (32, 2, 64),  # kv_mul 16 (Llama-3.1-405B's 128/8 at head_dim 128): two groups of 8 per KV head
]


@pytest.mark.parametrize("nh,nkv,hd", SHAPES)
@pytest.mark.parametrize("T,split", [(1, 0), (2, 0), (64, 0), (65, 64), (300, 128), (1000, 64),
                                     (2049, 0), (777, 256),
                                     # 32, 48 and 64 one-pass chunks: the asymmetric merge when the
                                     # launch puts two workgroups on every CU
                                     (2048, 64), (3072, 64), (4096, 64),
                                     # chunks that are not whole 64-row passes (rows past a chunk's
                                     # end masked), with the asymmetric merge at 64 chunks
                                     (3072, 48), (2048, 32), (1000, 40), (130, 8), (4000, 200),
                                     # 10 and 38 chunks without the asymmetric shape: one-level
                                     # folds compiled for 16 and 40 records, the rest empty
                                     (600, 64), (2400, 64),
                                     # automatic: 64 near-equal chunks of 33-64 rows for 8 KV heads,
                                     # then of two passes
                                     (2500, 0), (3001, 0), (5000, 0),
                                     # automatic short contexts: half-pass chunks where a group has
                                     # 2-8 one-pass chunks and the launch leaves CUs idle (2-wave
                                     # workgroups where the shape has them)
                                     (100, 0), (256, 0), (500, 0),
                                     # up to 32 positions: one 2-wave workgroup per group where the
                                     # shape has them; 33 takes a 4-wave one again; a forced 32-row
                                     # split keeps 4 waves
                                     (17, 0), (32, 0), (33, 0), (32, 32)])
def test_step_shapes_and_splits(nh, nkv, hd, T, split):
    theta = 10000.0 if hd == 64 else 500000.0
    rng = rng_for(nh, nkv, hd, T, split)
    seq_len = T + 5
    with HipAttention(nh, nkv, hd, seq_len, n_layers=2, rope_theta=theta) as att:
        if split:
            att.set_split(split)
        pos = T - 1
        att.kv_upload(0, 1, 0, normal(rng, (pos, nkv * hd), hd), normal(rng, (pos, nkv * hd), hd))
        q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
        out = att.step(1, pos, q, k, v)
        _step_and_check(att, 1, pos, q, k, v, theta, out=out)
        # the other layer is untouched
        k0, v0 = att.kv_download(0, 0, 0, seq_len)
        assert not k0.any() and not v0.any()


@pytest.mark.parametrize("nh,nkv,hd", SHAPES)
@pytest.mark.parametrize("T,split", [(1, 0), (65, 64), (1000, 64), (4096, 64), (2049, 0)])
def test_valu_products_shapes_and_splits(nh, nkv, hd, T, split):
    """The score and weighted-V products as VALU FMAs (the measurement knob
    set_products) meet the same bar, and write the same cache rows."""
    theta = 10000.0 if hd == 64 else 500000.0
    rng = rng_for(nh, nkv, hd, T, split, 1)
    with HipAttention(nh, nkv, hd, T + 5, rope_theta=theta) as att:
        att.set_products(True)
        if split:
            att.set_split(split)
        pos = T - 1
        att.kv_upload(0, 0, 0, normal(rng, (pos, nkv * hd), hd), normal(rng, (pos, nkv * hd), hd))
        q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
        out = att.step(0, pos, q, k, v)
        _step_and_check(att, 0, pos, q, k, v, theta, out=out)


@pytest.mark.parametrize("nh,nkv,hd", [(32, 8, 128), (32, 4, 64), (24, 8, 128), (8, 8, 128), (16, 8, 64),
                                       (64, 8, 128)])
@pytest.mark.parametrize("T", [1, 2, 33, 65, 257, 2080, 4096])
@pytest.mark.parametrize("sign", [1.0, -1.0])
def test_new_token_score_dominates_or_vanishes(nh, nkv, hd, T, sign):
    """The q heads of a group close to one direction u (u + 0.05 noise) and
    k_new = +-2000 u: the new token's score exceeds every cached score by far
    more than the lazy max's margin (the running max is raised for it, and
    the output is about v_new), or its weight underflows to zero.  RoPE
    rotates q and k by the same angles, so the score keeps its size."""
    theta = 10000.0 if hd == 64 else 500000.0
    rng = rng_for(nh, nkv, hd, T, int(sign > 0))
    g = nh // nkv
    with HipAttention(nh, nkv, hd, T + 3, rope_theta=theta) as att:
        pos = T - 1
        if pos:
            att.kv_upload(0, 0, 0, normal(rng, (pos, nkv * hd), hd), normal(rng, (pos, nkv * hd), hd))
        u = normal(rng, (nkv, 1, hd), hd)
        q = (u + 0.05 * normal(rng, (nkv, g, hd), hd)).astype(np.float32).reshape(-1)
        k = (sign * 2000.0 * u).astype(np.float32).reshape(-1)
        v = normal(rng, nkv * hd, hd)
        out = att.step(0, pos, q, k, v)
        _step_and_check(att, 0, pos, q, k, v, theta, out=out)
        if sign > 0:  # every head of a group takes (nearly) its group's v_new
            want = np.repeat(v.reshape(nkv, 1, hd), g, axis=1).reshape(-1)
            assert_close(out, want, rel=1e-3, what="dominant new token")


def test_first_position_returns_v_exactly():
    with HipAttention(32, 8, 128, 16) as att:
        rng = rng_for(5)
        q, k, v = normal(rng, 4096, 128), normal(rng, 1024, 128), normal(rng, 1024, 128)
        out = att.step(0, 0, q, k, v)
    want = np.concatenate([v.reshape(8, 128)[h // 4] for h in range(32)])
    assert np.array_equal(out, want)


def test_sequential_decode_matches_oracle_and_cache_bitwise():
    nh, nkv, hd, n = 16, 4, 128, 150
    rng = rng_for(77)
    orc = O.Oracle(2, nh, nkv, hd, 160)
    with HipAttention(nh, nkv, hd, 160, n_layers=2) as att:
        att.set_split(64)
        for pos in range(n):
            for layer in (0, 1):
                q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
                out = att.step(layer, pos, q, k, v)
                want, _ = orc.step(layer, pos, q, k, v)
                assert_close(out, want, what=f"pos {pos} layer {layer}")
        for layer in (0, 1):
            kr, vr = att.kv_download(0, layer, 0, 160)
            assert np.array_equal(kr, orc.key_cache[layer]) and np.array_equal(vr, orc.value_cache[layer])


# ---- full-size configurations -------------------------------------------------------

def test_llama3_8b_ctx4096_all_layers_all_heads():
    """32 layers, 32/8/128, T = 4096, theta 500000, seeded N(0,1)/sqrt(128)."""
    L, nh, nkv, hd, T = 32, 32, 8, 128, 4096
    with HipAttention(nh, nkv, hd, T, n_layers=L) as att:
        att.kv_fill_normal(0x4C454150 + 1, 1.0 / np.sqrt(hd))
        rng = rng_for(2, 4096)
        worst = 0.0
        for layer in range(L):
            q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
            out = att.step(layer, T - 1, q, k, v)
            worst = max(worst, _step_and_check(att, layer, T - 1, q, k, v, 500000.0, out=out))
    print(f"llama3-8b ctx4096: worst max|delta|/Linf over 32 layers = {worst:.2e}")


def test_tinyllama_ctx256_both_thetas():
    nh, nkv, hd, T = 32, 4, 64, 256
    for theta in (10000.0, 500000.0):
        with HipAttention(nh, nkv, hd, T, rope_theta=theta) as att:
            att.kv_fill_normal(0x4C454150 + 0, 1.0 / np.sqrt(hd))
            rng = rng_for(1, int(theta))
            q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
            out = att.step(0, T - 1, q, k, v)
            _step_and_check(att, 0, T - 1, q, k, v, theta, out=out)


def test_long_context_planted_keys():
    """Llama-3.1-8B head config at T = 131072 with planted high-score keys in
    the first chunk, a middle chunk, across a chunk boundary and the last
    chunk; one held layer."""
    nh, nkv, hd, T = 32, 8, 128, 131072
    with HipAttention(nh, nkv, hd, T, n_layers=32, layer_begin=17, layer_end=18) as att:
        att.kv_fill_normal(0x4C454150 + 4, 1.0 / np.sqrt(hd))
        rng = rng_for(4, T)
        q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
        c, s = O.rope_table(T, hd, 500000.0)
        qr = rope_f32(q, c[T - 1], s[T - 1]).reshape(nh, hd).astype(np.float64)
        plants = {0: (3, 300.0), 1: (65000, 420.0), 2: (98303, 520.0), 3: (98304, 500.0),
                  5: (T - 2, 460.0), 7: (1, 350.0)}
        for kvh, (p_pos, alpha) in plants.items():
            h = kvh * (nh // nkv)  # first q head of the group
            kr, _ = att.kv_download(0, 17, p_pos, p_pos + 1)
            kr = kr.reshape(nkv, hd)
            kr[kvh] = (qr[h] * alpha / np.dot(qr[h], qr[h])).astype(np.float32)
            att.kv_upload(0, 17, p_pos, kr.reshape(1, -1), None)
        out = att.step(17, T - 1, q, k, v)
        _step_and_check(att, 17, T - 1, q, k, v, 500000.0, out=out)


def test_batched_ragged_llama3_8b():
    """64 sequences, one layer, T_i ~ U[512, 8192] (the batched config's shape)."""
    nh, nkv, hd, S, T_max = 32, 8, 128, 64, 8192
    rng = rng_for(3, S)
    Ts = rng.integers(512, T_max + 1, size=S)
    with HipAttention(nh, nkv, hd, T_max, n_layers=32, layer_begin=5, layer_end=6,
                      max_batch=S) as att:
        att.kv_fill_normal(0x4C454150 + 2, 1.0 / np.sqrt(hd))
        q = normal(rng, (S, nh * hd), hd)
        k = normal(rng, (S, nkv * hd), hd)
        v = normal(rng, (S, nkv * hd), hd)
        out = att.step_batched(5, Ts - 1, q, k, v)
        for i in range(S):
            _step_and_check(att, 5, int(Ts[i]) - 1, q[i], k[i], v[i], 500000.0, seq=i, out=out[i])


def test_llama31_405b_heads_ragged_batch():
    """16 q heads per KV head (Llama-3.1-405B's 128/8/128), run as two groups
    of 8 per KV head: a ragged batch of 6 sequences over every launch regime,
    each sequence's output and appended cache row against the oracle."""
    nh, nkv, hd, S = 128, 8, 128, 6
    Ts = np.array([1, 65, 700, 3000, 4096, 9000])
    rng = rng_for(405, S)
    with HipAttention(nh, nkv, hd, 9000, n_layers=2, max_batch=S) as att:
        att.kv_fill_normal(0x4C454150 + 405, 1.0 / np.sqrt(hd))
        q = normal(rng, (S, nh * hd), hd)
        k = normal(rng, (S, nkv * hd), hd)
        v = normal(rng, (S, nkv * hd), hd)
        out = att.step_batched(1, Ts - 1, q, k, v)
        for i in range(S):
            _step_and_check(att, 1, int(Ts[i]) - 1, q[i], k[i], v[i], 500000.0, seq=i, out=out[i])
        # one sequence at a time: the launch shapes of batch 1 (two workgroups
        # per CU, near-equal chunks, the asymmetric merge at 4096)
        for i in (3, 4, 5):
            o1 = att.step(1, int(Ts[i]) - 1, q[i], k[i], v[i])
            _step_and_check(att, 1, int(Ts[i]) - 1, q[i], k[i], v[i], 500000.0, seq=0, out=o1)


@pytest.mark.parametrize("split", [64, 24])
def test_batched_small_ragged_with_tiny_contexts(split):
    nh, nkv, hd, S = 16, 2, 128, 9
    Ts = np.array([1, 2, 63, 64, 65, 128, 129, 700, 1500])
    rng = rng_for(33)
    with HipAttention(nh, nkv, hd, 1600, max_batch=12) as att:
        att.kv_fill_normal(99, 0.1)
        att.set_split(split)
        q = normal(rng, (S, nh * hd), hd)
        k = normal(rng, (S, nkv * hd), hd)
        v = normal(rng, (S, nkv * hd), hd)
        out = att.step_batched(0, Ts - 1, q, k, v)
        for i in range(S):
            _step_and_check(att, 0, int(Ts[i]) - 1, q[i], k[i], v[i], 500000.0, seq=i, out=out[i])


@pytest.mark.parametrize("nh,nkv,hd,Ts", [
    # 8 q heads per KV head: two launch groups of 4 per cache head up to 24 MiB
    # of K/V rows (TinyLlama: 12288 positions) over at most 8 groups
    (32, 4, 64, [12288]), (32, 4, 64, [12289]),
    (64, 8, 128, [3072]), (64, 8, 128, [3073]),
    (8, 1, 128, [24576]), (8, 1, 128, [24577]),        # one KV head: spread over the XCDs either way
    # 4 q heads per KV head: groups of 2 up to 8 MiB (Llama-3-8B heads: 1024)
    (32, 8, 128, [1024]), (32, 8, 128, [1025]), (16, 4, 64, [4096]), (16, 4, 64, [4097]),
    # batches: up to 8 (sequence, KV head) groups
    (32, 4, 64, [700, 33]), (32, 4, 64, [700, 33, 1]), (32, 8, 128, [40]), (32, 8, 128, [40, 40]),
    (16, 2, 128, [3000, 17, 2, 1]), (16, 2, 128, [3000, 17, 2, 1, 64]),
    # 8 q heads per KV head as four launch groups of 2: up to 2 MiB over four
    # groups (TinyLlama: 1024 positions; one KV head: 4 sequences)
    (32, 4, 64, [1024]), (32, 4, 64, [1025]), (32, 4, 64, [1]), (8, 1, 128, [2048]),
    (8, 1, 128, [500, 3, 1, 64]), (8, 1, 128, [500, 3, 1, 64, 2]), (16, 2, 64, [300, 9]), (16, 2, 64, [300]),
])
def test_twin_launch_group_limits(nh, nkv, hd, Ts):
    """Launches on either side of the twin and quarter launch groups' limits
    (K/V bytes, groups per launch), single and batched, against the oracle."""
    theta = 10000.0 if hd == 64 else 500000.0
    Ts = np.array(Ts)
    S = len(Ts)
    rng = rng_for(nh, nkv, hd, int(Ts.sum()), S)
    with HipAttention(nh, nkv, hd, int(Ts.max()) + 1, rope_theta=theta, max_batch=max(S, 1)) as att:
        att.kv_fill_normal(0x7417 + S, 1.0 / np.sqrt(hd))
        q = normal(rng, (S, nh * hd), hd)
        k = normal(rng, (S, nkv * hd), hd)
        v = normal(rng, (S, nkv * hd), hd)
        out = att.step_batched(0, Ts - 1, q, k, v)
        for i in range(S):
            _step_and_check(att, 0, int(Ts[i]) - 1, q[i], k[i], v[i], theta, seq=i, out=out[i])


@pytest.mark.parametrize("nh,nkv,hd,Ts,split", [
    # at least two groups per XCD take one workgroup per CU:
    (32, 8, 128, [1500, 1100], 0),       # 16 groups: 16 near-equal chunks each
    (32, 8, 128, [500] * 7 + [5], 0),    # 64 groups: 4 chunks each, the short sequence 4 of 1-2 rows
    (32, 8, 128, [6000, 5500], 0),       # 16 groups: 16 near-equal chunks of about six passes
    (32, 8, 128, [2048] * 4, 0),         # 32 groups: 8 whole chunks of four passes each
    (32, 32, 128, [2048], 0),            # 32 KV heads of one q head: the same
    # fewer groups, two per CU:
    (32, 4, 64, [6000], 0),              # 4 groups: 128 near-equal chunks, two-level merge
    (8, 1, 128, [20000], 0),             # one group: 512 near-equal chunks spread over the XCDs
    # forced: 32 one-pass chunks per sequence, 512 workgroups, the asymmetric merge of 32
    (32, 8, 128, [4096, 4096], 128),
])
def test_even_split_chunks(nh, nkv, hd, Ts, split):
    """Equal-length batches in the latency regime: whole or near-equal
    chunks, one or two workgroups per CU (and a forced chunk length)."""
    Ts = np.array(Ts)
    S = len(Ts)
    rng = rng_for(41, nh, nkv, hd, S)
    with HipAttention(nh, nkv, hd, int(Ts.max()) + 3, max_batch=S) as att:
        att.kv_fill_normal(0x4C454150 + 41, 1.0 / np.sqrt(hd))
        if split:
            att.set_split(split)
        q = normal(rng, (S, nh * hd), hd)
        k = normal(rng, (S, nkv * hd), hd)
        v = normal(rng, (S, nkv * hd), hd)
        out = att.step_batched(0, Ts - 1, q, k, v)
        for i in range(S):
            _step_and_check(att, 0, int(Ts[i]) - 1, q[i], k[i], v[i], 500000.0, seq=i, out=out[i])


def test_llama3_70b_stage_batch16_ctx8192():
    """64/8/128, batch 16, T = 8192: a handle holding the whole 20-layer
    stage [20, 40) of the 80-layer model; the first and the last held layer
    are stepped and every sequence is checked on both."""
    nh, nkv, hd, S, T = 64, 8, 128, 16, 8192
    rng = rng_for(5, S)
    with HipAttention(nh, nkv, hd, T, n_layers=80, layer_begin=20, layer_end=40,
                      max_batch=S) as att:
        att.kv_fill_normal(0x4C454150 + 3, 1.0 / np.sqrt(hd))
        for layer in (20, 39):
            q = normal(rng, (S, nh * hd), hd)
            k = normal(rng, (S, nkv * hd), hd)
            v = normal(rng, (S, nkv * hd), hd)
            out = att.step_batched(layer, np.full(S, T - 1), q, k, v)
            for i in range(S):
                _step_and_check(att, layer, T - 1, q[i], k[i], v[i], 500000.0, seq=i, out=out[i])


# ---- cache management and errors ----------------------------------------------------

def test_clear_upload_download_roundtrip():
    with HipAttention(8, 2, 64, 100, n_layers=3, max_batch=2) as att:
        rng = rng_for(9)
        k, v = normal(rng, (100, 128), 64), normal(rng, (100, 128), 64)
        att.kv_upload(1, 2, 0, k, v)
        kr, vr = att.kv_download(1, 2, 0, 100)
        assert np.array_equal(kr, k) and np.array_equal(vr, v)
        kr, _ = att.kv_download(1, 2, 10, 20)
        assert np.array_equal(kr, k[10:20])
        att.clear()
        kr, vr = att.kv_download(1, 2, 0, 100)
        assert not kr.any() and not vr.any()


def test_step_argument_errors():
    with HipAttention(8, 2, 64, 100, n_layers=4, layer_begin=1, layer_end=3) as att:
        z = np.zeros(8 * 64, np.float32)
        zk = np.zeros(2 * 64, np.float32)
        for layer, pos in ((0, 0), (3, 0), (1, 100), (1, -1)):
            with pytest.raises(LeapError):
                att.step(layer, pos, z, zk, zk)
        with pytest.raises(LeapError):
            att.step_batched(1, [5, 200], np.zeros((2, 512), np.float32),
                             np.zeros((2, 128), np.float32), np.zeros((2, 128), np.float32))
        with pytest.raises(LeapError):
            att.set_split(100)


def test_async_entry_points_on_a_torch_stream():
    import torch
    nh, nkv, hd, T = 32, 8, 128, 3000
    rng = rng_for(12)
    q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
    with HipAttention(nh, nkv, hd, T, max_batch=2) as att:
        att.kv_fill_normal(5, 0.1)
        ref = att.step(0, T - 1, q, k, v)
        dq, dk, dv = (torch.from_numpy(a).cuda() for a in (q, k, v))
        dout = torch.empty(nh * hd, device="cuda")
        s = torch.cuda.Stream()
        att.step_async(0, T - 1, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dout.data_ptr(),
                       s.cuda_stream)
        s.synchronize()
        assert np.array_equal(dout.cpu().numpy(), ref)
        # device pointers that are not 16-byte aligned are refused before any launch
        for shift in ((4, 0, 0, 0), (0, 8, 0, 0), (0, 0, 4, 0), (0, 0, 0, 12)):
            with pytest.raises(LeapError):
                att.step_async(0, T - 1, dq.data_ptr() + shift[0], dk.data_ptr() + shift[1],
                               dv.data_ptr() + shift[2], dout.data_ptr() + shift[3], s.cuda_stream)
        # batched async with device positions
        pos = torch.tensor([T - 1, 17], dtype=torch.int32, device="cuda")
        bq, bk, bv = (torch.stack([t, t]) for t in (dq, dk, dv))
        bout = torch.empty(2, nh * hd, device="cuda")
        att.step_batched_async(0, 2, pos.data_ptr(), T - 1, bq.data_ptr(), bk.data_ptr(),
                               bv.data_ptr(), bout.data_ptr(), s.cuda_stream)
        s.synchronize()
        # sized without the host's row count, this launch splits the positions
        # differently from the single step (fixed 64-row chunks against 64
        # near-equal ones): the same result up to fp32 summation order
        assert_close(bout[0].cpu().numpy(), ref)
        _step_and_check(att, 0, T - 1, q, k, v, 500000.0, seq=0, out=bout[0].cpu().numpy())
        _step_and_check(att, 0, 17, q, k, v, 500000.0, seq=1, out=bout[1].cpu().numpy())
        # the host's row count only changes how the positions are split
        hint = torch.empty_like(bout)
        att.step_batched_async(0, 2, pos.data_ptr(), T - 1, bq.data_ptr(), bk.data_ptr(),
                               bv.data_ptr(), hint.data_ptr(), s.cuda_stream, total_rows=T + 18)
        s.synchronize()
        assert_close(hint[0].cpu().numpy(), ref)
        assert_close(hint[1].cpu().numpy(), bout[1].cpu().numpy())
        with pytest.raises(LeapError):
            att.step_batched_async(0, 2, pos.data_ptr(), T - 1, bq.data_ptr(), bk.data_ptr(),
                                   bv.data_ptr(), hint.data_ptr(), s.cuda_stream, total_rows=2 * T + 1)


def _random_cases(n, seed):
    """Seeded draws over the supported space: head shape, context, forced
    chunk size (0 = the automatic choice) and batch with ragged positions."""
    shapes = [(32, 8, 128), (24, 8, 128), (16, 16, 64), (32, 4, 64), (64, 8, 128), (8, 8, 128),
              (16, 2, 128), (12, 4, 64), (8, 1, 64), (4, 2, 64), (128, 8, 128), (16, 1, 64)]
    rng = np.random.default_rng(seed)
    for i in range(n):
        nh, nkv, hd = shapes[rng.integers(len(shapes))]
        T = int(rng.choice([rng.integers(1, 200), rng.integers(200, 5000)]))
        split = int(rng.choice([0, 0, 64, 128, 192, 256, 512]))
        batch = int(rng.choice([1, 1, 2, 5]))
        yield pytest.param(nh, nkv, hd, T, split, batch, id=f"{i}-{nh}x{nkv}x{hd}-T{T}-s{split}-b{batch}")


@pytest.mark.parametrize("nh,nkv,hd,T,split,batch", list(_random_cases(40, 0x51AB)))
def test_random_shapes_positions_and_batches(nh, nkv, hd, T, split, batch):
    """Seeded random cases beyond the fixed grid; a batch holds sequences at
    ragged positions up to T - 1, the first at T - 1."""
    rng = rng_for(nh, nkv, hd, T, split, batch, 77)
    with HipAttention(nh, nkv, hd, T, max_batch=batch) as att:
        att.kv_fill_normal(int(rng.integers(1 << 30)), 1.0 / np.sqrt(hd))
        if split:
            att.set_split(split)
        pos = np.concatenate([[T - 1], rng.integers(0, T, size=batch - 1)]).astype(np.int32)
        q = normal(rng, (batch, nh * hd), hd)
        k = normal(rng, (batch, nkv * hd), hd)
        v = normal(rng, (batch, nkv * hd), hd)
        out = att.step(0, int(pos[0]), q[0], k[0], v[0])[None] if batch == 1 else att.step_batched(0, pos, q, k, v)
        for i in range(batch):
            _step_and_check(att, 0, int(pos[i]), q[i], k[i], v[i], 500000.0, seq=i, out=out[i])


def _random_cases_long(n, seed):
    """Seeded draws reaching the launch shapes of longer contexts: near-equal
    chunks of one to several passes (their pass order rotated), spread
    launches of few KV heads, forced chunk sizes that are not whole passes,
    and batches of near-equal lengths (cut into near-equal chunks too)."""
    shapes = [(32, 8, 128), (24, 8, 128), (16, 16, 64), (32, 4, 64), (64, 8, 128), (8, 8, 128),
              (16, 2, 128), (12, 4, 64), (8, 1, 64), (8, 1, 128), (32, 4, 128), (128, 8, 128), (16, 1, 128)]
    rng = np.random.default_rng(seed)
    for i in range(n):
        nh, nkv, hd = shapes[rng.integers(len(shapes))]
        T = int(rng.choice([rng.integers(2000, 20000), rng.integers(1, 3000)]))
        split = int(rng.choice([0, 0, 0, 8, 24, 40, 72, 136, 200]))
        batch = int(rng.choice([1, 1, 2, 4]))
        even = bool(rng.integers(2))
        yield pytest.param(nh, nkv, hd, T, split, batch, even,
                           id=f"{i}-{nh}x{nkv}x{hd}-T{T}-s{split}-b{batch}-{'even' if even else 'ragged'}")


@pytest.mark.parametrize("nh,nkv,hd,T,split,batch,even", list(_random_cases_long(40, 0x10A6)))
def test_random_long_contexts_and_chunkings(nh, nkv, hd, T, split, batch, even):
    """As test_random_shapes_positions_and_batches over longer contexts and
    finer forced chunk sizes; a batch's other sequences sit within 1/8 of
    the longest (even) or anywhere below it."""
    rng = rng_for(nh, nkv, hd, T, split, batch, int(even), 78)
    with HipAttention(nh, nkv, hd, T, max_batch=batch) as att:
        att.kv_fill_normal(int(rng.integers(1 << 30)), 1.0 / np.sqrt(hd))
        if split:
            att.set_split(split)
        lo = T - 1 - T // 8 if even else 0
        pos = np.concatenate([[T - 1], rng.integers(lo, T, size=batch - 1)]).astype(np.int32)
        q = normal(rng, (batch, nh * hd), hd)
        k = normal(rng, (batch, nkv * hd), hd)
        v = normal(rng, (batch, nkv * hd), hd)
        out = att.step(0, int(pos[0]), q[0], k[0], v[0])[None] if batch == 1 else att.step_batched(0, pos, q, k, v)
        for i in range(batch):
            _step_and_check(att, 0, int(pos[i]), q[i], k[i], v[i], 500000.0, seq=i, out=out[i])


# ---- few KV heads: a group's chunks spread over several XCDs ------------------------

@pytest.mark.parametrize("nh,nkv,hd,T,split", [
    (8, 1, 128, 4096, 0),     # one group over eight XCDs (4 MiB of K/V rows)
    (16, 2, 128, 4096, 0),    # two groups, four parts each
    (32, 4, 64, 8192, 0),     # TinyLlama heads at a long context, two parts each
    (32, 4, 128, 8000, 0),
    (8, 1, 64, 20000, 0),
    (8, 1, 128, 4096, 256),   # forced chunking: 16 chunks, eight parts of two
    (24, 3, 128, 9000, 0),    # three groups, two parts each (six XCDs)
    (32, 4, 64, 2048, 0),     # 2 MiB per group: no spread (the faster launch there)
    (32, 8, 128, 4096, 0),    # eight groups: no spread
])
def test_spread_over_xcds_few_kv_heads(nh, nkv, hd, T, split):
    theta = 500000.0
    rng = rng_for(nh, nkv, hd, T, split, 7)
    with HipAttention(nh, nkv, hd, T + 3, rope_theta=theta) as att:
        if split:
            att.set_split(split)
        pos = T - 1
        att.kv_upload(0, 0, 0, normal(rng, (pos, nkv * hd), hd), normal(rng, (pos, nkv * hd), hd))
        for rep in range(2):  # twice: the second launch finds the workspace as the first left it
            q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
            out = att.step(0, pos, q, k, v)
            _step_and_check(att, 0, pos, q, k, v, theta, out=out)


def test_spread_ragged_batch_with_empty_parts():
    """Two sequences of two KV heads (four groups, two parts each) at very
    different positions: the short one's second part has no chunks."""
    nh, nkv, hd = 16, 2, 128
    Ts = [9000, 100]
    rng = rng_for(8, 8)
    with HipAttention(nh, nkv, hd, 9003, max_batch=2) as att:
        rows = []
        for s, T in enumerate(Ts):
            kr, vr = normal(rng, (T - 1, nkv * hd), hd), normal(rng, (T - 1, nkv * hd), hd)
            att.kv_upload(s, 0, 0, kr, vr)
            rows.append((kr, vr))
        q = normal(rng, (2, nh * hd), hd)
        k, v = normal(rng, (2, nkv * hd), hd), normal(rng, (2, nkv * hd), hd)
        out = att.step_batched(0, [T - 1 for T in Ts], q, k, v)
        for s, T in enumerate(Ts):
            orc = O.Oracle(1, nh, nkv, hd, 9003)
            orc.key_cache[0, :T - 1], orc.value_cache[0, :T - 1] = rows[s]
            want, _ = orc.step(0, T - 1, q[s], k[s], v[s])
            assert_close(out[s], want, what=f"sequence {s}")
            kr, vr = att.kv_download(s, 0, T - 1, T)
            assert np.array_equal(kr[0], orc.key_cache[0, T - 1]) and np.array_equal(vr[0], orc.value_cache[0, T - 1])


# ---- the final fold shared by two workgroups --------------------------------------

@pytest.mark.parametrize("nh,nkv,hd,T", [
    (32, 8, 128, 4096),   # the asymmetric merge, 36 records
    (32, 8, 128, 2048),   # one level, 32 records
    (32, 8, 128, 1984),   # one level, 31 of 32 compiled records
    (24, 8, 128, 3000),   # three q heads per KV head (a padding head in the second half)
    (32, 4, 64, 1500),    # head_dim 64, eight q heads per KV head
    (64, 8, 128, 2048),   # eight q heads at head_dim 128 (a two-level tree: no shared fold)
    (16, 2, 128, 2048),   # two q heads per KV head
])
def test_fold_helper_modes_agree(nh, nkv, hd, T):
    """The final fold shared by the last two arrivals (mode 1), done by the
    last alone (0), and the fallback where the waiting workgroup gives up at
    once (2) give bitwise equal outputs, step after step (every mode leaves
    the arrival counters at zero), and meet the oracle."""
    theta = 10000.0 if hd == 64 else 500000.0
    rng = rng_for(301, nh, nkv, hd, T)
    pos = T - 1
    q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
    outs = []
    with HipAttention(nh, nkv, hd, T, rope_theta=theta) as att:
        att.kv_fill_normal(0x4C454150 + 301, 1.0 / np.sqrt(hd))
        for mode in (1, 0, 2, 1, 2, 0, 1):
            att.set_fold_helper(mode)
            outs.append(att.step(0, pos, q, k, v))
        _step_and_check(att, 0, pos, q, k, v, theta, out=outs[0])
        with pytest.raises(LeapError):
            att.set_fold_helper(3)
    for i, o in enumerate(outs[1:], 1):
        assert np.array_equal(o, outs[0]), f"step {i} differs from the first"


# ---- device positions the launch cannot serve --------------------------------------

@pytest.mark.parametrize("nh,nkv,hd,sl,Ts,bad", [
    (32, 8, 128, 3000, (2500, 1200, 2900, 700), (1, -1)),     # a negative position
    (32, 8, 128, 3000, (2500, 1200, 2900, 700), (2, 3000)),   # at seq_len
    (32, 8, 128, 3000, (2500, 1200, 2900, 700), (0, 2950)),   # past the launch's max_pos
    (32, 4, 64, 600, (400, 599, 64, 200), (3, -7)),           # TinyLlama heads, one chunk for some
    (128, 8, 128, 1000, (999, 300, 512, 64), (2, 1000)),      # sixteen q heads per KV head (two groups each)
    (16, 2, 128, 9100, (9000, 8800), (1, 9100)),              # few KV heads: spread over the XCDs
])
def test_batched_async_bad_position_writes_nan_rows(nh, nkv, hd, sl, Ts, bad):
    """step_batched_async with one sequence at a position the launch cannot
    serve (negative, at seq_len, or past max_pos): that sequence's output
    row is all NaN and its cache untouched; every other sequence matches the
    oracle as usual."""
    import torch
    n = len(Ts)
    bad_seq, bad_pos = bad
    rng = rng_for(77, nh, nkv, n, bad_seq, abs(bad_pos))
    theta = 500000.0
    with HipAttention(nh, nkv, hd, sl, max_batch=n) as att:
        rows = []
        for s, T in enumerate(Ts):
            kr, vr = normal(rng, (T - 1, nkv * hd), hd), normal(rng, (T - 1, nkv * hd), hd)
            att.kv_upload(s, 0, 0, kr, vr)
            rows.append((kr, vr))
        before = att.kv_download(bad_seq, 0, 0, sl)
        pos = np.array([T - 1 for T in Ts], np.int32)
        max_pos = int(pos.max())
        pos[bad_seq] = bad_pos
        q, k, v = normal(rng, (n, nh * hd), hd), normal(rng, (n, nkv * hd), hd), normal(rng, (n, nkv * hd), hd)
        dq, dk, dv = (torch.from_numpy(x).cuda() for x in (q, k, v))
        out = torch.zeros(n, nh * hd, device="cuda:0")
        dpos = torch.from_numpy(pos).cuda()
        s = torch.cuda.Stream()
        att.step_batched_async(0, n, dpos.data_ptr(), max_pos, dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
                               out.data_ptr(), s.cuda_stream)
        s.synchronize()
        got = out.cpu().numpy()
        assert np.isnan(got[bad_seq]).all(), "the skipped sequence's row is not all NaN"
        after = att.kv_download(bad_seq, 0, 0, sl)
        assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])
        for i, T in enumerate(Ts):
            if i == bad_seq:
                continue
            assert np.isfinite(got[i]).all()
            _step_and_check(att, 0, T - 1, q[i], k[i], v[i], theta, seq=i, out=got[i])
