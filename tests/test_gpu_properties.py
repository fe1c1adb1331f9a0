"""Size-independent properties of the HIP attention step at full sizes,
through the C ABI, checked without the oracle:

- every cached key equal to the new token's rotated key: all scores of a
  head are equal, the softmax is uniform, and each head's output is the mean
  of its KV head's value rows [0, pos].  The split-K merge (in-launch, and
  across XCDs for launches that spread a group) must weight every chunk
  exactly by its number of rows for this to hold at 131072 positions;
- permuting the cached positions [0, pos) leaves the output unchanged up to
  the order of fp32 sums: chunk boundaries and merge order do not matter;
- q heads of one GQA group given the same q produce bitwise identical
  outputs: a head's output depends only on its q and its KV head.

These are properties of the reference's attention loop
(FloatTransformer.cpp:496-662): the softmax of equal scores is uniform
(:216-238), the weighted sum over positions is order-free, and head h reads
KV head h / kv_mul (:499-500).
"""
import numpy as np
import pytest

from leap_amd.attention import HipAttention
from tests.helpers import REL_TOL, assert_close, normal, rng_for, rope_f32

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _needs_gpu(hip_device):
    return hip_device


def _rotated_row(att, pos, k_new):
    c, s = att.rope_download(pos, pos + 1)
    return rope_f32(k_new, c[0], s[0])


# (n_heads, n_kv_heads, head_dim, context, theta): the 131072-position and
# ctx 4096 Llama-3 shapes, TinyLlama at 256, and one KV head at 32768 (a launch
# that spreads each group over several XCDs and merges the parts in a second
# launch)
MEAN_SHAPES = [(32, 8, 128, 131072, 500000.0), (32, 8, 128, 4096, 500000.0), (32, 4, 64, 256, 10000.0),
               (8, 1, 128, 32768, 500000.0), (64, 8, 128, 8192, 500000.0),
               (128, 8, 128, 8192, 500000.0)]  # Llama-3.1-405B heads: 16 q heads per KV head


@pytest.mark.parametrize("nh,nkv,hd,T,theta", MEAN_SHAPES)
def test_identical_keys_give_mean_of_values(nh, nkv, hd, T, theta):
    rng = rng_for(201, nh, nkv, hd, T)
    pos = T - 1
    with HipAttention(nh, nkv, hd, T, rope_theta=theta) as att:
        att.kv_fill_normal(0x4C454150 + 201, 1.0 / np.sqrt(hd))
        q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
        kr = _rotated_row(att, pos, k)
        att.kv_upload(0, 0, 0, np.broadcast_to(kr, (pos, nkv * hd)), None)
        out = att.step(0, pos, q, k, v)
        k_rows, v_rows = att.kv_download(0, 0, 0, T)
    # the premise: every key row, the appended one included, is the same
    assert np.array_equal(k_rows[pos], kr), "the appended key is not the rotated k_new"
    assert np.array_equal(v_rows[pos], v)
    means = v_rows.reshape(T, nkv, hd).astype(np.float64).mean(axis=0)
    want = np.concatenate([means[h // (nh // nkv)] for h in range(nh)])
    assert_close(out, want, what=f"{nh}/{nkv}/{hd} T={T}")


@pytest.mark.parametrize("nh,nkv,hd,T", [(32, 8, 128, 4096), (32, 8, 128, 131072), (8, 1, 128, 32768)])
def test_permuting_cached_positions_leaves_output_unchanged(nh, nkv, hd, T):
    rng = rng_for(202, nh, nkv, hd, T)
    pos = T - 1
    q, k, v = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
    perm = rng.permutation(pos)
    with HipAttention(nh, nkv, hd, T) as att:
        att.kv_fill_normal(0x4C454150 + 202, 1.0 / np.sqrt(hd))
        out1 = att.step(0, pos, q, k, v)
        k_rows, v_rows = att.kv_download(0, 0, 0, pos)
        att.kv_upload(0, 0, 0, k_rows[perm], v_rows[perm])
        out2 = att.step(0, pos, q, k, v)
    assert_close(out2, out1, what=f"permuted {nh}/{nkv}/{hd} T={T}")


@pytest.mark.parametrize("nh,nkv,hd,T", [(32, 8, 128, 4096), (24, 8, 128, 4096), (64, 8, 128, 8192),
                                         (16, 8, 64, 300), (32, 4, 64, 256),
                                         # 16 q heads per KV head, run as two groups of 8
                                         (128, 8, 128, 4096), (128, 8, 128, 300), (32, 2, 64, 2000)])
def test_gqa_heads_with_equal_q_give_identical_outputs(nh, nkv, hd, T):
    rng = rng_for(203, nh, nkv, hd, T)
    g = nh // nkv
    pos = T - 1
    q = normal(rng, (nkv, 1, hd), hd)
    q = np.repeat(q, g, axis=1).reshape(-1)  # every head of a group gets its group's first q
    k, v = normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
    with HipAttention(nh, nkv, hd, T) as att:
        att.kv_fill_normal(0x4C454150 + 203, 1.0 / np.sqrt(hd))
        out = att.step(0, pos, q, k, v).reshape(nkv, g, hd)
    for j in range(1, g):
        assert np.array_equal(out[:, j], out[:, 0]), f"head {j} of a group differs from head 0"
