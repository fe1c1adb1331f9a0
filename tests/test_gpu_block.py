"""The attention sub-block on the GPU (rmsnorm, q/k/v projections, attention,
wo projection and residual: FloatTransformer.cpp:394-683) against the oracle.

The oracle's chain is bitwise equal to the reference's run_layer
(tests/test_oracle.py).  The GPU's projections sum in another order, so the
bar is the attention bar applied to the block's contribution x_out - x, and
the appended cache row agrees to 1e-5 of its largest element.
"""
import numpy as np
import pytest

from oracle import oracle as O
from leap_amd.attention import HipAttention, LeapError
from tests.helpers import assert_close, block_inputs, normal, rng_for

pytestmark = pytest.mark.gpu


def _setup(dim, nh, nkv, seq_len, L, layers, seed):
    hd = dim // nh
    kv = nkv * hd
    att = HipAttention(nh, nkv, hd, seq_len, n_layers=L)
    orc = O.Oracle(L, nh, nkv, hd, seq_len)
    weights = {}
    for layer in layers:
        w = block_inputs(rng_for(dim, nh, nkv, layer, seed), dim, kv)[1:]
        att.set_layer_weights(layer, *w)
        weights[layer] = w
    return att, orc, weights


@pytest.mark.parametrize("dim,nh,nkv,ctx", [
    (2048, 32, 4, 256),   # TinyLlama
    (4096, 32, 8, 300),   # Llama-3-8B
    (8192, 64, 8, 100),   # Llama-3-70B
    (4096, 32, 32, 50),   # multi-head
    (2048, 16, 2, 1),     # first token
    (3072, 24, 8, 200),   # Llama-3.2-3B (three q heads per KV head)
    (5120, 40, 40, 64),   # Llama-2-13B
])
def test_block_matches_oracle(hip_device, dim, nh, nkv, ctx):
    hd, L, layer = dim // nh, 2, 1
    att, orc, w = _setup(dim, nh, nkv, ctx + 7, L, [layer], 5)
    with att:
        pos = ctx - 1
        rng = rng_for(dim, ctx, 6)
        if pos > 0:
            k_rows = normal(rng, (pos, nkv * hd), hd)
            v_rows = normal(rng, (pos, nkv * hd), hd)
            att.kv_upload(0, layer, 0, k_rows, v_rows)
            orc.key_cache[layer, :pos] = k_rows
            orc.value_cache[layer, :pos] = v_rows
        x = rng.standard_normal(dim).astype(np.float32)
        got = att.block(layer, pos, x)
        want = orc.block(layer, pos, x, *w[layer])
        assert_close(got - x, want - x, what=f"block contribution dim {dim} pos {pos}")
        kr, vr = att.kv_download(0, layer, pos, pos + 1)
        assert_close(kr.reshape(-1), orc.key_cache[layer, pos], rel=1e-5, what="appended k")
        assert_close(vr.reshape(-1), orc.value_cache[layer, pos], rel=1e-5, what="appended v")
        if pos > 0:  # the rows before pos are untouched
            k0, v0 = att.kv_download(0, layer, 0, pos)
            assert np.array_equal(k0, orc.key_cache[layer, :pos])
            assert np.array_equal(v0, orc.value_cache[layer, :pos])


def test_block_sequential_decode(hip_device):
    """40 tokens through two layers, each block fed the GPU's own x."""
    dim, nh, nkv, L = 2048, 16, 4, 2
    att, orc, w = _setup(dim, nh, nkv, 64, L, [0, 1], 7)
    with att:
        x = rng_for(dim, 8).standard_normal(dim).astype(np.float32)
        for pos in range(40):
            for layer in range(L):
                got = att.block(layer, pos, x)
                want = orc.block(layer, pos, x, *w[layer])
                assert_close(got - x, want - x, what=f"pos {pos} layer {layer}")
                x = got
        k, v = att.kv_download(0, 1, 0, 40)
        assert_close(k, orc.key_cache[1, :40], rel=1e-5, what="layer 1 keys")
        assert_close(v, orc.value_cache[1, :40], rel=1e-5, what="layer 1 values")


def test_block_async_matches_sync(hip_device):
    import torch
    dim, nh, nkv = 4096, 32, 8
    att, _, _ = _setup(dim, nh, nkv, 128, 1, [0], 9)
    with att:
        rng = rng_for(dim, 10)
        k_rows = normal(rng, (99, nkv * 128), 128)
        v_rows = normal(rng, (99, nkv * 128), 128)
        att.kv_upload(0, 0, 0, k_rows, v_rows)
        x = rng.standard_normal(dim).astype(np.float32)
        ref = att.block(0, 99, x)
        att.kv_upload(0, 0, 0, k_rows, v_rows)
        dx = torch.from_numpy(x.copy()).cuda()
        s = torch.cuda.Stream()
        att.block_async(0, 99, dx.data_ptr(), s.cuda_stream)
        s.synchronize()
        assert np.array_equal(dx.cpu().numpy(), ref)


def test_block_argument_errors(hip_device):
    with HipAttention(8, 8, 64, 16) as att:  # dim 512: no projection kernel
        z = np.zeros(512 * 512, np.float32)
        with pytest.raises(LeapError):
            att.set_layer_weights(0, np.ones(512, np.float32), z, z, z, z)
    with HipAttention(32, 8, 64, 16) as att:  # dim 2048, no weights uploaded yet
        with pytest.raises(LeapError):
            att.block(0, 0, np.zeros(2048, np.float32))
        with pytest.raises(LeapError):
            att.block(0, 16, np.zeros(2048, np.float32))
