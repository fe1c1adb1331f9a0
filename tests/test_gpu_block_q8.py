"""The quantized engine's attention sub-block on the GPU (rmsnorm, per-group
int8 quantization, W8A8 q/k/v projections, attention, quantization of its
output, W8A8 wo projection and residual: QuantizedTransformer.cpp:654-945)
against the oracle, whose every stage is bitwise equal to the reference
(tests/test_oracle.py).

Each stage is checked on the GPU's own input to that stage, read back
through leap_hip_attention_block_views_get:
  - quantize(rmsnorm(x)): the GPU's rmsnorm rounds 1/sqrt exactly where the
    reference uses an approximate reciprocal square root plus a Newton step,
    so the two xb differ in the last bit or two; the group scales agree to
    1e-6 and a quantized value may differ by one step only where the oracle's
    x * id lies within 1e-3 of a rounding boundary;
  - the W8A8 q/k/v product of the GPU's quantized input: bitwise;
  - the attention step on the GPU's q/k/v: the attention bar (1e-4), with
    the rotated k and the v appended to the cache bitwise;
  - quantize(attention output): bitwise;
  - x + Wo . that: bitwise.
End to end, a one-step difference in a quantized input moves an output by up
to |W| times that group's scale (a few 1e-4 of the output's largest value at
these shapes), so x_out - x is held to 1e-3 of its largest element.
"""
import numpy as np
import pytest

from oracle import oracle as O
from leap_amd.attention import HipAttention, LeapError
from tests.helpers import assert_close, block_inputs, normal, rng_for

pytestmark = pytest.mark.gpu

END_TO_END = 1e-3


_hip = None


def _d2h(addr, n, dtype):
    """Copy n elements at device address addr into a new host array."""
    import ctypes
    global _hip
    if _hip is None:
        try:
            _hip = ctypes.CDLL("libamdhip64.so")
        except OSError:
            _hip = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipDeviceSynchronize.argtypes = []
    out = np.empty(n, dtype)
    assert _hip.hipDeviceSynchronize() == 0
    assert _hip.hipMemcpy(out.ctypes.data, addr, out.nbytes, 2) == 0  # device to host
    return out


def _views(att, dim, kv, gs):
    v = att.block_views()
    f, b = np.float32, np.int8
    return dict(q=_d2h(v["q"], dim, f), k=_d2h(v["k"], kv, f), v=_d2h(v["v"], kv, f),
                att=_d2h(v["att"], dim, f), xq=_d2h(v["xq"], dim, b), xs=_d2h(v["xs"], dim // gs, f),
                aq=_d2h(v["aq"], dim, b), as_=_d2h(v["as_"], dim // gs, f))


def _setup(dim, nh, nkv, seq_len, L, layers, gs, seed):
    hd = dim // nh
    kv = nkv * hd
    att = HipAttention(nh, nkv, hd, seq_len, n_layers=L)
    orc = O.Oracle(L, nh, nkv, hd, seq_len)
    weights = {}
    for layer in layers:
        _, rms, *wf = block_inputs(rng_for(dim, nh, nkv, layer, gs, seed), dim, kv)
        w8 = [O.quantize_weight(w, gs) for w in wf]
        att.set_layer_weights_q8(layer, gs, rms, *w8)
        weights[layer] = (rms, w8)
    return att, orc, weights


def _check_stages(att, orc, layer, pos, x, got, rms, w8, gs, what):
    dim, kv = orc.n_heads * orc.head_dim, orc.kv_dim
    st = _views(att, dim, kv, gs)
    # 1. quantize(rmsnorm(x)) up to boundary cases of the last-bit rmsnorm difference
    xb = O.rmsnorm(x, rms)
    oq, osc = O.quantize(xb, gs)
    assert_close(st["xs"], osc, rel=1e-6, what=f"{what}: activation scales")
    diff = np.nonzero(st["xq"] != oq)[0]
    if diff.size:
        assert np.all(np.abs(st["xq"][diff].astype(int) - oq[diff]) == 1), f"{what}: quantized values off by > 1"
        idv = np.where(osc > 0, 1.0 / osc.astype(np.float64), 0.0)
        t = xb[diff].astype(np.float64) * idv[diff // gs]
        assert np.all(np.abs(np.abs(t - np.trunc(t)) - 0.5) < 1e-3), f"{what}: a quantized value moved off a boundary"
        assert diff.size <= max(2, dim // 200), f"{what}: {diff.size} quantized values differ"
    # 2. W8A8 q/k/v on the GPU's quantized input: bitwise
    for w, key in zip(w8[:3], ("q", "k", "v")):
        assert np.array_equal(O.matmul_q8(*w, st["xq"], st["xs"], gs), st[key]), f"{what}: W8A8 {key} differs"
    # 3. the attention step on the GPU's q/k/v; the cache slot it appends
    want_att, _ = orc.step(layer, pos, st["q"], st["k"], st["v"])
    assert_close(st["att"], want_att, what=f"{what}: attention output")
    kr, vr = att.kv_download(0, layer, pos, pos + 1)
    assert np.array_equal(kr.reshape(-1), orc.key_cache[layer, pos]), f"{what}: appended k"
    assert np.array_equal(vr.reshape(-1), orc.value_cache[layer, pos]), f"{what}: appended v"
    # 4. quantize(attention output): bitwise
    aq, asc = O.quantize(st["att"], gs)
    assert np.array_equal(aq, st["aq"]) and np.array_equal(asc, st["as_"]), f"{what}: quantized attention output"
    # 5. x + Wo . that: bitwise
    assert np.array_equal(x + O.matmul_q8(*w8[3], st["aq"], st["as_"], gs), got), f"{what}: wo + residual"


@pytest.mark.parametrize("dim,nh,nkv,ctx,gs", [
    (2048, 32, 4, 256, 64),     # TinyLlama
    (4096, 32, 8, 300, 64),     # Llama-3-8B, the exporter's default group size
    (4096, 32, 8, 50, 32),
    (4096, 32, 32, 50, 256),    # multi-head, one group per 16 threads
    (2048, 32, 4, 40, 32),      # TinyLlama, the smallest group
    (8192, 64, 8, 100, 64),     # Llama-3-70B
    (8192, 64, 8, 20, 256),     # eight threads per group
    (8192, 64, 8, 33, 128),     # four threads per group
    (4096, 32, 8, 65, 128),     # eight threads per group at Llama-3-8B
    (2048, 16, 2, 1, 128),      # first token
    (3072, 24, 8, 200, 64),     # Llama-3.2-3B: 192 of a team's 256 threads own values
    (3072, 24, 8, 30, 32),
    (3072, 24, 8, 30, 128),
    (5120, 40, 40, 64, 64),     # Llama-2-13B: 160 threads of 32 values
    (5120, 40, 40, 9, 128),
])
def test_q8_block_stages_match_oracle(hip_device, dim, nh, nkv, ctx, gs):
    hd, L, layer = dim // nh, 2, 1
    att, orc, w = _setup(dim, nh, nkv, ctx + 7, L, [layer], gs, 5)
    rms, w8 = w[layer]
    with att:
        pos = ctx - 1
        rng = rng_for(dim, ctx, gs, 6)
        if pos > 0:
            k_rows = normal(rng, (pos, nkv * hd), hd)
            v_rows = normal(rng, (pos, nkv * hd), hd)
            att.kv_upload(0, layer, 0, k_rows, v_rows)
            orc.key_cache[layer, :pos] = k_rows
            orc.value_cache[layer, :pos] = v_rows
        x = rng.standard_normal(dim).astype(np.float32)
        got = att.block(layer, pos, x)
        _check_stages(att, orc, layer, pos, x, got, rms, w8, gs, f"dim {dim} gs {gs} pos {pos}")
        # end to end against the oracle's own chain on fresh caches
        e2e = O.Oracle(L, nh, nkv, hd, ctx + 7)
        if pos > 0:
            e2e.key_cache[layer, :pos] = k_rows
            e2e.value_cache[layer, :pos] = v_rows
        want = e2e.block_q8(layer, pos, x, rms, *w8, gs)
        assert_close(got - x, want - x, rel=END_TO_END, what="end to end")
        if pos > 0:  # the rows before pos are untouched
            k0, v0 = att.kv_download(0, layer, 0, pos)
            assert np.array_equal(k0, k_rows) and np.array_equal(v0, v_rows)


def test_q8_block_sequential_decode(hip_device):
    """24 tokens through two layers, each block fed the GPU's own x, every
    stage checked at every step."""
    dim, nh, nkv, L, gs = 2048, 16, 4, 2, 64
    att, orc, w = _setup(dim, nh, nkv, 32, L, [0, 1], gs, 7)
    with att:
        x = rng_for(dim, 8).standard_normal(dim).astype(np.float32)
        for pos in range(24):
            for layer in range(L):
                got = att.block(layer, pos, x)
                _check_stages(att, orc, layer, pos, x, got, *w[layer], gs, f"pos {pos} layer {layer}")
                x = got
        k, v = att.kv_download(0, 1, 0, 24)
        assert np.array_equal(k, orc.key_cache[1, :24]) and np.array_equal(v, orc.value_cache[1, :24])


def test_q8_block_async_matches_sync(hip_device):
    import torch
    dim, nh, nkv, gs = 4096, 32, 8, 64
    att, _, _ = _setup(dim, nh, nkv, 128, 1, [0], gs, 9)
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


def test_q8_weight_argument_errors(hip_device):
    dim, gs = 2048, 64
    z8 = np.zeros(dim * dim, np.int8)
    zs = np.zeros(dim * dim // gs, np.float32)
    ones = np.ones(dim, np.float32)
    with HipAttention(32, 8, 64, 16, n_layers=2) as att:  # dim 2048, kv_dim 512
        kv8 = (np.zeros(512 * dim, np.int8), np.zeros(512 * dim // gs, np.float32))
        with pytest.raises(LeapError):  # group size 256 at dim 2048: 32 threads per group
            att.set_layer_weights_q8(0, 256, ones, (z8, np.zeros(dim * dim // 256, np.float32)),
                                     (kv8[0], np.zeros(512 * dim // 256, np.float32)),
                                     (kv8[0], np.zeros(512 * dim // 256, np.float32)),
                                     (z8, np.zeros(dim * dim // 256, np.float32)))
        att.set_layer_weights_q8(0, gs, ones, (z8, zs), kv8, kv8, (z8, zs))
        with pytest.raises(LeapError):  # another group size on the same handle
            att.set_layer_weights_q8(1, 32, ones, (z8, np.zeros(dim * dim // 32, np.float32)),
                                     (kv8[0], np.zeros(512 * dim // 32, np.float32)),
                                     (kv8[0], np.zeros(512 * dim // 32, np.float32)),
                                     (z8, np.zeros(dim * dim // 32, np.float32)))
        with pytest.raises(LeapError):  # fp32 weights on an int8 handle
            zf = np.zeros(dim * dim, np.float32)
            att.set_layer_weights(1, ones, zf, np.zeros(512 * dim, np.float32), np.zeros(512 * dim, np.float32), zf)
        with pytest.raises(LeapError):  # layer 1 has no weights yet
            att.block(1, 0, np.zeros(dim, np.float32))
        # all-zero weights and scales: the block adds exactly zero
        x = rng_for(11).standard_normal(dim).astype(np.float32)
        assert np.array_equal(att.block(0, 0, x), x)
