"""LEAP checkpoint files (.bin): the header reader and the upload of every
held layer's attention weights (TransformerFactory.cpp:59-135,
memory_map_weights in FloatTransformer.cpp:947-978 and
QuantizedTransformer.cpp:102-134).

The files are written by tests.helpers.write_checkpoint.  That writer is
pinned against the reference's own factory: the engine Transformer::create
builds from a written file runs run_layer to the oracle's result bit for bit
(oracle/_ref), so the tensors sit where the reference reads them.  The GPU
tests then load the same files through leap_hip_attention_load_checkpoint.
"""
import os

import numpy as np
import pytest

from oracle import oracle as O
from leap_amd import attention as A
from tests.helpers import assert_close, block_inputs, normal, rng_for, write_checkpoint


def _model(dim, nh, nkv, L, seed, gs=None):
    """Per-layer (rms_att, wq, wk, wv, wo); int8 pairs for the projections when gs is set."""
    layers = []
    for layer in range(L):
        _, rms, *wf = block_inputs(rng_for(dim, nh, nkv, layer, seed), dim, nkv * (dim // nh))
        layers.append((rms, *(O.quantize_weight(w, gs) for w in wf)) if gs else (rms, *wf))
    return layers


def _attention_bytes(version, dim, nh, nkv, L, vocab, gs=64):
    kv = nkv * (dim // nh)
    head = 28 if version == 0 else 256
    if version != 2:
        return head + 4 * ((2 * L + 1) * dim + vocab * dim + L * (2 * dim * dim + 2 * kv * dim))
    per = lambda n: n + 4 * (n // gs)  # noqa: E731
    return head + 4 * (2 * L + 1) * dim + per(vocab * dim) + L * (2 * per(dim * dim) + 2 * per(kv * dim))


@pytest.mark.parametrize("version,shared", [(0, True), (0, False), (1, True), (2, True), (2, False)])
def test_header(tmp_path, version, shared):
    dim, nh, nkv, L, vocab, hidden, sl = 256, 4, 2, 2, 8, 64, 16
    gs = 64 if version == 2 else None
    layers = _model(dim, nh, nkv, L, 1, gs)
    path = tmp_path / "m.bin"
    size = write_checkpoint(path, version, dim, hidden, nh, nkv, vocab, sl, layers, shared=shared,
                            group_size=gs or 64)
    c = A.checkpoint_read(path)
    assert (c["version"], c["dim"], c["hidden_dim"], c["n_layers"], c["n_heads"], c["n_kv_heads"],
            c["vocab_size"], c["seq_len"]) == (version, dim, hidden, L, nh, nkv, vocab, sl)
    assert c["shared_classifier"] == (1 if shared or version == 1 else 0)
    assert c["group_size"] == (64 if version == 2 else 0)
    assert c["header_bytes"] == (28 if version == 0 else 256)
    assert c["file_bytes"] == size
    assert c["attention_bytes"] == _attention_bytes(version, dim, nh, nkv, L, vocab)


def test_header_rejects_non_checkpoints(tmp_path):
    bad = tmp_path / "bad.bin"
    bad.write_bytes(bytes(64))  # no magic and a zero Config
    with pytest.raises(A.LeapError):
        A.checkpoint_read(bad)
    import struct
    bad.write_bytes(struct.pack("<Ii", 0x616B3432, 3) + bytes(300))  # unknown version
    with pytest.raises(A.LeapError):
        A.checkpoint_read(bad)
    bad.write_bytes(struct.pack("<Ii7iBi", 0x616B3432, 2, 256, 64, 1, 4, 2, 8, 16, 1, 48) + bytes(256))
    with pytest.raises(A.LeapError):  # group size that does not divide dim
        A.checkpoint_read(bad)
    with pytest.raises(A.LeapError):
        A.checkpoint_read(tmp_path / "missing.bin")


@pytest.mark.parametrize("version", [0, 1, 2])
def test_writer_matches_reference_factory(tmp_path, version):
    if not O.ref_ckpt_available():
        pytest.skip("reference checkpoint driver not built (reference sources absent)")
    dim, nh, nkv, L, vocab, hidden, sl, gs = 256, 4, 2, 2, 8, 64, 40, 64
    hd = dim // nh
    layers = _model(dim, nh, nkv, L, 2, gs if version == 2 else None)
    path = tmp_path / "m.bin"
    write_checkpoint(path, version, dim, hidden, nh, nkv, vocab, sl, layers, group_size=gs)
    rng = rng_for(dim, version, 3)
    kc = normal(rng, (L, sl, nkv * hd), hd)
    vc = normal(rng, (L, sl, nkv * hd), hd)
    x = rng.standard_normal(dim).astype(np.float32)
    layer, pos = 1, 33
    kind, xr, kr, vr = O.ref_ckpt_run_layer(path, layer, pos, x, kc, vc)
    assert kind == (2 if version == 2 else 1)
    orc = O.Oracle(L, nh, nkv, hd, sl)
    orc.key_cache[:] = kc
    orc.value_cache[:] = vc
    if version == 2:
        got = orc.block_q8(layer, pos, x, *layers[layer], gs)
    else:
        got = orc.block(layer, pos, x, *layers[layer])
    assert np.array_equal(got, xr)
    assert np.array_equal(orc.key_cache, kr) and np.array_equal(orc.value_cache, vr)


# ---- upload to the device -------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("version,layer_begin", [(1, 0), (0, 1), (2, 0), (2, 1)])
def test_load_checkpoint_runs_the_block(tmp_path, hip_device, version, layer_begin):
    dim, nh, nkv, L, vocab, hidden, sl, gs = 2048, 16, 4, 2, 4, 64, 48, 64
    hd = dim // nh
    layers = _model(dim, nh, nkv, L, 4, gs if version == 2 else None)
    path = tmp_path / "m.bin"
    write_checkpoint(path, version, dim, hidden, nh, nkv, vocab, sl, layers, group_size=gs)
    layer, pos = 1, 40
    rng = rng_for(dim, version, 5)
    k_rows = normal(rng, (pos, nkv * hd), hd)
    v_rows = normal(rng, (pos, nkv * hd), hd)
    x = rng.standard_normal(dim).astype(np.float32)
    with A.HipAttention(nh, nkv, hd, sl, n_layers=L, layer_begin=layer_begin) as att:
        att.load_checkpoint(path)
        att.kv_upload(0, layer, 0, k_rows, v_rows)
        got = att.block(layer, pos, x)
    orc = O.Oracle(L, nh, nkv, hd, sl)
    orc.key_cache[layer, :pos] = k_rows
    orc.value_cache[layer, :pos] = v_rows
    if version == 2:
        want = orc.block_q8(layer, pos, x, *layers[layer], gs)
        assert_close(got - x, want - x, rel=1e-3, what="int8 block from the checkpoint")
    else:
        want = orc.block(layer, pos, x, *layers[layer])
        assert_close(got - x, want - x, what="fp32 block from the checkpoint")


@pytest.mark.gpu
def test_load_checkpoint_rejects_mismatches(tmp_path, hip_device):
    dim, nh, nkv, L = 2048, 16, 4, 2
    layers = _model(dim, nh, nkv, L, 6)
    path = tmp_path / "m.bin"
    size = write_checkpoint(path, 1, dim, 64, nh, nkv, 4, 32, layers)
    with A.HipAttention(nh, 8, dim // nh, 32, n_layers=L) as att:  # other KV heads
        with pytest.raises(A.LeapError):
            att.load_checkpoint(path)
    with A.HipAttention(nh, nkv, dim // nh, 32, n_layers=3) as att:  # other depth
        with pytest.raises(A.LeapError):
            att.load_checkpoint(path)
    short = tmp_path / "short.bin"
    with open(path, "rb") as f:
        short.write_bytes(f.read(size // 2))
    with A.HipAttention(nh, nkv, dim // nh, 32, n_layers=L) as att:
        with pytest.raises(A.LeapError):
            att.load_checkpoint(short)
        with pytest.raises(A.LeapError):
            att.load_checkpoint(tmp_path / "missing.bin")
        with pytest.raises(A.LeapError):  # nothing was uploaded by the failed loads
            att.block(0, 0, np.zeros(dim, np.float32))


@pytest.mark.parametrize("cfg", [
    (256, 64, 2, 4, 2, -2**31, 16),            # vocab_size INT_MIN: no magnitude (the fuzz's UBSan finding)
    (2**31 - 1, 64, 2**31 - 1, 1, 1, 8, 16),   # tensor bytes beyond any signed file size
])
def test_header_rejects_unrepresentable_sizes(tmp_path, cfg):
    import struct
    path = tmp_path / "x.bin"
    path.write_bytes(struct.pack("<7i", *cfg) + bytes(64))
    with pytest.raises(A.LeapError):
        A.checkpoint_read(path)
