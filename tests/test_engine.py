"""The C++20 engine-side wrapper and demo layer loop (leap_amd/host)."""
import os
import subprocess

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import gpu_available
from tests.helpers import assert_close

DEMO = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "leap_amd", "host",
                    "engine_demo")


def _demo():
    if not os.path.isfile(DEMO):
        pytest.fail(f"{DEMO} missing: build with `python -m leap_amd.build`")
    return DEMO


def test_engine_demo_usage_error():
    r = subprocess.run([_demo()], capture_output=True, text=True)
    assert r.returncode == 2 and "usage" in r.stderr


def test_engine_demo_reports_shim_errors_as_exceptions(tmp_path):
    if gpu_available():
        pytest.skip("a GPU is present")
    r = subprocess.run([_demo(), "2", "8", "2", "64", "16", "4", str(tmp_path)], capture_output=True,
                       text=True)
    assert r.returncode == 3 and "no HIP device" in r.stderr


@pytest.mark.gpu
def test_engine_demo_decode_matches_oracle(tmp_path, hip_device):
    L, nh, nkv, hd, seq_len, n_tok = 2, 16, 4, 128, 200, 150
    r = subprocess.run([_demo(), str(L), str(nh), str(nkv), str(hd), str(seq_len), str(n_tok),
                        str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rec = nh * hd * 2 + nkv * hd * 2
    trace = np.fromfile(tmp_path / "trace.bin", dtype=np.float32).reshape(n_tok, L, rec)
    orc = O.Oracle(L, nh, nkv, hd, seq_len)
    for pos in range(n_tok):
        for layer in range(L):
            t = trace[pos, layer]
            q, k, v, xb = np.split(t, [nh * hd, nh * hd + nkv * hd, nh * hd + 2 * nkv * hd])
            want, _ = orc.step(layer, pos, q, k, v)
            assert_close(xb, want, what=f"token {pos} layer {layer}")


@pytest.mark.gpu
def test_engine_demo_block_matches_oracle(tmp_path, hip_device):
    """The C++ wrapper's set_layer_weights/block path: 24 tokens x 2 layers of
    run_layer up to the attention residual, x fed back from step to step."""
    L, nh, nkv, hd, seq_len, n_tok = 2, 16, 4, 128, 32, 24
    r = subprocess.run([_demo(), str(L), str(nh), str(nkv), str(hd), str(seq_len), str(n_tok),
                        str(tmp_path), "block"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    dim, kv = nh * hd, nkv * hd
    wall = np.fromfile(tmp_path / "weights.bin", dtype=np.float32)
    sizes = [dim, dim * dim, kv * dim, kv * dim, dim * dim]
    assert wall.size == L * sum(sizes)
    weights = []
    for part in np.split(wall, L):
        rms, wq, wk, wv, wo = np.split(part, np.cumsum(sizes)[:-1])
        weights.append((rms, wq.reshape(dim, dim), wk.reshape(kv, dim), wv.reshape(kv, dim),
                        wo.reshape(dim, dim)))
    trace = np.fromfile(tmp_path / "trace.bin", dtype=np.float32).reshape(n_tok, L, 2, dim)
    orc = O.Oracle(L, nh, nkv, hd, seq_len)
    for pos in range(n_tok):
        for layer in range(L):
            x_in, x_out = trace[pos, layer]
            want = orc.block(layer, pos, x_in, *weights[layer])
            assert_close(x_out - x_in, want - x_in, what=f"token {pos} layer {layer}")


@pytest.mark.gpu
@pytest.mark.parametrize("version", [1, 2])
def test_engine_demo_checkpoint_matches_oracle(tmp_path, hip_device, version):
    """The engine loop with its weights loaded from a checkpoint file (fp32 or
    int8) through the C++ wrapper: 12 tokens x 2 layers against the oracle's
    chain on the same tensors."""
    from tests.helpers import block_inputs, rng_for, write_checkpoint
    L, nh, nkv, hd, seq_len, n_tok, gs = 2, 16, 4, 128, 16, 12, 64
    dim, kv = nh * hd, nkv * hd
    layers = []
    for layer in range(L):
        _, rms, *wf = block_inputs(rng_for(dim, layer, version, 31), dim, kv)
        layers.append((rms, *(O.quantize_weight(w, gs) for w in wf)) if version == 2 else (rms, *wf))
    path = tmp_path / "m.bin"
    write_checkpoint(path, version, dim, 64, nh, nkv, 4, seq_len, layers, group_size=gs)
    r = subprocess.run([_demo(), str(L), str(nh), str(nkv), str(hd), str(seq_len), str(n_tok), str(tmp_path),
                        "ckpt", str(path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    trace = np.fromfile(tmp_path / "trace.bin", dtype=np.float32).reshape(n_tok, L, 2, dim)
    orc = O.Oracle(L, nh, nkv, hd, seq_len)
    for pos in range(n_tok):
        for layer in range(L):
            x_in, x_out = trace[pos, layer]
            if version == 2:
                want = orc.block_q8(layer, pos, x_in, *layers[layer], gs)
                assert_close(x_out - x_in, want - x_in, rel=1e-3, what=f"int8 token {pos} layer {layer}")
            else:
                want = orc.block(layer, pos, x_in, *layers[layer])
                assert_close(x_out - x_in, want - x_in, what=f"token {pos} layer {layer}")


@pytest.mark.gpu
@pytest.mark.parametrize("version,split", [(1, 1), (2, 2)])
def test_engine_demo_pipeline_matches_oracle(tmp_path, hip_device, version, split):
    """The demo's two-node pipeline (master handle, tail worker handle, packets
    between them, x in device memory): each sent packet is the master's
    layers on the token's x, each reply the worker's layers on the sent x,
    the worker forwards by the reference's rule and the master takes x from
    the reply."""
    from tests.helpers import block_inputs, rng_for, write_checkpoint
    L, nh, nkv, hd, seq_len, n_tok, gs = 3, 16, 4, 128, 16, 9, 64
    dim, kv = nh * hd, nkv * hd
    q8 = version == 2
    layers = []
    for layer in range(L):
        _, rms, *wf = block_inputs(rng_for(dim, layer, version, 51), dim, kv)
        layers.append((rms, *(O.quantize_weight(w, gs) for w in wf)) if q8 else (rms, *wf))
    path = tmp_path / "m.bin"
    write_checkpoint(path, version, dim, 64, nh, nkv, 4, seq_len, layers, group_size=gs)
    r = subprocess.run([_demo(), str(L), str(nh), str(nkv), str(hd), str(seq_len), str(n_tok), str(tmp_path),
                        "pipeline", str(path), str(split)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    pk = 8 + 4 * dim
    rec = np.dtype([("x", "<f4", dim), ("sent", "u1", pk), ("fwd", "<i4"), ("reply", "u1", pk),
                    ("back", "<f4", dim)])
    trace = np.fromfile(tmp_path / "trace.bin", dtype=rec)
    assert trace.shape == (n_tok,)
    orc = O.Oracle(L, nh, nkv, hd, seq_len)

    def run(lo, hi, pos, x):
        for layer in range(lo, hi):
            x = orc.block_q8(layer, pos, x, *layers[layer], gs) if q8 else orc.block(layer, pos, x, *layers[layer])
        return x

    tol = 1e-3 if q8 else 1e-4
    for pos, t in enumerate(trace):
        flags = 0 if pos % 3 == 2 else 1
        p, f, sent_x = O.packet_unpack(t["sent"].tobytes(), dim)
        assert (p, f) == (pos, flags)
        if split == 1 or not q8:  # one layer per stage, or fp32: a tight bound holds
            assert_close(sent_x - t["x"], run(0, split, pos, t["x"]) - t["x"], rel=tol, what=f"sent, token {pos}")
        else:
            run(0, split, pos, t["x"])  # keep the oracle's cache in step
        want_reply = run(split, L, pos, sent_x)
        assert t["fwd"] == int(O.packet_forwards(True, flags))
        if t["fwd"]:
            rp, rf, rx = O.packet_unpack(t["reply"].tobytes(), dim)
            assert (rp, rf) == (pos, flags)
            if L - split == 1 or not q8:
                assert_close(rx - sent_x, want_reply - sent_x, rel=tol, what=f"reply, token {pos}")
            assert np.array_equal(t["back"], rx)
        else:
            assert not t["reply"].any() and not t["back"].any()
