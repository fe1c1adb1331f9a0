"""The stage hand-off of a pipeline: the packet {pos, flags} + x that the
master sends after its layers (FloatTransformer.cpp:775-788) and each worker
reads, runs its layers on and forwards (:925-939), and the entry points that
move it between a host packet and the device residual stream.

The oracle's packet restatement (oracle.packet_pack / packet_unpack /
packet_forwards) is pinned on the CPU against the reference itself: its
forward() as a master and its worker_loop(), each driven over a transport
that records what they send, built from checkpoint files whose FFN is zero
(run_layer is then exactly the attention sub-block, which the oracle's chain
reproduces bitwise).  The GPU tests check the device hand-off against the
oracle and a two-handle pipeline against one handle holding every layer.
"""
import struct

import numpy as np
import pytest

from oracle import oracle as O
from leap_amd import attention as A
from tests.helpers import assert_close, block_inputs, rng_for, write_checkpoint


def _layers(dim, nh, nkv, L, seed, gs=None):
    out = []
    for layer in range(L):
        _, rms, *wf = block_inputs(rng_for(dim, nh, nkv, layer, seed), dim, nkv * (dim // nh))
        out.append((rms, *(O.quantize_weight(w, gs) for w in wf)) if gs else (rms, *wf))
    return out


def _chain(orc, layers, lo, hi, pos, x, gs=None):
    for layer in range(lo, hi):
        x = orc.block_q8(layer, pos, x, *layers[layer], gs) if gs else orc.block(layer, pos, x, *layers[layer])
    return x


# ---- the restatement against the reference (CPU) -------------------------------

def _need_ref():
    if not O.ref_ckpt_available():
        pytest.skip("reference checkpoint driver not built (reference sources absent)")


def test_master_packets_match_reference(tmp_path):
    """forward() as the master of layers [0, 2) of 4: the packets it sends are
    the oracle's chain from the embedding row, packed, byte for byte; the
    forwards that ask for a reply take x from the reply packet."""
    _need_ref()
    dim, nh, nkv, L, vocab, sl, split = 256, 4, 2, 4, 7, 16, 2
    layers = _layers(dim, nh, nkv, L, 11)
    emb = rng_for(dim, 12).standard_normal((vocab, dim)).astype(np.float32)
    path = tmp_path / "m.bin"
    write_checkpoint(path, 1, dim, 64, nh, nkv, vocab, sl, layers, emb=emb)
    tokens, flags = [3, 1, 4, 1, 5, 6], [0, 1, 0, 1, 1, 0]
    pos = list(range(len(tokens)))
    rng = rng_for(dim, 13)
    replies = [O.packet_pack(p, 1, rng.standard_normal(dim).astype(np.float32))
               for p, f in zip(pos, flags) if f == 1]
    sent = O.ref_ckpt_master(path, split, dim, tokens, pos, flags, replies)
    assert len(sent) == len(tokens)
    orc = O.Oracle(L, nh, nkv, dim // nh, sl)
    for t, p, f, pkt in zip(tokens, pos, flags, sent):
        want = O.packet_pack(p, f, _chain(orc, layers, 0, split, p, emb[t]))
        assert pkt == want, f"token {t} at pos {p}"
        assert O.packet_unpack(pkt, dim)[:2] == (p, f)


@pytest.mark.parametrize("version,is_tail", [(1, True), (1, False), (2, True), (0, False)])
def test_worker_forwarding_matches_reference(tmp_path, version, is_tail):
    """worker_loop for layers [1, 3) of 4: which packets it forwards and what
    they hold are the oracle's rule and chain, byte for byte."""
    _need_ref()
    dim, nh, nkv, L, sl, lo, hi, gs = 256, 4, 2, 4, 16, 1, 3, 64
    layers = _layers(dim, nh, nkv, L, 21, gs if version == 2 else None)
    path = tmp_path / "m.bin"
    write_checkpoint(path, version, dim, 64, nh, nkv, 5, sl, layers, group_size=gs)
    rng = rng_for(dim, version, 22)
    flags = [1, 0, 0, 1, 1, 0, 1]
    packets = [O.packet_pack(p, f, rng.standard_normal(dim).astype(np.float32)) for p, f in enumerate(flags)]
    got = O.ref_ckpt_worker(path, lo, hi, is_tail, dim, packets)
    orc = O.Oracle(L, nh, nkv, dim // nh, sl)
    want = []
    for pkt in packets:
        p, f, x = O.packet_unpack(pkt, dim)
        x = _chain(orc, layers, lo, hi, p, x, gs if version == 2 else None)
        if O.packet_forwards(is_tail, f):
            want.append(O.packet_pack(p, f, x))
    assert len(got) == len(want) == (sum(flags) if is_tail else len(flags))
    for i, (g, w) in enumerate(zip(got, want)):
        assert g == w, f"forwarded packet {i}"


def test_packet_forwarding_rule():
    # every stage but the tail forwards; the tail only for a reply (FloatTransformer.cpp:937)
    assert [O.packet_forwards(t, f) for t in (False, True) for f in (0, 1)] == [True, True, False, True]


def test_packet_header_reads_packets():
    """The library's header reader (host only) on data, control and malformed packets."""
    dim = 64
    x = np.arange(dim, dtype=np.float32)
    for p, f in [(0, 0), (17, 1), (2**31 - 1, 5)]:
        assert A.packet_header(O.packet_pack(p, f, x), dim) == (p, f)
    ctrl = struct.pack("<H", 0xC0DE) + bytes(8 + 4 * dim - 2)  # ControlPacketHeader, padded
    assert A.packet_header(ctrl, dim) is None
    for bad in (b"", bytes(8 + 4 * dim - 4), bytes(8 + 4 * dim + 1)):
        with pytest.raises(A.LeapError):
            A.packet_header(bad, dim)


# ---- the device hand-off --------------------------------------------------------

@pytest.mark.gpu
def test_packet_upload_download_round_trip(hip_device):
    import torch
    nh, nkv, hd, sl = 16, 4, 128, 64
    dim = nh * hd
    rng = rng_for(dim, 31)
    with A.HipAttention(nh, nkv, hd, sl) as att:
        x = torch.zeros(dim, device="cuda:0")
        vals = rng.standard_normal(dim).astype(np.float32)
        pkt = O.packet_pack(37, 1, vals)
        assert att.packet_upload(pkt, x.data_ptr()) == (37, 1)
        assert np.array_equal(x.cpu().numpy(), vals)
        assert att.packet_download(x.data_ptr(), 37, 1) == pkt
        # a control packet copies nothing
        ctrl = struct.pack("<H", 0xC0DE) + bytes(len(pkt) - 2)
        assert att.packet_upload(ctrl, x.data_ptr()) is None
        assert np.array_equal(x.cpu().numpy(), vals)
        # on a caller's stream
        s = torch.cuda.Stream()
        vals2 = rng.standard_normal(dim).astype(np.float32)
        pkt2 = O.packet_pack(3, 0, vals2)
        assert att.packet_upload(pkt2, x.data_ptr(), s.cuda_stream) == (3, 0)
        s.synchronize()
        assert np.array_equal(x.cpu().numpy(), vals2)
        for bad in (pkt[:-4], pkt + b"\0", O.packet_pack(sl, 1, vals), O.packet_pack(-1, 1, vals)):
            with pytest.raises(A.LeapError):
                att.packet_upload(bad, x.data_ptr())
        with pytest.raises(A.LeapError):
            att.packet_download(x.data_ptr(), sl, 0)


@pytest.mark.gpu
@pytest.mark.parametrize("version,split", [(1, 2), (2, 1), (2, 3)])
def test_two_stage_pipeline(tmp_path, hip_device, version, split):
    """A master handle for layers [0, split) and a tail worker handle for the
    rest, connected by packets, against one handle that holds every layer
    (bitwise: the hand-off moves x without touching it), whose layers are
    each checked against the oracle on their own input; the worker forwards
    by the reference's rule."""
    import torch
    nh, nkv, hd, L, sl, gs = 16, 4, 128, 4, 32, 64
    dim = nh * hd
    q8 = version == 2
    layers = _layers(dim, nh, nkv, L, 41, gs if q8 else None)
    path = tmp_path / "m.bin"
    write_checkpoint(path, version, dim, 64, nh, nkv, 4, sl, layers, group_size=gs)
    rng = rng_for(dim, version, split, 42)
    orc = O.Oracle(L, nh, nkv, hd, sl)
    with A.HipAttention(nh, nkv, hd, sl, n_layers=L, layer_end=split) as master, \
            A.HipAttention(nh, nkv, hd, sl, n_layers=L, layer_begin=split) as worker, \
            A.HipAttention(nh, nkv, hd, sl, n_layers=L) as whole:
        for h in (master, worker, whole):
            h.load_checkpoint(path)
        xm = torch.empty(dim, device="cuda:0")
        xw = torch.empty(dim, device="cuda:0")
        xa = torch.empty(dim, device="cuda:0")
        for pos in range(10):
            flags = 0 if pos % 3 == 2 else 1
            x0 = rng.standard_normal(dim).astype(np.float32)
            xm.copy_(torch.from_numpy(x0))
            xa.copy_(torch.from_numpy(x0))
            for layer in range(split):
                master.block_async(layer, pos, xm.data_ptr())
            torch.cuda.synchronize()  # the packet calls run on the handle's own stream
            sent = master.packet_download(xm.data_ptr(), pos, flags)
            hdr = worker.packet_upload(sent, xw.data_ptr())
            assert hdr == (pos, flags)
            for layer in range(split, L):
                worker.block_async(layer, pos, xw.data_ptr())
            for layer in range(L):
                x_in = xa.cpu().numpy()
                whole.block_async(layer, pos, xa.data_ptr())
                torch.cuda.synchronize()
                x_out = xa.cpu().numpy()
                if layer == split - 1:
                    assert O.packet_unpack(sent, dim)[2].tobytes() == x_out.tobytes(), f"sent x, pos {pos}"
                want = (orc.block_q8(layer, pos, x_in, *layers[layer], gs) if q8 else
                        orc.block(layer, pos, x_in, *layers[layer]))
                assert_close(x_out - x_in, want - x_in, rel=1e-3 if q8 else 1e-4, what=f"pos {pos} layer {layer}")
                k, v = whole.kv_download(0, layer, pos, pos + 1)  # the oracle follows the device's cache
                orc.key_cache[layer, pos] = k[0]
                orc.value_cache[layer, pos] = v[0]
            torch.cuda.synchronize()
            assert np.array_equal(xw.cpu().numpy(), xa.cpu().numpy()), f"pos {pos}"
            if O.packet_forwards(True, flags):
                reply = worker.packet_download(xw.data_ptr(), pos, flags)
                assert O.packet_unpack(reply, dim)[:2] == (pos, flags)
                assert master.packet_upload(reply, xm.data_ptr()) == (pos, flags)
                assert np.array_equal(xm.cpu().numpy(), xa.cpu().numpy())
