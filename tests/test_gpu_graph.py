"""The async entry points under HIP graph capture.  They enqueue kernels only
(no allocation, copy or memset on the call path), so a caller can capture a
layer loop once and replay it.  Every replay is checked bitwise against the
same calls made eagerly, with other eager work and synchronisations between
the replays; the eager results themselves are the ones the parity tests hold
to the oracle."""
import numpy as np
import pytest

from oracle import oracle as O
from leap_amd.attention import HipAttention
from tests.helpers import block_inputs, normal, rng_for

pytestmark = pytest.mark.gpu


def _other_work():
    import torch
    a = torch.randn(1 << 20, device="cuda:0")
    assert np.isfinite((a * 2.0).sum().item())


def _capture(fn, stream):
    import torch
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        fn(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return graph


@pytest.mark.parametrize("nh,nkv,hd,sl,pos,poss", [
    (32, 8, 128, 3100, 2999, (2999, 17, 1200)),    # near-equal chunks of one pass, asymmetric merge
    (32, 8, 128, 8200, 8191, (8191, 8000, 300)),   # 128-row chunks of two passes, rotated
    (8, 1, 128, 20000, 19999, (19999, 5000, 40)),  # one KV head spread over the XCDs: two launches per step
    (32, 4, 64, 600, 255, (255, 40, 500)),         # TinyLlama's heads as four launch groups of 2 (the batch: 12 groups)
    (32, 8, 128, 1100, 1000, (1000, 3, 700)),      # Llama-3-8B's heads as two launch groups of 2
])
def test_step_loop_replays_match_eager(hip_device, nh, nkv, hd, sl, pos, poss):
    """Four layers of single-sequence steps (split-K merge over several
    chunks) and four of a ragged batch, captured once and replayed."""
    import torch
    L, batch = 4, 3
    poss = np.array(poss, np.int32)
    with HipAttention(nh, nkv, hd, sl, n_layers=L, max_batch=batch) as att:
        att.kv_fill_normal(21, 1.0 / np.sqrt(hd))
        g = torch.Generator(device="cuda:0")
        g.manual_seed(22)
        q = torch.randn(L, batch, nh * hd, device="cuda:0", generator=g) / np.sqrt(hd)
        k = torch.randn(L, batch, nkv * hd, device="cuda:0", generator=g) / np.sqrt(hd)
        v = torch.randn(L, batch, nkv * hd, device="cuda:0", generator=g) / np.sqrt(hd)
        out = torch.zeros(L, batch, nh * hd, device="cuda:0")
        pos_dev = torch.from_numpy(poss).cuda()
        s = torch.cuda.Stream()

        def loop(sp):
            for layer in range(L):
                att.step_async(layer, pos, q[layer, 0].data_ptr(), k[layer, 0].data_ptr(), v[layer, 0].data_ptr(),
                               out[layer, 0].data_ptr(), sp)
            for layer in range(L):
                att.step_batched_async(layer, batch, pos_dev.data_ptr(), int(poss.max()), q[layer].data_ptr(),
                                       k[layer].data_ptr(), v[layer].data_ptr(), out[layer].data_ptr(), sp,
                                       int(poss.sum() + batch))

        loop(s.cuda_stream)
        torch.cuda.synchronize()
        want = out.clone()
        rows = [(0, pos), (2, int(poss[2]))]  # (sequence, position) rows the loop appends
        want_kv = [att.kv_download(seq, L - 1, p, p + 1) for seq, p in rows]
        graph = _capture(loop, s)
        zero = np.zeros((1, nkv * hd), np.float32)
        for i in range(3):
            out.zero_()
            for seq, p in rows:
                att.kv_upload(seq, L - 1, p, zero, zero)
            _other_work()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want), f"replay {i}"
            for (seq, p), (wk, wv) in zip(rows, want_kv):
                gk, gv = att.kv_download(seq, L - 1, p, p + 1)
                assert np.array_equal(gk, wk) and np.array_equal(gv, wv), f"replay {i}: row {p} of sequence {seq}"


@pytest.mark.parametrize("q8", [False, True])
def test_block_loop_replays_match_eager(hip_device, q8):
    """Two layers of the attention sub-block, captured once; x is restored
    before each replay (the block adds into it)."""
    import torch
    dim, nh, nkv, L, sl, gs = 4096, 32, 8, 2, 160, 64
    hd, kv = dim // nh, nkv * (dim // nh)
    pos = 150
    with HipAttention(nh, nkv, hd, sl, n_layers=L) as att:
        for layer in range(L):
            _, rms, *wf = block_inputs(rng_for(dim, layer, 31), dim, kv)
            if q8:
                att.set_layer_weights_q8(layer, gs, rms, *(O.quantize_weight(w, gs) for w in wf))
            else:
                att.set_layer_weights(layer, rms, *wf)
        rng = rng_for(dim, 32)
        for layer in range(L):
            att.kv_upload(0, layer, 0, normal(rng, (pos, kv), hd), normal(rng, (pos, kv), hd))
        x0 = torch.from_numpy(rng.standard_normal(dim).astype(np.float32)).cuda()
        x = x0.clone()
        s = torch.cuda.Stream()

        def loop(sp):
            for layer in range(L):
                att.block_async(layer, pos, x.data_ptr(), sp)

        loop(s.cuda_stream)
        torch.cuda.synchronize()
        want = x.clone()
        assert not torch.equal(want, x0)
        graph = _capture(loop, s)
        for i in range(3):
            x.copy_(x0)
            _other_work()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(x, want), f"replay {i}"
