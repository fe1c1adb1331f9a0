"""leap_hip_attention_step_noalloc (no handle, no device allocation, a static
device workspace) against leap_hip_attention_step_async on the same cache
bytes, through the C ABI: bitwise equal outputs and appended cache rows on two
calls in a row, the second with a smaller context, within the oracle's bar,
and no change in the device's free memory."""
import errno

import numpy as np
import pytest

from leap_amd import attention as A
from leap_amd.attention import HipAttention, LeapError
from oracle import oracle as O
from tests.helpers import REL_TOL, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _needs_gpu(hip_device):
    return hip_device


def _packed_rope(att, torch):
    c, s = att.rope_download()
    return torch.from_numpy(np.stack([c, s], axis=-1).reshape(-1).copy()).cuda()


@pytest.mark.parametrize("nh,nkv,hd,seq_len,theta,positions", [
    (32, 8, 128, 4096, 500000.0, (4095, 1000)),   # Llama-3-8B: 64 chunks (asymmetric merge), then 16
    (32, 4, 64, 512, 10000.0, (255, 40, 20)),      # TinyLlama as four launch groups of 2 q heads per KV head: 8 half-pass chunks on 2-wave workgroups, then one chunk each
    (32, 2, 128, 4096, 500000.0, (4095, 700)),     # 16 q heads per KV head: four groups of 8, spread over the XCDs
    (64, 8, 128, 8192, 500000.0, (8191, 3000)),    # Llama-3-70B heads
])
def test_noalloc_matches_the_handle_step(nh, nkv, hd, seq_len, theta, positions):
    import torch
    dev = torch.device("cuda:0")
    with HipAttention(nh, nkv, hd, seq_len, rope_theta=theta) as att:
        att.kv_fill_normal(0x4E41 + nh, 1.0 / np.sqrt(hd))
        rope = _packed_rope(att, torch)
        k0, v0 = att.kv_download(0, 0, 0, seq_len)
        kc = torch.from_numpy(k0).cuda()
        vc = torch.from_numpy(v0).cuda()
        g = torch.Generator(device=dev)
        g.manual_seed(nh * 1000 + hd)
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):  # the runtime sets up a stream's queue on its first launch
            kc.add_(0.0)
        torch.cuda.synchronize()
        for i, pos in enumerate(positions):
            q = torch.randn(nh * hd, device=dev, generator=g) / np.sqrt(hd)
            k = torch.randn(nkv * hd, device=dev, generator=g) / np.sqrt(hd)
            v = torch.randn(nkv * hd, device=dev, generator=g) / np.sqrt(hd)
            out_n = torch.full((nh * hd,), float("nan"), device=dev)
            out_h = torch.full((nh * hd,), float("nan"), device=dev)
            torch.cuda.synchronize()
            free0, _ = torch.cuda.mem_get_info()
            A.step_noalloc(nh, nkv, hd, seq_len, pos, rope.data_ptr(), kc.data_ptr(), vc.data_ptr(), q.data_ptr(),
                           k.data_ptr(), v.data_ptr(), out_n.data_ptr(), s.cuda_stream)
            s.synchronize()
            free1, _ = torch.cuda.mem_get_info()
            assert free1 == free0, f"free device memory {free0} before the call, {free1} after"
            att.step_async(0, pos, q.data_ptr(), k.data_ptr(), v.data_ptr(), out_h.data_ptr(), s.cuda_stream)
            s.synchronize()
            on, oh = out_n.cpu().numpy(), out_h.cpu().numpy()
            assert np.array_equal(on, oh), f"call {i} (pos {pos}): outputs differ"
            kh, vh = att.kv_download(0, 0, pos, pos + 1)
            assert np.array_equal(kc[pos].cpu().numpy(), kh[0]) and np.array_equal(vc[pos].cpu().numpy(), vh[0])
            # and within the bar of the oracle on the caller's cache rows
            orc = O.Oracle(1, nh, nkv, hd, seq_len, theta=theta)
            orc.key_cache[0, :pos] = kc[:pos].cpu().numpy()
            orc.value_cache[0, :pos] = vc[:pos].cpu().numpy()
            want, _ = orc.step(0, pos, q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy())
            assert_close(on, want, rel=REL_TOL)
            assert np.array_equal(kh[0], orc.key_cache[0, pos])


def test_noalloc_rejects_what_the_workspace_cannot_hold():
    import torch
    buf = torch.zeros(1 << 16, device="cuda:0")
    p = buf.data_ptr()
    with pytest.raises(LeapError) as ei:  # 128 heads of 128: 4.7 MB of records
        A.step_noalloc(128, 16, 128, 64, 0, p, p, p, p, p, p, p)
    assert ei.value.code == -errno.EINVAL and "workspace" in str(ei.value)
    with pytest.raises(LeapError) as ei:
        A.step_noalloc(32, 8, 128, 64, 64, p, p, p, p, p, p, p)
    assert ei.value.code == -errno.EINVAL and "pos" in str(ei.value)
    with pytest.raises(LeapError) as ei:
        A.step_noalloc(32, 8, 128, 64, 0, p + 4, p, p, p, p, p, p)
    assert ei.value.code == -errno.EINVAL and "aligned" in str(ei.value)


def test_noalloc_alternating_shapes_share_the_workspace():
    """Shapes of different KV-head counts and chunk counts, called in turn on
    one device, against their handles: every shape's records leave the
    arrival counters of the others at zero."""
    import torch
    dev = torch.device("cuda:0")
    shapes = [(64, 8, 128, 8192, 500000.0), (32, 4, 64, 512, 10000.0), (32, 8, 128, 4096, 500000.0),
              (8, 2, 128, 2048, 500000.0), (8, 1, 128, 4096, 500000.0)]  # the last spreads over 8 XCDs
    atts, ropes, caches = [], [], []
    try:
        for i, (nh, nkv, hd, sl, th) in enumerate(shapes):
            att = HipAttention(nh, nkv, hd, sl, rope_theta=th)
            atts.append(att)
            att.kv_fill_normal(0x5A + i, 1.0 / np.sqrt(hd))
            ropes.append(_packed_rope(att, torch))
            k0, v0 = att.kv_download(0, 0, 0, sl)
            caches.append((torch.from_numpy(k0).cuda(), torch.from_numpy(v0).cuda()))
        s = torch.cuda.Stream()
        g = torch.Generator(device=dev)
        g.manual_seed(77)
        for rnd in range(3):
            for i, (nh, nkv, hd, sl, th) in enumerate(shapes):
                pos = sl - 1 - 37 * rnd
                q = torch.randn(nh * hd, device=dev, generator=g) / np.sqrt(hd)
                k = torch.randn(nkv * hd, device=dev, generator=g) / np.sqrt(hd)
                v = torch.randn(nkv * hd, device=dev, generator=g) / np.sqrt(hd)
                out_n = torch.full((nh * hd,), float("nan"), device=dev)
                out_h = torch.full((nh * hd,), float("nan"), device=dev)
                kc, vc = caches[i]
                A.step_noalloc(nh, nkv, hd, sl, pos, ropes[i].data_ptr(), kc.data_ptr(), vc.data_ptr(),
                               q.data_ptr(), k.data_ptr(), v.data_ptr(), out_n.data_ptr(), s.cuda_stream)
                atts[i].step_async(0, pos, q.data_ptr(), k.data_ptr(), v.data_ptr(), out_h.data_ptr(),
                                   s.cuda_stream)
                s.synchronize()
                assert torch.equal(out_n, out_h), f"round {rnd}, shape {shapes[i]}, pos {pos}: outputs differ"
                assert torch.isfinite(out_n).all()
    finally:
        for att in atts:
            att.close()


_FIRST_CALL_CAPTURED = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1])
from leap_amd import attention as A
from leap_amd.attention import HipAttention

nh, nkv, hd, sl, pos = 32, 8, 128, 4096, 4095   # 64 chunks: the asymmetric merge
dev = torch.device("cuda:0")
with HipAttention(nh, nkv, hd, sl) as att:
    att.kv_fill_normal(0x4341, 1.0 / np.sqrt(hd))
    c, s_ = att.rope_download()
    rope = torch.from_numpy(np.stack([c, s_], axis=-1).reshape(-1).copy()).cuda()
    k0, v0 = att.kv_download(0, 0, 0, sl)
    kc, vc = torch.from_numpy(k0).cuda(), torch.from_numpy(v0).cuda()
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    q = torch.randn(nh * hd, device=dev, generator=g) / np.sqrt(hd)
    k = torch.randn(nkv * hd, device=dev, generator=g) / np.sqrt(hd)
    v = torch.randn(nkv * hd, device=dev, generator=g) / np.sqrt(hd)
    out_n = torch.full((nh * hd,), float("nan"), device=dev)
    out_h = torch.full((nh * hd,), float("nan"), device=dev)
    st = torch.cuda.Stream()
    att.step_async(0, pos, q.data_ptr(), k.data_ptr(), v.data_ptr(), out_h.data_ptr(), st.cuda_stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=st):  # the process's first no-alloc call
        A.step_noalloc(nh, nkv, hd, sl, pos, rope.data_ptr(), kc.data_ptr(), vc.data_ptr(), q.data_ptr(),
                       k.data_ptr(), v.data_ptr(), out_n.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for rep in range(4):
        out_n.fill_(float("nan"))
        x = torch.randn(1 << 20, device=dev)  # other eager work between the replays
        assert np.isfinite((x * 2).sum().item())
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_n, out_h), f"replay {rep} differs from the handle's step"
    # eager calls after the replays still agree (the counters were left at zero)
    out_n.fill_(float("nan"))
    A.step_noalloc(nh, nkv, hd, sl, pos, rope.data_ptr(), kc.data_ptr(), vc.data_ptr(), q.data_ptr(),
                   k.data_ptr(), v.data_ptr(), out_n.data_ptr(), st.cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out_n, out_h), "eager call after the replays differs"
print("FIRST_CALL_CAPTURED_OK", flush=True)
"""


def test_noalloc_first_call_under_graph_capture():
    """In a fresh process, the first call on the device is captured into a
    HIP graph (so the static workspace's one-time clear is not recorded
    into it) and replayed four times, with other eager work between; every
    replay and a later eager call equal the handle's step bitwise."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _FIRST_CALL_CAPTURED, root], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and "FIRST_CALL_CAPTURED_OK" in r.stdout, r.stdout[-2000:] + r.stderr[-2000:]
