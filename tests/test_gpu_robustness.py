"""Device placement, allocation failure and stream-ordering rules of the
library, on the GPU, through the C ABI.

- The split-K merge keeps a (sequence, KV head) group's partials in one XCD's
  L2, which needs every workgroup id equal modulo 8 on the same XCD; create
  checks that with a probe launch, and the probe's map is checked here too.
- A create that runs out of device memory part-way returns -ENOMEM and frees
  what it had already allocated; a normal create then succeeds.
- After _async steps on a caller stream that the caller synchronised, the
  handle's own calls (clear, host-pointer step) see their results, and clear
  zeroes the cache rows and the merge counters.
"""
import errno

import numpy as np
import pytest

from leap_amd import attention as A
from leap_amd.attention import HipAttention, LeapError
from oracle import oracle as O
from tests.helpers import REL_TOL, assert_close, normal, rng_for

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _needs_gpu(hip_device):
    return hip_device


@pytest.mark.parametrize("n_wg", [8, 512, 4096])
def test_xcc_map_is_periodic_in_eight(n_wg):
    xcc = A.xcc_map(n_wg)
    assert xcc.shape == (n_wg,)
    assert ((xcc >= 0) & (xcc < 16)).all()
    first = xcc[:min(8, n_wg)]
    for i in range(8, n_wg):
        assert xcc[i] == first[i % 8], f"workgroup {i} on XCD {xcc[i]}, workgroup {i % 8} on {first[i % 8]}"


def test_oversize_create_returns_enomem_and_frees_everything():
    """create fails with -ENOMEM and frees what it had allocated: when its
    first allocation (the key cache) already exceeds free memory, so that
    nothing is held, and when the key cache fits and the value cache of the
    same size does not (the key cache sized at just over half of free
    memory, held only until the value cache's allocation fails)."""
    import torch
    torch.cuda.synchronize()
    free0, total = torch.cuda.mem_get_info()
    per_seq = 32 * 131072 * 1024 * 4  # one 16 GiB slab per cache
    for frac, what in ((1.0, "first allocation"), (0.52, "second allocation")):
        max_batch = int(frac * free0 // per_seq) + 1
        assert max_batch * per_seq <= free0 or frac == 1.0
        assert 2 * max_batch * per_seq > free0
        with pytest.raises(LeapError) as ei:
            HipAttention(32, 8, 128, 131072, n_layers=32, max_batch=max_batch)
        assert ei.value.code == -errno.ENOMEM, f"{what}: {ei.value}"
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert abs(free1 - free0) <= 64 << 20, f"{what}: free memory {free0} before, {free1} after the failed create"
    # a normal handle still works
    rng = rng_for(91)
    with HipAttention(8, 2, 128, 64) as att:
        q, k, v = normal(rng, 8 * 128, 128), normal(rng, 256, 128), normal(rng, 256, 128)
        out = att.step(0, 0, q, k, v)
    assert np.array_equal(out.reshape(8, 128), np.repeat(v.reshape(2, 1, 128), 4, axis=1).reshape(8, 128))


def test_async_on_a_caller_stream_then_clear_and_step():
    import torch
    nh, nkv, hd, T = 32, 8, 128, 4096
    rng = rng_for(92)
    with HipAttention(nh, nkv, hd, T) as att:
        att.kv_fill_normal(92, 1.0 / np.sqrt(hd))
        dev = torch.device("cuda:0")
        s = torch.cuda.Stream()
        q = torch.randn(nh * hd, device=dev) / np.sqrt(hd)
        k = torch.randn(nkv * hd, device=dev) / np.sqrt(hd)
        v = torch.randn(nkv * hd, device=dev) / np.sqrt(hd)
        out = torch.empty(nh * hd, device=dev)
        with torch.cuda.stream(s):
            for pos in (4095, 2047, 63, 4095):  # multi-chunk merges on the caller's stream
                att.step_async(0, pos, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), s.cuda_stream)
        s.synchronize()
        att.clear()
        kz, vz = att.kv_download(0, 0, 0, T)
        assert not kz.any() and not vz.any(), "clear left non-zero cache rows"
        kr, vr = normal(rng, (3000, nkv * hd), hd), normal(rng, (3000, nkv * hd), hd)
        att.kv_upload(0, 0, 0, kr, vr)
        qh, kh, vh = normal(rng, nh * hd, hd), normal(rng, nkv * hd, hd), normal(rng, nkv * hd, hd)
        got = att.step(0, 3000, qh, kh, vh)
        orc = O.Oracle(1, nh, nkv, hd, T)
        orc.key_cache[0, :3000] = kr
        orc.value_cache[0, :3000] = vr
        want, _ = orc.step(0, 3000, qh, kh, vh)
        assert_close(got, want, rel=REL_TOL)
        k_slot, v_slot = att.kv_download(0, 0, 3000, 3001)
        assert np.array_equal(k_slot[0], orc.key_cache[0, 3000])
        assert np.array_equal(v_slot[0], orc.value_cache[0, 3000])


@pytest.mark.parametrize("kind", [1, 2])
def test_floor_launches_write_nothing(kind):
    """The measurement launches (launch floor, bare stream floor) with a real
    step's shape leave the cache and the step's output untouched."""
    import torch
    nh, nkv, hd, T = 32, 8, 128, 2048
    with HipAttention(nh, nkv, hd, T, n_layers=2, max_batch=3) as att:
        att.kv_fill_normal(93, 1.0 / np.sqrt(hd))
        k0, v0 = att.kv_download(2, 1, 0, T)
        s = torch.cuda.Stream()
        att.floor_async(kind, 1, 1, T - 1, T, s.cuda_stream)
        att.floor_async(kind, 1, 3, 1000, 3 * 1001, s.cuda_stream)
        pos = torch.tensor([1000, 17, T - 1], dtype=torch.int32, device="cuda:0")
        att.floor_async(kind, 1, 3, T - 1, 1001 + 18 + T, s.cuda_stream, pos_ptr=pos.data_ptr())
        # short contexts, whose steps run 2-wave workgroups (the floors too)
        att.floor_async(kind, 1, 1, 20, 21, s.cuda_stream)
        att.floor_async(kind, 1, 1, 255, 256, s.cuda_stream)
        s.synchronize()
        k1, v1 = att.kv_download(2, 1, 0, T)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
        with pytest.raises(LeapError):
            att.floor_async(3, 1, 1, T - 1, T, s.cuda_stream)
        with pytest.raises(LeapError):
            att.floor_async(kind, 1, 4, T - 1, T, s.cuda_stream)
        with pytest.raises(LeapError):  # positions not 4-byte aligned
            att.floor_async(kind, 1, 1, T - 1, T, s.cuda_stream, pos_ptr=pos.data_ptr() + 2)
    # a step that spreads its groups over the XCDs (one KV head, 4 MiB of
    # rows) has no floor grid: refused rather than measured on another grid
    with HipAttention(8, 1, 128, 8192) as att:
        s = torch.cuda.Stream()
        att.floor_async(kind, 0, 1, 1999, 2000, s.cuda_stream)  # 2 MiB of rows: one XCD, no spread
        with pytest.raises(LeapError) as ei:
            att.floor_async(kind, 0, 1, 8191, 8192, s.cuda_stream)
        assert "spread" in str(ei.value)
    # four KV heads of 8 q heads at 24 MiB: as 4 groups the step would spread,
    # as the 8 twin launch groups it runs it does not, and the floor follows
    with HipAttention(32, 4, 64, 12288) as att:
        s = torch.cuda.Stream()
        att.floor_async(kind, 0, 1, 12287, 12288, s.cuda_stream)
        s.synchronize()
        s.synchronize()


@pytest.mark.parametrize("q8", [False, True])
def test_block_floor_launches_write_nothing(q8):
    """Floor kind 3, the sub-block's floor (both projections streaming their
    weights alone around the attention's bare K/V stream), for fp32 and
    int8 weights: runs, changes neither the cache nor the block's buffers,
    and refuses a layer without weights or a batch."""
    import torch
    from tests.helpers import block_inputs
    nh, nkv, hd, T, gs = 16, 4, 128, 512, 64
    dim = nh * hd
    rng = rng_for(94, int(q8))
    with HipAttention(nh, nkv, hd, T, n_layers=2) as att:
        att.kv_fill_normal(94, 1.0 / np.sqrt(hd))
        _, rms, *wf = block_inputs(rng, dim, nkv * hd)
        if q8:
            from oracle import oracle as O
            att.set_layer_weights_q8(0, gs, rms, *(O.quantize_weight(w, gs) for w in wf))
        else:
            att.set_layer_weights(0, rms, *wf)
        k0, v0 = att.kv_download(0, 0, 0, T)
        s = torch.cuda.Stream()
        for _ in range(3):
            att.floor_async(3, 0, 1, T - 1, T, s.cuda_stream)
        s.synchronize()
        k1, v1 = att.kv_download(0, 0, 0, T)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1)
        with pytest.raises(LeapError):  # no weights at layer 1
            att.floor_async(3, 1, 1, T - 1, T, s.cuda_stream)
        with pytest.raises(LeapError):  # one sequence only
            att.floor_async(3, 0, 2, T - 1, 2 * T, s.cuda_stream)
