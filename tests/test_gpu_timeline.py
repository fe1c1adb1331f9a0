"""The timeline build of the library (libleap_hip_attention_tl.so, the same
sources compiled with LEAP_TIMELINE): its decode launches compute the same
results as the library's, bit for bit, and record one row of device-clock
stamps per workgroup whose order follows the kernel's phases."""
import ctypes

import numpy as np
import pytest

from leap_amd import attention as A
from tests.helpers import normal, rng_for

pytestmark = pytest.mark.gpu

SLOTS, WGS, WORDS = 64, 2048, 16
START, PROLOGUE, SCORED, LOOP_END, COMBINED, STORED, DRAINED, COUNTED = range(8)
FOLD_ISSUED, FOLD_LOADED, FOLDED, SUB_COUNTED, SUB_FOLDED, END, ROLE = range(8, 15)
SINGLE, FINAL, HELPER, SUB = 1, 2, 4, 8


def _ring(lib):
    ring = np.zeros(SLOTS * WGS * WORDS, np.uint64)
    n = ctypes.c_longlong(0)
    assert lib.leap_hip_attention_timeline(ring.ctypes.data, ring.nbytes, ctypes.byref(n)) == 0
    return ring.reshape(SLOTS, WGS, WORDS).astype(np.int64), n.value


@pytest.mark.parametrize("nh,nkv,hd,T,n_wg", [
    (32, 8, 128, 4096, 512),  # 64 one-pass chunks per KV head: the asymmetric merge with the fold helper
    (24, 8, 128, 1000, 128),  # 16 chunks per KV head: the one-level merge
    (8, 4, 64, 50, 8),        # one chunk per KV head: the output written directly (4 of 8 workgroups idle)
    (32, 4, 64, 50, 16),      # 8 q heads per KV head: four launch groups of 2 per cache head, 16 workgroups
])
def test_timeline_build_matches_and_stamps_in_order(hip_device, nh, nkv, hd, T, n_wg):
    import torch
    tl = A.load_timeline_library()
    rng = rng_for(91, nh, T)
    k_rows = normal(rng, (T - 1, nkv * hd), hd)
    v_rows = normal(rng, (T - 1, nkv * hd), hd)
    q = torch.from_numpy(normal(rng, nh * hd, hd)).cuda()
    k = torch.from_numpy(normal(rng, nkv * hd, hd)).cuda()
    v = torch.from_numpy(normal(rng, nkv * hd, hd)).cuda()
    outs, caches = [], []
    for lib in (A.load_library(), tl):
        with A.HipAttention(nh, nkv, hd, T, lib=lib) as att:
            att.kv_upload(0, 0, 0, k_rows, v_rows)
            out = torch.zeros(nh * hd, device="cuda:0")
            s = torch.cuda.Stream()
            att.step_async(0, T - 1, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), s.cuda_stream)
            torch.cuda.synchronize()
            outs.append(out.cpu().numpy())
            caches.append(att.kv_download(0, 0, T - 1, T))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(caches[0][0], caches[1][0]) and np.array_equal(caches[0][1], caches[1][1])

    ring, launches = _ring(tl)
    assert launches >= 1
    t = ring[(launches - 1) % SLOTS, :n_wg]
    assert (t[:, START] > 0).all() and (t[:, END] >= t[:, START]).all()
    assert (ring[(launches - 1) % SLOTS, n_wg:, START] == 0).all()  # no workgroup beyond the grid
    # launch groups: small launches run 4 or 8 q heads per KV head as two
    # groups of 2 or 4 per cache head (up to 8 and 24 MiB of K/V rows), 8 as
    # four groups of 2 (up to 2 MiB over four groups)
    limit = {4: 8 << 20, 8: 24 << 20}.get(nh // nkv, -1)
    kv_bytes = T * nkv * hd * 8
    if nh // nkv == 8 and nkv == 4 and kv_bytes <= 2 << 20:
        groups = 4 * nkv
    else:
        groups = 2 * nkv if kv_bytes <= limit else nkv
    # workgroup ids equal modulo 8 are one KV head's chunks; ids of the
    # missing heads (fewer than 8) leave at once
    idle = (np.arange(n_wg) % 8) >= groups
    assert (t[idle, PROLOGUE] == 0).all()
    t = t[~idle]
    # every workgroup of a chunk passes the prologue, the main loop, the
    # combine and the store, in that order
    for a, b in ((START, PROLOGUE), (PROLOGUE, SCORED), (SCORED, LOOP_END), (LOOP_END, COMBINED),
                 (COMBINED, STORED), (STORED, END)):
        assert (t[:, a] > 0).all() and (t[:, b] >= t[:, a]).all(), (a, b)
    role = t[:, ROLE] & 0xFF
    if len(t) == groups:
        assert (role == SINGLE).all()
        return
    # one final fold per KV head (with the helper's share on top), after every
    # arrival of its group counted in
    assert ((role & FINAL) != 0).sum() == groups
    for g in range(groups):
        ids = np.arange(g, n_wg, 8)
        fin = ids[(role[ids] & FINAL) != 0]
        assert len(fin) == 1
        f = t[fin[0]]
        assert f[COUNTED] >= t[ids, DRAINED].max() or (t[ids, SUB_COUNTED] > 0).any()
        assert f[FOLD_ISSUED] >= f[COUNTED] and f[FOLD_LOADED] >= f[FOLD_ISSUED] and f[FOLDED] >= f[FOLD_LOADED]
