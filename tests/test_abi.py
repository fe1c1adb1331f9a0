"""The C-ABI library: loads, exports what the header declares, rejects bad
arguments with negative errno codes (host-side checks, no GPU needed)."""
import ctypes
import errno
import os
import re

import pytest

from leap_amd import attention as A
from tests.conftest import gpu_available

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "leap_hip_attention.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(leap_hip_attention_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = A.load_library()
    names = _declared()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(names) == set(A.EXPORTS)


def test_timeline_build_exports_the_same_symbols():
    tl = A.load_timeline_library()
    missing = [n for n in _declared() if not hasattr(tl, n)]
    assert not missing, missing


def test_timeline_is_refused_by_the_production_library():
    lib = A.load_library()
    buf = (ctypes.c_ulonglong * 16)()
    n = ctypes.c_longlong(-1)
    rc = lib.leap_hip_attention_timeline(ctypes.addressof(buf), ctypes.sizeof(buf), ctypes.byref(n))
    assert rc == -errno.ENOTSUP
    assert "timeline" in lib.leap_hip_attention_last_error(None).decode()
    assert n.value == -1


def _create(**kw):
    lib = A.load_library()
    base = dict(n_layers=2, layer_begin=0, layer_end=2, n_heads=8, n_kv_heads=2, head_dim=128,
                seq_len=64, rope_theta=500000.0, max_batch=1, device=0)
    base.update(kw)
    cfg = A.Config(*[base[f] for f, _ in A.Config._fields_])
    h = ctypes.c_void_p()
    rc = lib.leap_hip_attention_create(ctypes.byref(cfg), ctypes.byref(h))
    msg = lib.leap_hip_attention_last_error(None).decode()
    if rc == 0:
        lib.leap_hip_attention_destroy(h)
    return rc, msg


@pytest.mark.parametrize("kw,fragment", [
    (dict(n_kv_heads=3), "multiple"),
    (dict(n_heads=0), "multiple"),
    (dict(head_dim=96), "head_dim"),
    (dict(head_dim=128, n_heads=32, n_kv_heads=1), "head_dim"),  # 32 q heads per kv head
    (dict(head_dim=128, n_heads=24, n_kv_heads=4), "head_dim"),  # 6 q heads per kv head
    (dict(layer_begin=1, layer_end=1), "layer range"),
    (dict(layer_end=3), "layer range"),
    (dict(seq_len=0), "seq_len"),
    (dict(max_batch=0), "max_batch"),
])
def test_create_rejects_bad_config(kw, fragment):
    rc, msg = _create(**kw)
    assert rc == -errno.EINVAL
    assert fragment in msg


def test_create_without_gpu_reports_enodev():
    if gpu_available():
        pytest.skip("a GPU is present")
    rc, msg = _create()
    assert rc == -errno.ENODEV and "device" in msg


def test_null_arguments():
    lib = A.load_library()
    assert lib.leap_hip_attention_create(None, None) == -errno.EINVAL
    assert lib.leap_hip_attention_destroy(None) == 0
    assert lib.leap_hip_attention_step(None, 0, 0, None, None, None, None) == -errno.EINVAL
    assert lib.leap_hip_attention_clear(None) == -errno.EINVAL
    assert lib.leap_hip_attention_kv_upload(None, 0, 0, 0, 1, None, None) == -errno.EINVAL
    assert lib.leap_hip_attention_set_split(None, 64) == -errno.EINVAL
    assert lib.leap_hip_attention_set_products(None, 1) == -errno.EINVAL
    assert lib.leap_hip_attention_set_fold_helper(None, 1) == -errno.EINVAL
    assert lib.leap_hip_attention_floor_async(None, 1, 0, 1, None, 0, 1, None) == -errno.EINVAL


def test_python_binding_raises_leaperror():
    with pytest.raises(A.LeapError) as ei:
        A.HipAttention(n_heads=8, n_kv_heads=3, head_dim=128, seq_len=16)
    assert ei.value.code == -errno.EINVAL


def test_xcc_map_argument_checks():
    lib = A.load_library()
    buf = (ctypes.c_int * 8)()
    assert lib.leap_hip_attention_xcc_map(0, 0, buf) == -errno.EINVAL
    assert lib.leap_hip_attention_xcc_map(0, 8, None) == -errno.EINVAL
    if not gpu_available():
        assert lib.leap_hip_attention_xcc_map(0, 8, buf) == -errno.ENODEV


def test_step_noalloc_argument_checks():
    """The allocation-free step rejects bad shapes and arguments before it
    touches a device (through the Python binding, so its signature is
    exercised too)."""
    with pytest.raises(A.LeapError) as ei:
        A.step_noalloc(8, 3, 128, 64, 0, 16, 16, 16, 16, 16, 16, 16)
    assert ei.value.code == -errno.EINVAL and "multiple" in str(ei.value)
    with pytest.raises(A.LeapError) as ei:
        A.step_noalloc(8, 2, 96, 64, 0, 16, 16, 16, 16, 16, 16, 16)
    assert ei.value.code == -errno.EINVAL and "head_dim" in str(ei.value)
    with pytest.raises(A.LeapError) as ei:
        A.step_noalloc(8, 2, 128, 64, 64, 16, 16, 16, 16, 16, 16, 16)
    assert ei.value.code == -errno.EINVAL and "pos" in str(ei.value)
    with pytest.raises(A.LeapError) as ei:
        A.step_noalloc(8, 2, 128, 64, 0, 16, 16, 16, 0, 16, 16, 16)
    assert ei.value.code == -errno.EINVAL and "NULL" in str(ei.value)
    with pytest.raises(A.LeapError) as ei:
        A.step_noalloc(8, 2, 128, 64, 0, 20, 16, 16, 16, 16, 16, 16)
    assert ei.value.code == -errno.EINVAL and "aligned" in str(ei.value)
    with pytest.raises(A.LeapError) as ei:  # 128 heads of 128: 4.7 MB of records
        A.step_noalloc(128, 16, 128, 64, 0, 16, 16, 16, 16, 16, 16, 16)
    assert ei.value.code == -errno.EINVAL and "workspace" in str(ei.value)
    if not gpu_available():
        with pytest.raises(A.LeapError) as ei:
            A.step_noalloc(8, 2, 128, 64, 0, 16, 16, 16, 16, 16, 16, 16)
        assert ei.value.code == -errno.ENODEV
