"""Python binding of the C-ABI in include/leap_hip_attention.h.

``HipAttention`` owns one library handle: the device key/value caches in the
reference engine's layout and the RoPE table.  Its methods map one-to-one to
the C entry points and raise ``LeapError`` on a negative status, the way the
reference engine raises ``std::runtime_error`` around its layer step.

Host arrays are numpy float32; the ``*_async`` methods take raw device
addresses (integers, e.g. ``tensor.data_ptr()``) and a raw ``hipStream_t``
(``torch.cuda.Stream().cuda_stream``), so torch is plumbing only.
"""
from __future__ import annotations

import ctypes
import errno
import os

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libleap_hip_attention.so")
# the timeline build (the same sources compiled with LEAP_TIMELINE): decode
# launches record per-workgroup device-clock stamps (leap_hip_attention_timeline)
LIB_TL_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libleap_hip_attention_tl.so")

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.c_int
_P = ctypes.c_void_p
_B = ctypes.POINTER(ctypes.c_int8)

EXPORTS = (
    "leap_hip_attention_create", "leap_hip_attention_destroy", "leap_hip_attention_last_error",
    "leap_hip_attention_step", "leap_hip_attention_step_async",
    "leap_hip_attention_step_batched", "leap_hip_attention_step_batched_async",
    "leap_hip_attention_clear", "leap_hip_attention_kv_upload", "leap_hip_attention_kv_download",
    "leap_hip_attention_kv_fill_normal", "leap_hip_attention_rope_download",
    "leap_hip_attention_set_split", "leap_hip_attention_kv_device_ptr",
    "leap_hip_attention_set_layer_weights", "leap_hip_attention_block",
    "leap_hip_attention_block_async", "leap_hip_attention_set_layer_weights_q8",
    "leap_hip_attention_block_views_get", "leap_hip_attention_checkpoint_read",
    "leap_hip_attention_load_checkpoint", "leap_hip_attention_packet_header",
    "leap_hip_attention_packet_upload", "leap_hip_attention_packet_download",
    "leap_hip_attention_xcc_map", "leap_hip_attention_step_noalloc", "leap_hip_attention_floor_async",
    "leap_hip_attention_set_products", "leap_hip_attention_set_fold_helper", "leap_hip_attention_timeline",
)

PACKET_HEADER_BYTES = 8
FLAG_NO_REPLY, FLAG_NEED_REPLY = 0, 1


class Checkpoint(ctypes.Structure):
    """leap_hip_attention_checkpoint: a checkpoint file's header."""
    _fields_ = [(n, ctypes.c_int) for n in ("version", "dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads",
                                            "vocab_size", "seq_len", "shared_classifier", "group_size")] + \
               [(n, ctypes.c_longlong) for n in ("header_bytes", "attention_bytes", "file_bytes")]


class BlockViews(ctypes.Structure):
    """leap_hip_attention_block_views: device addresses of the sub-block's
    intermediates after the last block call."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("q", "k", "v", "att", "xq", "xs", "aq", "as_")]


class LeapError(RuntimeError):
    def __init__(self, code: int, msg: str):
        name = errno.errorcode.get(-code, str(code))
        super().__init__(f"{msg} ({name})")
        self.code = code


class Config(ctypes.Structure):
    _fields_ = [
        ("n_layers", _I), ("layer_begin", _I), ("layer_end", _I), ("n_heads", _I),
        ("n_kv_heads", _I), ("head_dim", _I), ("seq_len", _I), ("rope_theta", ctypes.c_float),
        ("max_batch", _I), ("device", _I),
    ]


_lib = None
_lib_tl = None


def load_library(path: str = LIB_PATH):
    """Load the HIP library; fails loudly when it has not been built."""
    global _lib
    if _lib is None:
        _lib = _open(path)
    return _lib


def load_timeline_library():
    """Load the timeline build of the library (its own copy of every entry
    point, with leap_hip_attention_timeline recording); handles made with it
    are passed `lib=` this library."""
    global _lib_tl
    if _lib_tl is None:
        _lib_tl = _open(LIB_TL_PATH)
    return _lib_tl


def _open(path: str):
    if not os.path.isfile(path):
        raise RuntimeError(f"{path} is missing: build it with `python -m leap_amd.build`")
    L = ctypes.CDLL(path)
    H = _P
    L.leap_hip_attention_create.argtypes = [ctypes.POINTER(Config), ctypes.POINTER(H)]
    L.leap_hip_attention_destroy.argtypes = [H]
    L.leap_hip_attention_last_error.argtypes = [H]
    L.leap_hip_attention_last_error.restype = ctypes.c_char_p
    L.leap_hip_attention_step.argtypes = [H, _I, _I, _F, _F, _F, _F]
    L.leap_hip_attention_step_async.argtypes = [H, _I, _I, _P, _P, _P, _P, _P]
    L.leap_hip_attention_step_batched.argtypes = [H, _I, _I, ctypes.POINTER(_I), _F, _F, _F, _F]
    L.leap_hip_attention_step_batched_async.argtypes = [H, _I, _I, _P, _I, ctypes.c_longlong, _P, _P,
                                                        _P, _P, _P]
    L.leap_hip_attention_clear.argtypes = [H]
    L.leap_hip_attention_kv_upload.argtypes = [H, _I, _I, _I, _I, _F, _F]
    L.leap_hip_attention_kv_download.argtypes = [H, _I, _I, _I, _I, _F, _F]
    L.leap_hip_attention_kv_fill_normal.argtypes = [H, ctypes.c_uint64, ctypes.c_float]
    L.leap_hip_attention_rope_download.argtypes = [H, _I, _I, _F, _F]
    L.leap_hip_attention_set_split.argtypes = [H, _I]
    L.leap_hip_attention_kv_device_ptr.argtypes = [H, _I, _I, ctypes.POINTER(_P),
                                                   ctypes.POINTER(_P)]
    L.leap_hip_attention_set_layer_weights.argtypes = [H, _I, _F, _F, _F, _F, _F]
    L.leap_hip_attention_block.argtypes = [H, _I, _I, _F]
    L.leap_hip_attention_block_async.argtypes = [H, _I, _I, _P, _P]
    L.leap_hip_attention_set_layer_weights_q8.argtypes = [H, _I, _I, _F] + [_B, _F] * 4
    L.leap_hip_attention_block_views_get.argtypes = [H, ctypes.POINTER(BlockViews)]
    L.leap_hip_attention_checkpoint_read.argtypes = [ctypes.c_char_p, ctypes.POINTER(Checkpoint)]
    L.leap_hip_attention_load_checkpoint.argtypes = [H, ctypes.c_char_p]
    _IP = ctypes.POINTER(_I)
    L.leap_hip_attention_packet_header.argtypes = [ctypes.c_char_p, ctypes.c_size_t, _I, _IP, _IP]
    L.leap_hip_attention_packet_upload.argtypes = [H, ctypes.c_char_p, ctypes.c_size_t, _P, _IP, _IP, _P]
    L.leap_hip_attention_packet_download.argtypes = [H, _P, _I, _I, _P, ctypes.c_size_t, _P]
    L.leap_hip_attention_xcc_map.argtypes = [_I, _I, ctypes.POINTER(_I)]
    L.leap_hip_attention_floor_async.argtypes = [H, _I, _I, _I, _P, _I, ctypes.c_longlong, _P]
    L.leap_hip_attention_set_products.argtypes = [H, _I]
    L.leap_hip_attention_set_fold_helper.argtypes = [H, _I]
    L.leap_hip_attention_step_noalloc.argtypes = [ctypes.POINTER(Config), _I] + [_P] * 8
    L.leap_hip_attention_timeline.argtypes = [_P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_longlong)]
    for name in EXPORTS:
        fn = getattr(L, name)
        if name != "leap_hip_attention_last_error":
            fn.restype = _I
    return L


def _fp(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _f32(a, n=None):
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    if n is not None and a.size != n:
        raise ValueError(f"expected {n} floats, got {a.size}")
    return a


def checkpoint_read(path) -> dict:
    """The header of a LEAP checkpoint file (no GPU needed)."""
    lib = load_library()
    c = Checkpoint()
    rc = lib.leap_hip_attention_checkpoint_read(os.fsencode(path), ctypes.byref(c))
    if rc != 0:
        raise LeapError(rc, f"{path}: {'cannot read' if rc == -errno.EIO else 'not a LEAP checkpoint'}")
    return {n: getattr(c, n) for n, _ in Checkpoint._fields_}


def xcc_map(n_wg: int, device: int = 0) -> np.ndarray:
    """The XCD each of n_wg workgroups of the decode kernel's size ran on."""
    lib = load_library()
    out = np.empty(n_wg, np.int32)
    rc = lib.leap_hip_attention_xcc_map(device, n_wg, out.ctypes.data_as(ctypes.POINTER(_I)))
    if rc != 0:
        raise LeapError(rc, lib.leap_hip_attention_last_error(None).decode())
    return out


def step_noalloc(n_heads, n_kv_heads, head_dim, seq_len, pos, rope_ptr, k_cache_ptr, v_cache_ptr, q_ptr,
                 k_ptr, v_ptr, out_ptr, stream=0, device=0):
    """leap_hip_attention_step_noalloc on caller-owned device buffers (raw
    addresses): no handle and no device allocation."""
    lib = load_library()
    cfg = Config(1, 0, 1, n_heads, n_kv_heads, head_dim, seq_len, 0.0, 1, device)
    rc = lib.leap_hip_attention_step_noalloc(ctypes.byref(cfg), pos, rope_ptr, k_cache_ptr, v_cache_ptr, q_ptr,
                                             k_ptr, v_ptr, out_ptr, stream)
    if rc != 0:
        raise LeapError(rc, lib.leap_hip_attention_last_error(None).decode())


def packet_header(packet: bytes, dim):
    """(pos, flags) of a stage packet, or None for a control packet (no GPU needed)."""
    pos, flags = _I(), _I()
    rc = load_library().leap_hip_attention_packet_header(packet, len(packet), dim, ctypes.byref(pos),
                                                         ctypes.byref(flags))
    if rc < 0:
        raise LeapError(rc, f"packet of {len(packet)} bytes is not 8 + 4*{dim}")
    return None if rc == 1 else (pos.value, flags.value)


class HipAttention:
    """One handle of the MI355X attention library (see the C header)."""

    def __init__(self, n_heads, n_kv_heads, head_dim, seq_len, n_layers=1, layer_begin=0,
                 layer_end=None, rope_theta=500000.0, max_batch=1, device=0, lib=None):
        self.lib = lib if lib is not None else load_library()
        self.cfg = Config(n_layers, layer_begin, n_layers if layer_end is None else layer_end,
                          n_heads, n_kv_heads, head_dim, seq_len, rope_theta, max_batch, device)
        self.n_heads, self.n_kv_heads, self.head_dim = n_heads, n_kv_heads, head_dim
        self.seq_len, self.max_batch = seq_len, max_batch
        self.q_dim, self.kv_dim = n_heads * head_dim, n_kv_heads * head_dim
        h = _P()
        rc = self.lib.leap_hip_attention_create(ctypes.byref(self.cfg), ctypes.byref(h))
        if rc != 0:
            raise LeapError(rc, self.lib.leap_hip_attention_last_error(None).decode())
        self.h = h

    # -- lifetime -----------------------------------------------------------
    def close(self):
        if getattr(self, "h", None):
            self.lib.leap_hip_attention_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc):
        if rc != 0:
            raise LeapError(rc, self.lib.leap_hip_attention_last_error(self.h).decode())

    # -- the step -----------------------------------------------------------
    def step(self, layer, pos, q, k_new, v_new):
        q, k, v = _f32(q, self.q_dim), _f32(k_new, self.kv_dim), _f32(v_new, self.kv_dim)
        out = np.empty(self.q_dim, np.float32)
        self._check(self.lib.leap_hip_attention_step(self.h, layer, pos, _fp(q), _fp(k), _fp(v),
                                                     _fp(out)))
        return out

    def step_async(self, layer, pos, q_ptr, k_ptr, v_ptr, out_ptr, stream=0):
        self._check(self.lib.leap_hip_attention_step_async(self.h, layer, pos, q_ptr, k_ptr,
                                                           v_ptr, out_ptr, stream))

    def step_batched(self, layer, pos, q, k_new, v_new):
        pos = np.ascontiguousarray(pos, dtype=np.int32).reshape(-1)
        n = pos.size
        q = _f32(q, n * self.q_dim)
        k, v = _f32(k_new, n * self.kv_dim), _f32(v_new, n * self.kv_dim)
        out = np.empty(n * self.q_dim, np.float32)
        self._check(self.lib.leap_hip_attention_step_batched(
            self.h, layer, n, pos.ctypes.data_as(ctypes.POINTER(_I)), _fp(q), _fp(k), _fp(v),
            _fp(out)))
        return out.reshape(n, self.q_dim)

    def step_batched_async(self, layer, n_seq, pos_ptr, max_pos, q_ptr, k_ptr, v_ptr, out_ptr,
                           stream=0, total_rows=0):
        """total_rows: sum of pos[i] + 1 if known on the host (sizes the split), else 0."""
        self._check(self.lib.leap_hip_attention_step_batched_async(
            self.h, layer, n_seq, pos_ptr, max_pos, total_rows, q_ptr, k_ptr, v_ptr, out_ptr,
            stream))

    # -- the attention sub-block (rmsnorm, q/k/v, attention, wo, residual) ---
    def set_layer_weights(self, layer, rms_att, wq, wk, wv, wo):
        """Upload one layer's weights, row-major as the reference holds them."""
        d, kv = self.q_dim, self.kv_dim
        arrs = (_f32(rms_att, d), _f32(wq, d * d), _f32(wk, kv * d), _f32(wv, kv * d), _f32(wo, d * d))
        self._check(self.lib.leap_hip_attention_set_layer_weights(self.h, layer, *(_fp(a) for a in arrs)))

    def set_layer_weights_q8(self, layer, group_size, rms_att, wq, wk, wv, wo):
        """Upload one layer's int8 weights: each of wq, wk, wv, wo is (int8
        values [d][n], float scales [d*n/group_size]) as the quantized engine
        holds them."""
        d, kv = self.q_dim, self.kv_dim
        arrs = [_f32(rms_att, d)]  # held here until the upload returns
        for (q, sc), rows in ((wq, d), (wk, kv), (wv, kv), (wo, d)):
            q = np.ascontiguousarray(q, np.int8).reshape(-1)
            if q.size != rows * d:
                raise ValueError(f"expected {rows * d} int8 values, got {q.size}")
            arrs += [q, _f32(sc, rows * d // group_size)]
        args = [a.ctypes.data_as(_B) if a.dtype == np.int8 else _fp(a) for a in arrs]
        self._check(self.lib.leap_hip_attention_set_layer_weights_q8(self.h, layer, group_size, *args))

    def load_checkpoint(self, path):
        """Upload every held layer's attention weights from a checkpoint file."""
        self._check(self.lib.leap_hip_attention_load_checkpoint(self.h, os.fsencode(path)))

    def block_views(self) -> dict:
        """Device addresses of the last block call's intermediates
        (q, k, v, att; xq, xs, aq, as_ with int8 weights, else None)."""
        bv = BlockViews()
        self._check(self.lib.leap_hip_attention_block_views_get(self.h, ctypes.byref(bv)))
        return {n: getattr(bv, n) for n, _ in BlockViews._fields_}

    def block(self, layer, pos, x):
        """x + Wo . attention(Wq/Wk/Wv . rmsnorm(x)); returns the new residual stream."""
        x = _f32(x, self.q_dim).copy()
        self._check(self.lib.leap_hip_attention_block(self.h, layer, pos, _fp(x)))
        return x

    def block_async(self, layer, pos, x_ptr, stream=0):
        self._check(self.lib.leap_hip_attention_block_async(self.h, layer, pos, x_ptr, stream))

    # -- stage hand-off -----------------------------------------------------
    def packet_upload(self, packet: bytes, x_ptr, stream=0):
        """Copy a data packet's x to device memory at x_ptr; returns (pos, flags),
        or None for a control packet.  stream 0: synchronous."""
        pos, flags = _I(), _I()
        rc = self.lib.leap_hip_attention_packet_upload(self.h, packet, len(packet), x_ptr, ctypes.byref(pos),
                                                       ctypes.byref(flags), stream)
        if rc == 1:
            return None
        self._check(rc)
        return pos.value, flags.value

    def packet_download(self, x_ptr, pos, flags) -> bytes:
        """The packet {pos, flags} + x (device memory at x_ptr), synchronously."""
        buf = ctypes.create_string_buffer(PACKET_HEADER_BYTES + 4 * self.q_dim)
        self._check(self.lib.leap_hip_attention_packet_download(self.h, x_ptr, pos, flags, buf, len(buf), None))
        return buf.raw

    # -- cache management ---------------------------------------------------
    def clear(self):
        self._check(self.lib.leap_hip_attention_clear(self.h))

    def kv_upload(self, seq, layer, pos_begin, k=None, v=None):
        rows = None
        if k is not None:
            k = _f32(k)
            rows = k.size // self.kv_dim
        if v is not None:
            v = _f32(v)
            rows = v.size // self.kv_dim if rows is None else rows
        if rows is None:
            return
        self._check(self.lib.leap_hip_attention_kv_upload(self.h, seq, layer, pos_begin,
                                                          pos_begin + rows, _fp(k), _fp(v)))

    def kv_download(self, seq, layer, pos_begin, pos_end):
        k = np.empty((pos_end - pos_begin, self.kv_dim), np.float32)
        v = np.empty_like(k)
        self._check(self.lib.leap_hip_attention_kv_download(self.h, seq, layer, pos_begin,
                                                            pos_end, _fp(k), _fp(v)))
        return k, v

    def kv_fill_normal(self, seed, scale):
        self._check(self.lib.leap_hip_attention_kv_fill_normal(self.h, seed, scale))

    def rope_download(self, pos_begin=0, pos_end=None):
        pos_end = self.seq_len if pos_end is None else pos_end
        c = np.empty((pos_end - pos_begin, self.head_dim // 2), np.float32)
        s = np.empty_like(c)
        self._check(self.lib.leap_hip_attention_rope_download(self.h, pos_begin, pos_end,
                                                              _fp(c), _fp(s)))
        return c, s

    def floor_async(self, kind, layer, n_seq, max_pos, total_rows, stream=0, pos_ptr=None):
        """Enqueue a floor launch of a step's shape: kind 1 launch only,
        kind 2 the bare K/V stream (measurement; writes nothing).  pos_ptr:
        device address of the n_seq positions, or None for every sequence
        at max_pos."""
        self._check(self.lib.leap_hip_attention_floor_async(self.h, kind, layer, n_seq, pos_ptr, max_pos,
                                                            total_rows, stream))

    def set_products(self, valu: bool):
        """Score and weighted-V products on the VALU (True) or the matrix cores."""
        self._check(self.lib.leap_hip_attention_set_products(self.h, 1 if valu else 0))

    def set_fold_helper(self, mode: int):
        """How a one-level merge's final fold is shared: 1 two workgroups (the
        default), 0 the last workgroup alone, 2 the fallback path (the helper
        gives up at once)."""
        self._check(self.lib.leap_hip_attention_set_fold_helper(self.h, mode))

    def set_split(self, chunk_positions):
        self._check(self.lib.leap_hip_attention_set_split(self.h, chunk_positions))

    def kv_device_ptr(self, seq, layer):
        k, v = _P(), _P()
        self._check(self.lib.leap_hip_attention_kv_device_ptr(self.h, seq, layer,
                                                              ctypes.byref(k), ctypes.byref(v)))
        return k.value, v.value
