"""ORACLE — test infrastructure only.

ctypes bindings for the CPU restatement (``liboracle_attn.so``, built from
``attn_oracle.c``) and for the driver around the reference's own code
(``_ref/libleap_ref.so``, built from ``ref_harness.cpp`` plus the reference's
``src/inference/FloatTransformer.cpp``; ``_ref/libleap_ref_q8.so``, built from
``ref_harness_q8.cpp`` plus ``src/inference/QuantizedTransformer.cpp``;
``_ref/libleap_ref_ckpt.so``, built from ``ref_harness_ckpt.cpp`` plus the
reference's checkpoint factory and both engines).  Only the tests, the smoke check and
the CPU-baseline leg of the benchmark import this module; the product package
``leap_amd`` never does.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle_attn.so")
# LEAP_REF_VARIANT=v4 selects the reference timing libraries built for an
# AVX-512 target (the CPU-baseline leg sets it on AVX-512 hosts).
_VARIANT = "_v4" if os.environ.get("LEAP_REF_VARIANT") == "v4" else ""
REF_SO = os.path.join(HERE, "_ref", f"libleap_ref{_VARIANT}.so")
REF_Q8_SO = os.path.join(HERE, "_ref", f"libleap_ref_q8{_VARIANT}.so")
REF_CKPT_SO = os.path.join(HERE, "_ref", "libleap_ref_ckpt.so")
REF_SRC = "/root/reference/src/inference"

_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.c_int
_B = ctypes.POINTER(ctypes.c_int8)


def build(ref: bool | None = None) -> None:
    """Compile the restatement, and the reference driver when the reference
    sources are present (they are not on machines that only run prebuilt
    libraries)."""
    targets = ["all"]
    if ref is None:
        ref = os.path.isfile(os.path.join(REF_SRC, "FloatTransformer.cpp"))
    if ref:
        targets.append("ref")
    subprocess.run(["make", "-s", "-B", "-C", HERE] + targets, check=True)


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _bp(a: np.ndarray):
    assert a.dtype == np.int8 and a.flags.c_contiguous
    return a.ctypes.data_as(_B)


_lib = None
_ref = None
_ref_q8 = None
_ref_ckpt = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.isfile(ORACLE_SO):
            raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run oracle.build())")
        L = ctypes.CDLL(ORACLE_SO)
        L.oracle_rope_table.argtypes = [_I, _I, ctypes.c_float, _F, _F]
        L.oracle_rope_table.restype = None
        step_args = [_I, _I, _I, _I, _I, _I, _F, _F, _F, _F, _F, _F, _F, _F, _F]
        L.oracle_attention_step.argtypes = step_args
        L.oracle_attention_step.restype = _I
        L.oracle_attention_step_mutant.argtypes = [_I] + step_args
        L.oracle_attention_step_mutant.restype = _I
        L.oracle_clear.argtypes = [_F, _F, ctypes.c_size_t]
        L.oracle_rmsnorm.argtypes = [_F, _F, _F, _I]
        L.oracle_rmsnorm.restype = None
        L.oracle_matmul.argtypes = [_F, _F, _F, _I, _I]
        L.oracle_matmul.restype = None
        L.oracle_quantize.argtypes = [_F, _I, _I, _B, _F]
        L.oracle_quantize.restype = None
        L.oracle_matmul_q8.argtypes = [_F, _B, _F, _B, _F, _I, _I, _I]
        L.oracle_matmul_q8.restype = None
        L.oracle_set_threads.argtypes = [_I]
        L.oracle_max_threads.restype = _I
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.isfile(REF_SO)


def ref():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"reference driver missing: {REF_SO}")
        L = ctypes.CDLL(REF_SO)
        L.leapref_rope_table.argtypes = [_I, _I, _I, _F, _F]
        L.leapref_rope_table.restype = _I
        L.leapref_run_layer.argtypes = [_I] * 7 + [_F] * 10
        L.leapref_run_layer.restype = _I
        L.leapref_clear_check.argtypes = [_I] * 5
        L.leapref_clear_check.restype = ctypes.c_long
        L.leapref_rmsnorm.argtypes = [_F, _F, _F, _I]
        L.leapref_rmsnorm.restype = _I
        L.leapref_matmul.argtypes = [_F, _F, _F, _I, _I]
        L.leapref_matmul.restype = _I
        L.leapref_block.argtypes = [_I] * 7 + [_F] * 8
        L.leapref_block.restype = _I
        L.leapref_block_timer_create.argtypes = [_I] * 5 + [_F] * 7 + [_I]
        L.leapref_block_timer_create.restype = ctypes.c_void_p
        L.leapref_block_timer_run.argtypes = [ctypes.c_void_p, _I, _F, _I]
        L.leapref_block_timer_run.restype = ctypes.c_double
        L.leapref_block_timer_destroy.argtypes = [ctypes.c_void_p]
        L.leapref_block_timer_destroy.restype = None
        _ref = L
    return _ref


def ref_q8_available() -> bool:
    return os.path.isfile(REF_Q8_SO)


def ref_q8():
    global _ref_q8
    if _ref_q8 is None:
        if not ref_q8_available():
            raise RuntimeError(f"reference driver missing: {REF_Q8_SO}")
        L = ctypes.CDLL(REF_Q8_SO)
        L.leapref_q8_quantize.argtypes = [_F, _I, _I, _B, _F]
        L.leapref_q8_quantize.restype = _I
        L.leapref_q8_matmul.argtypes = [_F, _B, _F, _B, _F, _I, _I, _I]
        L.leapref_q8_matmul.restype = _I
        L.leapref_q8_block.argtypes = [_I] * 8 + [_F, _B, _F, _B, _F, _B, _F, _B, _F, _F, _F, _F]
        L.leapref_q8_block.restype = _I
        L.leapref_q8_block_timer_create.argtypes = [_I] * 6 + [_F, _B, _F, _B, _F, _B, _F, _B, _F, _F, _F, _I]
        L.leapref_q8_block_timer_create.restype = ctypes.c_void_p
        L.leapref_q8_block_timer_run.argtypes = [ctypes.c_void_p, _I, _F, _I]
        L.leapref_q8_block_timer_run.restype = ctypes.c_double
        L.leapref_q8_block_timer_destroy.argtypes = [ctypes.c_void_p]
        L.leapref_q8_block_timer_destroy.restype = None
        _ref_q8 = L
    return _ref_q8


def ref_ckpt_available() -> bool:
    return os.path.isfile(REF_CKPT_SO)


def ref_ckpt_run_layer(path, layer, pos, x, key_cache, value_cache):
    """The reference engine built from the checkpoint at `path` by its own
    factory runs run_layer(layer, pos, x); returns (kind, x after, key cache,
    value cache) with kind 1 for fp32, 2 for int8."""
    kc = np.array(key_cache, np.float32, copy=True)
    vc = np.array(value_cache, np.float32, copy=True)
    xo = np.array(x, np.float32, copy=True).reshape(-1)
    kind = _ckpt_lib().leapref_ckpt_run_layer(os.fsencode(path), layer, pos, _fp(xo), _fp(kc), _fp(vc))
    if kind < 0:
        raise RuntimeError("reference checkpoint run failed")
    return kind, xo, kc, vc


def _ckpt_lib():
    global _ref_ckpt
    if _ref_ckpt is None:
        if not ref_ckpt_available():
            raise RuntimeError(f"reference driver missing: {REF_CKPT_SO}")
        L = ctypes.CDLL(REF_CKPT_SO)
        L.leapref_ckpt_run_layer.argtypes = [ctypes.c_char_p, _I, _I, _F, _F, _F]
        L.leapref_ckpt_run_layer.restype = _I
        _U = ctypes.c_char_p
        _IP = ctypes.POINTER(_I)
        L.leapref_ckpt_master.argtypes = [ctypes.c_char_p, _I, _I, _IP, _IP, _IP, _U, _I, ctypes.c_void_p]
        L.leapref_ckpt_master.restype = _I
        L.leapref_ckpt_worker.argtypes = [ctypes.c_char_p, _I, _I, _I, _I, _U, ctypes.c_void_p]
        L.leapref_ckpt_worker.restype = _I
        _ref_ckpt = L
    return _ref_ckpt


def _ints(a):
    a = np.ascontiguousarray(a, np.int32)
    return a, a.ctypes.data_as(ctypes.POINTER(_I))


def ref_ckpt_master(path, split, dim, tokens, pos, flags, replies=()):
    """The reference engine from `path` as a pipeline master that runs layers
    [0, split): forward(tokens[i], pos[i], flags[i]) for each i, with the
    packets that the forwards asking for a reply receive given in `replies`.
    Returns the packets it sent (bytes each)."""
    n = len(tokens)
    nb = PACKET_HEADER_BYTES + 4 * dim
    t, tp = _ints(tokens)
    p, pp = _ints(pos)
    f, fp = _ints(flags)
    rep = b"".join(replies)
    out = ctypes.create_string_buffer(n * nb)
    got = _ckpt_lib().leapref_ckpt_master(os.fsencode(path), split, n, tp, pp, fp, rep, len(replies), out)
    if got < 0:
        raise RuntimeError("reference master run failed")
    return [out.raw[i * nb:(i + 1) * nb] for i in range(got)]


def ref_ckpt_worker(path, split, end, is_tail, dim, packets):
    """The reference engine from `path` as a pipeline worker for layers
    [split, end), fed `packets` (bytes each) through worker_loop; returns
    the packets it forwarded."""
    nb = PACKET_HEADER_BYTES + 4 * dim
    out = ctypes.create_string_buffer(max(1, len(packets)) * nb)
    got = _ckpt_lib().leapref_ckpt_worker(os.fsencode(path), split, end, int(is_tail), len(packets),
                                          b"".join(packets), out)
    if got < 0:
        raise RuntimeError("reference worker run failed")
    return [out.raw[i * nb:(i + 1) * nb] for i in range(got)]


# ---- the stage hand-off (a restatement, pinned against the two above) ------------

PACKET_HEADER_BYTES = 8
FLAG_NO_REPLY, FLAG_NEED_REPLY = 0, 1
CONTROL_MAGIC = 0xC0DE


def packet_pack(pos, flags, x) -> bytes:
    """PacketHeader {int pos; int flags} then the dim floats of x, as forward
    sends them (Transformer.h:25-28; FloatTransformer.cpp:775-778)."""
    import struct
    return struct.pack("<ii", pos, flags) + np.ascontiguousarray(x, np.float32).tobytes()


def packet_unpack(packet: bytes, dim):
    """(pos, flags, x) of a data packet, as worker_loop reads it
    (FloatTransformer.cpp:925-926)."""
    import struct
    assert len(packet) == PACKET_HEADER_BYTES + 4 * dim
    pos, flags = struct.unpack_from("<ii", packet)
    return pos, flags, np.frombuffer(packet, np.float32, dim, PACKET_HEADER_BYTES).copy()


def packet_forwards(is_tail, flags) -> bool:
    """Whether a worker forwards the packet after its layers: every stage but
    the tail does, and the tail only when a reply is wanted
    (FloatTransformer.cpp:937-939)."""
    return (not is_tail) or flags == FLAG_NEED_REPLY


def rope_table(seq_len: int, head_dim: int, theta: float = 500000.0):
    """FloatTransformer.cpp:56-72 -> (cos, sin), each [seq_len, head_dim/2] fp32."""
    c = np.empty((seq_len, head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().oracle_rope_table(seq_len, head_dim, theta, _fp(c), _fp(s))
    return c, s


def _c32(a):
    return np.ascontiguousarray(a, np.float32)


def rmsnorm(x, w):
    """FloatTransformer.cpp:79-213 -> w * x / sqrt(mean(x^2) + 1e-5)."""
    x, w = _c32(x).reshape(-1), _c32(w).reshape(-1)
    o = np.empty_like(x)
    lib().oracle_rmsnorm(_fp(o), _fp(x), _fp(w), x.size)
    return o


def matmul(w, x):
    """FloatTransformer.cpp:240-382: W (d, n) @ x (n,) -> (d,)."""
    w = _c32(w)
    x = _c32(x).reshape(-1)
    d, n = w.shape
    o = np.empty(d, np.float32)
    lib().oracle_matmul(_fp(o), _fp(x), _fp(w), n, d)
    return o


def quantize(x, gs: int):
    """QuantizedTransformer.cpp:338-357 -> (int8 values [n], scales [ceil(n/gs)])."""
    x = _c32(x).reshape(-1)
    q = np.empty(x.size, np.int8)
    sc = np.empty(-(-x.size // gs), np.float32)
    lib().oracle_quantize(_fp(x), x.size, gs, _bp(q), _fp(sc))
    return q, sc


def quantize_weight(w, gs: int):
    """A weight matrix [d, n] (n a multiple of gs) in the quantized engine's
    format: int8 values [d, n] and one scale per group of a row, [d * n / gs]
    (the QuantizedTensor layout, QuantizedTransformer.h:9-12)."""
    w = _c32(w)
    assert w.ndim == 2 and w.shape[1] % gs == 0
    q, sc = quantize(w.reshape(-1), gs)
    return q.reshape(w.shape), sc


def matmul_q8(wq, ws, xq, xs, gs: int):
    """QuantizedTransformer.cpp:359-652: int8 W [d, n] with group scales ws,
    int8 x [n] with group scales xs -> float [d]."""
    wq = np.ascontiguousarray(wq, np.int8)
    d, n = wq.shape
    o = np.empty(d, np.float32)
    lib().oracle_matmul_q8(_fp(o), _bp(np.ascontiguousarray(xq, np.int8)), _fp(_c32(xs)), _bp(wq),
                           _fp(_c32(ws)), n, d, gs)
    return o


class Oracle:
    """One sequence's reference-layout cache plus the restated step.

    ``key_cache``/``value_cache`` are ``[n_layers, seq_len, kv_dim]`` fp32,
    exactly the reference's RunState layout (FloatTransformer.cpp:50-51).
    """

    def __init__(self, n_layers, n_heads, n_kv_heads, head_dim, seq_len, theta=500000.0,
                 rope=None):
        self.n_layers, self.n_heads, self.n_kv_heads = n_layers, n_heads, n_kv_heads
        self.head_dim, self.seq_len, self.theta = head_dim, seq_len, theta
        self.kv_dim = n_kv_heads * head_dim
        self.key_cache = np.zeros((n_layers, seq_len, self.kv_dim), np.float32)
        self.value_cache = np.zeros_like(self.key_cache)
        if rope is None:
            rope = rope_table(seq_len, head_dim, theta)
        self.cos, self.sin = (np.ascontiguousarray(r, np.float32) for r in rope)

    def step(self, layer, pos, q, k_new, v_new, mutant: int = 0):
        """Returns (out [n_heads*hd], q rotated).  Updates the cache slot."""
        q = np.array(q, np.float32, copy=True).reshape(-1)
        k_new = np.ascontiguousarray(k_new, np.float32).reshape(-1)
        v_new = np.ascontiguousarray(v_new, np.float32).reshape(-1)
        att = np.empty(self.n_heads * (pos + 1), np.float32)
        out = np.empty(self.n_heads * self.head_dim, np.float32)
        args = (self.n_heads, self.n_kv_heads, self.head_dim, self.seq_len, layer, pos,
                _fp(self.key_cache), _fp(self.value_cache), _fp(self.cos), _fp(self.sin),
                _fp(q), _fp(k_new), _fp(v_new), _fp(att), _fp(out))
        if mutant:
            rc = lib().oracle_attention_step_mutant(mutant, *args)
        else:
            rc = lib().oracle_attention_step(*args)
        if rc != 0:
            raise ValueError("oracle_attention_step rejected its arguments")
        return out, q

    def clear(self):
        lib().oracle_clear(_fp(self.key_cache), _fp(self.value_cache), self.key_cache.size)

    def block(self, layer, pos, x, rms_att, wq, wk, wv, wo):
        """run_layer up to the attention residual (FloatTransformer.cpp:394-683):
        returns x + wo . attention(q, k, v) with q, k, v = W . rmsnorm(x)."""
        x = _c32(x).reshape(-1)
        xb = rmsnorm(x, rms_att)
        q, k, v = matmul(wq, xb), matmul(wk, xb), matmul(wv, xb)
        out, _ = self.step(layer, pos, q, k, v)
        return x + matmul(wo, out)

    def block_q8(self, layer, pos, x, rms_att, wq, wk, wv, wo, gs, stages: bool = False):
        """The quantized engine's run_layer up to the attention residual
        (QuantizedTransformer.cpp:654-...): xb = rmsnorm(x), quantized per
        group; q, k, v = W8A8 matmuls; the fp32 attention step; its output
        quantized; x + wo . that.  Each weight is (int8 [d, n], scales).
        Returns x_out, or with stages=True a dict of every intermediate."""
        x = _c32(x).reshape(-1)
        xb = rmsnorm(x, rms_att)
        xq, xs = quantize(xb, gs)
        q, k, v = (matmul_q8(w[0], w[1], xq, xs, gs) for w in (wq, wk, wv))
        att, _ = self.step(layer, pos, q, k, v)
        aq, as_ = quantize(att, gs)
        x_out = x + matmul_q8(wo[0], wo[1], aq, as_, gs)
        if not stages:
            return x_out
        return dict(xb=xb, xq=xq, xs=xs, q=q, k=k, v=v, att=att, aq=aq, as_=as_, x_out=x_out)


def ref_run_layer(dim, n_heads, n_kv_heads, n_layers, seq_len, layer, pos, x, wq, wk, wv,
                  key_cache, value_cache):
    """Run the reference's run_layer; returns dict with q_pre, k_pre, v_pre,
    q_rot, out and the updated caches (copies)."""
    hd = dim // n_heads
    kv_dim = n_kv_heads * hd
    kc = np.array(key_cache, np.float32, copy=True)
    vc = np.array(value_cache, np.float32, copy=True)
    outs = {k: np.empty(n, np.float32) for k, n in
            (("q_pre", dim), ("k_pre", kv_dim), ("v_pre", kv_dim), ("q_rot", dim), ("out", dim))}
    rc = ref().leapref_run_layer(
        dim, n_heads, n_kv_heads, n_layers, seq_len, layer, pos,
        _fp(np.ascontiguousarray(x, np.float32)), _fp(np.ascontiguousarray(wq, np.float32)),
        _fp(np.ascontiguousarray(wk, np.float32)), _fp(np.ascontiguousarray(wv, np.float32)),
        _fp(kc), _fp(vc), _fp(outs["q_pre"]), _fp(outs["k_pre"]), _fp(outs["v_pre"]),
        _fp(outs["q_rot"]), _fp(outs["out"]))
    if rc != 0:
        raise RuntimeError("reference run_layer failed")
    outs["key_cache"], outs["value_cache"] = kc, vc
    return outs


def ref_rmsnorm(x, w):
    x, w = _c32(x).reshape(-1), _c32(w).reshape(-1)
    o = np.empty_like(x)
    ref().leapref_rmsnorm(_fp(o), _fp(x), _fp(w), x.size)
    return o


def ref_matmul(w, x):
    w = _c32(w)
    x = _c32(x).reshape(-1)
    d, n = w.shape
    o = np.empty(d, np.float32)
    ref().leapref_matmul(_fp(o), _fp(x), _fp(w), n, d)
    return o


def ref_block(dim, n_heads, n_kv_heads, n_layers, seq_len, layer, pos, x, rms_att, wq, wk, wv, wo,
              key_cache, value_cache):
    """The reference's run_layer with the given attention weights and a zero
    FFN: returns (x after the layer = x + wo . attention, key cache, value cache)."""
    kc = np.array(key_cache, np.float32, copy=True)
    vc = np.array(value_cache, np.float32, copy=True)
    xo = np.array(x, np.float32, copy=True).reshape(-1)
    rc = ref().leapref_block(dim, n_heads, n_kv_heads, n_layers, seq_len, layer, pos,
                             *(_fp(_c32(a)) for a in (rms_att, wq, wk, wv, wo)), _fp(kc), _fp(vc), _fp(xo))
    if rc != 0:
        raise RuntimeError("reference block failed")
    return xo, kc, vc


def ref_q8_quantize(x, gs: int):
    x = _c32(x).reshape(-1)
    q = np.empty(x.size, np.int8)
    sc = np.empty(-(-x.size // gs), np.float32)
    if ref_q8().leapref_q8_quantize(_fp(x), x.size, gs, _bp(q), _fp(sc)) != 0:
        raise RuntimeError("reference quantize failed")
    return q, sc


def ref_q8_matmul(wq, ws, xq, xs, gs: int):
    wq = np.ascontiguousarray(wq, np.int8)
    d, n = wq.shape
    o = np.empty(d, np.float32)
    if ref_q8().leapref_q8_matmul(_fp(o), _bp(np.ascontiguousarray(xq, np.int8)), _fp(_c32(xs)), _bp(wq),
                                  _fp(_c32(ws)), n, d, gs) != 0:
        raise RuntimeError("reference q8 matmul failed")
    return o


def ref_q8_block(dim, n_heads, n_kv_heads, n_layers, seq_len, gs, layer, pos, x, rms_att, wq, wk, wv, wo,
                 key_cache, value_cache):
    """The quantized reference's run_layer with the given attention weights
    (each (int8 [d, n], scales)) and a zero FFN: returns (x after the layer,
    key cache, value cache)."""
    kc = np.array(key_cache, np.float32, copy=True)
    vc = np.array(value_cache, np.float32, copy=True)
    xo = np.array(x, np.float32, copy=True).reshape(-1)
    ws = []
    for w in (wq, wk, wv, wo):
        ws += [_bp(np.ascontiguousarray(w[0], np.int8)), _fp(_c32(w[1]))]
    rc = ref_q8().leapref_q8_block(dim, n_heads, n_kv_heads, n_layers, seq_len, gs, layer, pos,
                                   _fp(_c32(rms_att)), *ws, _fp(kc), _fp(vc), _fp(xo))
    if rc != 0:
        raise RuntimeError("reference q8 block failed")
    return xo, kc, vc


class RefBlockTimer:
    """The reference's own run_layer (oracle/_ref) on an engine of n_layers
    layers that each hold the given attention weights (fp32 arrays, or (int8,
    scales) pairs with group size gs), a zero FFN of negligible size, and
    cache rows [0, rows) from key_rows/value_rows; each call runs the next
    layer.  The CPU baseline of the sub-block."""

    def __init__(self, dim, n_heads, n_kv_heads, seq_len, rms_att, wq, wk, wv, wo, key_rows, value_rows,
                 gs=None, n_layers=1):
        self._keep = [_c32(rms_att), _c32(key_rows), _c32(value_rows)]
        rows = key_rows.shape[0]
        if gs is None:
            self.lib = ref()
            ws = [_c32(w) for w in (wq, wk, wv, wo)]
            self._keep += ws
            self.h = self.lib.leapref_block_timer_create(dim, n_heads, n_kv_heads, seq_len, n_layers,
                                                         _fp(self._keep[0]),
                                                         *[_fp(w) for w in ws], _fp(self._keep[1]),
                                                         _fp(self._keep[2]), rows)
            self._run, self._free = self.lib.leapref_block_timer_run, self.lib.leapref_block_timer_destroy
        else:
            self.lib = ref_q8()
            args = []
            for w in (wq, wk, wv, wo):
                q, sc = np.ascontiguousarray(w[0], np.int8), _c32(w[1])
                self._keep += [q, sc]
                args += [_bp(q), _fp(sc)]
            self.h = self.lib.leapref_q8_block_timer_create(dim, n_heads, n_kv_heads, seq_len, n_layers, gs,
                                                            _fp(self._keep[0]), *args, _fp(self._keep[1]),
                                                            _fp(self._keep[2]), rows)
            self._run, self._free = self.lib.leapref_q8_block_timer_run, self.lib.leapref_q8_block_timer_destroy
        if not self.h:
            raise RuntimeError("reference block timer failed")

    def run(self, pos, x, iters):
        """Seconds per run_layer(l, pos, x) over `iters` calls, l cycling (x is updated)."""
        assert x.dtype == np.float32 and x.flags.c_contiguous
        return self._run(self.h, pos, _fp(x), iters)

    def close(self):
        if self.h:
            self._free(self.h)
            self.h = None


def ref_rope_table(dim, n_heads, seq_len):
    hd = dim // n_heads
    c = np.empty((seq_len, hd // 2), np.float32)
    s = np.empty_like(c)
    if ref().leapref_rope_table(dim, n_heads, seq_len, _fp(c), _fp(s)) != 0:
        raise RuntimeError("reference rope table failed")
    return c, s
