"""ctypes binding of the CPU parity oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the kuiperllama_amd package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

ROPE_INTERLEAVED, ROPE_HALF = 0, 1


def build(force: bool = False) -> None:
    cmd = ["make", "-C", HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        build()
    return C.CDLL(LIB_PATH)


lib = _load()
_i, _p, _f = C.c_int, C.c_void_p, C.c_float
_sigs = {
    "or_set_threads": (None, [_i]),
    "or_get_threads": (_i, []),
    "or_gemv_f32": (None, [_p, _p, _p, _i, _i, _f]),
    "or_gemv_q8": (None, [_p, _p, _p, _p, _i, _i, _i]),
    "or_gemv_q8_scalar": (None, [_p, _p, _p, _p, _i, _i, _i]),
    "or_quantize_q8": (None, [_p, C.c_int64, _i, _p, _p]),
    "or_dequant_q8": (None, [_p, _p, C.c_int64, _i, _p]),
    "or_rmsnorm": (None, [_p, _p, _p, _i, _f]),
    "or_rmsnorm_rows": (None, [_p, _p, _p, _i, _i, _f]),
    "or_sincos_table": (None, [_i, _i, _f, _p, _p]),
    "or_rope": (None, [_i, _i, _i, _i, _p, _p, _i, _p, _p]),
    "or_softmax": (None, [_p, _i]),
    "or_mha": (None, [_i, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p]),
    "or_scale": (None, [_f, _p, _i]),
    "or_scale_sum": (None, [_p, _p, _p, _i, _i, _i]),
    "or_swiglu": (None, [_p, _p, _p, _i]),
    "or_add": (None, [_p, _p, _p, _i]),
    "or_embedding": (_i, [_p, _i, _p, _i, _i, _p]),
    "or_argmax": (C.c_int64, [_p, C.c_int64]),
    "or_model_open": (_p, [_p, C.c_size_t, _i, _i, C.c_char_p, _i]),
    "or_model_close": (None, [_p]),
    "or_model_dims": (None, [_p, _p]),
    "or_model_step": (_i, [_p, C.c_int32, C.c_int32, _p]),
    "or_model_prompt": (_i, [_p, _p, _i, C.c_int32, _p]),
    "or_model_generate": (_i, [_p, _p, _i, _i, _p]),
    "or_model_kv_row": (None, [_p, _i, _i, _i, _p]),
}
for _n, (_r, _a) in _sigs.items():
    _fn = getattr(lib, _n)
    _fn.restype = _r
    _fn.argtypes = _a


def _f32(a):
    return np.ascontiguousarray(a, np.float32)


def set_threads(n: int):
    lib.or_set_threads(n)


def gemv_f32(x, W, scale=1.0):
    x, W = _f32(x), _f32(W)
    rows, cols = W.shape
    y = np.empty(rows, np.float32)
    lib.or_gemv_f32(x.ctypes.data, W.ctypes.data, y.ctypes.data, rows, cols, scale)
    return y


def gemv_q8(x, q, s, rows, cols, gs, scalar=False):
    x = _f32(x)
    q = np.ascontiguousarray(q, np.int8)
    s = _f32(s)
    y = np.empty(rows, np.float32)
    fn = lib.or_gemv_q8_scalar if scalar else lib.or_gemv_q8
    fn(x.ctypes.data, q.ctypes.data, s.ctypes.data, y.ctypes.data, rows, cols, gs)
    return y


def quantize_q8(w, gs):
    w = _f32(w).ravel()
    q = np.empty(w.size, np.int8)
    s = np.empty(w.size // gs, np.float32)
    lib.or_quantize_q8(w.ctypes.data, w.size, gs, q.ctypes.data, s.ctypes.data)
    return q, s


def dequant_q8(q, s, gs):
    q = np.ascontiguousarray(q, np.int8)
    s = _f32(s)
    out = np.empty(q.size, np.float32)
    lib.or_dequant_q8(q.ctypes.data, s.ctypes.data, q.size, gs, out.ctypes.data)
    return out


def rmsnorm(x, w, eps):
    x, w = _f32(x), _f32(w)
    y = np.empty_like(x)
    lib.or_rmsnorm(x.ctypes.data, w.ctypes.data, y.ctypes.data, x.size, eps)
    return y


def rmsnorm_rows(x, w, eps):
    x, w = _f32(x), _f32(w)
    rows, n = x.shape
    y = np.empty_like(x)
    lib.or_rmsnorm_rows(x.ctypes.data, w.ctypes.data, y.ctypes.data, rows, n, eps)
    return y


def sincos_table(hd, seq_len, theta):
    s = np.empty(seq_len * hd, np.float32)
    c = np.empty(seq_len * hd, np.float32)
    lib.or_sincos_table(hd, seq_len, theta, s.ctypes.data, c.ctypes.data)
    return s, c


def rope(style, dim, kv_dim, hd, q, k, pos, sin_t, cos_t):
    q, k = _f32(q).copy(), _f32(k).copy()
    sin_t, cos_t = _f32(sin_t), _f32(cos_t)
    lib.or_rope(style, dim, kv_dim, hd, q.ctypes.data, k.ctypes.data, pos, sin_t.ctypes.data,
                cos_t.ctypes.data)
    return q, k


def softmax(x):
    x = _f32(x).copy()
    lib.or_softmax(x.ctypes.data, x.size)
    return x


def mha(pos, head_num, layer, seq_len, kv_dim, kv_mul, hd, q, kcache, vcache):
    q, kcache, vcache = _f32(q), _f32(kcache), _f32(vcache)
    out = np.empty(head_num * hd, np.float32)
    score = np.empty(head_num * seq_len, np.float32)
    lib.or_mha(pos, head_num, layer, seq_len, kv_dim, kv_mul, hd, out.ctypes.data, q.ctypes.data,
               score.ctypes.data, kcache.ctypes.data, vcache.ctypes.data)
    return out


def scale(s, x):
    y = _f32(x).copy()
    lib.or_scale(s, y.ctypes.data, y.size)
    return y


def scale_sum(value, sc, out, pos, size, stride):
    """out[d] += sc[i] * value[i * stride + d] for i <= pos (value flat)."""
    v = _f32(value)
    s = _f32(sc)
    o = _f32(out).copy()
    lib.or_scale_sum(v.ctypes.data, s.ctypes.data, o.ctypes.data, pos, size, stride)
    return o


def swiglu(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib.or_swiglu(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def add(a, b):
    a, b = _f32(a), _f32(b)
    out = np.empty_like(a)
    lib.or_add(a.ctypes.data, b.ctypes.data, out.ctypes.data, a.size)
    return out


def embedding(tokens, table):
    tokens = np.ascontiguousarray(tokens, np.int32)
    table = _f32(table)
    vocab, dim = table.shape
    out = np.zeros((tokens.size, dim), np.float32)
    rc = lib.or_embedding(tokens.ctypes.data, tokens.size, table.ctypes.data, vocab, dim,
                          out.ctypes.data)
    if rc != 0:
        raise ValueError("token id out of range")
    return out


def argmax(x):
    x = _f32(x)
    return int(lib.or_argmax(x.ctypes.data, x.size))


class Model:
    """The reference decode step on the CPU, over a reference-format image."""

    def __init__(self, image: np.ndarray, family: int, quant: bool):
        self._image = np.ascontiguousarray(image)  # must outlive the handle
        err = C.create_string_buffer(256)
        h = lib.or_model_open(self._image.ctypes.data, self._image.nbytes, family, int(quant), err,
                              256)
        if not h:
            raise ValueError(err.value.decode())
        self.handle = h
        d = np.empty(10, np.int32)
        lib.or_model_dims(self.handle, d.ctypes.data)
        self.dims = [int(v) for v in d]
        self.vocab = self.dims[7]

    def step(self, token: int, pos: int) -> np.ndarray:
        logits = np.empty(self.vocab, np.float32)
        rc = lib.or_model_step(self.handle, int(token), int(pos), logits.ctypes.data)
        if rc != 0:
            raise ValueError(f"or_model_step rc={rc}")
        return logits

    def prompt(self, tokens, pos0: int = 0) -> np.ndarray:
        """Prompt tokens at positions pos0.. in one batched pass, bitwise equal
        to step() on each position in turn; the last position's logits."""
        t = np.ascontiguousarray(tokens, np.int32)
        logits = np.empty(self.vocab, np.float32)
        rc = lib.or_model_prompt(self.handle, t.ctypes.data, t.size, int(pos0), logits.ctypes.data)
        if rc != 0:
            raise ValueError(f"or_model_prompt rc={rc}")
        return logits

    def generate(self, prompt, n_new: int) -> np.ndarray:
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_new, np.int32)
        n = lib.or_model_generate(self.handle, p.ctypes.data, p.size, n_new, out.ctypes.data)
        if n != n_new:
            raise ValueError(f"or_model_generate returned {n}")
        return out

    def kv_row(self, layer: int, pos: int, which_v: bool) -> np.ndarray:
        out = np.empty(self.dims[2], np.float32)
        lib.or_model_kv_row(self.handle, layer, pos, int(which_v), out.ctypes.data)
        return out

    def close(self):
        if getattr(self, "handle", None):
            lib.or_model_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
