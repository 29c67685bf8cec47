"""kuiperllama_amd -- MI355X (gfx950) backend for KuiperLLama's batch-1
token-generation loop.

Python surface over the C ABI of include/kuiper_hip.h:
  * ``DeviceArray``: device memory with numpy upload/download,
  * op-level kernels (``gemv_f32``, ``rmsnorm``, ``rope``, ``mha`` ...), one per
    reference kernel typedef,
  * ``synth_image``: reference-format model images with seeded weights,
  * ``Engine``: the fused decode step (``step``) and the greedy loop
    (``generate``).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import MODE_MULTI, MODE_PERSISTENT, KlError, check, lib
from .configs import ALL, BASELINE, TINY, Config

__all__ = [
    "ALL", "BASELINE", "TINY", "Config", "DeviceArray", "Engine", "KlError", "Stream",
    "MODE_MULTI", "MODE_PERSISTENT",
    "synth_image", "synth_normal", "quantize_q8", "device_count",
]


def device_count() -> int:
    n = C.c_int(0)
    if lib.kl_device_count(C.byref(n)) != 0:
        return 0
    return n.value


def device_name(dev: int = 0) -> str:
    buf = C.create_string_buffer(256)
    check(lib.kl_device_name(dev, buf, 256), "kl_device_name")
    return buf.value.decode()


class Stream:
    def __init__(self):
        h = C.c_void_p()
        check(lib.kl_stream_create(C.byref(h)), "kl_stream_create")
        self.handle = h

    def sync(self):
        check(lib.kl_stream_sync(self.handle), "kl_stream_sync")

    def close(self):
        if self.handle:
            lib.kl_stream_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceArray:
    """A device allocation holding a 1-D array of `dtype`."""

    def __init__(self, n: int, dtype=np.float32, zero: bool = False):
        self.dtype = np.dtype(dtype)
        self.n = int(n)
        self.nbytes = self.n * self.dtype.itemsize
        p = C.c_void_p()
        check(lib.kl_malloc(C.byref(p), max(self.nbytes, 1)), "kl_malloc")
        self.ptr = p
        if zero:
            check(lib.kl_memset_zero(self.ptr, max(self.nbytes, 1), None), "kl_memset_zero")
            check(lib.kl_device_sync(), "kl_device_sync")

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.size, a.dtype)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.size == self.n
        check(lib.kl_memcpy_h2d(self.ptr, a.ctypes.data, self.nbytes, None), "kl_memcpy_h2d")
        check(lib.kl_device_sync(), "kl_device_sync")

    def numpy(self) -> np.ndarray:
        out = np.empty(self.n, self.dtype)
        check(lib.kl_device_sync(), "kl_device_sync")
        check(lib.kl_memcpy_d2h(out.ctypes.data, self.ptr, self.nbytes, None), "kl_memcpy_d2h")
        return out

    def offset(self, elems: int) -> C.c_void_p:
        return C.c_void_p(self.ptr.value + elems * self.dtype.itemsize)

    def free(self):
        if self.ptr:
            lib.kl_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# Synthetic model images (host only).
# ---------------------------------------------------------------------------
def synth_image(cfg: Config, seed: int = 1234, stddev: float = 0.02, threads: int = 0) -> np.ndarray:
    spec = cfg.spec()
    size = C.c_int64(0)
    check(lib.kl_synth_image_size(C.byref(spec), C.byref(size)), "kl_synth_image_size")
    buf = np.empty(size.value, np.uint8)
    check(lib.kl_synth_image(C.byref(spec), seed, stddev, buf.ctypes.data, size.value, threads),
          "kl_synth_image")
    return buf


def synth_normal(seed: int, role: int, layer: int, n: int, stddev: float = 0.02) -> np.ndarray:
    out = np.empty(n, np.float32)
    check(lib.kl_synth_normal(seed, role, layer, stddev, out.ctypes.data, n), "kl_synth_normal")
    return out


def quantize_q8(w: np.ndarray, group_size: int = 64):
    w = np.ascontiguousarray(w, np.float32).ravel()
    q = np.empty(w.size, np.int8)
    s = np.empty(w.size // group_size, np.float32)
    check(lib.kl_quantize_q8(w.ctypes.data, w.size, group_size, q.ctypes.data, s.ctypes.data),
          "kl_quantize_q8")
    return q, s


def prompt_tokens(cfg: Config, n: int | None = None, seed: int = 4321) -> np.ndarray:
    """Seeded uniform prompt ids in [3, vocab)."""
    rng = np.random.default_rng(seed)
    return rng.integers(3, cfg.vocab, size=n or cfg.prompt_len, dtype=np.int64).astype(np.int32)


# ---------------------------------------------------------------------------
# Fused decode engine.
# ---------------------------------------------------------------------------
class Engine:
    """The decode step of model::LLama2Model / Qwen2Model / Qwen3Model on the GPU."""

    def __init__(self, image: np.ndarray, cfg: Config):
        self.cfg = cfg
        h = C.c_void_p()
        img = np.ascontiguousarray(image)
        check(lib.kl_engine_create(img.ctypes.data, img.nbytes, cfg.family, int(cfg.quant),
                                   C.byref(h)), "kl_engine_create")
        self.handle = h
        dims = (C.c_int32 * 10)()
        check(lib.kl_engine_dims(self.handle, dims), "kl_engine_dims")
        self.dims = list(dims)
        self.vocab = self.dims[7]

    def set_graph(self, enable: bool):
        check(lib.kl_engine_set_graph(self.handle, int(enable)), "kl_engine_set_graph")

    def set_mode(self, mode: int):
        """_lib.MODE_PERSISTENT (one cooperative launch per token) or
        _lib.MODE_MULTI (5 kernels per layer, graph-replayed)."""
        check(lib.kl_engine_set_mode(self.handle, int(mode)), "kl_engine_set_mode")

    @property
    def mode(self) -> int:
        m = C.c_int(-1)
        check(lib.kl_engine_get_mode(self.handle, C.byref(m)), "kl_engine_get_mode")
        return m.value

    def launch_shape(self):
        """(workgroups, threads, dynamic LDS bytes) of the persistent step."""
        w, t, l = C.c_int32(0), C.c_int32(0), C.c_int64(0)
        check(lib.kl_engine_launch_shape(self.handle, C.byref(w), C.byref(t), C.byref(l)),
              "kl_engine_launch_shape")
        return w.value, t.value, l.value

    def step(self, token: int, pos: int, want_logits: bool = True):
        nxt = C.c_int32(-1)
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        check(lib.kl_engine_step(self.handle, int(token), int(pos), C.byref(nxt),
                                 logits.ctypes.data if want_logits else None), "kl_engine_step")
        return nxt.value, logits

    def generate(self, prompt, n_new: int):
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_new, np.int32)
        ms = C.c_float(0.0)
        check(lib.kl_engine_generate(self.handle, p.ctypes.data, p.size, n_new, out.ctypes.data,
                                     C.byref(ms)), "kl_engine_generate")
        return out, ms.value

    def prefill(self, prompt, want_logits: bool = True):
        """Batched prefill of the whole prompt (kl_engine_prefill): returns
        (next token, logits of the last position, device ms)."""
        p = np.ascontiguousarray(prompt, np.int32)
        nxt = C.c_int32(-1)
        logits = np.empty(self.vocab, np.float32) if want_logits else None
        ms = C.c_float(0.0)
        check(lib.kl_engine_prefill(self.handle, p.ctypes.data, p.size, C.byref(nxt),
                                    logits.ctypes.data if want_logits else None, C.byref(ms)),
              "kl_engine_prefill")
        return nxt.value, logits, ms.value

    def set_prefill(self, enable: bool):
        """Whether generate() runs the prompt through the batched prefill."""
        check(lib.kl_engine_set_prefill(self.handle, int(enable)), "kl_engine_set_prefill")

    def bench(self, prompt, n_warmup: int, n_timed: int):
        """Prompt + n_warmup untimed decode steps, then n_timed decode steps
        timed with HIP events on the engine's stream.  Returns (tokens, ms)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_warmup + n_timed, np.int32)
        ms = C.c_float(0.0)
        check(lib.kl_engine_bench(self.handle, p.ctypes.data, p.size, n_warmup, n_timed,
                                  out.ctypes.data, C.byref(ms)), "kl_engine_bench")
        return out, ms.value

    KERNEL_KINDS = ("embed", "qkv", "attn", "wo", "w13", "w2", "cls", "step")

    def profile(self, token: int, pos0: int, steps: int) -> dict:
        """Average device time per kernel kind over `steps` eager decode steps
        (HIP events between consecutive launches on the engine's stream)."""
        avg = (C.c_float * 8)()
        cnt = (C.c_int32 * 8)()
        check(lib.kl_engine_profile(self.handle, int(token), int(pos0), int(steps), avg, cnt),
              "kl_engine_profile")
        return {k: (float(avg[i]), int(cnt[i])) for i, k in enumerate(self.KERNEL_KINDS)}

    def trace_step(self, token: int, pos: int) -> np.ndarray:
        """Device-time trace of one persistent step: int64 ticks of the 100 MHz
        clock, shape [slots, workgroups] (see kl_engine_trace_step)."""
        ns, nw = C.c_int32(0), C.c_int32(0)
        rc = lib.kl_engine_trace_step(self.handle, int(token), int(pos), None, 0, C.byref(ns),
                                      C.byref(nw))
        if rc not in (0, _lib.KL_EWORKSPACE):
            check(rc, "kl_engine_trace_step")
        out = np.zeros((ns.value, nw.value), np.uint64)
        check(lib.kl_engine_trace_step(self.handle, int(token), int(pos), out.ctypes.data,
                                       out.size, C.byref(ns), C.byref(nw)), "kl_engine_trace_step")
        return out.astype(np.int64)

    def kv_row(self, layer: int, pos: int, which_v: bool) -> np.ndarray:
        lg, kc, vc = C.c_void_p(), C.c_void_p(), C.c_void_p()
        check(lib.kl_engine_buffers(self.handle, C.byref(lg), C.byref(kc), C.byref(vc)),
              "kl_engine_buffers")
        base = vc if which_v else kc
        kvd, S = self.dims[2], self.dims[8]
        off = ((layer * S) + pos) * kvd * 4
        out = np.empty(kvd, np.float32)
        check(lib.kl_device_sync(), "kl_device_sync")
        check(lib.kl_memcpy_d2h(out.ctypes.data, C.c_void_p(base.value + off), kvd * 4, None),
              "kl_memcpy_d2h")
        return out

    def weight_bytes(self) -> int:
        b = C.c_int64(0)
        check(lib.kl_engine_weight_bytes(self.handle, C.byref(b)), "kl_engine_weight_bytes")
        return b.value

    def close(self):
        if getattr(self, "handle", None):
            lib.kl_engine_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
