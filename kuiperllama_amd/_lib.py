"""ctypes binding of libkuiper_hip.so (the C ABI declared in include/kuiper_hip.h).

The library is built in-tree (kuiperllama_amd/lib/) by ``build.py``; there is
no fallback: if it is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes as C
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libkuiper_hip.so")

KL_OK = 0
KL_EINVAL = -1
KL_ENOMEM = -2
KL_EFORMAT = -3
KL_EUNSUPP = -4
KL_ETOKEN = -5
KL_EWORKSPACE = -6
KL_EDEVICE = -7
MODE_PERSISTENT, MODE_MULTI = 0, 1

FAMILY_LLAMA2, FAMILY_LLAMA3, FAMILY_QWEN2, FAMILY_QWEN3 = 0, 1, 2, 3
ROPE_INTERLEAVED, ROPE_HALF = 0, 1


class KlError(RuntimeError):
    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what} failed: {code} ({_errstr(code)})")


class ModelSpec(C.Structure):
    _fields_ = [
        ("family", C.c_int32),
        ("dim", C.c_int32),
        ("q_dim", C.c_int32),
        ("hidden_dim", C.c_int32),
        ("layers", C.c_int32),
        ("heads", C.c_int32),
        ("kv_heads", C.c_int32),
        ("vocab", C.c_int32),
        ("seq_len", C.c_int32),
        ("tied", C.c_int32),
        ("group_size", C.c_int32),
        ("norm_stddev", C.c_float),
    ]


def _load() -> C.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is not built; run __graft_entry__.build() (make -C kuiperllama_amd/csrc)"
        )
    return C.CDLL(LIB_PATH)


lib = _load()

_i, _p, _sz, _f = C.c_int, C.c_void_p, C.c_size_t, C.c_float
_i32p, _i64p, _fp = C.POINTER(C.c_int32), C.POINTER(C.c_int64), C.POINTER(C.c_float)

_SIGS = {
    "kl_error_string": (C.c_char_p, [_i]),
    "kl_device_count": (_i, [C.POINTER(_i)]),
    "kl_set_device": (_i, [_i]),
    "kl_device_name": (_i, [_i, C.c_char_p, _i]),
    "kl_malloc": (_i, [C.POINTER(_p), _sz]),
    "kl_free": (_i, [_p]),
    "kl_host_alloc": (_i, [C.POINTER(_p), _sz]),
    "kl_host_free": (_i, [_p]),
    "kl_memcpy_h2d": (_i, [_p, _p, _sz, _p]),
    "kl_memcpy_d2h": (_i, [_p, _p, _sz, _p]),
    "kl_memcpy_d2d": (_i, [_p, _p, _sz, _p]),
    "kl_memset_zero": (_i, [_p, _sz, _p]),
    "kl_stream_create": (_i, [C.POINTER(_p)]),
    "kl_stream_destroy": (_i, [_p]),
    "kl_stream_sync": (_i, [_p]),
    "kl_device_sync": (_i, []),
    "kl_event_create": (_i, [C.POINTER(_p)]),
    "kl_event_destroy": (_i, [_p]),
    "kl_event_record": (_i, [_p, _p]),
    "kl_event_elapsed_ms": (_i, [_p, _p, _fp]),
    "kl_gemv_f32": (_i, [_p, _p, _p, _i, _i, _f, _p]),
    "kl_gemv_q8": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "kl_dequant_q8": (_i, [_p, _p, C.c_int64, _i, _p, _p]),
    "kl_rmsnorm": (_i, [_p, _p, _p, _i, _f, _p]),
    "kl_rmsnorm_rows": (_i, [_p, _p, _p, _i, _i, _f, _p]),
    "kl_sincos_table": (_i, [_i, _i, _f, _p, _p]),
    "kl_rope": (_i, [_i, _i, _i, _i, _p, _p, _i, _p, _p, _p]),
    "kl_mha_workspace_size": (_i, [_i, _i, _i, _i, C.POINTER(_sz)]),
    "kl_mha": (_i, [_i, _i, _i, _i, _i, _i, _i, _p, _p, _p, _sz, _p, _p, _p]),
    "kl_mha_noalloc_max_bytes": (_sz, []),
    "kl_mha_noalloc": (_i, [_i, _i, _i, _i, _i, _i, _i, _p, _p, _p, _p, _p]),
    "kl_gemm_f32": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _i, _p]),
    "kl_gemm_f32_grouped": (_i, [_p, _i, _i, _i, _i, _p, _p, _p, _p, _p, _p, _i, _p]),
    "kl_gemm_f32_splitk": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _i, _i, _p, _sz, _p]),
    "kl_gemm_q8": (_i, [_p, _p, _p, _i, _p, _i, _i, _i, _i, _i, _p, _i, _i, _p, _sz, _p]),
    "kl_split_bf16x3_bytes": (_sz, [_i, _i]),
    "kl_split_bf16x3": (_i, [_p, _i, _i, _i, _p, _p]),
    "kl_gemm_x6": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _i, _p, _sz, _p]),
    "kl_gemm_x6w": (_i, [_p, _p, _i, _p, _i, _i, _i, _i, _p, _i, _p, _sz, _p]),
    "kl_x6_weight_planes": (_i, [_p, _i, _i, C.POINTER(C.c_int), _p]),
    "kl_q8s_packed_bytes": (_sz, [_i, _i, _i]),
    "kl_q8s_pack": (_i, [_p, _p, _i, _i, _i, _p, _p]),
    "kl_gemm_q8s": (_i, [_p, _i, _i, _i, _p, _i, _i, _p, _i, _p, _i, _p, _sz, _p]),
    "kl_rope_rows": (_i, [_i, _i, _i, _i, _p, _i, _p, _i, _i, _i, _p, _p, _p]),
    "kl_attn_prefill": (_i, [_i, _i, _i, _i, _i, _p, _i, _p, _p, _i, _p, _i, _p]),
    "kl_hbm_probe": (_i, [C.c_size_t, _i, _fp, _fp]),
    "kl_qk_norm_rope_rows": (_i, [_i, _i, _i, _i, _p, _i, _p, _i, _p, _p, C.c_float, _i, _i, _p, _p,
                                  _p]),
    "kl_attn_prefill_workspace_size": (_i, [_i, _i, _i, C.POINTER(C.c_size_t)]),
    "kl_attn_prefill_ws": (_i, [_i, _i, _i, _i, _i, _p, _i, _p, _p, _i, _p, _i, _p, C.c_size_t,
                                _p]),
    "kl_swiglu": (_i, [_p, _p, _p, _i, _p]),
    "kl_add": (_i, [_p, _p, _p, _i, _p]),
    "kl_scale": (_i, [C.c_float, _p, _i, _p]),
    "kl_softmax": (_i, [_p, _i, _p]),
    "kl_scale_sum": (_i, [_p, _p, _p, _i, _i, _i, _p]),
    "kl_embedding": (_i, [_p, _i, _p, _i, _i, _p, _p, _p]),
    "kl_argmax_workspace_size": (_i, [_i, C.POINTER(_sz)]),
    "kl_argmax": (_i, [_p, _i, _p, _p, _sz, _p]),
    "kl_synth_image_size": (_i, [C.POINTER(ModelSpec), _i64p]),
    "kl_synth_image": (_i, [C.POINTER(ModelSpec), C.c_uint64, _f, _p, C.c_int64, _i]),
    "kl_synth_normal": (_i, [C.c_uint64, C.c_int32, C.c_int32, _f, _p, C.c_int64]),
    "kl_quantize_q8": (_i, [_p, C.c_int64, _i, _p, _p]),
    "kl_engine_create": (_i, [_p, _sz, _i, _i, C.POINTER(_p)]),
    "kl_engine_destroy": (_i, [_p]),
    "kl_engine_dims": (_i, [_p, _i32p]),
    "kl_engine_weight_bytes": (_i, [_p, _i64p]),
    "kl_engine_set_graph": (_i, [_p, _i]),
    "kl_engine_set_mode": (_i, [_p, _i]),
    "kl_engine_get_mode": (_i, [_p, C.POINTER(_i)]),
    "kl_engine_launch_shape": (_i, [_p, _i32p, _i32p, _i64p]),
    "kl_engine_step": (_i, [_p, C.c_int32, C.c_int32, _i32p, _p]),
    "kl_engine_generate": (_i, [_p, _p, _i, _i, _p, _fp]),
    "kl_engine_bench": (_i, [_p, _p, _i, _i, _i, _p, _fp]),
    "kl_engine_prefill": (_i, [_p, _p, _i, _i32p, _p, _fp]),
    "kl_engine_set_prefill": (_i, [_p, _i]),
    "kl_engine_profile": (_i, [_p, C.c_int32, C.c_int32, _i, _fp, _i32p]),
    "kl_engine_trace_step": (_i, [_p, C.c_int32, C.c_int32, _p, C.c_int64, _i32p, _i32p]),
    "kl_engine_buffers": (_i, [_p, C.POINTER(_p), C.POINTER(_p), C.POINTER(_p)]),
    "kl_engine_stream": (_i, [_p, C.POINTER(_p)]),
}

for _name, (_res, _args) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.restype = _res
    _fn.argtypes = _args

EXPORTED = tuple(_SIGS)


def _errstr(code: int) -> str:
    s = lib.kl_error_string(code)
    return s.decode() if s else "?"


def check(code: int, what: str) -> None:
    if code != KL_OK:
        raise KlError(code, what)
