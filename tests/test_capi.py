"""CPU checks of the drop-in boundary: the library loads, exports every entry
point include/kuiper_hip.h declares, rejects bad arguments on the host, and
writes model images in the reference byte layouts."""
import ctypes as C
import os
import re

import numpy as np
import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "kuiper_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kl_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported(K):
    from kuiperllama_amd import _lib

    names = declared_functions()
    assert len(names) >= 40
    for n in names:
        assert hasattr(_lib.lib, n), f"{n} declared in kuiper_hip.h but not exported"
    assert set(names) == set(_lib.EXPORTED), "python binding and header disagree"


def test_error_strings(K):
    from kuiperllama_amd import _lib

    for code in (0, -1, -2, -3, -4, -5, -6):
        assert _lib.lib.kl_error_string(code)


def test_host_side_argument_checks(K):
    """Shape errors are rejected before any launch (no device needed)."""
    lib = K.lib
    assert lib.kl_gemv_f32(None, None, None, 4, 4, 1.0, None) == -1
    assert lib.kl_gemv_q8(None, None, None, None, 4, 64, 64, None) == -1
    assert lib.kl_rope(0, 10, 4, 3, None, None, 0, None, None, None) == -1
    sz = C.c_size_t(0)
    assert lib.kl_mha_workspace_size(8, 3, 64, 64, C.byref(sz)) == -1  # 8 % 3
    assert lib.kl_mha_workspace_size(8, 16, 64, 64, C.byref(sz)) == -1  # kv_mul > 8
    assert lib.kl_mha_workspace_size(32, 4, 320, 64, C.byref(sz)) == 0 and sz.value > 0
    assert lib.kl_argmax_workspace_size(128256, C.byref(sz)) == 0 and sz.value > 0
    bad = np.zeros(64, np.uint8)
    h = C.c_void_p()
    assert lib.kl_engine_create(bad.ctypes.data, 8, 0, 0, C.byref(h)) == -3
    assert lib.kl_split_bf16x3(None, 4, 32, 32, None, None) == -1
    assert lib.kl_split_bf16x3_bytes(17, 64) == 32 * 64 * 6 and lib.kl_split_bf16x3_bytes(0, 64) == 0
    assert lib.kl_gemm_x6(None, None, None, 4, 4, 32, 4, None, 0, None, 0, None) == -1
    assert lib.kl_q8s_packed_bytes(40, 128, 64) == 64 * 128 + 2 * 2 * 128
    assert lib.kl_q8s_pack(None, None, 32, 64, 64, None, None) == -1
    rd, cp = C.c_float(0), C.c_float(0)
    assert lib.kl_hbm_probe(1 << 19, 1, C.byref(rd), C.byref(cp)) == -1  # under 1 MiB
    assert lib.kl_hbm_probe(1 << 20, 0, C.byref(rd), C.byref(cp)) == -1  # no passes


# ------------------------------------------------------------ formats ------
def _hdr(img, n):
    return list(np.frombuffer(img[: 4 * n].tobytes(), np.int32))


# synth.cpp norm roles: attention, ffn, final, Qwen3 q and k norms
RMS_ATT, RMS_FFN, RMS_FINAL, Q_NORM, K_NORM = 13, 14, 15, 16, 17


def _norms(K, cfg, role, layers, n):
    """The norm vectors the writer emits for `role` over `layers`: 1 + N(0,
    norm_std) per layer, concatenated."""
    return np.concatenate([1.0 + K.synth_normal(1234, role, l, n, cfg.norm_std)
                           for l in layers]).astype(np.float32)


def test_llama_v0_layout(K):
    cfg = K.TINY["tiny_llama2"]
    img = K.synth_image(cfg)
    D, F, L, V, S, hd = cfg.dim, cfg.hidden_dim, cfg.layers, cfg.vocab, cfg.seq_len, cfg.head_size
    Dkv = cfg.kv_dim
    # export_llama.py:91-93: negative vocab marks a separate classifier
    assert _hdr(img, 7) == [D, F, L, cfg.heads, cfg.kv_heads, -V, S]
    f = np.frombuffer(img[28:].tobytes(), np.float32)
    emb = K.synth_normal(1234, 1, 0, V * D)
    assert np.array_equal(f[: V * D], emb)
    off = V * D
    assert np.array_equal(f[off: off + L * D], _norms(K, cfg, RMS_ATT, range(L), D))
    assert not np.all(f[off: off + L * D] == 1.0)
    off += L * D
    assert np.array_equal(f[off: off + D * D], K.synth_normal(1234, 2, 0, D * D))  # wq[0]
    off += L * D * D + 2 * L * Dkv * D + L * D * D
    assert np.array_equal(f[off: off + L * D], _norms(K, cfg, RMS_FFN, range(L), D))
    off += L * D + 3 * L * F * D
    assert np.array_equal(f[off: off + D], _norms(K, cfg, RMS_FINAL, [0], D))
    off += D + S * hd  # freq tables
    assert np.array_equal(f[off:], K.synth_normal(1234, 9, 0, V * D))  # classifier
    assert f.size == off + V * D


def test_llama_int8_layout(K, O):
    cfg = K.TINY["tiny_q8"]
    img = K.synth_image(cfg)
    D, gs = cfg.dim, cfg.group_size
    assert _hdr(img, 8) == [D, cfg.hidden_dim, cfg.layers, cfg.heads, cfg.kv_heads, -cfg.vocab,
                            cfg.seq_len, gs]
    raw = img[32:].tobytes()
    n = D * D
    q = np.frombuffer(raw[:n], np.int8)
    s = np.frombuffer(raw[n: n + 4 * n // gs], np.float32)
    q_ref, s_ref = O.quantize_q8(K.synth_normal(1234, 2, 0, n), gs)
    assert np.array_equal(q, q_ref) and np.array_equal(s, s_ref)
    # fp32 embedding then (2L + 1) norm vectors close the file
    L = cfg.layers
    tail = np.frombuffer(raw[-4 * (2 * L + 1) * D:], np.float32)
    want = np.concatenate([_norms(K, cfg, RMS_ATT, range(L), D), _norms(K, cfg, RMS_FFN, range(L), D),
                           _norms(K, cfg, RMS_FINAL, [0], D)])
    assert np.array_equal(tail, want)


def test_qwen2_bias_follows_weight(K):
    cfg = K.TINY["tiny_qwen2"]
    img = K.synth_image(cfg)
    D, V, L = cfg.dim, cfg.vocab, cfg.layers
    assert _hdr(img, 7)[5] == V  # tied: positive vocab
    f = np.frombuffer(img[28:].tobytes(), np.float32)
    off = V * D + L * D
    assert np.array_equal(f[off: off + D * D], K.synth_normal(1234, 2, 0, D * D))
    off += D * D
    assert np.array_equal(f[off: off + D], K.synth_normal(1234, 10, 0, D))  # bq[0]
    off += D
    assert np.array_equal(f[off: off + D * D], K.synth_normal(1234, 2, 1, D * D))  # wq[1]


def test_qwen3_layout(K):
    cfg = K.TINY["tiny_qwen3"]
    img = K.synth_image(cfg)
    D, Dq, L, V, hd = cfg.dim, cfg.qd, cfg.layers, cfg.vocab, cfg.head_size
    # export_qwen3.py:55-78: {q_dim, dim, L, H, KVH, V, seq, ffn}
    assert _hdr(img, 8) == [Dq, D, L, cfg.heads, cfg.kv_heads, V, cfg.seq_len, cfg.hidden_dim]
    f = np.frombuffer(img[32:].tobytes(), np.float32)
    want = np.concatenate([_norms(K, cfg, RMS_ATT, range(L), D), _norms(K, cfg, RMS_FFN, range(L), D),
                           _norms(K, cfg, RMS_FINAL, [0], D)])
    assert np.array_equal(f[: (2 * L + 1) * D], want)
    off = (2 * L + 1) * D
    assert np.array_equal(f[off: off + V * D], K.synth_normal(1234, 1, 0, V * D))
    off += V * D + L * Dq * D
    assert np.array_equal(f[off: off + L * hd], _norms(K, cfg, Q_NORM, range(L), hd))  # q norms
    off += L * hd + L * cfg.kv_dim * D
    assert np.array_equal(f[off: off + L * hd], _norms(K, cfg, K_NORM, range(L), hd))  # k norms
    assert np.array_equal(f[-V * D:], K.synth_normal(1234, 9, 0, V * D))  # lm_head


def test_image_sizes_of_baseline_configs(K):
    """Sizes match the per-config weight bytes (no allocation needed)."""
    for name, cfg in K.BASELINE.items():
        spec = cfg.spec()
        n = C.c_int64(0)
        assert K.lib.kl_synth_image_size(C.byref(spec), C.byref(n)) == 0
        wb = cfg.weight_bytes_per_token()
        extra = n.value - wb
        # the image also holds the embedding matrix (untied), freq tables,
        # header; it never holds less than the streamed weights
        assert extra >= -4 * cfg.dim, name
    gb = K.BASELINE["llama32_1b"].weight_bytes_per_token() / 1e9
    assert 4.94 < gb < 4.95  # 4943.3 MB of weights per token


def test_mha_workspace_fits_reference_score_buffer(K):
    """kl_mha's split partials fit the reference's score tensor, head_num x
    seq_len floats (llama3.cpp:485-487, qwen2.cpp:550, qwen3.cpp:367), at
    every BASELINE shape and over a sweep of sequence lengths; a context that
    one workgroup per kv head covers needs none."""
    for cfg in K.BASELINE.values():
        sz = C.c_size_t(0)
        assert K.lib.kl_mha_workspace_size(cfg.heads, cfg.heads // cfg.kv_heads, cfg.seq_len,
                                           cfg.head_size, C.byref(sz)) == 0
        assert 0 < sz.value <= cfg.heads * cfg.seq_len * 4, cfg.name
    for H, kvm, hd in ((12, 6, 128), (32, 4, 64), (4, 2, 32), (2, 2, 256), (32, 1, 128)):
        for S in (1, 2, 31, 64, 65, 130, 300, 1000, 4096, 8192, 20000):
            sz = C.c_size_t(0)
            assert K.lib.kl_mha_workspace_size(H, kvm, S, hd, C.byref(sz)) == 0
            assert sz.value <= H * S * 4, (H, kvm, hd, S, sz.value)
    sz = C.c_size_t(0)
    assert K.lib.kl_mha_workspace_size(8, 2, 64, 64, C.byref(sz)) == 0 and sz.value == 0
