"""Pins the CPU oracle before anything is compared against it.

Sources of truth, per function:
  * known-answer tests of the reference's own test suite (test/test_op/*),
    with the fixture tmp/test.bin copied to tests/golden/ref_test.bin;
  * closed forms and invariants (pos 0 RoPE is the identity, a one-element
    softmax is 1, identical keys average V, ...);
  * fp64 brute force on small inputs, written from the mathematics;
  * an independent fp64 numpy model (tests/npmodel.py) for the whole step.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN


def rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ---------------------------------------------------------------- GEMV ------
def test_gemv_kat_ref_fixture(O):
    # test/test_op/test_load.cpp:11-105: header (16, 128, 256, ...) then
    # float(0..2047); MatmulLayer with W = arange(2048).reshape(16, 128), x = 1.
    raw = open(os.path.join(GOLDEN, "ref_test.bin"), "rb").read()
    hdr = np.frombuffer(raw[:28], np.int32)
    assert list(hdr[:3]) == [16, 128, 256]
    w = np.frombuffer(raw[28:], np.float32)
    assert np.array_equal(w, np.arange(2048, dtype=np.float32))
    y = O.gemv_f32(np.ones(128, np.float32), w.reshape(16, 128))
    assert y[0] == 8128 and y[1] == 24512 and y[14] == 237504 and y[15] == 253888


def test_gemv_kat_small(O):
    # test/test_op/test_cu_matmul.cpp:48-76: [[1..9]] . [1, 1, -1] = [0, 3, 6]
    y = O.gemv_f32(np.array([1, 1, -1], np.float32), np.arange(1, 10, dtype=np.float32).reshape(3, 3))
    assert list(y) == [0, 3, 6]
    # :10-46: 4x4 arange, x = [0, 1, 2, 3]
    y = O.gemv_f32(np.arange(4, dtype=np.float32), np.arange(16, dtype=np.float32).reshape(4, 4))
    assert list(y) == [14, 38, 62, 86]


@pytest.mark.parametrize("rows,cols", [(7, 13), (64, 768), (33, 2048), (5, 11008)])
def test_gemv_brute_force(O, rows, cols):
    rng = np.random.default_rng(rows * cols)
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = O.gemv_f32(x, W, 0.5)
    ref = 0.5 * (W.astype(np.float64) @ x.astype(np.float64))
    bound = 1e-6 * np.sqrt(cols) * (np.abs(W) @ np.abs(x)).max()
    assert np.max(np.abs(y - ref)) < bound + 1e-6


# ---------------------------------------------------------------- INT8 ------
def test_quantize_closed_form(O, K):
    # scale = max|w| / 127, round half to even (torch.round), per group
    w = np.zeros(64, np.float32)
    w[0] = 127.0  # scale 1.0
    w[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.49, -126.6]
    for quant in (O.quantize_q8, K.quantize_q8):
        q, s = quant(w, 64)
        assert s[0] == 1.0
        assert list(q[:9]) == [127, 0, 2, 2, 0, -2, -2, 3, -127]
    # an all-zero group quantises to zeros (documented choice, torch gives NaN)
    q, s = O.quantize_q8(np.zeros(64, np.float32), 64)
    assert s[0] == 0 and not q.any()


def test_quantize_product_matches_oracle(O, K):
    w = K.synth_normal(7, 2, 0, 64 * 500)
    q1, s1 = O.quantize_q8(w, 64)
    q2, s2 = K.quantize_q8(w, 64)
    assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.int32), s2.view(np.int32))
    # quantisation error bound: |w - s q| <= s / 2
    deq = O.dequant_q8(q1, s1, 64)
    assert np.all(np.abs(deq - w) <= np.repeat(s1, 64) * 0.5 * (1 + 1e-6))


def test_dequant_exact_for_grid_values(O):
    rng = np.random.default_rng(3)
    s = (rng.random(10) * 0.01 + 1e-3).astype(np.float32)
    k = rng.integers(-127, 128, 640).astype(np.int8)
    k[::64] = 127  # max of each group
    w = (np.repeat(s, 64) * k.astype(np.float32)).astype(np.float32)
    q, s2 = O.quantize_q8(w, 64)
    assert np.array_equal(q, k)
    assert np.array_equal(O.dequant_q8(q, s2, 64), w)


@pytest.mark.parametrize("rows,cols,gs", [(8, 256, 64), (33, 4096, 64), (4, 96, 32), (5, 100, 20),
                                           (7, 120, 40)])
def test_gemv_q8_brute_force(O, rows, cols, gs):
    rng = np.random.default_rng(cols)
    q = rng.integers(-127, 128, rows * cols).astype(np.int8)
    s = (rng.random(rows * cols // gs) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = O.gemv_q8(x, q, s, rows, cols, gs)
    Wd = (np.repeat(s.astype(np.float64), gs) * q).reshape(rows, cols)
    ref = Wd @ x.astype(np.float64)
    assert rel_err(y, ref) < 1e-5
    # the vector path (gs and cols multiples of 8) and the element loop agree bit for bit
    assert np.array_equal(y, O.gemv_q8(x, q, s, rows, cols, gs, scalar=True))


# ------------------------------------------------------------- RMSNorm ------
def test_rmsnorm_closed_form(O):
    for c, eps in ((0.5, 1e-5), (-3.0, 1e-6), (1e-3, 1e-5)):
        x = np.full(2048, c, np.float32)
        w = np.linspace(0.5, 1.5, 2048).astype(np.float32)
        y = O.rmsnorm(x, w, eps)
        ref = w.astype(np.float64) * c / np.sqrt(c * c + eps)
        assert rel_err(y, ref) < 2e-6


def test_rmsnorm_brute_force_and_rows(O):
    rng = np.random.default_rng(5)
    x = rng.random(72480).astype(np.float32)  # size used by test_cu_rmsnorm.cpp:138-176
    w = rng.random(72480).astype(np.float32)
    y = O.rmsnorm(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = w * xd / np.sqrt(np.mean(xd * xd) + 1e-5)
    assert rel_err(y, ref) < 1e-5
    # row kernel == 1-D kernel per row (test_cu_rmsnorm.cpp:41-104), arange data
    X = np.tile(np.arange(1024, dtype=np.float32), (4, 1))
    W = np.arange(1024, dtype=np.float32)
    Y = O.rmsnorm_rows(X, W, 1e-6)
    for r in range(4):
        assert np.array_equal(Y[r], O.rmsnorm(X[r], W, 1e-6))


# ---------------------------------------------------------------- RoPE ------
@pytest.mark.parametrize("hd,theta", [(64, 1e4), (128, 1e6), (64, 5e5)])
def test_sincos_table(O, hd, theta):
    s, c = O.sincos_table(hd, 300, theta)
    d = np.arange(hd)
    freq = 1.0 / theta ** (d / hd)
    pos = np.arange(300)[:, None]
    ang = pos * freq
    # float angle rounding grows with pos * freq: compare in absolute terms
    tol = 4e-7 * (1 + np.abs(ang))
    assert np.all(np.abs(s.reshape(300, hd) - np.sin(ang)) < tol)
    assert np.all(np.abs(c.reshape(300, hd) - np.cos(ang)) < tol)


@pytest.mark.parametrize("style", [0, 1])
def test_rope_pos0_identity_and_norm(O, style):
    hd, dim, kv = 64, 256, 128
    s, c = O.sincos_table(hd, 40, 1e4)
    rng = np.random.default_rng(1)
    q = rng.standard_normal(dim).astype(np.float32)
    k = rng.standard_normal(kv).astype(np.float32)
    q0, k0 = O.rope(style, dim, kv, hd, q, k, 0, s, c)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    q1, _ = O.rope(style, dim, kv, hd, q, k, 37, s, c)
    if style == 0:
        pairs = [(i, i + 1) for i in range(0, dim, 2)]
    else:
        pairs = [(h + j, h + j + hd // 2) for h in range(0, dim, hd) for j in range(hd // 2)]
    for a, b in pairs:
        n0 = np.hypot(np.float64(q[a]), q[b])
        n1 = np.hypot(np.float64(q1[a]), q1[b])
        assert abs(n1 - n0) <= 3e-7 * n0 + 1e-12


@pytest.mark.parametrize("style", [0, 1])
def test_rope_brute_force(O, style):
    hd, dim, kv, pos, theta = 32, 128, 64, 11, 1e4
    s, c = O.sincos_table(hd, 16, theta)
    rng = np.random.default_rng(2)
    q = rng.standard_normal(dim).astype(np.float32)
    k = rng.standard_normal(kv).astype(np.float32)
    q1, k1 = O.rope(style, dim, kv, hd, q, k, pos, s, c)

    def rot(v):
        v = v.astype(np.float64).reshape(-1, hd).copy()
        j = np.arange(hd // 2)
        ang = pos * theta ** (-(2.0 * j) / hd)
        if style == 1:
            a, b = v[:, : hd // 2].copy(), v[:, hd // 2 :].copy()
            v[:, : hd // 2] = a * np.cos(ang) - b * np.sin(ang)
            v[:, hd // 2 :] = a * np.sin(ang) + b * np.cos(ang)
        else:
            a, b = v[:, 0::2].copy(), v[:, 1::2].copy()
            v[:, 0::2] = a * np.cos(ang) - b * np.sin(ang)
            v[:, 1::2] = a * np.sin(ang) + b * np.cos(ang)
        return v.ravel()

    assert np.max(np.abs(q1 - rot(q))) < 1e-5
    assert np.max(np.abs(k1 - rot(k))) < 1e-5


# ------------------------------------------------------- softmax / MHA -----
def test_softmax_closed_form(O):
    p = O.softmax(np.array([0.0, np.log(3.0)], np.float32))
    assert abs(p[0] - 0.25) < 1e-7 and abs(p[1] - 0.75) < 1e-7
    assert O.softmax(np.array([42.0], np.float32))[0] == 1.0


def _rand_cache(rng, L, S, kvd):
    return (rng.standard_normal((L, S, kvd)).astype(np.float32),
            rng.standard_normal((L, S, kvd)).astype(np.float32))


def test_mha_pos0_is_v0(O):
    rng = np.random.default_rng(4)
    H, kvm, hd, S, L = 8, 4, 64, 32, 3
    kvd = H // kvm * hd
    kc, vc = _rand_cache(rng, L, S, kvd)
    q = rng.standard_normal(H * hd).astype(np.float32)
    out = O.mha(0, H, 2, S, kvd, kvm, hd, q, kc, vc)
    for h in range(H):
        g = h // kvm
        assert np.array_equal(out[h * hd:(h + 1) * hd], vc[2, 0, g * hd:(g + 1) * hd])


def test_mha_identical_keys_average_v(O):
    rng = np.random.default_rng(6)
    H, kvm, hd, S, L, pos = 4, 2, 32, 20, 1, 9
    kvd = H // kvm * hd
    kc, vc = _rand_cache(rng, L, S, kvd)
    kc[0, : pos + 1] = kc[0, 0]
    q = rng.standard_normal(H * hd).astype(np.float32)
    out = O.mha(pos, H, 0, S, kvd, kvm, hd, q, kc, vc)
    for h in range(H):
        g = h // kvm
        ref = vc[0, : pos + 1, g * hd:(g + 1) * hd].astype(np.float64).mean(0)
        assert np.max(np.abs(out[h * hd:(h + 1) * hd] - ref)) < 1e-6


@pytest.mark.parametrize("H,kvm,hd", [(4, 1, 32), (8, 4, 64), (12, 6, 128)])
def test_mha_brute_force(O, H, kvm, hd):
    rng = np.random.default_rng(H * hd)
    S, L, pos, layer = 40, 2, 29, 1
    kvd = H // kvm * hd
    kc, vc = _rand_cache(rng, L, S, kvd)
    q = rng.standard_normal(H * hd).astype(np.float32)
    out = O.mha(pos, H, layer, S, kvd, kvm, hd, q, kc, vc)
    for h in range(H):
        g = h // kvm
        K_ = kc[layer, : pos + 1, g * hd:(g + 1) * hd].astype(np.float64)
        V_ = vc[layer, : pos + 1, g * hd:(g + 1) * hd].astype(np.float64)
        s = K_ @ q[h * hd:(h + 1) * hd] / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.max(np.abs(out[h * hd:(h + 1) * hd] - p @ V_)) < 2e-6


# ------------------------------------------- SwiGLU / add / emb / argmax ----
def test_scale_closed_form(O):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(513).astype(np.float32)
    # a power of two scales exactly; otherwise one fp32 rounding per element
    assert np.array_equal(O.scale(0.25, x), x / np.float32(4))
    assert np.array_equal(O.scale(np.float32(0.3), x), x * np.float32(0.3))


def test_scale_sum_pins(O):
    """One-hot weights pick one value row exactly (catches a wrong stride or
    row index); integer data sums exactly; fp64 brute force otherwise; and
    rows past pos are never read."""
    rng = np.random.default_rng(5)
    pos, size, stride = 9, 24, 40
    value = rng.standard_normal(pos * stride + size).astype(np.float32)
    out0 = rng.standard_normal(size).astype(np.float32)
    for i in (0, 4, pos):
        sc = np.zeros(pos + 1, np.float32)
        sc[i] = 1.0
        got = O.scale_sum(value, sc, np.zeros(size, np.float32), pos, size, stride)
        assert np.array_equal(got, value[i * stride:i * stride + size])
    vi = rng.integers(-50, 50, value.size).astype(np.float32)
    si = rng.integers(-3, 4, pos + 1).astype(np.float32)
    oi = rng.integers(-50, 50, size).astype(np.float32)
    want = oi.astype(np.int64) + sum(int(si[i]) * vi[i * stride:i * stride + size].astype(np.int64)
                                     for i in range(pos + 1))
    assert np.array_equal(O.scale_sum(vi, si, oi, pos, size, stride), want.astype(np.float32))
    sc = rng.random(pos + 1).astype(np.float32)
    ref = out0.astype(np.float64) + sum(float(sc[i]) * value[i * stride:i * stride + size].astype(np.float64)
                                        for i in range(pos + 1))
    assert rel_err(O.scale_sum(value, sc, out0, pos, size, stride), ref) < 1e-6
    # a NaN past pos would poison the sum if it were read
    bad = value.copy()
    bad = np.concatenate([bad, np.full(stride, np.nan, np.float32)])
    assert np.all(np.isfinite(O.scale_sum(bad, sc, out0, pos, size, stride)))


def test_swiglu(O):
    a = np.array([0.0, 30.0, -30.0, 1.0], np.float32)
    b = np.array([5.0, 2.0, 2.0, 3.0], np.float32)
    y = O.swiglu(a, b)
    assert y[0] == 0.0 and abs(y[1] - 60.0) < 1e-5 and abs(y[2]) < 1e-10
    assert abs(y[3] - 3.0 / (1.0 + np.exp(-1.0))) < 1e-6
    rng = np.random.default_rng(8)
    a, b = rng.random(4832).astype(np.float32), rng.random(4832).astype(np.float32)
    ad = a.astype(np.float64)
    assert rel_err(O.swiglu(a, b), ad / (1 + np.exp(-ad)) * b) < 1e-6


def test_add_exact(O):
    # test/test_op/test_cu_add.cpp:7-75
    assert np.all(O.add(np.full(32, 2.0, np.float32), np.full(32, 3.0, np.float32)) == 5.0)
    a = np.random.default_rng(9).standard_normal(1000).astype(np.float32)
    assert np.array_equal(O.add(a, a), a + a)


def test_embedding_kat(O):
    # test/test_op/test_cu_emb.cpp:6-89: W = arange(2048).reshape(4, 512)
    W = np.arange(2048, dtype=np.float32).reshape(4, 512)
    out = O.embedding([1, 2], W)
    assert np.array_equal(out[0], 512 + np.arange(512, dtype=np.float32))
    assert np.array_equal(out[1], 1024 + np.arange(512, dtype=np.float32))
    for bad in (4, -1):
        with pytest.raises(ValueError):
            O.embedding([bad], W)


def test_argmax_first_max(O):
    assert O.argmax(np.array([1, 3, 2, 3], np.float32)) == 1
    assert O.argmax(np.array([-0.0, 0.0], np.float32)) == 0
    assert O.argmax(np.array([0.0, -0.0], np.float32)) == 0
    assert O.argmax(np.full(7, -np.inf, np.float32)) == 0
    x = np.random.default_rng(1).standard_normal(128256).astype(np.float32)
    assert O.argmax(x) == int(np.argmax(x))


# --------------------------------------------------------- whole model -----
TINY_NAMES = ["tiny_llama2", "tiny_llama3", "tiny_q8", "tiny_qwen2", "tiny_qwen2_q8", "tiny_qwen3"]


@pytest.mark.parametrize("name", TINY_NAMES)
def test_model_step_vs_fp64_model(K, O, name):
    from npmodel import NpModel

    cfg = K.TINY[name]
    img = K.synth_image(cfg)
    om = O.Model(img, cfg.family, cfg.quant)
    nm = NpModel(K, cfg)
    toks = K.prompt_tokens(cfg, 12)
    for pos, t in enumerate(toks):
        lo = om.step(int(t), pos)
        ln = nm.step(int(t), pos)
        assert rel_err(lo, ln) < 2e-5, (name, pos)
    # the K cache row holds the rotated key
    assert rel_err(om.kv_row(1, 5, False), nm.kc[1, 5]) < 1e-4
    assert rel_err(om.kv_row(0, 3, True), nm.vc[0, 3]) < 1e-4


def _norm_offsets(cfg):
    """Byte offsets of the norm vectors in an image: {(role, layer): (offset,
    floats)} for the attention ("att"), ffn ("ffn"), final ("fin") and Qwen3
    q/k ("qn", "kn") norms, in the writers' layouts (export_llama.py:79-210,
    export_qwen2.py:79-210, export_qwen3.py:55-102)."""
    D, Dq, Dkv, F, L, V, hd = (cfg.dim, cfg.qd, cfg.kv_dim, cfg.hidden_dim, cfg.layers, cfg.vocab,
                               cfg.head_size)
    out = {}
    if cfg.family == 3:
        off = 32
        for l in range(L):
            out[("att", l)] = (off + 4 * l * D, D)
            out[("ffn", l)] = (off + 4 * (L + l) * D, D)
        out[("fin", 0)] = (off + 4 * 2 * L * D, D)
        off += 4 * ((2 * L + 1) * D + V * D + L * Dq * D)
        for l in range(L):
            out[("qn", l)] = (off + 4 * l * hd, hd)
        off += 4 * (L * hd + L * Dkv * D)
        for l in range(L):
            out[("kn", l)] = (off + 4 * l * hd, hd)
    elif cfg.quant:
        gs = cfg.group_size
        q8 = lambda n: n + n // gs * 4
        off = 32 + L * (q8(Dq * D) + 2 * q8(Dkv * D) + q8(D * Dq) + 3 * q8(F * D)) + q8(V * D)
        off += 4 * V * D
        for l in range(L):
            out[("att", l)] = (off + 4 * l * D, D)
            out[("ffn", l)] = (off + 4 * (L + l) * D, D)
        out[("fin", 0)] = (off + 4 * 2 * L * D, D)
    else:
        b = (Dq + 2 * Dkv) if cfg.family == 2 else 0
        off = 28 + 4 * V * D
        for l in range(L):
            out[("att", l)] = (off + 4 * l * D, D)
        off += 4 * (L * D + L * (Dq * D + 2 * Dkv * D + b + D * Dq))
        for l in range(L):
            out[("ffn", l)] = (off + 4 * l * D, D)
        out[("fin", 0)] = (off + 4 * (L * D + 3 * L * F * D), D)
    return out


@pytest.mark.parametrize("name,a,b", [
    ("tiny_llama3", ("att", 0), ("ffn", 0)),   # layer l's ffn norm used for attention
    ("tiny_llama2", ("att", 0), ("att", 1)),   # off-by-one layer index
    ("tiny_qwen2", ("ffn", 1), ("fin", 0)),    # final norm taken from the wrong slot
    ("tiny_q8", ("att", 1), ("ffn", 1)),
    ("tiny_qwen3", ("qn", 0), ("kn", 0)),      # q_norm and k_norm swapped
    ("tiny_qwen3", ("qn", 0), ("qn", 1)),
])
def test_fp64_pin_catches_swapped_norms(K, O, name, a, b):
    """A planted mistake in the oracle's input: two norm vectors of the image
    swapped (what a wrong offset in a parser would read) make the oracle
    disagree with the fp64 model, which takes every norm from its own stream.
    So the pin sees the norm weights, and the same swap in any GPU path fails
    its comparison with the oracle."""
    from npmodel import NpModel

    cfg = K.TINY[name]
    img = K.synth_image(cfg).copy()
    offs = _norm_offsets(cfg)
    (oa, na), (ob, nb) = offs[a], offs[b]
    n = min(na, nb)
    va = img[oa: oa + 4 * n].copy()
    vb = img[ob: ob + 4 * n].copy()
    assert not np.array_equal(va, vb)
    nm = NpModel(K, cfg)
    good = O.Model(K.synth_image(cfg), cfg.family, cfg.quant)
    img[oa: oa + 4 * n], img[ob: ob + 4 * n] = vb, va
    bad = O.Model(img, cfg.family, cfg.quant)
    toks = K.prompt_tokens(cfg, 4)
    worst_bad = worst_good = 0.0
    for pos, t in enumerate(toks):
        ln = nm.step(int(t), pos)
        worst_good = max(worst_good, rel_err(good.step(int(t), pos), ln))
        worst_bad = max(worst_bad, rel_err(bad.step(int(t), pos), ln))
    assert worst_good < 2e-5
    assert worst_bad > 1e-3, (name, a, b, worst_bad)


def test_model_generate_follows_demo_loop(K, O):
    # demo/main.cpp:18-41: prompt positions run without sampling, the last
    # prompt token and every sampled token are fed back one at a time.
    cfg = K.TINY["tiny_qwen3"]
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg, 6)
    toks = O.Model(img, cfg.family, cfg.quant).generate(prompt, 10)
    m = O.Model(img, cfg.family, cfg.quant)
    seq = list(prompt)
    for pos in range(len(prompt) + 10 - 1):
        lg = m.step(seq[pos], pos)
        if pos >= len(prompt) - 1:
            seq.append(O.argmax(lg))
    assert list(toks) == seq[len(prompt):]


def test_model_rejects_truncated_image(K, O):
    cfg = K.TINY["tiny_llama2"]
    img = K.synth_image(cfg)
    with pytest.raises(ValueError):
        O.Model(img[:-4], cfg.family, cfg.quant)
    with pytest.raises(ValueError):
        O.Model(img[:20], cfg.family, cfg.quant)


# Shapes beyond the tiny set for the batched prompt: widths that are not a
# multiple of 8 (dot8's scalar tail), int8 groups of 40 (vector path) and of
# 20 (a group boundary inside an 8-column step: the scalar int8 path), and a
# prompt longer than one 512-position pass.
PROMPT_EXTRA = {
    "odd_llama2": dict(base="tiny_llama2", dim=108, hidden_dim=230, heads=6, kv_heads=3, vocab=301),
    "q8_g40": dict(base="tiny_q8", dim=120, hidden_dim=200, heads=4, kv_heads=2, vocab=500,
                   group_size=40),
    "q8_g20": dict(base="tiny_qwen2_q8", dim=120, hidden_dim=200, heads=4, kv_heads=2, vocab=500,
                   group_size=20),
    "long_llama3": dict(base="tiny_llama3", seq_len=700),
}


def _prompt_cfg(K, name):
    if name in K.TINY:
        return K.TINY[name]
    kw = dict(PROMPT_EXTRA[name])
    return K.TINY[kw.pop("base")].with_(name=name, **kw)


@pytest.mark.parametrize("name", TINY_NAMES + list(PROMPT_EXTRA))
def test_model_prompt_bitwise_equals_steps(K, O, name):
    """or_model_prompt (each weight row applied to many positions while
    cached) against or_model_step position by position: the last logits and
    every cache row bit for bit, for a prompt from position 0 and for one
    continuing a cache that steps filled; and generate() (which runs its
    prompt batched) against the demo loop made of steps."""
    cfg = _prompt_cfg(K, name)
    img = K.synth_image(cfg)
    P = 600 if name == "long_llama3" else min(37, cfg.seq_len - 12)
    toks = [int(t) for t in K.prompt_tokens(cfg, P)]
    a = O.Model(img, cfg.family, cfg.quant)
    b = O.Model(img, cfg.family, cfg.quant)
    for pos, t in enumerate(toks):
        ref = a.step(t, pos)
    got = b.prompt(toks)
    assert np.array_equal(got, ref), name
    # a continuation from a filled cache: 5 more positions as one batch
    more = [int(t) for t in K.prompt_tokens(cfg, P + 5)[P:]]
    for i, t in enumerate(more):
        ref = a.step(t, P + i)
    assert np.array_equal(b.prompt(more, P), ref), name
    for layer in range(cfg.layers):
        for pos in range(P + 5):
            for v in (False, True):
                assert np.array_equal(a.kv_row(layer, pos, v), b.kv_row(layer, pos, v)), (layer, pos, v)
    if name != "long_llama3":
        prompt = toks[:9]
        gen = O.Model(img, cfg.family, cfg.quant).generate(prompt, 6)
        m = O.Model(img, cfg.family, cfg.quant)
        seq = list(prompt)
        for pos in range(len(prompt) + 6 - 1):
            lg = m.step(seq[pos], pos)
            if pos >= len(prompt) - 1:
                seq.append(O.argmax(lg))
        assert list(gen) == seq[len(prompt):]


def test_model_prompt_rejects_bad_input(K, O):
    cfg = K.TINY["tiny_llama2"]
    m = O.Model(K.synth_image(cfg), cfg.family, cfg.quant)
    with pytest.raises(ValueError):
        m.prompt([1, cfg.vocab])
    with pytest.raises(ValueError):
        m.prompt([1, 2], cfg.seq_len - 1)
