"""Op-level parity: every C-ABI kernel against the CPU oracle on the same inputs.

Bars: bit-exact for embedding, argmax, add, int8 dequant, RoPE and the sin/cos
tables (elementwise, no reduction); fp32 reductions (GEMV, RMSNorm, MHA,
SwiGLU's expf) within the tolerance written in each test.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def D(K, a):
    return K.DeviceArray.from_numpy(np.ascontiguousarray(a))


def ok(rc, what="call"):
    assert rc == 0, f"{what}: rc={rc}"


def sync(K):
    ok(K.lib.kl_device_sync(), "sync")


def gemv_tol(W, x):
    """fp32 GEMV error bound used for both orders: ~ sqrt(cols) eps |W||x|."""
    return 4e-7 * np.sqrt(W.shape[1]) * (np.abs(W) @ np.abs(x)).max() + 1e-30


# ---------------------------------------------------------------- GEMV ------
def test_gemv_kat_exact(K, O, gpu):
    for W, x, want in (
        (np.arange(2048, dtype=np.float32).reshape(16, 128), np.ones(128, np.float32),
         {0: 8128, 1: 24512, 14: 237504, 15: 253888}),
        (np.arange(1, 10, dtype=np.float32).reshape(3, 3), np.array([1, 1, -1], np.float32),
         {0: 0, 1: 3, 2: 6}),
        (np.arange(16, dtype=np.float32).reshape(4, 4), np.arange(4, dtype=np.float32),
         {0: 14, 1: 38, 2: 62, 3: 86}),
    ):
        dW, dx, dy = D(K, W), D(K, x), K.DeviceArray(W.shape[0])
        ok(K.lib.kl_gemv_f32(dx.ptr, dW.ptr, dy.ptr, W.shape[0], W.shape[1], 1.0, None))
        y = dy.numpy()
        for i, v in want.items():
            assert y[i] == v
        assert np.array_equal(y, O.gemv_f32(x, W))


SHAPES = [
    (768, 768), (2048, 768), (768, 2048),            # cfg 1
    (3072, 2048), (2048, 8192), (512, 2048),          # cfg 2 (fused qkv rows, w2, wk)
    (256, 1536), (1536, 8960),                       # cfg 4
    (1000, 2560), (2560, 9728),                      # cfg 5
    (37, 100), (5, 6), (129, 4),                     # odd shapes (scalar path)
]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_gemv_f32_vs_oracle(K, O, gpu, rows, cols):
    rng = np.random.default_rng(rows + cols)
    W = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    dW, dx, dy = D(K, W), D(K, x), K.DeviceArray(rows)
    ok(K.lib.kl_gemv_f32(dx.ptr, dW.ptr, dy.ptr, rows, cols, 0.5, None))
    y = dy.numpy()
    ref = O.gemv_f32(x, W, 0.5)
    assert np.max(np.abs(y - ref)) <= 0.5 * 2 * gemv_tol(W, x)


@pytest.mark.parametrize("rows,cols,gs", [(4096, 4096, 64), (11008, 4096, 64), (4096, 11008, 64),
                                          (64, 256, 32), (10, 96, 48)])
def test_gemv_q8_vs_oracle(K, O, gpu, rows, cols, gs):
    rng = np.random.default_rng(rows)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    q, s = O.quantize_q8(w, gs)
    x = rng.standard_normal(cols).astype(np.float32)
    dq, ds, dx, dy = D(K, q), D(K, s), D(K, x), K.DeviceArray(rows)
    ok(K.lib.kl_gemv_q8(dx.ptr, dq.ptr, ds.ptr, dy.ptr, rows, cols, gs, None))
    y = dy.numpy()
    ref = O.gemv_q8(x, q, s, rows, cols, gs)
    Wd = O.dequant_q8(q, s, gs).reshape(rows, cols)
    assert np.max(np.abs(y - ref)) <= 2 * gemv_tol(Wd, x)


def test_dequant_q8_bit_exact(K, O, gpu):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal(64 * 4096) * 0.02).astype(np.float32)
    q, s = O.quantize_q8(w, 64)
    dq, ds, do = D(K, q), D(K, s), K.DeviceArray(q.size)
    ok(K.lib.kl_dequant_q8(dq.ptr, ds.ptr, q.size, 64, do.ptr, None))
    assert np.array_equal(do.numpy().view(np.int32), O.dequant_q8(q, s, 64).view(np.int32))


# ------------------------------------------------------------- RMSNorm ------
@pytest.mark.parametrize("n", [480, 32, 72480, 2048, 2560])
def test_rmsnorm_vs_oracle(K, O, gpu, n):
    # sizes of test/test_op/test_cu_rmsnorm.cpp (480, 32, 72480) + model widths
    rng = np.random.default_rng(n)
    x = rng.random(n).astype(np.float32)
    w = rng.random(n).astype(np.float32)
    dx, dw, dy = D(K, x), D(K, w), K.DeviceArray(n)
    ok(K.lib.kl_rmsnorm(dx.ptr, dw.ptr, dy.ptr, n, 1e-5, None))
    assert np.max(np.abs(dy.numpy() - O.rmsnorm(x, w, 1e-5))) < 1e-5  # test_cu_rmsnorm.cpp:37
    # in place
    ok(K.lib.kl_rmsnorm(dx.ptr, dw.ptr, dx.ptr, n, 1e-5, None))
    assert np.max(np.abs(dx.numpy() - O.rmsnorm(x, w, 1e-5))) < 1e-5


def test_rmsnorm_rows_vs_oracle(K, O, gpu):
    X = np.tile(np.arange(1024, dtype=np.float32), (4, 1))
    W = np.arange(1024, dtype=np.float32)
    dX, dW, dY = D(K, X.ravel()), D(K, W), K.DeviceArray(X.size)
    ok(K.lib.kl_rmsnorm_rows(dX.ptr, dW.ptr, dY.ptr, 4, 1024, 1e-6, None))
    Y = dY.numpy().reshape(4, 1024)
    ref = O.rmsnorm_rows(X, W, 1e-6)
    assert np.max(np.abs(Y - ref) / np.maximum(np.abs(ref), 1)) < 1e-5
    rng = np.random.default_rng(2)
    q = rng.standard_normal((32, 128)).astype(np.float32)
    w = rng.random(128).astype(np.float32)
    dq, dw = D(K, q.ravel()), D(K, w)
    ok(K.lib.kl_rmsnorm_rows(dq.ptr, dw.ptr, dq.ptr, 32, 128, 1e-6, None))  # in place
    assert np.max(np.abs(dq.numpy().reshape(32, 128) - O.rmsnorm_rows(q, w, 1e-6))) < 1e-5


# ---------------------------------------------------------------- RoPE ------
def test_sincos_table_bit_exact(K, O, gpu):
    for hd, S, theta in ((64, 1024, 1e4), (128, 4096, 1e6), (64, 320, 5e5)):
        ds, dc = K.DeviceArray(hd * S), K.DeviceArray(hd * S)
        ok(K.lib.kl_sincos_table(hd, S, theta, ds.ptr, dc.ptr))
        s, c = O.sincos_table(hd, S, theta)
        assert np.array_equal(ds.numpy(), s) and np.array_equal(dc.numpy(), c)


@pytest.mark.parametrize("style,dim,kv,hd", [(0, 768, 768, 64), (1, 2048, 512, 64),
                                             (1, 1536, 256, 128), (1, 4096, 1024, 128),
                                             (0, 4096, 4096, 128)])
def test_rope_bit_exact(K, O, gpu, style, dim, kv, hd):
    S = 64
    s, c = O.sincos_table(hd, S, 1e4 if style == 0 else 1e6)
    rng = np.random.default_rng(dim + kv)
    q = rng.standard_normal(dim).astype(np.float32)
    k = rng.standard_normal(kv).astype(np.float32)
    dq, dk, dsn, dcs = D(K, q), D(K, k), D(K, s), D(K, c)
    for pos in (0, 1, 63):
        dq.upload(q)
        dk.upload(k)
        ok(K.lib.kl_rope(style, dim, kv, hd, dq.ptr, dk.ptr, pos, dsn.ptr, dcs.ptr, None))
        rq, rk = O.rope(style, dim, kv, hd, q, k, pos, s, c)
        assert np.array_equal(dq.numpy(), rq) and np.array_equal(dk.numpy(), rk)


# ----------------------------------------------------------------- MHA ------
@pytest.mark.parametrize("H,kvm,hd,S,pos", [(12, 1, 64, 1024, 0), (12, 1, 64, 1024, 143),
                                            (32, 4, 64, 1024, 319), (32, 4, 64, 1024, 1023),
                                            (12, 6, 128, 4096, 4095), (12, 6, 128, 4096, 4000),
                                            (12, 6, 128, 4096, 191), (32, 4, 128, 1024, 639),
                                            (32, 1, 128, 160, 77), (4, 2, 32, 50, 17),
                                            (2, 2, 256, 300, 299), (32, 4, 128, 1024, 511)])
def test_mha_vs_oracle(K, O, gpu, H, kvm, hd, S, pos):
    """kl_mha with the reference's own score buffer, exactly head_num x
    seq_len floats (llama3.cpp:485-487), left uninitialised (filled with NaN
    bit patterns here): cfg 2's shape (32/8 heads of 64, seq 1024) and cfg
    4's (12/2 heads of 128, seq 4096) among them."""
    rng = np.random.default_rng(H * S + pos)
    L, layer = 2, 1
    kvd = H // kvm * hd
    kc = rng.standard_normal((L, S, kvd)).astype(np.float32)
    vc = rng.standard_normal((L, S, kvd)).astype(np.float32)
    q = rng.standard_normal(H * hd).astype(np.float32)
    sz = C.c_size_t(0)
    ok(K.lib.kl_mha_workspace_size(H, kvm, S, hd, C.byref(sz)))
    score_bytes = H * S * 4
    assert sz.value <= score_bytes
    ws = D(K, np.full(H * S, np.nan, np.float32))
    dk, dv, dq, do = D(K, kc.ravel()), D(K, vc.ravel()), D(K, q), K.DeviceArray(H * hd)
    ref = O.mha(pos, H, layer, S, kvd, kvm, hd, q, kc, vc)
    for _ in range(2):  # the second call reuses the workspace as the first left it
        ok(K.lib.kl_mha(pos, H, layer, S, kvd, kvm, hd, do.ptr, dq.ptr, ws.ptr, score_bytes,
                        dk.ptr, dv.ptr, None))
        out = do.numpy()
        assert np.max(np.abs(out - ref)) < 2e-5
    if pos == 0:  # softmax of one element: V0 exactly
        for h in range(H):
            g = h // kvm
            assert np.array_equal(out[h * hd:(h + 1) * hd], vc[layer, 0, g * hd:(g + 1) * hd])


def test_mha_workspace_too_small(K, gpu):
    sz = C.c_size_t(0)
    ok(K.lib.kl_mha_workspace_size(8, 2, 1024, 64, C.byref(sz)))
    assert sz.value > 16
    ws = K.DeviceArray(16, np.uint8, zero=True)
    buf = K.DeviceArray(8 * 1024 * 64)
    assert K.lib.kl_mha(3, 8, 0, 1024, 256, 2, 64, buf.ptr, buf.ptr, ws.ptr, 16, buf.ptr, buf.ptr,
                        None) == -6


# ------------------------------------------------------ elementwise --------
def test_swiglu_vs_oracle(K, O, gpu):
    rng = np.random.default_rng(4832)
    a, b = rng.random(4832).astype(np.float32), rng.random(4832).astype(np.float32)
    da, db, do = D(K, a), D(K, b), K.DeviceArray(4832)
    ok(K.lib.kl_swiglu(da.ptr, db.ptr, do.ptr, 4832, None))
    assert np.max(np.abs(do.numpy() - O.swiglu(a, b))) < 1e-5  # test_cu_swiglu.cpp tolerance
    ok(K.lib.kl_swiglu(da.ptr, db.ptr, da.ptr, 4832, None))  # in place, as the models call it
    assert np.max(np.abs(da.numpy() - O.swiglu(a, b))) < 1e-5


def test_add_exact(K, O, gpu):
    rng = np.random.default_rng(1)
    a = rng.standard_normal(8191).astype(np.float32)
    b = rng.standard_normal(8191).astype(np.float32)
    da, db, do = D(K, a), D(K, b), K.DeviceArray(8191)
    ok(K.lib.kl_add(da.ptr, db.ptr, do.ptr, 8191, None))
    assert np.array_equal(do.numpy(), O.add(a, b))
    ok(K.lib.kl_add(da.ptr, db.ptr, da.ptr, 8191, None))  # x = x + y in place
    assert np.array_equal(da.numpy(), O.add(a, b))


def test_scale_bit_exact(K, O, gpu):
    rng = np.random.default_rng(41)
    x = rng.standard_normal(10001).astype(np.float32)
    for sc in (0.125, 1.0 / np.sqrt(128.0), -3.7):
        d = D(K, x)
        ok(K.lib.kl_scale(C.c_float(sc), d.ptr, x.size, None), "kl_scale")
        assert np.array_equal(d.numpy(), O.scale(np.float32(sc), x))


@pytest.mark.parametrize("n", [1, 7, 1000, 4096, 70001])
def test_softmax_vs_oracle(K, O, gpu, n):
    """One vector in place: max-subtract, exp, sum, divide.  The sum runs in
    another order than the CPU's (which adds in two running sums), so every
    element differs by about the same factor, bounded by the sums' rounding
    (~4e-7 sqrt(n) relative), plus the device expf; both sides are also held
    to an fp64 softmax.  A single element is exactly 1."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 4).astype(np.float32)
    d = D(K, x)
    ok(K.lib.kl_softmax(d.ptr, n, None), "kl_softmax")
    got, want = d.numpy(), O.softmax(x)
    bound = 4e-7 * np.sqrt(n) + 1e-6
    assert np.max(np.abs(got / want - 1)) <= bound, np.max(np.abs(got / want - 1))
    e = np.exp(x.astype(np.float64) - x.max())
    exact = e / e.sum()
    for y in (got, want):
        assert np.max(np.abs(y / exact - 1)) <= bound
    if n == 1:
        assert got[0] == 1.0


@pytest.mark.parametrize("pos,size,stride", [(0, 64, 512), (17, 64, 512), (300, 128, 256), (5, 1000, 1000)])
def test_scale_sum_bit_exact(K, O, gpu, pos, size, stride):
    """The MHA's weighted sum of V rows (value rows at a stride, as in the
    cache): bit-exact, the products and sums rounded in the reference's order."""
    rng = np.random.default_rng(pos + size)
    value = rng.standard_normal(pos * stride + size).astype(np.float32)
    sc = rng.random(pos + 1).astype(np.float32)
    out0 = rng.standard_normal(size).astype(np.float32)
    dv, ds, do = D(K, value), D(K, sc), D(K, out0)
    ok(K.lib.kl_scale_sum(dv.ptr, ds.ptr, do.ptr, pos, size, stride, None), "kl_scale_sum")
    assert np.array_equal(do.numpy(), O.scale_sum(value, sc, out0, pos, size, stride))
    # overlapping rows are refused
    assert K.lib.kl_scale_sum(dv.ptr, ds.ptr, do.ptr, 1, size, size - 1, None) == -1


def test_embedding_kat_and_bounds(K, O, gpu):
    W = np.arange(2048, dtype=np.float32).reshape(4, 512)
    toks = np.array([1, 2], np.int32)
    dW, dt, do = D(K, W.ravel()), D(K, toks), K.DeviceArray(2 * 512)
    flag = K.DeviceArray(1, np.int32, zero=True)
    ok(K.lib.kl_embedding(dt.ptr, 2, dW.ptr, 4, 512, do.ptr, flag.ptr, None))
    assert np.array_equal(do.numpy().reshape(2, 512), O.embedding(toks, W))
    assert flag.numpy()[0] == 0
    # more than 512 tokens (the reference CUDA kernel silently stops at 512)
    rng = np.random.default_rng(0)
    E = rng.standard_normal((1000, 64)).astype(np.float32)
    toks = rng.integers(0, 1000, 700).astype(np.int32)
    dE, dt, do = D(K, E.ravel()), D(K, toks), K.DeviceArray(700 * 64)
    ok(K.lib.kl_embedding(dt.ptr, 700, dE.ptr, 1000, 64, do.ptr, flag.ptr, None))
    assert np.array_equal(do.numpy().reshape(700, 64), O.embedding(toks, E))
    bad = D(K, np.array([4], np.int32))
    ok(K.lib.kl_embedding(bad.ptr, 1, dW.ptr, 4, 512, do.ptr, flag.ptr, None))
    assert flag.numpy()[0] == 1


def test_hbm_probe_rates_plausible(K, gpu):
    """kl_hbm_probe (the bench's on-box bandwidth reference): a read rate and a
    copy rate between 1 TB/s and the 8 TB/s HBM3E specification."""
    rd, cp = C.c_float(0), C.c_float(0)
    ok(K.lib.kl_hbm_probe(256 << 20, 3, C.byref(rd), C.byref(cp)), "kl_hbm_probe")
    print(f"read {rd.value:.0f} GB/s, copy {cp.value:.0f} GB/s", flush=True)
    assert 1000 < rd.value < 8000 and 1000 < cp.value < 8000


@pytest.mark.parametrize("n", [1, 7, 32000, 128256, 151936])
def test_argmax_exact(K, O, gpu, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    if n > 10:
        x[n // 3] = x[2 * n // 3] = x.max() + 1.0  # tie: the first index wins
    sz = C.c_size_t(0)
    ok(K.lib.kl_argmax_workspace_size(n, C.byref(sz)))
    ws = K.DeviceArray(sz.value, np.uint8, zero=True)
    dx, di = D(K, x), K.DeviceArray(1, np.int32)
    for _ in range(2):
        ok(K.lib.kl_argmax(dx.ptr, n, di.ptr, ws.ptr, sz.value, None))
        assert di.numpy()[0] == O.argmax(x)
    z = np.array([-0.0, 0.0, -0.0], np.float32)
    dz = D(K, z)
    ok(K.lib.kl_argmax(dz.ptr, 3, di.ptr, ws.ptr, sz.value, None))
    assert di.numpy()[0] == 0
