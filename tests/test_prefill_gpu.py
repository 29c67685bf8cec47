"""Batched prompt prefill: the MFMA GEMM, batched RoPE and causal attention
ops, and kl_engine_prefill, against the CPU oracle (which, like the
reference, runs the prompt token by token).

Bars: GEMM rows within the fp32 GEMV bound of the oracle's MatmulKernel on the
same row; RoPE rows bit-exact (elementwise); attention within 2e-5 of the
oracle's MHA at each position; whole-prompt logits within 1e-4 relative
(max |gpu - cpu| / max |cpu|) and the greedy tokens identical.  cfg 5's shape
at 2 layers (narrow FFN and vocabulary) runs its 512-token prefill here; the
full-size cfg 3 / 4 / 5 workloads are in test_fullsize_gpu.py.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LOGIT_RTOL = 1e-4


def D(K, a):
    return K.DeviceArray.from_numpy(np.ascontiguousarray(a))


def ok(rc, what="call"):
    assert rc == 0, f"{what}: rc={rc}"


def rel(a, b):
    return float(np.max(np.abs(a.astype(np.float64) - b)) / max(np.max(np.abs(b)), 1e-30))


def gemm(K, A, W, bias=None, C0=None):
    M, Kd = A.shape
    N = W.shape[0]
    dA, dW = D(K, A), D(K, W)
    dC = D(K, C0) if C0 is not None else K.DeviceArray(M * N)
    db = D(K, bias) if bias is not None else None
    ok(K.lib.kl_gemm_f32(dA.ptr, dW.ptr, dC.ptr, M, N, Kd, Kd, Kd, N, db.ptr if db else None,
                         int(C0 is not None), None), "kl_gemm_f32")
    return dC.numpy().reshape(M, N)


# ---------------------------------------------------------------- GEMM ------
def test_gemm_kat_exact(K, O, gpu):
    # test_load.cpp:49-105 and test_cu_matmul.cpp's 4x4 arange, as GEMM rows.
    W = np.arange(2048, dtype=np.float32).reshape(16, 128)
    y = gemm(K, np.ones((3, 128), np.float32), W)
    for r in range(3):
        for i, v in {0: 8128, 1: 24512, 14: 237504, 15: 253888}.items():
            assert y[r, i] == v
    W4 = np.arange(16, dtype=np.float32).reshape(4, 4)
    y = gemm(K, np.arange(4, dtype=np.float32).reshape(1, 4), W4)
    assert list(y[0]) == [14, 38, 62, 86]


@pytest.mark.parametrize("M,N,Kd", [(1, 3, 4), (5, 37, 12), (64, 64, 64), (77, 300, 256),
                                    (512, 1024, 2560), (130, 2560, 4096), (512, 9728, 512),
                                    (1000, 256, 1536), (33, 70, 100), (65, 129, 36),
                                    (512, 16384, 96), (300, 33000, 64)])
def test_gemm_vs_oracle_rows(K, O, gpu, M, N, Kd):
    """fp32 GEMM rows against the oracle's GEMV within the fp32 rounding bound.
    (512, 16384) and (300, 33000) have at least 1024 tiles of 128 x 64 and
    run the tall-tile kernel (the latter with partial tiles in both dims)."""
    rng = np.random.default_rng(M * 7 + N + Kd)
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    W = (rng.standard_normal((N, Kd)) * 0.02).astype(np.float32)
    y = gemm(K, A, W)
    rows = sorted(set(np.linspace(0, M - 1, min(M, 24)).astype(int)))
    for m in rows:
        ref = O.gemv_f32(A[m], W)
        tol = 4e-7 * np.sqrt(Kd) * (np.abs(W) @ np.abs(A[m])).max() + 1e-30
        assert np.max(np.abs(y[m] - ref)) <= tol, (m, np.max(np.abs(y[m] - ref)), tol)


def test_gemm_bias_and_accumulate(K, O, gpu):
    rng = np.random.default_rng(5)
    M, N, Kd = 70, 200, 96
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    W = rng.standard_normal((N, Kd)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    yb = gemm(K, A, W, bias=b)      # matmul.cpp:74-77: y = W x, then y += b
    ya = gemm(K, A, W, C0=C0)       # llama3.cpp:682-683: x = x + W x'
    for m in range(M):
        g = O.gemv_f32(A[m], W)
        tol = 4e-7 * np.sqrt(Kd) * (np.abs(W) @ np.abs(A[m])).max()
        assert np.max(np.abs(yb[m] - O.add(g, b))) <= tol + 1e-6
        assert np.max(np.abs(ya[m] - O.add(C0[m], g))) <= tol + 1e-6


def test_gemm_grouped_matches_single(K, O, gpu):
    """Three outputs over one A (the Q, K, V projections) in one launch."""
    rng = np.random.default_rng(9)
    M, Kd = 90, 160
    Ns = [256, 64, 64]
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    Ws = [(rng.standard_normal((n, Kd)) * 0.05).astype(np.float32) for n in Ns]
    bs = [rng.standard_normal(n).astype(np.float32) for n in Ns]
    dA = D(K, A)
    dW = [D(K, w) for w in Ws]
    dC = [K.DeviceArray(M * n) for n in Ns]
    db = [D(K, b) for b in bs]
    P3 = C.c_void_p * 3
    I3 = C.c_int * 3
    ok(K.lib.kl_gemm_f32_grouped(dA.ptr, M, Kd, Kd, 3, P3(*[w.ptr for w in dW]),
                                 P3(*[c.ptr for c in dC]), P3(*[b.ptr for b in db]), I3(*Ns),
                                 I3(Kd, Kd, Kd), I3(*Ns), 0, None), "grouped")
    for w, b, c, n in zip(Ws, bs, dC, Ns):
        y = c.numpy().reshape(M, n)
        assert np.array_equal(y, gemm(K, A, w, bias=b))  # same kernel, same order


# --------------------------------------------- split-product GEMM (x6) ------
def _bf16_rne(x):
    """fp32 -> the nearest bf16 (ties to even), as fp32 (finite inputs)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)


def _split3_ref(x):
    """x0 = bf16(x), x1 = bf16(x - x0), x2 = bf16(x - x0 - x1); the fp32
    differences are exact (x0 holds x's leading bits)."""
    x = np.asarray(x, np.float32)
    x0 = _bf16_rne(x)
    r1 = (x - x0).astype(np.float32)
    x1 = _bf16_rne(r1)
    x2 = _bf16_rne((r1 - x1).astype(np.float32))
    return x0, x1, x2


def _as_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def _untile(buf, rows, cols):
    """Planes [3][rows][cols] from the tiled plane format: tiles of 16 rows x
    32 columns, row-tile-major, each tile plane 0, 1, 2 of 16 x 32 in turn."""
    rt, kt = (rows + 15) // 16, cols // 32
    t = buf[: rt * kt * 1536].reshape(rt, kt, 3, 16, 32)
    return t.transpose(2, 0, 3, 1, 4).reshape(3, rt * 16, cols)[:, :rows]


def _split_dev(K, X):
    """kl_split_bf16x3 of X (rows x cols, row stride cols + 4)."""
    rows, cols = X.shape
    Xp = np.zeros((rows, cols + 4), np.float32)
    Xp[:, :cols] = X
    dX = D(K, Xp)
    nbytes = K.lib.kl_split_bf16x3_bytes(rows, cols)
    assert nbytes == ((rows + 15) // 16) * 16 * cols * 6
    dP = K.DeviceArray(nbytes // 2, np.uint16)
    ok(K.lib.kl_split_bf16x3(dX.ptr, rows, cols, cols + 4, dP.ptr, None), "split")
    return dP


def test_split_bf16x3_bit_exact(K, gpu):
    rng = np.random.default_rng(11)
    rows, cols = 37, 256
    X = (rng.standard_normal((rows, cols)) * 10.0 ** rng.integers(-20, 20, (rows, cols))).astype(np.float32)
    X[0, :8] = [0.0, -0.0, 1.0, -1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -9, 3.0e38, -1.5e-30]
    got = _untile(_split_dev(K, X).numpy(), rows, cols)
    refs = _split3_ref(X)
    for p in range(3):
        assert np.array_equal(_as_f32(got[p]).view(np.uint32), refs[p].view(np.uint32)), f"plane {p}"
    # the planes hold x exactly (24 significand bits in 8 + 8 + 8)
    x0, x1, x2 = (r.astype(np.float64) for r in refs)
    finite = np.abs(X) < 1e37
    assert np.array_equal((x0 + x1 + x2)[finite], X.astype(np.float64)[finite])


def gemm_x6(K, A, W, bias=None, C0=None, ws=True, ldc=None):
    """C (M x N, row stride ldc) = A W^T (+ bias) (+ C0); returns the M x N part."""
    M, Kd = A.shape
    N = W.shape[0]
    ldc = ldc or N
    dA, dW = _split_dev(K, A), _split_dev(K, W)
    C = np.full((M, ldc), np.nan, np.float32)
    if C0 is not None:
        C[:, :N] = C0
    dC = D(K, C)
    db = D(K, bias) if bias is not None else None
    wsa = K.DeviceArray(8 * M * N) if ws else None
    ok(K.lib.kl_gemm_x6(dA.ptr, dW.ptr, dC.ptr, M, N, Kd, ldc, db.ptr if db else None,
                        int(C0 is not None), wsa.ptr if wsa else None, wsa.nbytes if wsa else 0,
                        None), "kl_gemm_x6")
    out = dC.numpy().reshape(M, ldc)
    assert np.all(np.isnan(out[:, N:])), "columns past N of a row were written"
    return out[:, :N]


def test_gemm_x6_kat_six_terms_exact(K, gpu):
    """a = s_m sigma_k c, w = t_n sigma_k c with c = 1 + 2^-9 + 2^-17 (planes
    exactly 1, 2^-9, 2^-17), K = 32: every partial sum is exact in fp32, so
    the product is exactly 32 s_m t_n (1 + 2^-8 + 2^-16 + 2^-18), the six
    terms Ai Wj with i + j <= 2 (x0 w0; x0 w1 + x1 w0 = 2^-8; x0 w2 + x2 w0 =
    2^-16; x1 w1 = 2^-18).  A missing or mis-paired term moves it by at least
    32 |s t| 2^-18, a whole number of fp32 ulps."""
    c = np.float32(1 + 2 ** -9 + 2 ** -17)
    M, N, Kd = 130, 200, 32
    s = np.array([(-1) ** (m % 3) * 2.0 ** (m % 5 - 2) for m in range(M)], np.float32)
    t = np.array([(-1) ** (n % 2) * 2.0 ** (n % 7 - 3) for n in range(N)], np.float32)
    sig = np.array([(-1) ** (k % 3 == 1) for k in range(Kd)], np.float32)
    A = (s[:, None] * sig[None, :] * c).astype(np.float32)
    W = (t[:, None] * sig[None, :] * c).astype(np.float32)
    assert [float(v[0, 0]) for v in _split3_ref(np.array([[c]]))] == [1.0, 2 ** -9, 2 ** -17]
    want = (32 * (1 + 2 ** -8 + 2 ** -16 + 2 ** -18) * np.outer(s.astype(np.float64), t)).astype(np.float32)
    for ws in (False, True):
        y = gemm_x6(K, A, W, ws=ws)
        assert np.array_equal(y, want), np.max(np.abs(y - want))
    # each of the six terms is visible in fp32: dropping any one changes every output
    st = np.outer(s.astype(np.float64), t)
    for term in (1.0, 2 ** -9, 2 ** -17, 2 ** -18):
        less = (32 * (1 + 2 ** -8 + 2 ** -16 + 2 ** -18 - term) * st).astype(np.float32)
        assert not np.any(less == want)


X6_TOL = 1e-6  # |C - A W^T| <= X6_TOL * (|A| |W|^T), elementwise (fp32 GEMMs here: <= 2.2e-7)


@pytest.mark.parametrize("M,N,Kd", [(1, 64, 32), (37, 200, 96), (300, 1000, 256), (513, 130, 1024),
                                    (512, 2560, 4096), (1024, 1536, 1536), (129, 257, 64),
                                    (512, 20000, 512), (300, 33000, 128)])
def test_gemm_x6_vs_fp64(K, gpu, M, N, Kd):
    """Within an fp32 GEMM's error of the exact product, with and without the
    split-K workspace (the launcher picks the tile and the split count; the
    narrow, deep shapes split; (512, 20000) and (300, 33000) have more than a
    round of 256 x 128 tiles and run whole rounds plus a split-K launch over
    the last columns, the latter with ragged rows and columns)."""
    rng = np.random.default_rng(M + 3 * N + Kd)
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    W = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float32)
    exact = A.astype(np.float64) @ W.astype(np.float64).T
    mag = np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64).T
    for ws in (False, True):
        y = gemm_x6(K, A, W, ws=ws)
        err = np.max(np.abs(y - exact) / mag)
        print(f"x6 {M}x{N}x{Kd} ws={ws}: max err / sum|aw| {err:.2e}", flush=True)
        assert err <= X6_TOL


@pytest.mark.parametrize("M,N,Kd,ldc", [(70, 200, 96, 200), (70, 200, 96, 212), (300, 33000, 128, 33012)])
def test_gemm_x6_bias_accumulate(K, gpu, M, N, Kd, ldc):
    """Bias and accumulation into C with a row stride past N; (300, 33000)
    runs whole rounds of 256 x 128 tiles plus a split-K launch over the last
    columns, whose output, bias and weight planes start past column 0."""
    rng = np.random.default_rng(21 + N)
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    W = rng.standard_normal((N, Kd)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    exact = A.astype(np.float64) @ W.astype(np.float64).T
    mag = np.abs(A).astype(np.float64) @ np.abs(W).astype(np.float64).T
    yb = gemm_x6(K, A, W, bias=b, ldc=ldc)
    ya = gemm_x6(K, A, W, bias=b, C0=C0, ldc=ldc)
    assert np.max(np.abs(yb - (exact + b)) / (mag + np.abs(b))) <= X6_TOL
    assert np.max(np.abs(ya - (exact + b + C0)) / (mag + np.abs(b) + np.abs(C0))) <= X6_TOL


def test_gemm_x6_refusals(K, gpu):
    rng = np.random.default_rng(21)
    M, N, Kd = 70, 200, 96
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    dP = _split_dev(K, A)
    dC = K.DeviceArray(M * N)
    # K not a multiple of 32; ldc < N; a missing operand (all refused before any launch)
    assert K.lib.kl_gemm_x6(dP.ptr, dP.ptr, dC.ptr, M, N, 80, N, None, 0, None, 0, None) == -4
    assert K.lib.kl_gemm_x6(dP.ptr, dP.ptr, dC.ptr, M, N, Kd, N - 1, None, 0, None, 0, None) == -1
    assert K.lib.kl_gemm_x6(dP.ptr, None, dC.ptr, M, N, Kd, N, None, 0, None, 0, None) == -1
    assert K.lib.kl_split_bf16x3(dC.ptr, M, 80, 80, dP.ptr, None) == -4  # cols % 32


def _bf16_exact(x):
    """x rounded to the nearest bf16 value (ties to even), kept as fp32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).reshape(np.shape(x))


@pytest.mark.parametrize("M,N,Kd", [(37, 200, 96), (512, 2560, 4096), (300, 33000, 128), (1024, 1536, 1536)])
def test_gemm_x6w_one_plane(K, gpu, M, N, Kd):
    """bf16-exact W (as exported from bf16 checkpoints): kl_x6_weight_planes
    finds planes 1 and 2 zero, and the one-plane product (three terms) gives
    exactly kl_gemm_x6's values, with and without the split-K workspace (the
    (300, 33000) shape runs the tail launch).  On W that is not bf16-exact the
    planes are reported as needed, and the one-plane product drops their
    terms (about 2^-9 of each product)."""
    rng = np.random.default_rng(M + N + Kd)
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    Wf = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float32)
    W = _bf16_exact(Wf)
    dA, dW, dWf = _split_dev(K, A), _split_dev(K, W), _split_dev(K, Wf)
    used = C.c_int(0)
    ok(K.lib.kl_x6_weight_planes(dW.ptr, N, Kd, C.byref(used), None), "kl_x6_weight_planes")
    assert used.value == 1
    ok(K.lib.kl_x6_weight_planes(dWf.ptr, N, Kd, C.byref(used), None), "kl_x6_weight_planes")
    assert used.value == 3
    for ws in (False, True):
        wsa = K.DeviceArray(8 * M * N) if ws else None
        outs = []
        for fn in ("x6", "x6w"):
            dC = K.DeviceArray(M * N)
            args = (dC.ptr, M, N, Kd, N, None, 0, wsa.ptr if wsa else None, wsa.nbytes if wsa else 0, None)
            if fn == "x6":
                ok(K.lib.kl_gemm_x6(dA.ptr, dW.ptr, *args), "kl_gemm_x6")
            else:
                ok(K.lib.kl_gemm_x6w(dA.ptr, dW.ptr, 1, *args), "kl_gemm_x6w")
            outs.append(dC.numpy().reshape(M, N))
        assert np.array_equal(outs[0], outs[1]), (ws, np.max(np.abs(outs[0] - outs[1])))
    # not bf16-exact: the one-plane product leaves out W's planes 1 and 2
    d6, d1 = K.DeviceArray(M * N), K.DeviceArray(M * N)
    ok(K.lib.kl_gemm_x6(dA.ptr, dWf.ptr, d6.ptr, M, N, Kd, N, None, 0, None, 0, None), "kl_gemm_x6")
    ok(K.lib.kl_gemm_x6w(dA.ptr, dWf.ptr, 1, d1.ptr, M, N, Kd, N, None, 0, None, 0, None), "kl_gemm_x6w")
    y6, y1 = d6.numpy().reshape(M, N), d1.numpy().reshape(M, N)
    mag = np.abs(A).astype(np.float64) @ np.abs(Wf).astype(np.float64).T
    assert np.max(np.abs(y1 - y6) / mag) > 1e-6 and np.max(np.abs(y1 - y6) / mag) < 2 ** -8
    assert K.lib.kl_gemm_x6w(dA.ptr, dW.ptr, 2, d1.ptr, M, N, Kd, N, None, 0, None, 0, None) == -1


@pytest.mark.parametrize("splits", [1, 2, 3, 4])
def test_gemm_splitk_vs_oracle(K, O, gpu, splits):
    rng = np.random.default_rng(splits)
    M, N, Kd = 100, 192, 1024
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    W = (rng.standard_normal((N, Kd)) * 0.02).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    dA, dW, dC = D(K, A), D(K, W), D(K, C0)
    ws = K.DeviceArray(splits * M * N)
    ok(K.lib.kl_gemm_f32_splitk(dA.ptr, dW.ptr, dC.ptr, M, N, Kd, Kd, Kd, N, None, 1, splits,
                                ws.ptr, ws.nbytes, None), "splitk")
    y = dC.numpy().reshape(M, N)
    for m in range(0, M, 7):
        g = O.gemv_f32(A[m], W)
        tol = 4e-7 * np.sqrt(Kd) * (np.abs(W) @ np.abs(A[m])).max() + 1e-6
        assert np.max(np.abs(y[m] - O.add(C0[m], g))) <= tol
    if splits > 1:  # a workspace too small is refused before any launch
        assert K.lib.kl_gemm_f32_splitk(dA.ptr, dW.ptr, dC.ptr, M, N, Kd, Kd, Kd, N, None, 1,
                                        splits, ws.ptr, ws.nbytes - 4, None) == -6


@pytest.mark.parametrize("M,N,Kd,splits", [(1, 1, 32, 1), (3, 65, 64, 1), (65, 1, 96, 1), (64, 64, 32, 1),
                                            (70, 130, 160, 1), (5, 200, 32, 4), (129, 96, 96, 2),
                                            (200, 70, 2560, 3)])
def test_gemm_k32_blocks_vs_oracle(K, O, gpu, M, N, Kd, splits):
    """K a whole number of 32-column blocks (the direct-to-LDS kernel): one
    block, odd and even block counts (the loop runs blocks in pairs), single
    rows and columns (edge tiles clamp their loads), and more splits than
    blocks (empty splits contribute zeros); accumulate into C with a bias."""
    rng = np.random.default_rng(M * 131 + N * 7 + Kd + splits)
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    W = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    dA, dW, dC, db = D(K, A), D(K, W), D(K, C0), D(K, b)
    ws = K.DeviceArray(max(1, splits * M * N))
    ok(K.lib.kl_gemm_f32_splitk(dA.ptr, dW.ptr, dC.ptr, M, N, Kd, Kd, Kd, N, db.ptr, 1, splits,
                                ws.ptr, ws.nbytes, None), "splitk")
    y = dC.numpy().reshape(M, N)
    for m in range(M):
        want = C0[m].astype(np.float64) + O.gemv_f32(A[m], W) + b
        tol = 4e-7 * np.sqrt(Kd) * (np.abs(W) @ np.abs(A[m])).max() + 1e-6
        assert np.max(np.abs(y[m] - want)) <= tol, (m, np.max(np.abs(y[m] - want)))


def test_gemm_rejects_unaligned_k(K, gpu):
    buf = K.DeviceArray(64)
    assert K.lib.kl_gemm_f32(buf.ptr, buf.ptr, buf.ptr, 2, 2, 3, 3, 3, 2, None, 0, None) == -4
    assert K.lib.kl_gemm_f32(buf.ptr, buf.ptr, buf.ptr, 0, 2, 4, 4, 4, 2, None, 0, None) == -1


# ---------------------------------------------------------------- RoPE ------
@pytest.mark.parametrize("style,dim,kv,hd,pos0,n", [(0, 768, 768, 64, 0, 16), (1, 2048, 512, 64, 5, 33),
                                                    (1, 4096, 1024, 128, 0, 70)])
def test_rope_rows_bit_exact(K, O, gpu, style, dim, kv, hd, pos0, n):
    S = pos0 + n
    s, c = O.sincos_table(hd, S, 1e4 if style == 0 else 1e6)
    rng = np.random.default_rng(dim + n)
    q = rng.standard_normal((n, dim)).astype(np.float32)
    k = rng.standard_normal((n, kv)).astype(np.float32)
    dq, dk, dsn, dcs = D(K, q), D(K, k), D(K, s), D(K, c)
    ok(K.lib.kl_rope_rows(style, dim, kv, hd, dq.ptr, dim, dk.ptr, kv, pos0, n, dsn.ptr, dcs.ptr,
                          None))
    gq, gk = dq.numpy().reshape(n, dim), dk.numpy().reshape(n, kv)
    for r in range(n):
        rq, rk = O.rope(style, dim, kv, hd, q[r], k[r], pos0 + r, s, c)
        assert np.array_equal(gq[r], rq) and np.array_equal(gk[r], rk), r


# ----------------------------------------------------------- attention ------
@pytest.mark.parametrize("H,kvm,hd,S,pos0,n", [(12, 1, 64, 160, 0, 143), (32, 4, 128, 256, 0, 200),
                                              (4, 2, 32, 80, 17, 50), (12, 6, 128, 4096, 3900, 100),
                                              (8, 8, 64, 70, 0, 1), (8, 2, 64, 300, 130, 70),
                                              (4, 2, 256, 200, 0, 150), (2, 2, 256, 160, 37, 100)])
@pytest.mark.parametrize("attn", ["split", "f32"])
def test_attn_prefill_vs_oracle(K, O, gpu, monkeypatch, attn, H, kvm, hd, S, pos0, n):
    """Head size 128 runs the split-bf16-product kernel by default and the
    fp32 matrix-core one with KL_PREFILL_ATTN=f32 (read per launch); both
    against the oracle's MHA."""
    if attn == "f32":
        if hd != 128:
            pytest.skip("one kernel for this head size")
        monkeypatch.setenv("KL_PREFILL_ATTN", "f32")
    rng = np.random.default_rng(H * S + pos0 + n)
    kvd = H // kvm * hd
    kc = rng.standard_normal((1, S, kvd)).astype(np.float32)
    vc = rng.standard_normal((1, S, kvd)).astype(np.float32)
    q = rng.standard_normal((n, H * hd)).astype(np.float32)
    dk, dv, dq, do = D(K, kc.ravel()), D(K, vc.ravel()), D(K, q), K.DeviceArray(n * H * hd)
    ok(K.lib.kl_attn_prefill(pos0, n, H, kvm, hd, dq.ptr, H * hd, dk.ptr, dv.ptr, kvd, do.ptr,
                             H * hd, None), "kl_attn_prefill")
    out = do.numpy().reshape(n, H * hd)
    rows = sorted(set(np.linspace(0, n - 1, min(n, 16)).astype(int)))
    for r in rows:
        ref = O.mha(pos0 + r, H, 0, S, kvd, kvm, hd, q[r], kc, vc)
        assert np.max(np.abs(out[r] - ref)) < 2e-5, r
    if pos0 == 0:  # position 0 attends only key 0: V0 exactly up to the 1/l factor (l = 1)
        for h in range(H):
            g = h // kvm
            assert np.allclose(out[0, h * hd:(h + 1) * hd], vc[0, 0, g * hd:(g + 1) * hd], rtol=0,
                               atol=1e-7)


def _fa_workers(pos0, n, H, cus=256):
    """Stream-K workgroups the launcher picks (0: one workgroup per segment):
    a unit is one (head, 64-row block, 64-key block); row block i < nqb - 1
    walks a + i key blocks, the last one (pos0 + n - 1) // 64 + 1."""
    nqb, a, nk_last = (n + 63) // 64, (pos0 + 63) // 64 + 1, (pos0 + n - 1) // 64 + 1
    m = nqb - 1
    W = (m * a + m * (m - 1) // 2 + nk_last) * H
    G = min(cus, 256, W)
    plain = nk_last if nqb * H <= cus else -(-W // cus) + nk_last
    return G if -(-W // G) < plain else 0


@pytest.mark.parametrize("H,kvm,hd,S,pos0,n", [(4, 2, 128, 3200, 3000, 64), (12, 6, 128, 600, 0, 512),
                                              (12, 6, 128, 1100, 1000, 70), (8, 8, 128, 4096, 3968, 128),
                                              (32, 4, 128, 520, 0, 512), (8, 2, 64, 300, 130, 70),
                                              (6, 3, 128, 400, 30, 300), (2, 1, 128, 2100, 0, 2048),
                                              (16, 4, 64, 700, 0, 640), (64, 8, 128, 64, 0, 16)])
@pytest.mark.parametrize("attn", ["split", "f32"])
def test_attn_prefill_ws_vs_oracle(K, O, gpu, monkeypatch, attn, H, kvm, hd, S, pos0, n):
    """kl_attn_prefill_ws: where the causal segments (64-row block, head) are
    unequal or fewer than the CUs, equal ranges of (row block, key block)
    units per workgroup, cut segments merged afterwards; a second launch on
    the same workspace gives the same bits; rows against the
    oracle's MHA and within 2e-5 of kl_attn_prefill (one workgroup per
    segment).  Cases: one row block far into the context (48 pieces per
    segment), ranges crossing segment boundaries (512 rows from position 0),
    head size 64, a start off the 64 grid (pieces where a row's keys are all
    masked), 2048 rows (long segments over many workgroups), and 16 rows x
    64 heads (one unit per segment: no split).  Head size 128 with both its
    kernels (split bf16 products, default; fp32 products)."""
    if attn == "f32":
        if hd != 128:
            pytest.skip("one kernel for this head size")
        monkeypatch.setenv("KL_PREFILL_ATTN", "f32")
    rng = np.random.default_rng(H * S + pos0 + n + 7)
    kvd = H // kvm * hd
    kc = rng.standard_normal((1, S, kvd)).astype(np.float32)
    vc = rng.standard_normal((1, S, kvd)).astype(np.float32)
    q = rng.standard_normal((n, H * hd)).astype(np.float32)
    dk, dv, dq = D(K, kc.ravel()), D(K, vc.ravel()), D(K, q)
    do, du = K.DeviceArray(n * H * hd), K.DeviceArray(n * H * hd)
    need = C.c_size_t(0)
    ok(K.lib.kl_attn_prefill_workspace_size(n, H, hd, C.byref(need)), "workspace size")
    assert need.value == 2 * 256 * 64 * (hd + 4) * 4
    ws = K.DeviceArray(need.value // 4)
    split = _fa_workers(pos0, n, H) > 0
    assert split == ((H, n) != (64, 16))
    ok(K.lib.kl_attn_prefill_ws(pos0, n, H, kvm, hd, dq.ptr, H * hd, dk.ptr, dv.ptr, kvd, do.ptr,
                                H * hd, ws.ptr, need.value, None), "kl_attn_prefill_ws")
    ok(K.lib.kl_attn_prefill(pos0, n, H, kvm, hd, dq.ptr, H * hd, dk.ptr, dv.ptr, kvd, du.ptr,
                             H * hd, None), "kl_attn_prefill")
    out = do.numpy().reshape(n, H * hd)
    whole = du.numpy().reshape(n, H * hd)
    assert np.all(np.isfinite(out))
    assert np.max(np.abs(out - whole)) < 2e-5
    # a second launch on the same (now dirty) workspace gives the same bits
    ok(K.lib.kl_attn_prefill_ws(pos0, n, H, kvm, hd, dq.ptr, H * hd, dk.ptr, dv.ptr, kvd, du.ptr,
                                H * hd, ws.ptr, need.value, None), "kl_attn_prefill_ws again")
    assert np.array_equal(du.numpy().reshape(n, H * hd), out)
    if split:  # a workspace short of one float is refused before any launch
        assert K.lib.kl_attn_prefill_ws(pos0, n, H, kvm, hd, dq.ptr, H * hd, dk.ptr, dv.ptr, kvd,
                                        do.ptr, H * hd, ws.ptr, need.value - 4, None) == -6
    rows = range(n) if n <= 512 else sorted(set(np.linspace(0, n - 1, 96).astype(int)))
    for r in rows:
        ref = O.mha(pos0 + r, H, 0, S, kvd, kvm, hd, q[r], kc, vc)
        assert np.max(np.abs(out[r] - ref)) < 2e-5, r


@pytest.mark.parametrize("style,hd,H,KVH,pos0,n", [(1, 128, 32, 8, 0, 40), (1, 128, 16, 8, 300, 17),
                                                  (0, 128, 8, 2, 5, 9), (1, 64, 8, 4, 7, 33),
                                                  (0, 64, 4, 4, 0, 5), (1, 128, 3, 2, 4, 3),
                                                  (0, 64, 3, 2, 0, 3), (1, 64, 5, 1, 2, 7)])
def test_qk_norm_rope_rows_matches_two_step(K, O, gpu, style, hd, H, KVH, pos0, n):
    """The fused Qwen3 q/k RMSNorm + RoPE of the prefill against the two-step
    path it replaces (kl_rmsnorm_rows per head, then kl_rope_rows, both pinned
    to the oracle): every element within a few float roundings.  The kernel
    packs 64 / (hd / 4) (row, head) pairs per wave; the last three cases leave
    the last wave partly empty (15, 15 and 42 pairs)."""
    rng = np.random.default_rng(hd * H + pos0 + n + style)
    S = pos0 + n + 4
    q = rng.standard_normal((n, H * hd)).astype(np.float32)
    k = rng.standard_normal((n, KVH * hd)).astype(np.float32)
    qn = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + 0.1 * rng.standard_normal(hd)).astype(np.float32)
    sin_t, cos_t = K.DeviceArray(S * hd), K.DeviceArray(S * hd)
    ok(K.lib.kl_sincos_table(hd, S, 1e6, sin_t.ptr, cos_t.ptr), "kl_sincos_table")
    dq, dk, dqn, dkn = D(K, q), D(K, k), D(K, qn), D(K, kn)
    dq2, dk2 = D(K, q), D(K, k)
    ok(K.lib.kl_qk_norm_rope_rows(style, hd, H, KVH, dq.ptr, H * hd, dk.ptr, KVH * hd, dqn.ptr, dkn.ptr,
                                  1e-6, pos0, n, sin_t.ptr, cos_t.ptr, None), "kl_qk_norm_rope_rows")
    ok(K.lib.kl_rmsnorm_rows(dq2.ptr, dqn.ptr, dq2.ptr, n * H, hd, C.c_float(1e-6), None), "norm q")
    ok(K.lib.kl_rmsnorm_rows(dk2.ptr, dkn.ptr, dk2.ptr, n * KVH, hd, C.c_float(1e-6), None), "norm k")
    ok(K.lib.kl_rope_rows(style, H * hd, KVH * hd, hd, dq2.ptr, H * hd, dk2.ptr, KVH * hd, pos0, n,
                          sin_t.ptr, cos_t.ptr, None), "kl_rope_rows")
    for a, b in ((dq, dq2), (dk, dk2)):
        x, y = a.numpy(), b.numpy()
        assert np.max(np.abs(x - y)) <= 4e-7 * np.max(np.abs(y)), np.max(np.abs(x - y))
    # tables not 16-byte aligned are refused before any launch
    assert K.lib.kl_qk_norm_rope_rows(style, hd, H, KVH, dq.ptr, H * hd, dk.ptr, KVH * hd, dqn.ptr,
                                      dkn.ptr, 1e-6, pos0, n, C.c_void_p(sin_t.ptr.value + 4), cos_t.ptr,
                                      None) == -4


# ------------------------------------------------------- whole prompt -------
PREFILL_TINY = ["tiny_llama2", "tiny_llama3", "tiny_qwen2", "tiny_qwen3", "tiny_q8", "tiny_qwen2_q8"]


def test_engine_prefill_f32_gemm_path(K, O, gpu, monkeypatch):
    """KL_PREFILL_GEMM=f32 keeps the fp32 matrix-core GEMMs: same bars, and
    logits close to the default (split-product) engine's."""
    cfg = K.TINY["tiny_llama3"]
    img = K.synth_image(cfg)
    P = 40
    prompt = [int(t) for t in K.prompt_tokens(cfg, P)]
    _, lg6, _ = K.Engine(img, cfg).prefill(prompt)
    monkeypatch.setenv("KL_PREFILL_GEMM", "f32")
    nxt, lg, _ = K.Engine(img, cfg).prefill(prompt)
    om = O.Model(img, cfg.family, cfg.quant)
    for pos in range(P - 1):
        om.step(prompt[pos], pos)
    ref = om.step(prompt[P - 1], P - 1)
    assert rel(lg, ref) < LOGIT_RTOL and rel(lg6, ref) < LOGIT_RTOL
    assert not np.array_equal(lg, lg6)  # the two paths did run
    assert nxt == int(np.argmax(lg))


@pytest.mark.parametrize("name", ["tiny_llama3", "tiny_qwen3", "tiny_qwen2_q8"])
def test_engine_prefill_small_chunks_vs_oracle(K, O, gpu, monkeypatch, name):
    """A prompt longer than a prefill pass (KL_PREFILL_CHUNK=64: passes of 64,
    64 and 22 rows, each attending the cache rows of the passes before it)
    against the oracle's token-by-token run: the last logits, the cache rows
    on both sides of each pass boundary, and decoding on from the cache."""
    monkeypatch.setenv("KL_PREFILL_CHUNK", "64")
    cfg = K.TINY[name].with_(seq_len=256)
    img = K.synth_image(cfg)
    P = 150
    prompt = [int(t) for t in K.prompt_tokens(cfg, P)]
    eng = K.Engine(img, cfg)
    nxt, lg, _ = eng.prefill(prompt)
    om = O.Model(img, cfg.family, cfg.quant)
    for pos in range(P - 1):
        om.step(prompt[pos], pos)
    ref = om.step(prompt[P - 1], P - 1)
    assert rel(lg, ref) < LOGIT_RTOL
    for layer in (0, cfg.layers - 1):
        for pos in (0, 63, 64, 127, 128, P - 1):
            for which_v in (False, True):
                a, b = eng.kv_row(layer, pos, which_v), om.kv_row(layer, pos, which_v)
                assert np.max(np.abs(a - b)) <= 1e-5 * max(np.max(np.abs(b)), 1.0), (layer, pos)
    tok = O.argmax(ref)
    for pos in range(P, P + 4):
        _, lg2 = eng.step(tok, pos)
        ref2 = om.step(tok, pos)
        assert rel(lg2, ref2) < LOGIT_RTOL
        tok = O.argmax(ref2)


@pytest.mark.parametrize("name", ["tiny_llama3", "tiny_qwen3", "qwen3_shape"])
def test_engine_prefill_bf16_exact_weights(K, O, gpu, name):
    """An image whose weights are all bf16 values (every float past the
    header rounded to bf16): the engine finds every projection's planes 1 and
    2 zero and runs the one-plane products; the prompt's last logits and cache
    rows against the oracle on the same image."""
    if name == "qwen3_shape":
        cfg = K.BASELINE["qwen3_4b"].with_(name="qwen3_shape_bf16", layers=2, hidden_dim=1024,
                                           vocab=2048, norm_std=0.1)
        P = 512
    else:
        cfg = K.TINY[name]
        P = 40
    img = K.synth_image(cfg).copy()
    body = img[256:256 + (img.size - 256) // 4 * 4].view(np.float32)
    img[256:256 + body.size * 4] = _bf16_exact(body).view(np.uint8)
    prompt = [int(t) for t in K.prompt_tokens(cfg, P)]
    eng = K.Engine(img, cfg)
    nxt, lg, ms = eng.prefill(prompt)
    om = O.Model(img, cfg.family, cfg.quant)
    ref = om.prompt(prompt) if P > 64 else None
    if ref is None:
        for pos in range(P - 1):
            om.step(prompt[pos], pos)
        ref = om.step(prompt[P - 1], P - 1)
    r = rel(lg, ref)
    print(f"{name} bf16-exact weights: prefill P={P} in {ms:.2f} ms, logits rel err {r:.2e}", flush=True)
    assert r < LOGIT_RTOL
    for layer in (0, cfg.layers - 1):
        for pos in (0, P - 1):
            for which_v in (False, True):
                a, b = eng.kv_row(layer, pos, which_v), om.kv_row(layer, pos, which_v)
                assert np.max(np.abs(a - b)) <= 1e-5 * max(np.max(np.abs(b)), 1.0)


def _prefill_cfg(K, name):
    if name == "tiny_hd256":  # head size 256 (the VALU attention with 32-key blocks)
        return K.TINY["tiny_llama2"].with_(name="tiny_hd256", dim=512, hidden_dim=768, heads=2,
                                          kv_heads=1, vocab=600, seq_len=96)
    return K.TINY[name]


@pytest.mark.parametrize("name", PREFILL_TINY + ["tiny_hd256"])
def test_engine_prefill_vs_oracle(K, O, gpu, name):
    cfg = _prefill_cfg(K, name)
    assert name != "tiny_hd256" or cfg.head_size == 256
    img = K.synth_image(cfg)
    P = min(40, cfg.seq_len - 10)
    prompt = [int(t) for t in K.prompt_tokens(cfg, P)]
    eng = K.Engine(img, cfg)
    nxt, lg, ms = eng.prefill(prompt)
    om = O.Model(img, cfg.family, cfg.quant)
    for pos in range(P - 1):
        om.step(prompt[pos], pos)
    ref = om.step(prompt[P - 1], P - 1)
    r = rel(lg, ref)
    print(f"{name}: prefill P={P} logits rel err {r:.2e}, {ms:.3f} ms", flush=True)
    assert r < LOGIT_RTOL
    assert nxt == int(np.argmax(lg))
    want = O.argmax(ref)
    if nxt != want:
        assert abs(float(ref[nxt]) - float(ref[want])) <= LOGIT_RTOL * np.max(np.abs(ref))
    # The cache rows the prefill wrote are the ones the step path writes.
    for layer in (0, cfg.layers - 1):
        for pos in (0, P // 2, P - 1):
            for which_v in (False, True):
                a, b = eng.kv_row(layer, pos, which_v), om.kv_row(layer, pos, which_v)
                assert np.max(np.abs(a - b)) <= 1e-5 * max(np.max(np.abs(b)), 1.0)
    # Decoding continues from the prefilled cache (teacher-forced on the oracle's tokens).
    tok = want
    for pos in range(P, P + 4):
        n2, lg2 = eng.step(tok, pos)
        ref2 = om.step(tok, pos)
        assert rel(lg2, ref2) < LOGIT_RTOL
        tok = O.argmax(ref2)


@pytest.mark.parametrize("shape", ["llama2_7b_q8", "qwen25_15b"])
def test_engine_prefill_q8_short_prompt_vs_oracle(K, O, gpu, shape):
    """A 32-token int8 prompt (the short-prompt int8 GEMMs, split along K) on
    two layers of a full-width shape: Llama2-7B (interleaved RoPE) and
    Qwen2.5-1.5B with int8 weights (QKV bias, rotate-half RoPE).  Q/K/V's
    partials are summed, biased and rotated in one pass.  Last logits, cache
    rows and four decode steps against the oracle."""
    cfg = K.BASELINE[shape].with_(name=f"{shape}_int8_2l", layers=2, vocab=2048, group_size=64,
                                  norm_std=0.1, tied=False)  # int8 images keep their classifier
    assert cfg.quant
    img = K.synth_image(cfg)
    P = 32
    prompt = [int(t) for t in K.prompt_tokens(cfg, P)]
    eng = K.Engine(img, cfg)
    nxt, lg, ms = eng.prefill(prompt)
    om = O.Model(img, cfg.family, cfg.quant)
    for pos in range(P - 1):
        om.step(prompt[pos], pos)
    ref = om.step(prompt[P - 1], P - 1)
    r = rel(lg, ref)
    print(f"{cfg.name}: prefill P={P} logits rel err {r:.2e}, {ms:.3f} ms", flush=True)
    assert r < LOGIT_RTOL
    for layer in (0, cfg.layers - 1):
        for pos in (0, 17, P - 1):
            for which_v in (False, True):
                a, b = eng.kv_row(layer, pos, which_v), om.kv_row(layer, pos, which_v)
                assert np.max(np.abs(a - b)) <= 1e-5 * max(np.max(np.abs(b)), 1.0), (layer, pos, which_v)
    tok = O.argmax(ref)
    for pos in range(P, P + 4):
        _, lg2 = eng.step(tok, pos)
        ref2 = om.step(tok, pos)
        assert rel(lg2, ref2) < LOGIT_RTOL
        tok = O.argmax(ref2)


def test_qwen3_shape_prefill_512_vs_oracle(K, O, gpu):
    """cfg 5's layer shape (Qwen3: dim 2560, 32 Q / 8 KV heads of 128, q/k
    norms) at 2 layers with non-unit norm weights: the 512-token prompt as one
    batched prefill against the oracle's token-by-token run, then 8 greedy
    decode steps in the persistent mode from the prefilled cache."""
    cfg = K.BASELINE["qwen3_4b"].with_(name="qwen3_shape_2l", layers=2, hidden_dim=1024,
                                       vocab=2048, norm_std=0.1)
    img = K.synth_image(cfg)
    P = 512
    prompt = [int(t) for t in K.prompt_tokens(cfg, P)]
    eng = K.Engine(img, cfg)
    eng.set_mode(K.MODE_PERSISTENT)
    assert eng.mode == K.MODE_PERSISTENT
    nxt, lg, ms = eng.prefill(prompt)
    om = O.Model(img, cfg.family, cfg.quant)
    ref = om.prompt(prompt)
    r = rel(lg, ref)
    print(f"qwen3 shape: prefill of {P} tokens in {ms:.2f} ms, logits rel err {r:.2e}", flush=True)
    assert r < LOGIT_RTOL
    want = O.argmax(ref)
    assert nxt == want, float(ref[want]) - float(ref[nxt])
    for layer in (0, 1):
        for pos in (0, 255, 511):
            for which_v in (False, True):
                a, b = eng.kv_row(layer, pos, which_v), om.kv_row(layer, pos, which_v)
                assert np.max(np.abs(a - b)) <= 1e-5 * max(np.max(np.abs(b)), 1.0)
    tok = want
    for pos in range(P, P + 8):
        n2, lg2 = eng.step(tok, pos)
        ref2 = om.step(tok, pos)
        assert rel(lg2, ref2) < LOGIT_RTOL, pos
        tok = O.argmax(ref2)
        assert n2 == tok, pos


@pytest.mark.parametrize("name", PREFILL_TINY)
def test_generate_with_prefill_matches_oracle(K, O, gpu, name):
    cfg = K.TINY[name]
    img = K.synth_image(cfg)
    prompt = K.prompt_tokens(cfg, 12)
    eng = K.Engine(img, cfg)
    eng.set_prefill(True)
    got, _ = eng.generate(prompt, 10)
    want = O.Model(img, cfg.family, cfg.quant).generate(prompt, 10)
    assert list(got) == list(want)


@pytest.mark.parametrize("M,N,Kd,gs,splits", [(1, 5, 64, 64, 1), (37, 200, 256, 64, 1),
                                              (100, 192, 1024, 64, 4), (64, 96, 128, 32, 2),
                                              (7, 33, 4096, 128, 3), (32, 300, 512, 64, 8),
                                              (32, 1024, 2048, 64, 16)])
def test_gemm_q8_vs_oracle(K, O, gpu, M, N, Kd, gs, splits):
    """int8 weights (group-wise scales over the flattened matrix): every row of
    C within the fp32 GEMV bound of the oracle's int8 MatmulKernel on that
    row, with bias and accumulate, with and without split-K; M <= 32 runs the
    32 x 128 tiles (N = 300: a partial last tile)."""
    rng = np.random.default_rng(M * 7 + N)
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    Wf = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float32)
    q, s = O.quantize_q8(Wf.reshape(-1), gs)
    bias = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    dA, dq, ds, db, dC = D(K, A), D(K, q), D(K, s), D(K, bias), D(K, C0)
    ws = K.DeviceArray(max(1, splits * M * N))
    ok(K.lib.kl_gemm_q8(dA.ptr, dq.ptr, ds.ptr, gs, dC.ptr, M, N, Kd, Kd, N, db.ptr, 1, splits,
                        ws.ptr, ws.nbytes, None), "kl_gemm_q8")
    y = dC.numpy().reshape(M, N)
    wd = O.dequant_q8(q, s, gs).reshape(N, Kd).astype(np.float64)
    for m in range(M):
        g = O.gemv_q8(A[m], q, s, N, Kd, gs)
        want = C0[m].astype(np.float64) + g + bias
        tol = 4e-7 * np.sqrt(Kd) * (np.abs(wd) @ np.abs(A[m])).max() + 1e-6
        assert np.max(np.abs(y[m] - want)) <= tol, m


def gemm_q8s(K, A, q, s, gs, N, bias=None, C0=None, ws=True):
    M, Kd = A.shape
    pb = K.lib.kl_q8s_packed_bytes(N, Kd, gs)
    assert pb == ((N + 31) // 32) * (Kd * 32 + (Kd // gs) * 128)
    dq, ds, dP = D(K, q), D(K, s), K.DeviceArray(pb, np.uint8)
    ok(K.lib.kl_q8s_pack(dq.ptr, ds.ptr, N, Kd, gs, dP.ptr, None), "kl_q8s_pack")
    dA = D(K, A)
    dC = D(K, C0) if C0 is not None else K.DeviceArray(M * N)
    db = D(K, bias) if bias is not None else None
    wsb = Kd * 192 + (64 * 32 * N * 4 + 256 if ws else 0)
    w = K.DeviceArray(wsb, np.uint8)
    rc = K.lib.kl_gemm_q8s(dA.ptr, M, Kd, Kd, dP.ptr, N, gs, dC.ptr, N, db.ptr if db else None,
                           int(C0 is not None), w.ptr, wsb, None)
    if not ws and Kd > 832:  # one split holds at most 832 columns of K
        assert rc == -6
        return None
    ok(rc, "kl_gemm_q8s")
    return dC.numpy().reshape(M, N)


def test_gemm_q8s_kat_exact(K, gpu):
    """a = s_m sigma_k c (c = 1 + 2^-9 + 2^-17: three exact bf16 planes),
    q = t_n sigma_k, group scales powers of two: every partial sum is exact, so
    C = s_m t_n c 32 (sc_0 + sc_1) exactly; without the third plane it would
    miss 32 |s t| 2^-17 per group."""
    c = np.float32(1 + 2 ** -9 + 2 ** -17)
    M, N, Kd, gs = 19, 100, 64, 32
    sm = np.array([(-1) ** (m % 3) * 2.0 ** (m % 5 - 2) for m in range(M)], np.float32)
    tn = np.array([(-1) ** (n % 2) * (1 << (n % 4)) for n in range(N)], np.int64)
    sig = np.array([(-1) ** (k % 3 == 1) for k in range(Kd)], np.int64)
    A = (sm[:, None] * sig[None, :].astype(np.float32) * c).astype(np.float32)
    q = (tn[:, None] * sig[None, :]).astype(np.int8)
    sc = np.array([[1.0, 2.0] if n % 2 else [0.5, 4.0] for n in range(N)], np.float32).reshape(-1)
    want = np.array([[float(sm[m]) * float(tn[n]) * float(c) * 32 * (sc[2 * n] + sc[2 * n + 1])
                      for n in range(N)] for m in range(M)]).astype(np.float32)
    for ws in (False, True):
        y = gemm_q8s(K, A, q.reshape(-1), sc, gs, N, ws=ws)
        assert np.array_equal(y, want), np.max(np.abs(y - want))


@pytest.mark.parametrize("M,N,Kd,gs", [(1, 64, 64, 64), (5, 300, 256, 32), (32, 1000, 512, 64),
                                       (17, 4096, 4096, 64), (32, 4096, 11008, 64), (3, 100, 1024, 32),
                                       (32, 12288, 4096, 64)])
def test_gemm_q8s_vs_oracle(K, O, gpu, M, N, Kd, gs):
    """The short-prompt int8 GEMM against the oracle's int8 MatmulKernel row by
    row within the fp32 GEMV bound, with bias and accumulate, with and without
    the split-K workspace."""
    rng = np.random.default_rng(M * 13 + N + gs)
    A = rng.standard_normal((M, Kd)).astype(np.float32)
    Wf = (rng.standard_normal((N, Kd)) * 0.05).astype(np.float32)
    q, s = O.quantize_q8(Wf.reshape(-1), gs)
    bias = rng.standard_normal(N).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    wd = O.dequant_q8(q, s, gs).reshape(N, Kd).astype(np.float64)
    for ws in (False, True):
        y = gemm_q8s(K, A, q, s, gs, N, bias=bias, C0=C0, ws=ws)
        if y is None:
            continue
        for m in range(M):
            g = O.gemv_q8(A[m], q, s, N, Kd, gs)
            want = C0[m].astype(np.float64) + g + bias
            tol = 4e-7 * np.sqrt(Kd) * (np.abs(wd) @ np.abs(A[m])).max() + 1e-6
            assert np.max(np.abs(y[m] - want)) <= tol, (ws, m)


def test_gemm_q8s_refusals(K, gpu):
    buf = K.DeviceArray(1 << 16, np.uint8)
    # 33 rows; group size 16; K not a multiple of the group; a workspace short of A's planes
    assert K.lib.kl_gemm_q8s(buf.ptr, 33, 64, 64, buf.ptr, 32, 64, buf.ptr, 32, None, 0, buf.ptr,
                             buf.nbytes, None) == -1
    assert K.lib.kl_gemm_q8s(buf.ptr, 4, 64, 64, buf.ptr, 32, 16, buf.ptr, 32, None, 0, buf.ptr,
                             buf.nbytes, None) == -4
    assert K.lib.kl_gemm_q8s(buf.ptr, 4, 96, 96, buf.ptr, 32, 64, buf.ptr, 32, None, 0, buf.ptr,
                             buf.nbytes, None) == -4
    assert K.lib.kl_gemm_q8s(buf.ptr, 4, 64, 64, buf.ptr, 32, 64, buf.ptr, 32, None, 0, buf.ptr,
                             64 * 192 - 1, None) == -6
    assert K.lib.kl_q8s_packed_bytes(32, 96, 64) == 0
    assert K.lib.kl_q8s_packed_bytes(32, 256, 128) == 0  # groups of 128 take kl_gemm_q8


def test_gemm_q8_rejects_bad_shapes(K, gpu):
    buf = K.DeviceArray(4096)
    # K not a whole number of 32-column blocks; group size not a power of two
    assert K.lib.kl_gemm_q8(buf.ptr, buf.ptr, buf.ptr, 64, buf.ptr, 2, 2, 48, 48, 2, None, 0, 1,
                            None, 0, None) == -4
    assert K.lib.kl_gemm_q8(buf.ptr, buf.ptr, buf.ptr, 48, buf.ptr, 2, 2, 64, 64, 2, None, 0, 1,
                            None, 0, None) == -1
    # split-K without a large enough workspace
    assert K.lib.kl_gemm_q8(buf.ptr, buf.ptr, buf.ptr, 64, buf.ptr, 2, 2, 64, 64, 2, None, 0, 2,
                            buf.ptr, 4, None) == -6
