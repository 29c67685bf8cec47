"""kl_mha_noalloc: kl_mha for callers that cannot allocate.  Its split
partials live in the library's own per-device array, so the caller passes
only the inputs and the output.  Checked against kl_mha (same kernels and
plan, so bit for bit) on two calls in a row, the second on a smaller input,
and its size limit is refused on the host before any launch."""
import ctypes as C

import numpy as np
import pytest


def _shape_args(H, kvm, hd, S, pos, seed):
    rng = np.random.default_rng(seed)
    L, layer = 2, 1
    kvd = H // kvm * hd
    kc = rng.standard_normal((L, S, kvd)).astype(np.float32)
    vc = rng.standard_normal((L, S, kvd)).astype(np.float32)
    q = rng.standard_normal(H * hd).astype(np.float32)
    return layer, kvd, kc, vc, q


def test_noalloc_refuses_oversized_partials_on_host(K):
    lib = K.lib
    cap = lib.kl_mha_noalloc_max_bytes()
    assert cap == 1 << 20
    sz = C.c_size_t(0)
    H, kvm, hd, S = 32, 1, 128, 32768
    assert lib.kl_mha_workspace_size(H, kvm, S, hd, C.byref(sz)) == 0
    assert sz.value > cap
    dummy = C.c_void_p(16)  # never dereferenced: the size check comes first
    assert lib.kl_mha_noalloc(S - 1, H, 0, S, H // kvm * hd, kvm, hd, dummy, dummy, dummy,
                              dummy, None) == -6
    assert lib.kl_mha_noalloc(0, 8, 0, 64, 256, 3, 64, dummy, dummy, dummy, dummy, None) == -4


@pytest.mark.gpu
def test_noalloc_matches_kl_mha_twice(K, O, gpu):
    lib = K.lib
    cases = [(12, 6, 128, 4096, 4000), (32, 4, 64, 1024, 700), (4, 2, 64, 96, 40)]
    for i, (H, kvm, hd, S, pos) in enumerate(cases):
        print(f"noalloc case {i}: H={H} kvm={kvm} hd={hd} S={S} pos={pos}", flush=True)
        layer, kvd, kc, vc, q = _shape_args(H, kvm, hd, S, pos, 100 + i)
        sz = C.c_size_t(0)
        assert lib.kl_mha_workspace_size(H, kvm, S, hd, C.byref(sz)) == 0
        assert sz.value <= lib.kl_mha_noalloc_max_bytes()
        dk, dv, dq = (K.DeviceArray.from_numpy(a) for a in (kc.ravel(), vc.ravel(), q))
        ws = K.DeviceArray.from_numpy(np.full(H * S, np.nan, np.float32))
        want_d, got_d = K.DeviceArray(H * hd), K.DeviceArray(H * hd)
        assert lib.kl_mha(pos, H, layer, S, kvd, kvm, hd, want_d.ptr, dq.ptr, ws.ptr, H * S * 4,
                          dk.ptr, dv.ptr, None) == 0
        assert lib.kl_mha_noalloc(pos, H, layer, S, kvd, kvm, hd, got_d.ptr, dq.ptr, dk.ptr,
                                  dv.ptr, None) == 0
        want, got = want_d.numpy(), got_d.numpy()
        assert np.array_equal(got, want), (i, float(np.max(np.abs(got - want))))
        ref = O.mha(pos, H, layer, S, kvd, kvm, hd, q, kc, vc)
        assert np.max(np.abs(got - ref)) < 2e-5
