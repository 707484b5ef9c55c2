"""The ggml CPU path (Q8_K activations, vec_dot_q4_K_q8_K): scalar and AVX2
forms agree, and both compute the dequantised product of the Q8_K-quantised
activation.  Upstream bit-exactness is unpinned (ggml is not available)."""
import numpy as np

import _common


def _q8K_fields(yq, K):
    b = yq.reshape(-1, K // 256, 292)
    d = b[..., 0:4].copy().view(np.float32)[..., 0]
    qs = b[..., 4:260].view(np.int8)
    bs = b[..., 260:292].copy().view(np.int16)
    return d, qs, bs


def test_q8_K_invariants(O):
    x = _common.activations(2, 1024, seed=31) * np.float32(3.0)
    yq = O.quantize_q8_K(x)
    d, qs, bs = _q8K_fields(yq, 1024)
    assert np.abs(qs.astype(np.int32)).max() <= 127
    assert np.array_equal(bs, qs.reshape(2, 4, 16, 16).astype(np.int32).sum(-1).astype(np.int16))
    xb = x.reshape(2, 4, 256)
    err = np.abs(xb - d[..., None] * qs)
    assert (err <= np.abs(d)[..., None] * 0.5 * (1 + 1e-5)).all()


def test_scalar_and_avx2_agree_with_dequantised_product(O):
    if not O.lib().orc_cpu_has_avx2():
        import pytest
        pytest.skip("no AVX2")
    M, K = 48, 4096
    wq = O.quantize_q4_K(_common.weights(M, K, seed=32))
    x = _common.activations(3, K, seed=32)
    yq = O.quantize_q8_K(x)
    import test_oracle_gemv as T
    q, sc, mm, d, dmin = T.np_unpack_q4K(wq, K)
    w = (np.repeat(d, 8, 1) * sc)[:, :, None] * q.reshape(M, -1, 32) - (np.repeat(dmin, 8, 1) * mm)[:, :, None]
    dy, qs, _ = _q8K_fields(yq, K)
    a = (dy.astype(np.float64)[..., None] * qs).reshape(3, K)
    exact = a @ w.reshape(M, K).T
    scale = np.abs(a) @ np.abs(w.reshape(M, K)).T
    for c in range(3):
        for r in range(M):
            s = O.vec_dot_q4_K_q8_K(wq[r], yq[c], K, "scalar")
            v = O.vec_dot_q4_K_q8_K(wq[r], yq[c], K, "avx2")
            assert abs(s - exact[c, r]) <= 1e-5 * scale[c, r]
            assert abs(v - exact[c, r]) <= 1e-5 * scale[c, r]
    dst, isa = O.cpu_mul_mat_q4_K(wq, K, x, nthreads=4)
    assert isa == "avx2"
    assert np.allclose(dst, exact, rtol=0, atol=1e-5 * scale.max())
    # against the Q8_1 path: the activation quantisations differ, so the
    # outputs agree only to the activation-quantisation error
    ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    assert np.abs(dst - ref["y64"]).max() < 0.02 * np.abs(ref["y64"]).max()


def test_q6_K_scalar_and_avx2_agree_with_dequantised_product(O):
    """The same for ggml's vec_dot_q6_K_q8_K (the CPU baseline of the Q6_K
    configs): scalar and AVX2 forms and the threaded product against the f64
    dot of the decoded weights (d * scale * (q - 32), a numpy decode of the
    dequantize_row_q6_K layout) and the dequantised Q8_K activation; every
    6-bit value and scale extreme included."""
    import pytest
    if not O.lib().orc_cpu_has_avx2():
        pytest.skip("no AVX2")
    import test_oracle_q6K as T6
    M, K = 40, 4352
    rng = np.random.default_rng(36)
    wq = np.concatenate([O.quantize_q6_K(_common.weights(M // 2, K, seed=36)),
                         T6.random_q6_blocks(rng, M // 2, K)])
    x = _common.activations(3, K, seed=36)
    yq = O.quantize_q8_K(x)
    q, sc, d = T6.decode(wq, K)
    w = (np.repeat(d.astype(np.float64), 16, 1) * sc)[:, :, None] * (q.reshape(M, -1, 16) - 32)
    w = w.reshape(M, K)
    dy, qs, _ = _q8K_fields(yq, K)
    a = (dy.astype(np.float64)[..., None] * qs).reshape(3, K)
    exact = a @ w.T
    scale = np.abs(a) @ np.abs(w).T
    for c in range(3):
        for r in range(M):
            s = O.vec_dot_q6_K_q8_K(wq[r], yq[c], K, "scalar")
            v = O.vec_dot_q6_K_q8_K(wq[r], yq[c], K, "avx2")
            assert abs(s - exact[c, r]) <= 1e-5 * scale[c, r], (c, r, s, exact[c, r])
            assert abs(v - exact[c, r]) <= 1e-5 * scale[c, r], (c, r, v, exact[c, r])
    dst, isa = O.cpu_mul_mat_q4_K(wq, K, x, nthreads=4, wtype="q6_K")
    assert isa == "avx2"
    assert np.allclose(dst, exact, rtol=0, atol=1e-5 * scale.max())
    # the Q8_1 path of the GPU kernels agrees to the activation-quantisation error
    ref = O.gemv_q6K_q8_1(wq[: M // 2], K, O.quantize_q8_1(x), want_sums=False)
    assert np.abs(dst[:, : M // 2] - ref["y64"]).max() < 0.02 * np.abs(ref["y64"]).max()

