"""Pins the oracle's Q4_K x Q8_1 GEMV (the vec-dot's structure,
kernels/vecdotq.cuh:457-483 and :775-819) against the textbook product of the
dequantised operands, written here from the block layout alone."""
import numpy as np
import pytest

import _common


def np_unpack_q4K(wq, K):
    """Q4_K bytes [M, K/256*144] -> (q [M,K] 0..15, sc [M,K/32], m [M,K/32],
    d [M,K/256], dmin [M,K/256]) from the layout: qs[32c+l] low nibble is
    element 64c+l, high nibble element 64c+32+l; 6-bit fields as in ggml."""
    M = wq.shape[0]
    nb = K // 256
    b = wq.reshape(M, nb, 144)
    d = b[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    dmin = b[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    s = b[:, :, 4:16].astype(np.int32)
    sc = np.empty((M, nb, 8), np.int32)
    mm = np.empty((M, nb, 8), np.int32)
    for j in range(8):
        if j < 4:
            sc[..., j] = s[..., j] & 63
            mm[..., j] = s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 15) | ((s[..., j - 4] >> 6) << 4)
            mm[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    qs = b[:, :, 16:].astype(np.int32).reshape(M, nb, 4, 32)
    q = np.concatenate([qs & 15, qs >> 4], axis=-1)  # [M, nb, 4, 64]
    return q.reshape(M, K), sc.reshape(M, -1), mm.reshape(M, -1), d, dmin


def np_unpack_q8_1(q8, K):
    N = q8.shape[0]
    b = q8.reshape(N, -1, 36)[:, : K // 32]
    d8 = b[..., 0:2].copy().view(np.float16)[..., 0].astype(np.float64)
    qs = b[..., 4:].view(np.int8).astype(np.int32).reshape(N, K)
    return qs, d8


def np_reference(wq, K, q8):
    q, sc, mm, d, dmin = np_unpack_q4K(wq, K)
    a, d8 = np_unpack_q8_1(q8, K)
    M, N = q.shape[0], a.shape[0]
    sqq = np.einsum("mse,nse->nms", q.reshape(M, -1, 32), a.reshape(N, -1, 32))
    sq = a.reshape(N, -1, 32).sum(-1)
    w = (np.repeat(d, 8, 1) * sc)[:, :, None] * q.reshape(M, -1, 32) - (np.repeat(dmin, 8, 1) * mm)[:, :, None]
    x = d8[:, :, None] * a.reshape(N, -1, 32)
    y = x.reshape(N, K) @ w.reshape(M, K).T
    return sqq, sq, y


@pytest.mark.parametrize("M,K,N", [(7, 256, 1), (16, 768, 3), (33, 2048, 8), (5, 4352, 2)])
def test_gemv_matches_dequantised_product(O, M, K, N):
    W = _common.weights(M, K, seed=M + K)
    x = _common.activations(N, K, seed=N)
    wq = O.quantize_q4_K(W)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q4K_q8_1(wq, K, q8)
    sqq, sq, y = np_reference(wq, K, q8)
    assert (ref["sqq"] == sqq).all()
    assert (ref["sq"] == sq).all()
    assert np.allclose(ref["y64"], y.T.T, rtol=1e-12, atol=1e-12 * np.abs(y).max())


def test_extreme_values(O):
    # q4 in {0, 15}, q8 in {-127, 127}, 6-bit fields at 63, large fp16 d
    K, M = 512, 4
    rng = np.random.default_rng(1)
    wq = np.zeros((M, K // 256 * 144), np.uint8)
    blocks = wq.reshape(M, -1, 144)
    blocks[..., 0:2] = np.frombuffer(np.float16(1024.0).tobytes(), np.uint8)
    blocks[..., 2:4] = np.frombuffer(np.float16(-0.5).tobytes(), np.uint8)
    blocks[..., 4:16] = 0xFF
    blocks[0, :, 16:] = 0xFF
    blocks[1, :, 16:] = 0x00
    blocks[2, :, 16:] = 0xF0
    blocks[3, :, 16:] = rng.choice([0x00, 0x0F, 0xF0, 0xFF], size=blocks[3, :, 16:].shape)
    q8 = np.zeros((2, K // 32 * 36), np.uint8)
    b8 = q8.reshape(2, -1, 36)
    b8[..., 0:2] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    b8[0, :, 4:] = np.uint8(127)
    b8[1, :, 4:] = rng.choice([127, 129], size=b8[1, :, 4:].shape).astype(np.uint8)  # +-127
    ref = O.gemv_q4K_q8_1(wq, K, q8)
    sqq, sq, y = np_reference(wq, K, q8)
    assert (ref["sqq"] == sqq).all() and (ref["sq"] == sq).all()
    assert ref["sqq"].max() == 32 * 15 * 127 and ref["sq"].max() == 32 * 127
    assert np.allclose(ref["y64"], y, rtol=1e-12)


def test_row_and_column_independence(O):
    M, K, N = 24, 1024, 4
    wq = O.quantize_q4_K(_common.weights(M, K, seed=3))
    q8 = O.quantize_q8_1(_common.activations(N, K, seed=3))
    full = O.gemv_q4K_q8_1(wq, K, q8)
    for r in (0, 7, 23):
        one = O.gemv_q4K_q8_1(wq[r:r + 1], K, q8)
        assert (one["y64"][:, 0] == full["y64"][:, r]).all()
        assert (one["sqq"][:, 0] == full["sqq"][:, r]).all()
    for c in range(N):
        one = O.gemv_q4K_q8_1(wq, K, q8[c:c + 1])
        assert (one["y64"][0] == full["y64"][c]).all()


def test_linearity_in_activation_scale(O):
    # scaling x by 2^k leaves q8 unchanged and scales every d8 exactly
    M, K = 8, 1024
    wq = O.quantize_q4_K(_common.weights(M, K, seed=4))
    x = _common.activations(1, K, seed=4)
    base = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x))
    for k in (-3, 2):
        scaled = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x * np.float32(2.0 ** k)))
        assert (scaled["sqq"] == base["sqq"]).all()
        assert np.array_equal(scaled["y64"], base["y64"] * 2.0 ** k)


def test_tolerance_catches_a_dropped_term(O):
    # the parity tolerance must be far tighter than one sub-block term
    M, K = 64, 4096
    wq = O.quantize_q4_K(_common.weights(M, K, seed=5))
    q8 = O.quantize_q8_1(_common.activations(1, K, seed=5))
    ref = O.gemv_q4K_q8_1(wq, K, q8)
    tol = O.parity_tolerance(ref["y64"], ref["l1"])
    # smallest sub-block term magnitude scale: l1 / number of terms
    assert (tol < 0.05 * ref["l1"] / (2 * K / 32)).all()
