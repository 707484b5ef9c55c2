"""Pins the Q6_K part of the oracle (oracle/q6k_oracle.c).

The byte and bit layout is stated twice, independently: the oracle's GEMV
follows the index arithmetic of the reference's vec-dot
(kernels/vecdotq.cuh:867-891, :580-600: bq8_offset, scale_offset, vh_shift
from iqs), while `decode` below follows the loops of ggml's
dequantize_row_q6_K (ql low/high nibbles and qh bit pairs per l < 32 of each
128-weight half).  Agreement on random blocks with every field at its
extremes pins the layout; the integer group sums are compared exactly and the
f64 result to 1e-12.  The quantiser (quantize_row_q6_K_ref restated) is
checked for the properties its output must have; byte-exactness against
upstream ggml is unpinned (ggml is not available here), and it is compared
byte for byte with the product library's host quantiser, a second
restatement.
"""
import numpy as np
import pytest

import _common

QK = 256
B6 = 210


def decode(wq: np.ndarray, K: int):
    """Q6_K bytes [M, K/256*210] -> (q [M, K] int in [0, 63], sc [M, K/16]
    int8 scale of each 16-weight group, d [M, K/256] float32)."""
    M = wq.shape[0]
    nb = K // QK
    blk = wq.reshape(M, nb, B6)
    ql = blk[:, :, :128].astype(np.int32)
    qh = blk[:, :, 128:192].astype(np.int32)
    sc = blk[:, :, 192:208].view(np.int8).astype(np.int32)
    d = blk[:, :, 208:210].copy().view(np.float16).astype(np.float32)[:, :, 0]
    q = np.empty((M, nb, QK), dtype=np.int32)
    for h in range(2):
        lo = ql[:, :, 64 * h:64 * h + 64]
        hb = qh[:, :, 32 * h:32 * h + 32]
        base = 128 * h
        q[:, :, base + 0:base + 32] = (lo[:, :, :32] & 0xF) | (((hb >> 0) & 3) << 4)
        q[:, :, base + 32:base + 64] = (lo[:, :, 32:] & 0xF) | (((hb >> 2) & 3) << 4)
        q[:, :, base + 64:base + 96] = (lo[:, :, :32] >> 4) | (((hb >> 4) & 3) << 4)
        q[:, :, base + 96:base + 128] = (lo[:, :, 32:] >> 4) | (((hb >> 6) & 3) << 4)
    return q.reshape(M, K), sc.reshape(M, K // 16), d


def random_q6_blocks(rng, M, K, extremes=True):
    """Random Q6_K bytes with finite fp16 d; with `extremes` most 6-bit
    values are 0 or 63 and most scales -128 or 127."""
    nb = K // QK
    blk = rng.integers(0, 256, size=(M, nb, B6), dtype=np.uint8)
    if extremes:
        q = np.where(rng.random((M, nb, QK)) < 0.7, rng.choice([0, 63], size=(M, nb, QK)),
                     rng.integers(0, 64, size=(M, nb, QK)))
        # pack q with the dequantiser's layout (the inverse of decode)
        for h in range(2):
            b = 128 * h
            q1, q2, q3, q4 = (q[:, :, b + 32 * t:b + 32 * t + 32] for t in range(4))
            blk[:, :, 64 * h:64 * h + 32] = (q1 & 0xF) | ((q3 & 0xF) << 4)
            blk[:, :, 64 * h + 32:64 * h + 64] = (q2 & 0xF) | ((q4 & 0xF) << 4)
            blk[:, :, 128 + 32 * h:128 + 32 * h + 32] = ((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4)
                                                         | ((q4 >> 4) << 6))
        sc = np.where(rng.random((M, nb, 16)) < 0.5, rng.choice([-128, 127], size=(M, nb, 16)),
                      rng.integers(-128, 128, size=(M, nb, 16)))
        blk[:, :, 192:208] = sc.astype(np.int8).view(np.uint8)
    d = (rng.random((M, nb)) * 0.01 + 1e-4).astype(np.float16)
    blk[:, :, 208:210] = d.reshape(M, nb, 1).view(np.uint8)
    return blk.reshape(M, nb * B6)


def random_q8_1(rng, N, K):
    """Random Q8_1 columns [N, Kp/32*36] with q8 mostly at +-127."""
    kp = (K + 511) // 512 * 512
    nblk = kp // 32
    blk = np.zeros((N, nblk, 36), dtype=np.uint8)
    q = np.where(rng.random((N, nblk, 32)) < 0.6, rng.choice([-127, 127], size=(N, nblk, 32)),
                 rng.integers(-127, 128, size=(N, nblk, 32)))
    blk[:, :, 4:] = q.astype(np.int8).view(np.uint8)
    d8 = (rng.random((N, nblk)) * 0.05 + 1e-3).astype(np.float16)
    s = rng.standard_normal((N, nblk)).astype(np.float16)
    blk[:, :, 0:2] = d8.reshape(N, nblk, 1).view(np.uint8)
    blk[:, :, 2:4] = s.reshape(N, nblk, 1).view(np.uint8)
    return blk.reshape(N, nblk * 36)


def reference_sums(wq, K, q8):
    """numpy: int sums of (q - 32) * q8 per 16-weight group and the f64 dot."""
    q, sc, d = decode(wq, K)
    N = q8.shape[0]
    nblk = q8.shape[1] // 36
    qb = q8.reshape(N, nblk, 36)
    a = qb[:, :, 4:].view(np.int8).astype(np.int64).reshape(N, -1)[:, :K]
    d8 = qb[:, :, 0:2].copy().view(np.float16).astype(np.float64)[:, :, 0][:, :K // 32]
    M = wq.shape[0]
    s16 = ((q - 32).astype(np.int64)[None, :, :] * a[:, None, :]).reshape(N, M, K // 16, 16).sum(-1)
    d8g = np.repeat(d8, 2, axis=1)                          # d8 of each 16-weight group
    dg = np.repeat(d.astype(np.float64), 16, axis=1)        # d of each group
    y = (dg[None] * d8g[:, None, :] * sc[None].astype(np.float64) * s16).sum(-1)
    return s16, y


@pytest.mark.parametrize("M,K,N", [(1, 256, 1), (3, 512, 2), (5, 1024, 3), (2, 2304, 4)])
def test_gemv_matches_dequantiser_layout(O, M, K, N):
    rng = np.random.default_rng([M, K, N, 6])
    wq = random_q6_blocks(rng, M, K)
    q8 = random_q8_1(rng, N, K)
    ref = O.gemv_q6K_q8_1(wq, K, q8)
    assert ref["mismatches"] == 0
    s16, y = reference_sums(wq, K, q8)
    np.testing.assert_array_equal(ref["s16"], s16)
    np.testing.assert_allclose(ref["y64"], y, rtol=1e-12, atol=1e-12 * np.abs(y).max())


def test_gemv_detects_a_swapped_bit_field(O):
    """A layout mistake planted in the decode (qh bit pairs of weights +32
    and +64 exchanged) is caught by the comparison above."""
    rng = np.random.default_rng(7)
    K = 512
    wq = random_q6_blocks(rng, 2, K)
    q8 = random_q8_1(rng, 1, K)
    ref = O.gemv_q6K_q8_1(wq, K, q8)
    bad = wq.reshape(2, 2, B6).copy()
    qh = bad[:, :, 128:192].astype(np.int32)
    swapped = (qh & 0b11000011) | ((qh >> 2) & 0b00001100) | ((qh << 2) & 0b00110000)
    bad[:, :, 128:192] = swapped.astype(np.uint8)
    s16_bad, _ = reference_sums(bad.reshape(2, -1), K, q8)
    assert not np.array_equal(ref["s16"], s16_bad)


def test_dequantize_matches_decode(O):
    rng = np.random.default_rng(11)
    K = 1024
    wq = random_q6_blocks(rng, 4, K, extremes=False)
    q, sc, d = decode(wq, K)
    expect = (np.repeat(d, QK, axis=1) * np.repeat(sc, 16, axis=1).astype(np.float32)) * (q - 32).astype(np.float32)
    got = O.dequantize_q6_K(wq, K)
    np.testing.assert_array_equal(got, expect.astype(np.float32))


@pytest.mark.parametrize("dist", ["normal", "uniform", "heavy"])
def test_quantize_properties(O, dist):
    rng = np.random.default_rng({"normal": 1, "uniform": 2, "heavy": 3}[dist])
    M, K = 8, 2048
    if dist == "normal":
        w = rng.standard_normal((M, K)).astype(np.float32) * np.float32(0.02)
    elif dist == "uniform":
        w = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    else:
        w = (rng.standard_t(2, (M, K)) * 0.05).astype(np.float32)
    wq = O.quantize_q6_K(w)
    q, sc, d = decode(wq, K)
    assert q.min() >= 0 and q.max() <= 63
    # every block's largest scale is stored as -128 (iscale = -128 / max scale)
    assert (sc.reshape(M, K // QK, 16).min(-1) == -128).all()
    # each value sits on the nearest level of its group's grid d * sc * (l - 32)
    step = np.repeat(d, QK, axis=1).astype(np.float64) * np.repeat(sc, 16, axis=1)
    deq = step * (q - 32)
    levels = step[..., None] * (np.arange(64) - 32)[None, None, :]
    best = np.abs(w[..., None].astype(np.float64) - levels).min(-1)
    err = np.abs(w - deq)
    assert (err <= best + 1e-6 * np.abs(step) + 1e-12).all()
    # 64 levels per group: about 1% relative RMS error for light tails; a
    # heavy tail stretches the grid of the groups holding its outliers
    rel = np.sqrt(((w - deq) ** 2).mean()) / np.sqrt((w ** 2).mean())
    assert rel < (0.05 if dist == "heavy" else 0.02)


def test_quantize_zero_block_and_matches_host_quantiser(O, Q):
    rng = np.random.default_rng(5)
    w = rng.standard_normal((6, 1024)).astype(np.float32) * np.float32(0.02)
    w[2, 256:512] = 0.0
    wq = O.quantize_q6_K(w)
    assert not wq.reshape(6, 4, B6)[2, 1].any()
    np.testing.assert_array_equal(Q.quantize_rows_q6_K(w, nthreads=3), wq)
