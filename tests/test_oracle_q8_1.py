"""Pins the oracle's F32 -> Q8_1 quantiser (ggml-cuda quantize_q8_1
arithmetic) by its invariants and exact special cases."""
import numpy as np


def _split(q8, nblk):
    b = q8.reshape(-1, nblk, 36)
    d = b[..., 0:2].copy().view(np.uint16)[..., 0]
    s = b[..., 2:4].copy().view(np.uint16)[..., 0]
    qs = b[..., 4:].view(np.int8)
    return d, s, qs


def test_invariants(O):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((3, 4096)) * rng.uniform(0.01, 100, size=(3, 1))).astype(np.float32)
    q8 = O.quantize_q8_1(x)
    d16, s16, qs = _split(q8, 4096 // 32)
    d = O.f16_bits_to_f32(d16)
    xb = x.reshape(3, -1, 32)
    amax = np.abs(xb).max(-1)
    assert np.abs(qs.astype(np.int32)).max() <= 127
    # d is half(amax/127) with the f32 quotient
    assert (d16 == O.f32_to_f16_bits((amax / np.float32(127)).astype(np.float32))).all()
    # the largest-magnitude value maps to +-127
    imax = np.abs(xb).argmax(-1)
    top = np.take_along_axis(qs.astype(np.int32), imax[..., None], -1)[..., 0]
    sign = np.sign(np.take_along_axis(xb, imax[..., None], -1)[..., 0])
    assert (top == 127 * sign).all()
    # rounding error at most half a step of the f32 scale
    d32 = (amax / np.float32(127)).astype(np.float64)
    err = np.abs(xb.astype(np.float64) - d32[..., None] * qs)
    assert (err <= d32[..., None] * 0.5 * (1 + 1e-6)).all()
    # ds.y is half of the block sum
    ssum = xb.astype(np.float64).sum(-1)
    s = O.f16_bits_to_f32(s16).astype(np.float64)
    assert (np.abs(s - ssum) <= np.abs(ssum) * 2.0 ** -10 + 1e-6).all()


def test_zero_blocks_and_padding(O):
    x = np.zeros((1, 1024), dtype=np.float32)
    x[0, 100] = 3.0
    q8 = O.quantize_q8_1(x, k_padded=2048)
    assert q8.shape == (1, 2048 // 32 * 36)
    d16, s16, qs = _split(q8, 64)
    # block 3 holds the only non-zero value
    nz = [i for i in range(64) if d16[0, i] != 0]
    assert nz == [3]
    assert (qs[0, [i for i in range(64) if i != 3]] == 0).all()
    assert (s16[0, 32:] == 0).all() and (d16[0, 32:] == 0).all()


def test_exact_multiples_roundtrip(O):
    rng = np.random.default_rng(9)
    q = rng.integers(-127, 128, size=(2, 512)).astype(np.int32)
    q[:, ::32] = 127  # every block reaches amax = 127 * 2^-e
    for e in (0, 3, 10):
        x = (q * 2.0 ** -e).astype(np.float32)
        d16, _, qs = _split(O.quantize_q8_1(x), 16)
        assert (qs.reshape(2, -1) == q).all()
        assert (O.f16_bits_to_f32(d16) == np.float32(2.0 ** -e)).all()


def test_division_by_127_identity(O):
    """The GPU quantiser's division-free d = amax/127 (product with the
    rounded reciprocal plus one fma correction) must equal the IEEE quotient.
    Every 61st float bit pattern here (35M values, a few seconds); the
    same function run with stride 1 over [0, 0x7f800000) is the exhaustive
    check and reports no mismatch either.  A planted error -- the correction
    step dropped -- is caught by the same sample."""
    L = O.lib()
    assert L.orc_check_div127(0, 0x7F800000, 61) == 0
    # the first 2^20 patterns (zero and the subnormals) exhaustively
    assert L.orc_check_div127(0, 1 << 20, 1) == 0
    # without the correction (q0 alone) many quotients are off by one ulp
    rcp = np.float32(1.0 / 127.0)
    a = np.random.default_rng(0).uniform(1e-3, 1e3, 100000).astype(np.float32)
    assert ((a * rcp).astype(np.float32) != a / np.float32(127)).sum() > 1000


def _fast_round_agrees(d, xs, threshold):
    """The in-launch quantiser's fast rounding: y = x * r with r any float
    within one ulp of 1/d (the accuracy of v_rcp_f32), rint(y) accepted when
    |y - rint(y)| <= threshold.  Returns the number of accepted values whose
    rint(y) differs from ggml's roundf(x / d) (IEEE quotient)."""
    d = np.float32(d)
    r0 = np.float32(1.0) / d
    bad = 0
    q_ref = np.float32(xs / d)
    q_ref = np.sign(q_ref) * np.floor(np.abs(q_ref) + np.float32(0.5))
    for r in (r0, np.nextafter(r0, np.float32(0)), np.nextafter(r0, np.float32(np.inf))):
        y = (xs * r).astype(np.float32)
        ry = np.rint(y)
        fast = np.abs(y - ry) <= threshold
        bad += int(np.sum(fast & (ry != q_ref)))
    return bad


def _tie_adversaries(rng, d, n=4000):
    """x whose x/d lies within a few units of 2^-20 of a half-integer."""
    k = rng.integers(-127, 127, size=n) + 0.5
    off = rng.integers(-64, 65, size=n) * 2.0 ** -20
    return (np.float32(d) * (k + off)).astype(np.float32)


def test_fast_rounding_threshold_is_safe():
    """|y - x/d| <= 127 (2^-23 + 2^-24) < 2^-15.4 and |fl(x/d) - x/d| <= 2^-17,
    so rint(y) = roundf(fl(x/d)) whenever y is more than 2^-15 from a
    half-integer; the kernel accepts up to 0.5 - 2^-14 (twice that margin).
    Checked over random and near-tie quotients with the three reciprocals a
    one-ulp rcp can return; a threshold without the margin fails."""
    rng = np.random.default_rng(42)
    thr = np.float32(0.5 - 2.0 ** -14)
    too_loose = np.float32(0.5 - 2.0 ** -19)
    loose_bad = 0
    for _ in range(300):
        amax = np.float32(np.exp(rng.uniform(-40, 40)))
        d = np.float32(amax / np.float32(127.0))
        xs = np.concatenate([rng.uniform(-1, 1, 2000).astype(np.float32) * amax,
                             _tie_adversaries(rng, d)]).astype(np.float32)
        xs = xs[np.abs(xs) <= amax]
        assert _fast_round_agrees(d, xs, thr) == 0
        loose_bad += _fast_round_agrees(d, xs, too_loose)
    assert loose_bad > 0
