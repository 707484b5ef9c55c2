"""Pins the oracle's quantisers against the published ggml algorithms, without
ggml (not available here: see the oracle's header).

Weight quantisers (the inputs of every workload):
  * quantize_row_q4_K_ref, stage 1 (make_qkx2_quants per 32-value
    sub-block): a numpy walk over ggml's candidate inverse scales
    ((rmin + rdelta*is + nmax) / (max - min), is = 0..nstep, after the
    min-max fit), whose fits and errors are computed in f64.  The oracle's f32
    choice must agree wherever no accept/reject decision on the way is within
    1 % of a tie; planted mistakes (rdelta 0.2, rmin -0.5, x^2 weights, no
    candidate walk) each disagree far from any tie on hundreds of sub-blocks.
  * stage 2 (6-bit scales and mins, fp16 d and dmin) and stage 3 (levels):
    each stored field is the nearest one to what the fit asked for, and each
    level is the nearest of the 16 levels its sub-block offers.
  * quantize_row_q6_K_ref, stage 1 (make_qx_quants per 16-value group):
    argmax of sum(w x l)^2 / sum(w l^2) over ggml's 19 candidates, in f64,
    with the same tie rule (agreement required wherever no decision is within
    1e-5 of a tie; the disagreements seen are all within 4e-7, f32 rounding);
    planted mistakes (rdelta 0.2, |x| weights, no neighbours) fail.
  * both quantisers reproduce values on an exact grid bit for bit (a wrong
    nibble order, sub-block pairing, scale packing or sign fails).
Activation quantisers:
  * Q8_1 (ggml-cuda quantize_q8_1, call site kernels/mmvq.cu:728-735): exact
    ties x/d = k + 1/2 round away from zero (roundf); numpy's rint, the
    plausible mistake, rounds them to even and differs on the same inputs.
  * Q8_K (quantize_row_q8_K_ref): the signed value of largest magnitude, the
    first one on ties, maps to -127; an amax-based scale would give +127 on
    the blocks whose extreme value is positive, which the inputs include.
"""
import numpy as np
import pytest

import _common
import test_oracle_gemv as G

f32 = np.float32


# ----------------------------------------------------------------- Q4_K ----
def walk_qkx2(x, rmin=-1.0, rdelta=0.1, nstep=20, nmax=15):
    """ggml make_qkx2_quants on rows of x [n, 32] (float32): levels from f32
    arithmetic as ggml forms them, fits (weighted least squares with min <= 0)
    and weighted squared errors in f64.  ggml keeps a candidate only when its
    error is below the best so far and then generates the next candidates
    around the new min, so the walk is sequential.  Returns (L, scale, -min,
    margin, constant): margin is the smallest relative gap between a
    candidate's error and the best error at any decision of the walk."""
    x = np.asarray(x, np.float32)
    xd = x.astype(np.float64)
    w = np.sqrt((xd * xd).mean(1))[:, None] + np.abs(xd)
    lo = np.minimum(x.min(1), f32(0))
    hi = x.max(1)
    constant = hi == lo
    hi_lo = np.where(constant, f32(1), hi - lo).astype(np.float32)
    iscale = (f32(nmax) / hi_lo).astype(np.float32)
    L = np.clip(np.rint((iscale[:, None] * (x - lo[:, None])).astype(np.float32)), 0, nmax)
    scale = (f32(1) / iscale).astype(np.float64)
    mn = lo.astype(np.float64)
    best = (w * (scale[:, None] * L + mn[:, None] - xd) ** 2).sum(1)
    cur_min = lo.copy()
    sw, sx = w.sum(1), (w * xd).sum(1)
    margin = np.full(len(x), np.inf)
    for i in range(nstep + 1):
        a = f32(f32(f32(rmin) + f32(f32(rdelta) * f32(i))) + f32(nmax))
        span = np.where(constant, f32(1), hi - cur_min).astype(np.float32)
        isc = (a / span).astype(np.float32)
        La = np.clip(np.rint((isc[:, None] * (x - cur_min[:, None])).astype(np.float32)), 0, nmax)
        sl, sl2, sxl = (w * La).sum(1), (w * La * La).sum(1), (w * La * xd).sum(1)
        D = sw * sl2 - sl * sl
        ok = D > 0
        Ds = np.where(ok, D, 1.0)
        sc = (sw * sxl - sx * sl) / Ds
        m = (sl2 * sx - sl * sxl) / Ds
        pos = m > 0
        sc = np.where(pos, sxl / np.where(sl2 > 0, sl2, 1.0), sc)
        m = np.where(pos, 0.0, m)
        err = (w * (sc[:, None] * La + m[:, None] - xd) ** 2).sum(1)
        margin = np.where(ok, np.minimum(margin, np.abs(err - best) / np.maximum(best, 1e-300)), margin)
        acc = ok & (err < best)
        L = np.where(acc[:, None], La, L)
        best = np.where(acc, err, best)
        scale = np.where(acc, sc, scale)
        mn = np.where(acc, m, mn)
        cur_min = np.where(acc, m.astype(np.float32), cur_min)
    L = np.where(constant[:, None], 0, L)
    return L, scale, -mn, margin, constant


def q4K_fit_disagreements(O, W, tie_margin=1e-2, **planted):
    """Sub-blocks where the oracle's stage-1 fit (with `planted` parameters)
    differs from the walk with ggml's parameters: (all, those whose walk
    has no decision within tie_margin of a tie, total)."""
    sc, mn, L = O.q4K_fit(W, **planted)
    xs = W.reshape(-1, 32)
    Lr, sr, mr, margin, const = walk_qkx2(xs)
    sc = sc.reshape(-1).astype(np.float64)
    mn = mn.reshape(-1).astype(np.float64)
    same = (Lr == L.reshape(-1, 32)).all(1)
    same &= np.abs(sr - sc) <= 1e-4 * np.abs(sr) + 1e-30
    same &= np.abs(mr - mn) <= 1e-4 * (np.abs(mr) + 15 * np.abs(sr)) + 1e-30
    same |= const & (sc == 0)
    diff = ~same
    return int(diff.sum()), int((diff & (margin >= tie_margin)).sum()), len(same)


def _weight_sets():
    rng = np.random.default_rng(101)
    return {
        "normal": _common.weights(64, 4096, seed=3),
        "heavy": (rng.standard_t(2, (64, 4096)) * 0.02).astype(np.float32),
        "uniform": rng.uniform(-1, 1, (64, 4096)).astype(np.float32),
        "positive": np.abs(_common.weights(16, 4096, seed=4)) + f32(0.01),
    }


@pytest.mark.parametrize("dist", ["normal", "heavy", "uniform", "positive"])
def test_q4K_fit_follows_the_candidate_walk(O, dist):
    W = _weight_sets()[dist]
    total, far, n = q4K_fit_disagreements(O, W)
    assert far == 0, f"{far} sub-blocks differ from ggml's candidate walk away from any near-tie"
    assert total <= n // 100, f"{total} of {n} sub-blocks differ (near-ties only expected, under 1 %)"


@pytest.mark.parametrize("planted", [dict(rdelta=0.2), dict(rmin=-0.5), dict(weight_mode=1), dict(nstep=0)],
                         ids=["rdelta0.2", "rmin-0.5", "x2weights", "no_walk"])
def test_q4K_fit_check_catches_planted_mistakes(O, planted):
    W = _weight_sets()["normal"]
    total, far, n = q4K_fit_disagreements(O, W, **planted)
    assert far >= 100 and total >= 1000, (far, total, n)


def test_q4K_stage2_and_stage3_are_nearest(O):
    """The stored 6-bit scale/min of each sub-block is the nearest to
    63 * (fit / block maximum); d and dmin are half(max / 63); every level
    is the nearest of its sub-block's 16 levels d*sc*l - dmin*m (sub-blocks
    with d*sc = 0 keep the fit's levels)."""
    for W in _weight_sets().values():
        M, K = W.shape
        wq = O.quantize_q4_K(W)
        fsc, fmn, fL = O.q4K_fit(W)
        nb = K // 256
        fsc = fsc.reshape(M, nb, 8).astype(np.float64)
        fmn = fmn.reshape(M, nb, 8).astype(np.float64)
        q, sc, mm, d, dmin = G.np_unpack_q4K(wq, K)
        sc = sc.reshape(M, nb, 8)
        mm = mm.reshape(M, nb, 8)
        max_sc = np.maximum(fsc.max(-1), 0)
        max_mn = np.maximum(fmn.max(-1), 0)
        h = lambda v: O.f16_bits_to_f32(O.f32_to_f16_bits((v / f32(63)).astype(np.float32))).astype(np.float64)
        assert np.array_equal(d, h(max_sc.astype(np.float32)))
        assert np.array_equal(dmin, h(max_mn.astype(np.float32)))
        want_sc = np.where(max_sc[..., None] > 0, 63 * fsc / np.where(max_sc > 0, max_sc, 1)[..., None], 0)
        want_m = np.where(max_mn[..., None] > 0, 63 * fmn / np.where(max_mn > 0, max_mn, 1)[..., None], 0)
        assert (np.abs(sc - np.clip(want_sc, 0, 63)) <= 0.5 + 1e-4).all()
        assert (np.abs(mm - np.clip(want_m, 0, 63)) <= 0.5 + 1e-4).all()
        assert ((sc.max(-1) == 63) | (max_sc == 0)).all()
        # levels: nearest of 16 in f64 (an f32 tie may go either way)
        step = (d[..., None] * sc).astype(np.float32).astype(np.float64)        # d*sc as the f32 product
        off = (dmin[..., None] * mm).astype(np.float32).astype(np.float64)
        x = W.reshape(M, nb, 8, 32).astype(np.float64)
        ql = q.reshape(M, nb, 8, 32)
        lv = step[..., None, None] * np.arange(16) - off[..., None, None]       # [M, nb, 8, 1, 16]
        dist = np.abs(x[..., None] - lv)
        got = np.take_along_axis(dist, ql[..., None], -1)[..., 0]
        live = (step != 0)[..., None]
        assert ((got <= dist.min(-1) * (1 + 1e-6) + 1e-6 * step[..., None]) | ~live).all()
        fL = fL.reshape(M, nb, 8, 32)
        assert ((ql == fL) | live).all()


def test_q4K_exact_grid_round_trips(O):
    """Sub-blocks x = sc_s 2^-10 L - m_s 2^-12 with integer L covering 0..15
    and 6-bit (sc_s, m_s) whose block maxima are 63: every stage is exact,
    so dequantising gives x back bit for bit."""
    rng = np.random.default_rng(8)
    M, K = 16, 1024
    nb = K // 256
    L = rng.integers(0, 16, size=(M, nb, 8, 32))
    L[..., 0], L[..., 1] = 0, 15
    sc = rng.integers(1, 64, size=(M, nb, 8))
    mm = rng.integers(0, 64, size=(M, nb, 8))
    sc[..., rng.integers(0, 8)] = 63
    mm[..., rng.integers(0, 8)] = 63
    x = (sc[..., None] * 2.0 ** -10 * L - mm[..., None] * 2.0 ** -12).astype(np.float32).reshape(M, K)
    wq = O.quantize_q4_K(x)
    assert np.array_equal(O.dequantize_q4_K(wq, K), x)
    q, s2, m2, d, dmin = G.np_unpack_q4K(wq, K)
    assert np.array_equal(q.reshape(M, nb, 8, 32), L)
    assert np.array_equal(s2.reshape(M, nb, 8), sc) and np.array_equal(m2.reshape(M, nb, 8), mm)
    assert (d == 2.0 ** -10).all() and (dmin == 2.0 ** -12).all()


# ----------------------------------------------------------------- Q6_K ----
def walk_qx(x, nmax=32, rdelta=0.1, nstep=9):
    """ggml make_qx_quants (rmse_type 1: weights x^2) on rows of x [n, 16]:
    candidates iscale = -(nmax + rdelta*is)/x_max for is = 0, -nstep..nstep
    (x_max the first value of largest magnitude), levels from f32, the
    objective sum(w x l)^2 / sum(w l^2) in f64; a candidate replaces the best
    only when strictly better.  Returns (L + nmax, scale, margin, zero)."""
    x = np.asarray(x, np.float32)
    xd = x.astype(np.float64)
    w = xd * xd
    imax = np.abs(x).argmax(1)
    xm = x[np.arange(len(x)), imax]
    zero = np.abs(xm) < f32(1e-15)
    xm_s = np.where(zero, f32(1), xm).astype(np.float32)

    def cand(isc):
        l = np.clip(np.rint((isc[:, None] * x).astype(np.float32)), -nmax, nmax - 1)
        return l, (w * xd * l).sum(1), (w * l * l).sum(1)

    l, slx, sl2 = cand((f32(-nmax) / xm_s).astype(np.float32))
    L, scale = l, np.where(sl2 > 0, slx / np.where(sl2 > 0, sl2, 1), 0)
    best = scale * slx
    margin = np.full(len(x), np.inf)
    for i in [k for k in range(-nstep, nstep + 1) if k != 0]:
        isc = (-(f32(nmax) + f32(f32(rdelta) * f32(i))) / xm_s).astype(np.float32)
        l, slx, sl2 = cand(isc)
        obj = np.where(sl2 > 0, slx * slx / np.where(sl2 > 0, sl2, 1), -np.inf)
        margin = np.minimum(margin, np.abs(obj - best) / np.maximum(np.abs(best), 1e-300))
        acc = (sl2 > 0) & (obj > best)
        L = np.where(acc[:, None], l, L)
        scale = np.where(acc, slx / np.where(sl2 > 0, sl2, 1), scale)
        best = np.where(acc, scale * slx, best)
    L = np.where(zero[:, None], -nmax, L)
    return (L + nmax).astype(np.int8), np.where(zero, 0, scale), margin, zero


def q6K_fit_disagreements(O, W, tie_margin=1e-5, **planted):
    sc, L = O.q6K_fit(W, **planted)
    xs = W.reshape(-1, 16)
    Lr, sr, margin, zero = walk_qx(xs)
    sc = sc.reshape(-1).astype(np.float64)
    same = (Lr == L.reshape(-1, 16)).all(1) & (np.abs(sr - sc) <= 1e-4 * np.abs(sr) + 1e-30)
    diff = ~same
    return int(diff.sum()), int((diff & (margin >= tie_margin)).sum()), len(same)


@pytest.mark.parametrize("dist", ["normal", "heavy", "uniform", "positive"])
def test_q6K_fit_is_ggml_candidate_argmax(O, dist):
    W = _weight_sets()[dist]
    total, far, n = q6K_fit_disagreements(O, W)
    assert far == 0, f"{far} groups differ from ggml's candidates away from any near-tie"
    # 16-value groups often have two candidates within f32 rounding (< 1e-6
    # relative) of each other; about 2 % of N(0, 0.02) groups
    assert total <= n // 20, (total, n)


@pytest.mark.parametrize("planted", [dict(rdelta=0.2), dict(weight_mode=1), dict(nstep=0)],
                         ids=["rdelta0.2", "abs_weights", "no_neighbours"])
def test_q6K_fit_check_catches_planted_mistakes(O, planted):
    W = _weight_sets()["normal"]
    total, far, n = q6K_fit_disagreements(O, W, **planted)
    assert far >= 100 and total >= 1000, (far, total, n)


def test_q6K_stage2_is_nearest(O):
    """Each group's stored int8 scale is the nearest to -128 * fit / (fit of
    largest magnitude), clamped to 127; d = half(max / -128)."""
    import test_oracle_q6K as Q6
    for W in _weight_sets().values():
        M, K = W.shape
        wq = O.quantize_q6_K(W)
        _, sc, d = Q6.decode(wq, K)
        fsc, _ = O.q6K_fit(W)
        fsc = fsc.reshape(M, K // 256, 16).astype(np.float64)
        imax = np.abs(fsc).argmax(-1)
        mx = np.take_along_axis(fsc, imax[..., None], -1)[..., 0]
        want = np.clip(-128.0 * fsc / mx[..., None], -128, 127)
        assert (np.abs(sc.reshape(M, K // 256, 16) - want) <= 0.5 + 1e-4).all()
        dh = O.f16_bits_to_f32(O.f32_to_f16_bits((f32(1) / (f32(-128) / mx.astype(np.float32))).astype(np.float32)))
        assert np.array_equal(d, dh)


def test_q6K_exact_grid_round_trips(O):
    """Groups x = -k_j 2^-10 l with integer l in [-32, 31] (l = -32 present,
    so it is the group's value of largest magnitude) and k_j in 1..128 with
    128 in every block: the fit, the int8 scales (-k_j) and d = 2^-10 are
    exact, and dequantising gives x back bit for bit."""
    import test_oracle_q6K as Q6
    rng = np.random.default_rng(12)
    M, K = 8, 1024
    nb = K // 256
    l = rng.integers(-31, 32, size=(M, nb, 16, 16))
    l[..., 0] = -32
    k = rng.integers(1, 129, size=(M, nb, 16))
    k[..., rng.integers(0, 16)] = 128
    x = (-k[..., None] * 2.0 ** -10 * l).astype(np.float32).reshape(M, K)
    wq = O.quantize_q6_K(x)
    assert np.array_equal(O.dequantize_q6_K(wq, K), x)
    q, sc, d = Q6.decode(wq, K)
    assert np.array_equal(q.reshape(M, nb, 16, 16) - 32, l)
    assert np.array_equal(sc.reshape(M, nb, 16), -k) and (d == 2.0 ** -10).all()


# ----------------------------------------------------------------- Q8_1 ----
def test_q8_1_ties_round_half_away_from_zero(O):
    """Blocks with amax = 127 * 2^e (so d = 2^e exactly) and values
    (k + 1/2) 2^e: x / d is an exact tie and ggml-cuda's roundf takes it away
    from zero.  The planted alternative, round-half-even (rint), gives a
    different byte on about half of these values."""
    rng = np.random.default_rng(77)
    nblk = 64
    e = rng.integers(-20, 10, size=nblk)
    k = rng.integers(-127, 127, size=(nblk, 32)).astype(np.float64)
    t = k + 0.5
    t[:, 0] = 127.0
    t[:, 1] = -127.0
    x = (t * 2.0 ** e[:, None]).astype(np.float32).reshape(1, -1)
    _, _, qs = _split_q81(O.quantize_q8_1(x), nblk)
    qs = qs.reshape(nblk, 32).astype(np.int32)
    away = (np.sign(t) * np.floor(np.abs(t) + 0.5)).astype(np.int32)
    assert np.array_equal(qs, away)
    half_even = np.rint(t).astype(np.int32)
    assert (half_even != away).sum() > 500


def _split_q81(q8, nblk):
    b = q8.reshape(-1, nblk, 36)
    d = b[..., 0:2].copy().view(np.uint16)[..., 0]
    s = b[..., 2:4].copy().view(np.uint16)[..., 0]
    return d, s, b[..., 4:].view(np.int8)


# ----------------------------------------------------------------- Q8_K ----
def test_q8_K_signed_max_maps_to_minus_127(O):
    """quantize_row_q8_K_ref scales by -127 / x_max with x_max the signed
    value of largest magnitude (the first one on ties): that value maps to
    -127, whatever its sign, and d = 1 / iscale carries the sign.  About half
    the blocks have a positive extreme, where an amax-based scale would give
    +127; the tie blocks fix which of two equal magnitudes wins."""
    rng = np.random.default_rng(31)
    nb = 64
    x = rng.standard_normal((nb, 256)).astype(np.float32)
    for b in range(nb):  # a clear extreme, positive in even blocks
        x[b, rng.integers(0, 256)] = (8.0 if b % 2 == 0 else -8.0)
    x[0, :] = 0.25
    x[0, 7], x[0, 200] = 3.0, -3.0   # tie in |x|: the first (+3) wins
    x[1, :] = 0.25
    x[1, 9], x[1, 100] = -3.0, 3.0   # tie: the first (-3) wins
    yq = O.quantize_q8_K(x.reshape(1, -1))
    b = yq.reshape(nb, 292)
    d = b[:, 0:4].copy().view(np.float32)[:, 0]
    qs = b[:, 4:260].view(np.int8).astype(np.int32)
    first = np.abs(x).argmax(1)  # numpy returns the first index of the maximum
    assert (qs[np.arange(nb), first] == -127).all()
    assert (np.sign(d) == -np.sign(x[np.arange(nb), first])).all()
    assert qs[0, 7] == -127 and qs[0, 200] == 127
    assert qs[1, 9] == -127 and qs[1, 100] == 127
    assert (x[np.arange(nb), first] > 0).sum() >= nb // 2 - 1
