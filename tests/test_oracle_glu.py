"""Pins the oracle's GLU epilogue (oracle.glu) to what the mathematics fixes:
the tanh-form GELU stays within its published 1e-3 of the erf-form GELU,
silu(g) = g * logistic(g) with its limits, SWIGLU_OAI's clamps, and the
glu_tolerance bound holds for perturbations inside its box."""
import math

import numpy as np

import _common


def test_geglu_tanh_form_close_to_erf_gelu(O):
    g = np.linspace(-8, 8, 4001)
    erf_gelu = 0.5 * g * (1.0 + np.array([math.erf(v / math.sqrt(2.0)) for v in g]))
    tanh_gelu = O.glu(O.GLU_GEGLU, np.ones_like(g), g)
    assert np.max(np.abs(tanh_gelu - erf_gelu)) < 1e-3
    # exact at 0, odd part cancels: gelu(g) - gelu(-g) = g
    assert tanh_gelu[2000] == 0.0
    np.testing.assert_allclose(tanh_gelu - tanh_gelu[::-1], g, atol=1e-12)


def test_swiglu_is_up_times_g_logistic(O):
    g = np.array([-30.0, -1.0, 0.0, 0.5, 30.0])
    up = np.array([2.0, -3.0, 5.0, 1.0, 0.25])
    y = O.glu(O.GLU_SWIGLU, up, g)
    np.testing.assert_allclose(y, up * g / (1.0 + np.exp(-g)), rtol=1e-15)
    assert y[2] == 0.0
    np.testing.assert_allclose(y[4], up[4] * g[4], rtol=1e-12)  # silu(g) -> g for large g
    assert abs(y[0]) < 1e-10                                      # silu(g) -> 0 for very negative g


def test_swiglu_oai_clamps(O):
    # gate clamped above at 7 (not below), up clamped to [-7, 7]
    a = O.glu(O.GLU_SWIGLU_OAI, np.array([1.0, 1.0, 100.0, -100.0]), np.array([7.0, 50.0, 1.0, 1.0]))
    s7 = 7.0 / (1.0 + math.exp(-1.702 * 7.0))
    s1 = 1.0 / (1.0 + math.exp(-1.702))
    np.testing.assert_allclose(a, [s7 * 2, s7 * 2, s1 * 8, s1 * -6], rtol=1e-15)
    b = O.glu(O.GLU_SWIGLU_OAI, np.array([0.0]), np.array([-50.0]))
    assert abs(b[0]) < 1e-30 + 1e-20


def test_tolerance_covers_its_box(O):
    rng = np.random.default_rng(0)
    up = rng.standard_normal(2000) * 2
    g = rng.standard_normal(2000) * 3
    tu = np.abs(up) * 1e-5 + 1e-6
    tg = np.abs(g) * 1e-5 + 1e-6
    for op in (O.GLU_SWIGLU, O.GLU_GEGLU, O.GLU_SWIGLU_OAI):
        tol = O.glu_tolerance(op, up, g, tu, tg)
        for _ in range(4):
            du = rng.uniform(-1, 1, up.shape) * tu
            dg = rng.uniform(-1, 1, g.shape) * tg
            assert np.all(np.abs(O.glu(op, up + du, g + dg) - O.glu(op, up, g)) <= tol)
