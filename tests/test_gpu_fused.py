"""GPU parity of the fused epilogue (kernels/mmvq.cu:182-227, :309-336):
bias on the product, gate weight streamed in the same launch with its own
bias, and the GLU of the pair, for Q4_K and Q6_K weights.

Bar: the two products are checked against the oracle's f64 results through
the GLU -- glu_tolerance propagates each product's parity tolerance through
the GLU and adds 16 f32 epsilons of the epilogue's magnitude for the
device's expf/tanhf.  The bias-only epilogue is one f32 add after the
product, so it must equal the unfused product plus the bias bit for bit, and
the fused products themselves round exactly like the unfused kernel's (the
GLU of SWIGLU with the gate's output recovered is not invertible, so that
part is checked through the tolerance).
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

_cache = {}


def weights_q(Q, wtype, M, K, seed):
    key = (wtype, M, K, seed)
    if key not in _cache:
        if len(_cache) > 8:
            _cache.clear()
        W = _common.weights(M, K, seed)
        quant = Q.quantize_rows_q4_K if wtype == Q.GGML_TYPE_Q4_K else Q.quantize_rows_q6_K
        _cache[key] = quant(W, nthreads=16)
    return _cache[key]


def oracle_product(O, Q, wtype, wq, K, q8):
    f = O.gemv_q4K_q8_1 if wtype == Q.GGML_TYPE_Q4_K else O.gemv_q6K_q8_1
    r = f(wq, K, q8, want_sums=False)
    return r["y64"][0], O.parity_tolerance(r["y64"], r["l1"])[0]


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


SHAPES = [(1, 256), (17, 4352), (1000, 4096), (14336, 4096), (300, 14336), (777, 768), (3000, 2048)]
TYPES = [12, 14]


@pytest.mark.parametrize("wtype", TYPES)
@pytest.mark.parametrize("M,K", SHAPES)
@pytest.mark.parametrize("op", [2, 1, 3])
def test_gate_glu_against_oracle(Q, O, gpu, wtype, M, K, op):
    wu = weights_q(Q, wtype, M, K, seed=1)
    wg = weights_q(Q, wtype, M, K, seed=2)
    x = _common.activations(1, K, seed=3)
    rng = np.random.default_rng([M, K, op])
    bu = rng.standard_normal(M).astype(np.float32) * np.float32(0.1)
    bg = rng.standard_normal(M).astype(np.float32) * np.float32(0.1)
    use_bias = op != 3 or M % 2 == 1      # some cases without biases
    q8 = O.quantize_q8_1(x)
    up, tu = oracle_product(O, Q, wtype, wu, K, q8)
    g, tg = oracle_product(O, Q, wtype, wg, K, q8)
    if use_bias:
        up = up + bu.astype(np.float64)
        g = g + bg.astype(np.float64)
    expect = O.glu(op, up, g)
    tol = O.glu_tolerance(op, up, g, tu, tg)
    y = Q.mul_mat_vec_q_fused(to_dev(wu, gpu), K, to_dev(x, gpu), gate=to_dev(wg, gpu),
                              x_bias=to_dev(bu, gpu) if use_bias else None,
                              gate_bias=to_dev(bg, gpu) if use_bias else None, glu_op=op,
                              wtype=wtype).cpu().numpy()[0]
    err = np.abs(y - expect)
    bad = np.flatnonzero(err > tol)
    assert bad.size == 0, (f"{bad.size} outputs outside tolerance, e.g. row {bad[0]}: {y[bad[0]]} vs "
                           f"{expect[bad[0]]} (tol {tol[bad[0]]})")


@pytest.mark.parametrize("wtype", TYPES)
def test_bias_only_is_product_plus_bias(Q, O, gpu, wtype):
    M, K = 1000, 4096
    wu = weights_q(Q, wtype, M, K, seed=1)
    x = _common.activations(1, K, seed=3)
    b = np.random.default_rng(9).standard_normal(M).astype(np.float32)
    wd, xd = to_dev(wu, gpu), to_dev(x, gpu)
    plain = Q.mul_mat_vec_q(wd, K, xd, wtype=wtype).cpu().numpy()[0]
    y = Q.mul_mat_vec_q_fused(wd, K, xd, x_bias=to_dev(b, gpu), wtype=wtype).cpu().numpy()[0]
    assert np.array_equal(y, plain + b)
    # no epilogue at all: the plain product
    y0 = Q.mul_mat_vec_q_fused(wd, K, xd, wtype=wtype).cpu().numpy()[0]
    assert np.array_equal(y0, plain)


@pytest.mark.parametrize("wtype", TYPES)
def test_gate_products_round_like_unfused(Q, O, gpu, wtype):
    """With the plain-product GLU (gate 'op' 0 is not fused, so use SWIGLU
    with the gate weight equal to the weight): dst = up * silu(up), where up
    must be the unfused product bit for bit; checked by recomputing the
    epilogue from the unfused product in f64 and requiring agreement to a few
    ulps, far inside the tolerance of the oracle test."""
    M, K = 777, 4096
    wu = weights_q(Q, wtype, M, K, seed=1)
    x = _common.activations(1, K, seed=3)
    wd, xd = to_dev(wu, gpu), to_dev(x, gpu)
    plain = Q.mul_mat_vec_q(wd, K, xd, wtype=wtype).cpu().numpy()[0].astype(np.float64)
    y = Q.mul_mat_vec_q_fused(wd, K, xd, gate=wd, glu_op=2, wtype=wtype).cpu().numpy()[0]
    expect = plain * (plain / (1.0 + np.exp(-plain)))
    assert np.all(np.abs(y - expect) <= 8 * np.spacing(np.abs(expect).astype(np.float32)) + 1e-30)


@pytest.mark.parametrize("wtype", TYPES)
def test_fused_geometry_variants_agree(Q, O, gpu, wtype):
    M, K = 2000, 4096
    wu = weights_q(Q, wtype, M, K, seed=1)
    wg = weights_q(Q, wtype, M, K, seed=2)
    x = _common.activations(1, K, seed=3)
    wd, gd, xd = to_dev(wu, gpu), to_dev(wg, gpu), to_dev(x, gpu)
    outs = []
    try:
        for waves, wgs, slots in ((8, 0, 1), (16, 0, 1), (8, 0, 2), (16, 5, 2), (0, 1, 0)):
            Q.set_geometry_override(waves_per_wg=waves, workgroups=wgs)
            Q.set_pipeline_override(slots, -1)
            outs.append(Q.mul_mat_vec_q_fused(wd, K, xd, gate=gd, glu_op=2, wtype=wtype).cpu().numpy())
    finally:
        Q.set_geometry_override()
        Q.set_pipeline_override()
    for y in outs[1:]:
        assert np.array_equal(y, outs[0])


def test_descriptor_fusion(Q, O, gpu):
    import ctypes
    import torch
    M, K = 500, 4096
    wt = Q.GGML_TYPE_Q4_K
    wu = weights_q(Q, wt, M, K, seed=1)
    wg = weights_q(Q, wt, M, K, seed=2)
    x = _common.activations(1, K, seed=3)
    b = np.random.default_rng(4).standard_normal(M).astype(np.float32)
    wd, gd, xd, bd = to_dev(wu, gpu), to_dev(wg, gpu), to_dev(x, gpu), to_dev(b, gpu)
    dst = torch.empty((1, M), dtype=torch.float32, device=gpu)
    s0 = Q.make_tensor(wt, [K, M], [144, wu.shape[1]], wd.data_ptr())
    sg = Q.make_tensor(wt, [K, M], [144, wu.shape[1]], gd.data_ptr())
    s1 = Q.make_tensor(Q.GGML_TYPE_F32, [K, 1], [4, K * 4], xd.data_ptr())
    d = Q.make_tensor(Q.GGML_TYPE_F32, [M, 1], [4, M * 4], dst.data_ptr())
    tb = Q.make_tensor(Q.GGML_TYPE_F32, [M], [4], bd.data_ptr())
    fa = Q.q4k_fusion_args(ctypes.pointer(tb), ctypes.pointer(sg), None, Q.GLU_OP_GEGLU)
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, fusion=fa) == Q.Q4K_OK
    ref = Q.mul_mat_vec_q_fused(wd, K, xd, gate=gd, x_bias=bd, glu_op=Q.GLU_OP_GEGLU)
    assert torch.equal(dst, ref)
