"""GPU parity of the batched launches of the descriptor entry
(q4k_ggml_mul_mat_vec_q): channel/sample broadcasting of GGML_OP_MUL_MAT and
GGML_OP_MUL_MAT_ID for one token (kernels/mmvq.cu:174-180, :396-398,
:739-755), for Q4_K and Q6_K weights, with and without the fused epilogue.

Each dst slice is checked against the oracle's 2-D product of the weight
matrix and activation column the reference's index mapping selects:
weight channel c / (ne12/ne02) (MUL_MAT) or ids[j] (MUL_MAT_ID), sample
s / (ne13/ne03), activation channel c (MUL_MAT) or j % ne11 (MUL_MAT_ID).
An expert id outside [0, ne02) must give a zero column (the reference
would read out of bounds; here no weight byte is read).
"""
import ctypes

import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

BB = {12: 144, 14: 210}


def quant(Q, wtype, W):
    return (Q.quantize_rows_q4_K if wtype == 12 else Q.quantize_rows_q6_K)(W, nthreads=16)


def oracle(O, wtype, wq, K, x):
    f = O.gemv_q4K_q8_1 if wtype == 12 else O.gemv_q6K_q8_1
    return f(wq, K, O.quantize_q8_1(x), want_sums=False)


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def tensor(Q, t, ne, nb, ptr):
    return Q.make_tensor(t, list(ne), list(nb), ptr)


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("M,K,ne02,ne03,ne11,ne12,ne13", [
    (300, 1024, 2, 1, 3, 4, 1),       # channel broadcast 2:1, 3 columns
    (64, 4352, 1, 2, 1, 3, 4),        # one matrix per sample, sample broadcast 2:1
    (777, 4096, 3, 1, 8, 3, 1),       # 8 columns, a matrix per channel
    (5000, 2048, 2, 2, 2, 2, 2),      # both dims, one matrix each
])
def test_broadcast_mul_mat(Q, O, gpu, wtype, M, K, ne02, ne03, ne11, ne12, ne13):
    import torch
    rng = np.random.default_rng([M, K, ne02, ne12])
    mats = {}
    wq = np.empty((ne03, ne02, M, K // 256 * BB[wtype]), np.uint8)
    for s in range(ne03):
        for c in range(ne02):
            wq[s, c] = quant(Q, wtype, _common.weights(M, K, seed=10 * s + c))
    x = rng.standard_normal((ne13, ne12, ne11, K)).astype(np.float32)
    # padded strides: 64 extra floats per activation channel, 16 per dst channel
    xs = np.zeros((ne13, ne12, ne11 * K + 64), np.float32)
    xs[:, :, :ne11 * K] = x.reshape(ne13, ne12, -1)
    wd, xd = to_dev(wq, gpu), to_dev(xs, gpu)
    dst = torch.full((ne13, ne12, ne11 * M + 16), 3.0, dtype=torch.float32, device=gpu)
    rb = wq.shape[-1]
    s0 = tensor(Q, wtype, (K, M, ne02, ne03), (BB[wtype], rb, rb * M, rb * M * ne02), wd.data_ptr())
    s1 = tensor(Q, 0, (K, ne11, ne12, ne13), (4, 4 * K, 4 * (ne11 * K + 64), 4 * (ne11 * K + 64) * ne12),
                xd.data_ptr())
    d = tensor(Q, 0, (M, ne11, ne12, ne13), (4, 4 * M, 4 * (ne11 * M + 16), 4 * (ne11 * M + 16) * ne12),
               dst.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s0, s1, d) == Q.Q4K_OK
    out = dst.cpu().numpy()
    for s in range(ne13):
        for c in range(ne12):
            ref = oracle(O, wtype, wq[s // (ne13 // ne03), c // (ne12 // ne02)], K, x[s, c])
            y = out[s, c, :ne11 * M].reshape(ne11, M)
            _common.assert_within_tolerance(O, y, ref, f"sample {s} channel {c}")
            assert (out[s, c, ne11 * M:] == 3.0).all()


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("ne11", [1, 4])
def test_mul_mat_id(Q, O, gpu, wtype, ne11):
    import torch
    M, K, nexp = 768, 2048, 8
    ids = np.array([5, 0, 5, 99], np.int32)          # repeated expert, one invalid id
    nused = len(ids)
    wq = np.stack([quant(Q, wtype, _common.weights(M, K, seed=20 + e)) for e in range(nexp)])
    x = _common.activations(ne11, K, seed=21)
    wd, xd, idd = to_dev(wq, gpu), to_dev(x, gpu), to_dev(ids, gpu)
    dst = torch.full((nused, M), 7.0, dtype=torch.float32, device=gpu)
    rb = wq.shape[-1]
    s0 = tensor(Q, wtype, (K, M, nexp), (BB[wtype], rb, rb * M), wd.data_ptr())
    s1 = tensor(Q, 0, (K, ne11, 1), (4, 4 * K, 4 * K * ne11), xd.data_ptr())
    ti = tensor(Q, 26, (nused, 1), (4, 4 * nused), idd.data_ptr())
    d = tensor(Q, 0, (M, nused, 1), (4, 4 * M, 4 * M * nused), dst.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, ids=ti) == Q.Q4K_OK
    out = dst.cpu().numpy()
    for j, e in enumerate(ids):
        if 0 <= e < nexp:
            ref = oracle(O, wtype, wq[e], K, x[j % ne11:j % ne11 + 1])
            _common.assert_within_tolerance(O, out[j:j + 1], ref, f"slot {j} expert {e}")
        else:
            assert (out[j] == 0.0).all()
    assert np.array_equal(out[0], out[2]) or ne11 > 1   # same expert, same activation


@pytest.mark.parametrize("wtype", [12, 14])
def test_mul_mat_id_fused_swiglu_oai(Q, O, gpu, wtype):
    """MUL_MAT_ID with per-expert biases on both products, a gate weight and
    SWIGLU_OAI (the gpt-oss expert FFN at batch 1)."""
    import torch
    M, K, nexp = 512, 2048, 6
    ids = np.array([3, 1, 4], np.int32)
    nused = len(ids)
    wu = np.stack([quant(Q, wtype, _common.weights(M, K, seed=30 + e)) for e in range(nexp)])
    wg = np.stack([quant(Q, wtype, _common.weights(M, K, seed=40 + e)) for e in range(nexp)])
    rng = np.random.default_rng(5)
    bu = (rng.standard_normal((nexp, M)) * 0.5).astype(np.float32)
    bg = (rng.standard_normal((nexp, M)) * 0.5).astype(np.float32)
    x = _common.activations(1, K, seed=31)
    dev = [to_dev(a, gpu) for a in (wu, wg, bu, bg, x, ids)]
    dst = torch.empty((nused, M), dtype=torch.float32, device=gpu)
    rb = wu.shape[-1]
    s0 = tensor(Q, wtype, (K, M, nexp), (BB[wtype], rb, rb * M), dev[0].data_ptr())
    sg = tensor(Q, wtype, (K, M, nexp), (BB[wtype], rb, rb * M), dev[1].data_ptr())
    tbu = tensor(Q, 0, (M, nexp), (4, 4 * M), dev[2].data_ptr())
    tbg = tensor(Q, 0, (M, nexp), (4, 4 * M), dev[3].data_ptr())
    s1 = tensor(Q, 0, (K, 1, 1), (4, 4 * K, 4 * K), dev[4].data_ptr())
    ti = tensor(Q, 26, (nused, 1), (4, 4 * nused), dev[5].data_ptr())
    d = tensor(Q, 0, (M, nused, 1), (4, 4 * M, 4 * M * nused), dst.data_ptr())
    fa = Q.q4k_fusion_args(ctypes.pointer(tbu), ctypes.pointer(sg), ctypes.pointer(tbg), Q.GLU_OP_SWIGLU_OAI)
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, ids=ti, fusion=fa) == Q.Q4K_OK
    out = dst.cpu().numpy()
    for j, e in enumerate(ids):
        ru = oracle(O, wtype, wu[e], K, x)
        rg = oracle(O, wtype, wg[e], K, x)
        up = ru["y64"][0] + bu[e]
        g = rg["y64"][0] + bg[e]
        tu = O.parity_tolerance(ru["y64"], ru["l1"])[0]
        tg = O.parity_tolerance(rg["y64"], rg["l1"])[0]
        expect = O.glu(O.GLU_SWIGLU_OAI, up, g)
        tol = O.glu_tolerance(O.GLU_SWIGLU_OAI, up, g, tu, tg)
        assert np.all(np.abs(out[j] - expect) <= tol), f"slot {j}"


def test_broadcast_with_fused_bias(Q, O, gpu):
    """Channels with one column each and a bias per channel: equals the
    unfused batched product plus the bias, bit for bit."""
    import torch
    M, K, nch = 1000, 4096, 3
    wq = quant(Q, 12, _common.weights(M, K, seed=50))
    x = _common.activations(nch, K, seed=51)
    b = np.random.default_rng(6).standard_normal((nch, M)).astype(np.float32)
    wd, xd, bd = to_dev(wq, gpu), to_dev(x, gpu), to_dev(b, gpu)
    rb = wq.shape[1]
    s0 = tensor(Q, 12, (K, M, 1), (144, rb, rb * M), wd.data_ptr())
    s1 = tensor(Q, 0, (K, 1, nch), (4, 4 * K, 4 * K), xd.data_ptr())
    dst = torch.empty((nch, M), dtype=torch.float32, device=gpu)
    dst2 = torch.empty((nch, M), dtype=torch.float32, device=gpu)
    d = tensor(Q, 0, (M, 1, nch), (4, 4 * M, 4 * M), dst.data_ptr())
    d2 = tensor(Q, 0, (M, 1, nch), (4, 4 * M, 4 * M), dst2.data_ptr())
    tb = tensor(Q, 0, (M, 1, nch), (4, 4 * M, 4 * M), bd.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s0, s1, d2) == Q.Q4K_OK
    fa = Q.q4k_fusion_args(ctypes.pointer(tb), None, None, 0)
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, fusion=fa) == Q.Q4K_OK
    assert np.array_equal(dst.cpu().numpy(), dst2.cpu().numpy() + b)
    # and the unfused batched product matches the 2-D entry per channel
    for c in range(nch):
        y = Q.mul_mat_vec_q(wd, K, xd[c:c + 1]).cpu().numpy()[0]
        assert np.array_equal(dst2.cpu().numpy()[c], y)
