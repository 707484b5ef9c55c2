"""Q4_K weight quantiser: invariants of the oracle's restatement of
quantize_row_q4_K_ref (its stages are pinned against ggml's published
algorithm in test_oracle_quantiser_pins.py); the product's host quantiser
must equal it byte for byte."""
import numpy as np
import pytest

import _common


def _fields(wq, K):
    import test_oracle_gemv as T
    return T.np_unpack_q4K(wq, K)


def test_reconstruction_error_bound(O):
    M, K = 64, 2048
    W = _common.weights(M, K, seed=21)
    wq = O.quantize_q4_K(W)
    q, sc, mm, d, dmin = _fields(wq, K)
    dsub = np.repeat(d, 8, 1) * sc              # per sub-block step
    msub = np.repeat(dmin, 8, 1) * mm
    rec = dsub[..., None] * q.reshape(M, -1, 32) - msub[..., None]
    err = np.abs(rec - W.reshape(M, -1, 32))
    interior = (q.reshape(M, -1, 32) > 0) & (q.reshape(M, -1, 32) < 15)
    # re-quantisation picks the nearest level unless clamped to 0 or 15
    assert (err[interior] <= (dsub[..., None] * np.ones_like(err))[interior] * 0.5 * (1 + 1e-3) + 1e-7).all()
    rel = np.sqrt((err ** 2).mean()) / np.sqrt((W ** 2).mean())
    assert rel < 0.1
    # dequantisation agrees with the oracle's own dequantiser
    assert np.allclose(O.dequantize_q4_K(wq, K), rec.reshape(M, K), rtol=1e-6, atol=1e-7)
    assert (d >= 0).all() and (dmin >= 0).all()


def test_special_blocks(O):
    K = 256
    z = np.zeros((1, K), np.float32)
    assert (O.quantize_q4_K(z) == 0).all()
    c = np.full((1, K), 0.5, np.float32)
    rec = O.dequantize_q4_K(O.quantize_q4_K(c), K)
    assert np.abs(rec - 0.5).max() < 0.5 / 30
    neg = -np.abs(_common.weights(1, K, 7))
    rec = O.dequantize_q4_K(O.quantize_q4_K(neg), K)
    assert np.abs(rec - neg).max() < 0.02


@pytest.mark.parametrize("M,K,scale", [(33, 256, 0.02), (8, 4096, 1.0), (17, 1280, 1e-4),
                                       (4, 512, 300.0)])
def test_host_quantiser_equals_oracle(O, Q, M, K, scale):
    W = _common.weights(M, K, seed=M) * np.float32(scale / 0.02)
    W[0, :32] = 0.0                     # zero sub-block
    W[1 % M, 32:64] = 1e-30             # tiny values
    W[2 % M, 64:96] = np.float32(scale)  # constant sub-block
    assert np.array_equal(Q.quantize_rows_q4_K(W, nthreads=3), O.quantize_q4_K(W))
