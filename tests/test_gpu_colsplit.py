"""GPU parity of several columns over few rows per CU, which the op runs as
one-column channels of one broadcast batched launch (the weight shared,
one column per dst channel): on the F32 route the batched one-column
K-split kernel, on the pre-quantised route the batched one-column tile
kernel.

Bar: every column bit for bit equal to the one-column op on that column
(the one-column tile kernel's bits), on both routes; within the parity
tolerance of the oracle; the parity variant's int32 sums bit for bit
against the oracle, its outputs equal to the product's; the geometry query
reports one column per launch.
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def inputs(Q, M, K, N, seed, wtype):
    W = _common.weights(M, K, seed)
    wq = (Q.quantize_rows_q4_K if wtype == Q4 else Q.quantize_rows_q6_K)(W, nthreads=16)
    return wq, _common.activations(N, K, seed + 1)


@pytest.mark.parametrize("wtype,M,K,N", [(Q4, 1024, 4096, 2), (Q4, 1024, 4096, 3), (Q4, 1024, 4096, 5),
                                         (Q4, 1024, 4096, 8), (Q4, 3000, 4096, 4), (Q4, 37, 4096, 6),
                                         (Q4, 512, 14336, 4), (Q4, 1000, 2048, 7), (Q4, 700, 8192, 3),
                                         (Q6, 1024, 4096, 4), (Q6, 1024, 4096, 8), (Q6, 300, 14336, 5)])
def test_columns_as_channels_equal_one_column_products(Q, O, gpu, wtype, M, K, N):
    import torch
    g = Q.geometry(K, M, N, wtype)
    assert g["cols_per_launch"] == 1 and g["kernel"] == 5, g
    wq, x = inputs(Q, M, K, N, 70 + N, wtype)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd, wtype=wtype).cpu().numpy()
    for c in range(N):
        yc = Q.mul_mat_vec_q(wd, K, xd[c:c + 1], wtype=wtype).cpu().numpy()
        assert np.array_equal(y[c], yc[0]), f"column {c} differs from its one-column product"
    q8 = O.quantize_q8_1(x)
    ref = (O.gemv_q4K_q8_1 if wtype == Q4 else O.gemv_q6K_q8_1)(wq, K, q8, want_sums=False)
    _common.assert_within_tolerance(O, y, ref, f"columns as channels {M}x{K} N={N}")
    # the pre-quantised route and a workspace: the same bits
    q8d = Q.quantize_row_q8_1(xd)
    assert np.array_equal(Q.op_mul_mat_vec_q(wd, K, q8d, N, wtype=wtype).cpu().numpy(), y)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    assert np.array_equal(Q.mul_mat_vec_q(wd, K, xd, workspace=ws, wtype=wtype).cpu().numpy(), y)
    # the parity variant: per column, the same kernel and geometry
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, min(M, 60), replace=False)]))
    ys, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=wtype)
    assert np.array_equal(ys.cpu().numpy(), y)
    got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
    if wtype == Q4:
        r = O.gemv_q4K_q8_1(wq[rows], K, q8)
        assert np.array_equal(got, r["sqq"]) and np.array_equal(sq.cpu().numpy(), r["sq"])
    else:
        assert np.array_equal(got, O.gemv_q6K_q8_1(wq[rows], K, q8)["s16"])


@pytest.mark.parametrize("M,K,N", [(1024, 4096, 4), (512, 14336, 3)])
def test_columns_as_channels_unaligned_activation(Q, gpu, M, K, N):
    """Column strides that are not 16-byte multiples (the batched one-column
    tile kernel on the F32 route) and an unaligned base: every column still
    equals its one-column product."""
    import torch
    wq, x = inputs(Q, M, K, N, 90 + N, Q4)
    wd = to_dev(wq, gpu)
    xb = torch.zeros((N, K + 1), dtype=torch.float32, device=gpu)
    xb[:, :K] = to_dev(x, gpu)
    xv = xb[:, :K]  # ldx = K + 1
    y = Q.mul_mat_vec_q(wd, K, xv).cpu().numpy()
    xa = to_dev(x, gpu)
    for c in range(N):
        assert np.array_equal(y[c], Q.mul_mat_vec_q(wd, K, xa[c:c + 1]).cpu().numpy()[0]), f"column {c}"


def test_columns_as_channels_not_at_many_rows(Q, gpu):
    """From 13 rows per CU (8 with two columns) several columns stay in one
    launch (4096 x 4096: the several-column K-split and tile kernels)."""
    for M, K, N in [(4096, 4096, 2), (4096, 4096, 4), (3072, 4096, 2), (14336, 4096, 8)]:
        assert Q.geometry(K, M, N)["cols_per_launch"] == N, (M, K, N)
