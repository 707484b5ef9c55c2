"""GPU parity of the matrix-core Q4_K and Q6_K kernels that read their A
operand (the q8 of up to eight activation columns) straight from the Q8_1
buffer instead of an LDS copy of the whole activation (kernel 6: the
pre-quantised route).

Bar: on rows of 4096 values, where the staged matrix-core kernel also runs,
outputs bit for bit equal to it (both sum a row's super-blocks in the same
segments and tree, which depend on K alone); on long rows, which the staged
kernel cannot hold in LDS, within the parity tolerance of the oracle; the
int32 sub-block sums S_qq and the block sums S_q of q8 (formed here by a
second MFMA against a B of ones) bit for bit against the oracle.
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

_wcache = {}


def inputs(Q, M, K, N, seed):
    key = (M, K, seed)
    if key not in _wcache:
        _wcache.clear()
        _wcache[key] = Q.quantize_rows_q4_K(_common.weights(M, K, seed), nthreads=16)
    return _wcache[key], _common.activations(N, K, seed)


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def run_pre(Q, wd, K, q8d, N, kernel, wgs=0, inflight=0):
    try:
        Q.set_geometry_override(kernel=kernel, workgroups=wgs)
        Q.set_pipeline_override(slots=inflight)
        g = Q.geometry(K, wd.shape[0], N, route="q8_1")
        assert g["kernel"] == (6 if kernel == 6 else 4), g
        return Q.op_mul_mat_vec_q(wd, K, q8d, N).cpu().numpy()
    finally:
        Q.set_geometry_override()
        Q.set_pipeline_override()


@pytest.mark.parametrize("M,N", [(14336, 8), (4096, 8), (1000, 6), (37, 5), (16, 8), (300, 3), (129, 1)])
def test_ga_bits_equal_staged_mfma(Q, O, gpu, M, N):
    """Rows of 4096 values, 1..8 columns, partial last tiles: the GA kernel
    with 2 and 4 items in flight against the staged matrix-core kernel bit
    for bit on the same Q8_1 columns, with one workgroup per CU and with 7
    workgroups (several rounds per workgroup); the staged kernel against the
    oracle."""
    K = 4096
    wq, x = inputs(Q, M, K, N, seed=51)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    q8d = Q.quantize_row_q8_1(xd)
    y4 = run_pre(Q, wd, K, q8d, N, 4)
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y4[:, rows], ref, f"staged mfma {M}x{K} N={N}")
    for wgs in (0, 7):
        for nif in (2, 4):
            y6 = run_pre(Q, wd, K, q8d, N, 6, wgs, nif)
            if not np.array_equal(y6, y4):
                bad = np.argwhere(y6 != y4)
                raise AssertionError(f"GA {M}x{K} N={N} wgs {wgs} in flight {nif}: {len(bad)} outputs differ, "
                                     f"e.g. {bad[:4].tolist()}")


@pytest.mark.parametrize("M,K,N", [(4096, 14336, 8), (4096, 14336, 6), (1000, 14336, 5), (300, 28672, 8),
                                   (33, 12544, 7), (64, 20480, 8)])
def test_ga_long_rows_against_oracle(Q, O, gpu, M, K, N):
    """Rows too long for the staged kernel's LDS copy of eight columns: the
    GA kernel (forced, and on the automatic choice where it is made) within
    tolerance of the oracle; the pre-quantised launch and the F32 launch
    with a workspace (which quantises separately) give the same bits."""
    import torch
    wq, x = inputs(Q, M, K, N, seed=52)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    q8d = Q.quantize_row_q8_1(xd)
    y6 = run_pre(Q, wd, K, q8d, N, 6)
    assert np.array_equal(run_pre(Q, wd, K, q8d, N, 6, inflight=2), y6)
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y6[:, rows], ref, f"GA {M}x{K} N={N}")
    if Q.geometry(K, M, N, route="q8_1")["kernel"] == 6:
        assert np.array_equal(Q.op_mul_mat_vec_q(wd, K, q8d, N).cpu().numpy(), y6)
        ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
        assert np.array_equal(Q.mul_mat_vec_q(wd, K, xd, workspace=ws).cpu().numpy(), y6)


@pytest.mark.parametrize("M,K,N", [(4096, 14336, 8), (333, 8192, 6), (50, 28672, 3)])
def test_ga_sums_exact(Q, O, gpu, M, K, N):
    """The GA parity variant (through the op with a workspace, so the same
    quantiser and route as production): S_qq of every sampled row and
    sub-block, and S_q of every block and column, bit for bit against the
    oracle; its outputs equal the product launch's."""
    import torch
    wq, x = inputs(Q, M, K, N, seed=53)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, min(M, 120), replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    try:
        Q.set_geometry_override(kernel=6)
        y, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd, workspace=ws)
        y_prod = Q.mul_mat_vec_q(wd, K, xd, workspace=ws)
        assert Q.geometry(K, M, N, route="q8_1")["kernel"] == 6
    finally:
        Q.set_geometry_override()
    assert torch.equal(y, y_prod)
    got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
    assert np.array_equal(got, ref["sqq"]), f"GA {M}x{K} N={N}: S_qq differ"
    assert np.array_equal(sq.cpu().numpy(), ref["sq"]), f"GA {M}x{K} N={N}: S_q differ"


def test_ga_is_the_automatic_choice_for_eight_long_columns(Q):
    """4096 x 14336 with eight columns (the mistral down projection's batch
    shape) runs the GA kernel on the pre-quantised route, in one launch."""
    g = Q.geometry(14336, 4096, 8, route="q8_1")
    assert g["kernel"] == 6 and g["cols_per_launch"] == 8 and g["waves_per_wg"] == 8, g


# ------------------------------------------------------------------ Q6_K ----
_w6cache = {}


def inputs6(Q, M, K, N, seed):
    key = (M, K, seed)
    if key not in _w6cache:
        _w6cache.clear()
        _w6cache[key] = Q.quantize_rows_q6_K(_common.weights(M, K, seed), nthreads=16)
    return _w6cache[key], _common.activations(N, K, seed)


def run_pre6(Q, wd, K, q8d, N, kernel, wgs=0):
    t6 = Q.GGML_TYPE_Q6_K
    try:
        Q.set_geometry_override(kernel=kernel, workgroups=wgs)
        g = Q.geometry(K, wd.shape[0], N, t6, route="q8_1")
        assert g["kernel"] == (6 if kernel == 6 else 4), g
        return Q.op_mul_mat_vec_q(wd, K, q8d, N, wtype=t6).cpu().numpy()
    finally:
        Q.set_geometry_override()


@pytest.mark.parametrize("M,N", [(14336, 8), (4096, 8), (1000, 6), (37, 5), (16, 8), (300, 3), (129, 1)])
def test_q6k_ga_bits_equal_staged_mfma(Q, O, gpu, M, N):
    """Q6_K rows of 4096 values: the GA kernel against the staged Q6_K
    matrix-core kernel bit for bit on the same Q8_1 columns (one and two
    column halves per MFMA), with one workgroup per CU and with 7; the
    staged kernel against the oracle."""
    K = 4096
    wq, x = inputs6(Q, M, K, N, seed=61)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    q8d = Q.quantize_row_q8_1(xd)
    y4 = run_pre6(Q, wd, K, q8d, N, 4)
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y4[:, rows], ref, f"Q6_K staged mfma {M}x{K} N={N}")
    for wgs in (0, 7):
        y6 = run_pre6(Q, wd, K, q8d, N, 6, wgs)
        if not np.array_equal(y6, y4):
            bad = np.argwhere(y6 != y4)
            raise AssertionError(f"Q6_K GA {M}x{K} N={N} wgs {wgs}: {len(bad)} outputs differ, e.g. {bad[:4].tolist()}")


@pytest.mark.parametrize("M,K,N", [(4096, 14336, 8), (4096, 14336, 6), (300, 28672, 8), (33, 12544, 7)])
def test_q6k_ga_long_rows_against_oracle(Q, O, gpu, M, K, N):
    """Q6_K rows too long for the staged kernel's LDS copy: the GA kernel
    within tolerance of the oracle; where it is the automatic choice the
    pre-quantised launch and the F32 launch with a workspace give its bits."""
    import torch
    t6 = Q.GGML_TYPE_Q6_K
    wq, x = inputs6(Q, M, K, N, seed=62)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    q8d = Q.quantize_row_q8_1(xd)
    y6 = run_pre6(Q, wd, K, q8d, N, 6)
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y6[:, rows], ref, f"Q6_K GA {M}x{K} N={N}")
    if Q.geometry(K, M, N, t6, route="q8_1")["kernel"] == 6:
        assert np.array_equal(Q.op_mul_mat_vec_q(wd, K, q8d, N, wtype=t6).cpu().numpy(), y6)
        ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
        assert np.array_equal(Q.mul_mat_vec_q(wd, K, xd, workspace=ws, wtype=t6).cpu().numpy(), y6)


@pytest.mark.parametrize("M,K,N", [(4096, 14336, 8), (333, 8192, 6), (50, 28672, 3)])
def test_q6k_ga_group_sums_exact(Q, O, gpu, M, K, N):
    """The Q6_K GA parity variant through the op with a workspace: the int32
    group sums of (q - 32) * q8 bit for bit against the oracle; its outputs
    equal the product launch's."""
    import torch
    t6 = Q.GGML_TYPE_Q6_K
    wq, x = inputs6(Q, M, K, N, seed=63)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, min(M, 120), replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    try:
        Q.set_geometry_override(kernel=6)
        y, s16, _ = Q.mul_mat_vec_q_sums(wd, K, xd, workspace=ws, wtype=t6)
        y_prod = Q.mul_mat_vec_q(wd, K, xd, workspace=ws, wtype=t6)
        assert Q.geometry(K, M, N, t6, route="q8_1")["kernel"] == 6
    finally:
        Q.set_geometry_override()
    assert torch.equal(y, y_prod)
    got = s16[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
    assert np.array_equal(got, ref["s16"]), f"Q6_K GA {M}x{K} N={N}: group sums differ"
