"""GPU parity of the matrix-core (MFMA) Q6_K GEMV kernel, called through the C
ABI and forced through the geometry override.

The shapes cover one to eight columns (the MFMA's second column half only
from five), rows of one to 64 super-blocks (odd counts: rows and every other
block 2-byte aligned), ragged tiles, one tile shared by 2, 4 or 8 waves,
several rounds per workgroup and the column-chunked path.  Each is checked
against the oracle (every output, or a row sample on the largest), its int32
group sums of (q - 32) * q8 bit for bit (the kernel's parity variant, the same
launch), against the pre-quantised launch bit for bit, and against a second
run bit for bit.
"""
import numpy as np
import pytest

import _common
from test_gpu_q6K import inputs, to_dev
from test_oracle_q6K import random_q6_blocks, random_q8_1

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 256, 1),        # one tile, one super-block
    (17, 768, 3),       # two tiles, ragged; 3 super-blocks per row
    (300, 4096, 8),
    (1000, 4096, 5),
    (4096, 4096, 8),    # one tile per workgroup, 8 waves per tile
    (14336, 4096, 8),   # 3-4 tiles per workgroup
    (2000, 14336, 7),   # 56 super-blocks per row; two launches of 4 and 3 columns
    (8000, 2048, 6),
    (4099, 1280, 2),    # 5 super-blocks per row
    (64, 16384, 4),     # 64 super-blocks per row
    (33000, 4096, 8),   # several rounds of tiles per workgroup
    (4000, 8192, 7),    # 32 super-blocks per row, seven columns in one launch
]


def _force(Q, **kw):
    Q.set_geometry_override(kernel=4, **kw)


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_q6_mfma_kernel_against_oracle(Q, O, gpu, M, K, N):
    import torch
    wq, x = inputs(Q, M, K, N, seed=31)
    q8 = O.quantize_q8_1(x)
    if M <= 4099:
        rows = np.arange(M)
    else:
        rng = np.random.default_rng(M + N)
        rows = np.unique(np.concatenate([[0, 1, 15, 16, M - 17, M - 2, M - 1], rng.choice(M, 400, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, q8)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    t6 = Q.GGML_TYPE_Q6_K
    try:
        _force(Q)
        geo = Q.geometry(K, M, N, t6)
        assert geo["kernel"] == 4, geo
        y = Q.mul_mat_vec_q(wd, K, xd, wtype=t6)
        _common.assert_within_tolerance(O, y.cpu().numpy()[:, rows], ref, f"q6 mfma {M}x{K} N={N}")
        assert torch.equal(y, Q.mul_mat_vec_q(wd, K, xd, wtype=t6)), "two runs differ"
        y_q8 = Q.op_mul_mat_vec_q(wd, K, Q.quantize_row_q8_1(xd), N, wtype=t6)
        assert torch.equal(y, y_q8), "pre-quantised launch differs"
        ys, sums, _ = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=t6)
        assert torch.equal(ys, y), "parity variant's outputs differ"
        got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["s16"]), "group sums differ"
    finally:
        Q.set_geometry_override()
    print(f"[q6 mfma] {M}x{K} N={N} {geo}: exact sums, outputs within tolerance", flush=True)


def test_q6_mfma_extreme_blocks(Q, O, gpu):
    """Every 6-bit value and the scale extremes (-128 and 127): group sums
    exact through the F32 route, and outputs of the pre-quantised route with
    extreme q8 values within tolerance."""
    import torch
    rng = np.random.default_rng(33)
    M, K, N = 600, 4352, 8
    wq = random_q6_blocks(rng, M, K)
    x = _common.activations(N, K, 33)
    q8x = O.quantize_q8_1(x)
    q8r = random_q8_1(rng, N, K)
    ref_x = O.gemv_q6K_q8_1(wq, K, q8x)
    ref_r = O.gemv_q6K_q8_1(wq, K, q8r, want_sums=False)
    wd = to_dev(wq, gpu)
    t6 = Q.GGML_TYPE_Q6_K
    try:
        _force(Q)
        ys, sums, _ = Q.mul_mat_vec_q_sums(wd, K, to_dev(x, gpu), wtype=t6)
        assert np.array_equal(sums.cpu().numpy(), ref_x["s16"]), "group sums differ"
        _common.assert_within_tolerance(O, ys.cpu().numpy(), ref_x, "extreme weights")
        y = Q.op_mul_mat_vec_q(wd, K, to_dev(q8r, gpu), N, wtype=t6).cpu().numpy()
        _common.assert_within_tolerance(O, y, ref_r, "extreme weights and q8")
    finally:
        Q.set_geometry_override()


def test_q6_mfma_zero_inputs(Q, O, gpu):
    """Zero activation and zero weights give exact zeros (no stray values
    from the zero area, the padding columns or the bytes past each block)."""
    import torch
    M, K, N = 515, 4096, 6
    wq, _ = inputs(Q, M, K, N, seed=34)
    t6 = Q.GGML_TYPE_Q6_K
    try:
        _force(Q)
        z = torch.zeros((N, K), dtype=torch.float32, device=gpu)
        assert (Q.mul_mat_vec_q(to_dev(wq, gpu), K, z, wtype=t6) == 0).all()
        wz = torch.zeros_like(to_dev(wq, gpu))
        x = to_dev(_common.activations(N, K, 34), gpu)
        assert (Q.mul_mat_vec_q(wz, K, x, wtype=t6) == 0).all()
    finally:
        Q.set_geometry_override()


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 8), (1100, 14336, 6), (2048, 768, 5)])
def test_q6_mfma_result_independent_of_work_split(Q, O, gpu, M, K, N):
    """The summation order depends on K alone: launches over 256, 64, 16 and
    4 workgroups, the 8-wave variant and row slices at odd offsets give the
    same bits."""
    import torch
    wq, x = inputs(Q, M, K, N, seed=35)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    q8d = Q.quantize_row_q8_1(xd)
    t6 = Q.GGML_TYPE_Q6_K
    try:
        _force(Q)
        y = Q.mul_mat_vec_q(wd, K, xd, wtype=t6)
        _, sums16, _ = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=t6)
        for wgs in (64, 16, 4):
            _force(Q, workgroups=wgs)
            assert torch.equal(Q.mul_mat_vec_q(wd, K, xd, wtype=t6), y), f"{wgs} workgroups"
        for wgs in (0, 16):
            _force(Q, waves_per_wg=8, workgroups=wgs)
            assert Q.geometry(K, M, N, t6)["waves_per_wg"] == 8
            assert torch.equal(Q.mul_mat_vec_q(wd, K, xd, wtype=t6), y), f"8 waves, {wgs} workgroups"
            ys, sums, _ = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=t6)
            assert torch.equal(ys, y) and torch.equal(sums, sums16)
        _force(Q)
        cut = M // 3 + 5
        top = Q.op_mul_mat_vec_q(wd[:cut], K, q8d, N, row_low=0, row_high=cut, wtype=t6)
        bot = Q.op_mul_mat_vec_q(wd[cut:], K, q8d, N, row_low=cut, row_high=M, wtype=t6)
        assert torch.equal(torch.cat([top, bot], dim=1), y), "row slices"
    finally:
        Q.set_geometry_override()


def test_q6_automatic_choice(Q, gpu):
    """The automatic geometry takes the matrix-core kernel for eight columns
    from 896 row tiles and six or more from 2048 on rows of up to 4096
    values, seven or eight from 512 tiles on longer rows (and at 5120 values
    six from 512 and five from 864), the variant that reads its A operand
    from a Q8_1 copy for eight columns the staged kernel cannot hold (4096 x
    14336), the tile kernel elsewhere;
    the Q6_K workloads' eight-column launches of 32768 and 128256 rows (whose
    sums and outputs the workload tests check) are matrix-core launches."""
    t6 = Q.GGML_TYPE_Q6_K
    for M, K, N, kern in [(128256, 4096, 8, 4), (32768, 4096, 8, 4), (14336, 4096, 8, 4), (65536, 4096, 6, 4),
                          (32768, 4096, 6, 4), (128256, 4096, 4, 1), (14336, 4096, 6, 1), (4096, 14336, 8, 6),
                          (4096, 4096, 8, 1), (128256, 4096, 1, 1), (28672, 3584, 8, 4), (13824, 3584, 8, 1),
                          (8192, 8192, 8, 4), (8192, 8192, 7, 4), (28672, 8192, 6, 1), (8192, 5120, 6, 4),
                          (13824, 5120, 5, 4), (8192, 5120, 5, 1), (4096, 8192, 8, 1)]:
        assert Q.geometry(K, M, N, t6)["kernel"] == kern, (M, K, N)
