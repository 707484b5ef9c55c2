"""GPU parity of the matrix-core (MFMA) Q4_K GEMV kernel, called through the C
ABI and forced through the geometry override on shapes where the automatic
geometry would pick another kernel too.

The shapes cover every work split the kernel has: one to eight columns
(columns past the count padded with zeros inside the MFMA), rows of one to
56 super-blocks, ragged tiles (M not a multiple of 16), one tile per
workgroup shared by 2, 4 or 8 waves, and several rounds of tiles per
workgroup.  Each is checked against the oracle (every output, or a row
sample on the largest), with its int32 sub-block sums bit for bit (the
kernel's parity variant, the same launch), against the pre-quantised launch
bit for bit, and against a second run bit for bit (the partial results of
the waves sharing a tile are summed in a fixed order).
"""
import numpy as np
import pytest

import _common
from test_gpu_parity import inputs, to_dev

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 256, 1),        # one tile, one super-block: one wave per tile
    (17, 768, 3),       # two tiles, ragged; 3 super-blocks
    (300, 4096, 8),
    (1000, 4096, 5),
    (4096, 4096, 8),    # one tile per workgroup, 8 waves per tile
    (14336, 4096, 8),   # 3-4 tiles per workgroup
    (2000, 14336, 7),   # 56 super-blocks per row
    (8000, 2048, 6),
    (4099, 1280, 2),
    (64, 16384, 4),
    (33000, 4096, 8),   # several rounds of tiles per workgroup
    (8192, 8192, 6),    # 32 super-blocks per row, chosen automatically
]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_mfma_kernel_against_oracle(Q, O, gpu, M, K, N):
    import torch
    wq, x = inputs(Q, M, K, N, seed=21)
    q8 = O.quantize_q8_1(x)
    if M <= 4099:
        rows = np.arange(M)
    else:
        rng = np.random.default_rng(M + N)
        rows = np.unique(np.concatenate([[0, 1, 15, 16, M - 17, M - 2, M - 1], rng.choice(M, 400, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, q8)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=4)
        geo = Q.geometry(K, M, N)
        assert geo["kernel"] == 4, geo
        y = Q.mul_mat_vec_q(wd, K, xd)
        _common.assert_within_tolerance(O, y.cpu().numpy()[:, rows], ref, f"mfma {M}x{K} N={N}")
        y_again = Q.mul_mat_vec_q(wd, K, xd)
        assert torch.equal(y, y_again), "two runs differ"
        y_q8 = Q.op_mul_mat_vec_q(wd, K, Q.quantize_row_q8_1(xd), N)
        assert torch.equal(y, y_q8), "pre-quantised launch differs"
        ys, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd)
        assert torch.equal(ys, y), "parity variant's outputs differ"
        assert np.array_equal(sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy(), ref["sqq"]), "S_qq differ"
        assert np.array_equal(sq.cpu().numpy(), ref["sq"]), "S_q differ"
    finally:
        Q.set_geometry_override()
    print(f"[mfma] {M}x{K} N={N} {geo}: exact sums, outputs within tolerance", flush=True)


def test_mfma_kernel_zero_inputs(Q, O, gpu):
    """Zero activation and zero weights give exact zeros (no stray values
    from the zero area or the padding columns)."""
    import torch
    M, K, N = 515, 4096, 6
    wq, _ = inputs(Q, M, K, N, seed=22)
    try:
        Q.set_geometry_override(kernel=4)
        z = torch.zeros((N, K), dtype=torch.float32, device=gpu)
        assert (Q.mul_mat_vec_q(to_dev(wq, gpu), K, z) == 0).all()
        wz = torch.zeros_like(to_dev(wq, gpu))
        x = to_dev(_common.activations(N, K, 22), gpu)
        assert (Q.mul_mat_vec_q(wz, K, x) == 0).all()
    finally:
        Q.set_geometry_override()


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 8), (1100, 14336, 6), (2048, 768, 5)])
def test_mfma_result_independent_of_work_split(Q, O, gpu, M, K, N):
    """The summation order depends on K alone: launches over 256, 64, 16 and
    4 workgroups (8, 4, 2 and 1 waves per tile, one to several rounds), the
    8-wave variant and row slices at odd offsets give the same bits."""
    import torch
    wq, x = inputs(Q, M, K, N, seed=23)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    q8d = Q.quantize_row_q8_1(xd)
    try:
        Q.set_geometry_override(kernel=4)
        y = Q.mul_mat_vec_q(wd, K, xd)
        _, sums16, _ = Q.mul_mat_vec_q_sums(wd, K, xd)
        for wgs in (64, 16, 4):
            Q.set_geometry_override(kernel=4, workgroups=wgs)
            assert torch.equal(Q.mul_mat_vec_q(wd, K, xd), y), f"{wgs} workgroups"
        for wgs in (0, 16):
            Q.set_geometry_override(kernel=4, waves_per_wg=8, workgroups=wgs)
            assert Q.geometry(K, M, N)["waves_per_wg"] == 8
            assert torch.equal(Q.mul_mat_vec_q(wd, K, xd), y), f"8 waves, {wgs} workgroups"
            ys, sums, _ = Q.mul_mat_vec_q_sums(wd, K, xd)
            assert torch.equal(ys, y) and torch.equal(sums, sums16)
        Q.set_geometry_override(kernel=4)
        cut = M // 3 + 5
        top = Q.op_mul_mat_vec_q(wd[:cut], K, q8d, N, row_low=0, row_high=cut)
        bot = Q.op_mul_mat_vec_q(wd[cut:], K, q8d, N, row_low=cut, row_high=M)
        assert torch.equal(torch.cat([top, bot], dim=1), y), "row slices"
    finally:
        Q.set_geometry_override()


def test_automatic_choice(Q, gpu):
    """The automatic geometry takes the matrix-core kernel where it measured
    faster: eight columns from 896 row tiles and six to eight from 4096 at
    4096-value rows; six to eight from 512 tiles and five from 864 at longer
    rows whose eight columns fit one launch; never below 4096 values; and
    where the columns do not fit the staged kernel's LDS (4096 x 14336, eight
    columns), the variant that reads its A operand from a Q8_1 copy."""
    for M, K, N, kern in [(14336, 4096, 8, 4), (14336, 4096, 6, 1), (128256, 4096, 6, 4), (4096, 4096, 8, 1),
                          (11008, 4096, 8, 1), (8192, 8192, 8, 4), (8192, 8192, 6, 4), (8192, 8192, 4, 1),
                          (13824, 5120, 5, 4), (8192, 5120, 5, 1), (5120, 5120, 8, 1), (4096, 14336, 8, 6),
                          (18944, 3584, 8, 1), (28672, 10240, 5, 4)]:
        assert Q.geometry(K, M, N)["kernel"] == kern, (M, K, N)
