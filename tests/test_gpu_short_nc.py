"""GPU parity of the several-column short-team kernel: two to four columns of
rows of 3 to 8 super-blocks (768 .. 2048 values), one team of as few waves as
the row needs per row tile (three or four columns over 5 to 8 blocks: four
waves, each with super-blocks w and w + 4, the tile kernel's four-column
tree).

Bar: every instantiated launch shape (super-blocks per wave, waves, tiles in
flight) at one workgroup per CU, 7 and 300 workgroups, bit for bit against
the several-column tile kernel (whose reduction tree, for these rows, is the
one-column tree the short teams form); the tile kernel within the parity
tolerance of the oracle; the parity variant's int32 sums and the
activation's block sums bit for bit against the oracle, its outputs equal to
the product's.
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

# instantiated team sizes per super-blocks per wave
TEAMS = {1: (4, 8), 2: (2, 4, 5, 6, 7), 4: (1, 2, 3)}


def team(nb, sbw):
    """The fewest waves that cover nb super-blocks where that team is
    instantiated, else the next power of two."""
    need = -(-nb // sbw)
    if need in TEAMS[sbw]:
        return need
    t = 1
    while t < need:
        t *= 2
    return t


def nc_exists(nc, sbw, kt, waves, slots):
    pair = (sbw, kt) in {(2, 2), (2, 4), (4, 1), (4, 2)} if nc == 2 else (sbw, kt) == (4, 1)
    return pair and waves in (4, 8, 16) and waves % kt == 0 and slots in (1, 2)


def variants(nc, K):
    nb = K // 256
    if nc > 2 and nb > 4:  # super-blocks w and w + 4 per wave, teams of 4
        return [(8, w, s) for w in (4, 8, 16) for s in (1, 2)]
    out = []
    for tr in (8, 4):
        sbw = 16 // tr
        if nc > 2 and sbw != 4:
            continue
        kt = team(nb, sbw)
        out += [(tr, w, s) for w in (4, 8, 16) for s in (1, 2) if nc_exists(nc, sbw, kt, w, s)]
    return out


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def forced(Q, K, M, N, tr, waves, slots, wgs=0):
    Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, workgroups=wgs, kernel=5)
    Q.set_pipeline_override(slots=slots)
    g = Q.geometry(K, M, N)
    assert g["kernel"] == 5 and g["rows_per_step"] == tr and g["waves_per_wg"] == waves, g
    assert g["cols_per_launch"] == N, g


def release(Q):
    Q.set_geometry_override()
    Q.set_pipeline_override()


SHAPES = [(1000, 768, 2), (4096, 1024, 2), (300, 1280, 2), (2048, 1536, 2), (37, 1792, 2), (5, 2048, 2),
          (1030, 2048, 2), (1000, 768, 3), (257, 1024, 3), (4096, 768, 4), (129, 1024, 4), (3, 1024, 4),
          (1000, 1280, 3), (300, 1536, 3), (4096, 1792, 3), (2048, 2048, 4), (37, 2048, 4), (1030, 2048, 3)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_short_nc_bits_equal_tile_kernel(Q, O, gpu, M, K, N):
    assert variants(N, K), (M, K, N)
    wq = Q.quantize_rows_q4_K(_common.weights(M, K, 80 + N), nthreads=16)
    x = _common.activations(N, K, 81 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        assert Q.geometry(K, M, N)["cols_per_launch"] == N
        y_tile = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        release(Q)
    ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile, ref, f"tile {M}x{K} N={N}")
    for tr, waves, slots in variants(N, K):
        for wgs in (0, 7, 300):
            try:
                forced(Q, K, M, N, tr, waves, slots, wgs)
                y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
            finally:
                release(Q)
            if not np.array_equal(y, y_tile):
                bad = np.argwhere(y != y_tile)
                raise AssertionError(f"{M}x{K} N={N} rows/step {tr} waves {waves} slots {slots} wgs {wgs}: "
                                     f"{len(bad)} outputs differ from the tile kernel, e.g. (col, row) "
                                     f"{bad[:5].tolist()}")


@pytest.mark.parametrize("M,K,N", [(1000, 1024, 2), (300, 2048, 2), (257, 768, 3), (129, 1024, 4), (300, 2048, 3),
                                   (129, 1536, 4)])
def test_short_nc_sums_exact(Q, O, gpu, M, K, N):
    import torch
    wq = Q.quantize_rows_q4_K(_common.weights(M, K, 90 + N), nthreads=16)
    x = _common.activations(N, K, 91 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x))
    for tr, waves, slots in variants(N, K):
        try:
            forced(Q, K, M, N, tr, waves, slots)
            y, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd)
            y_prod = Q.mul_mat_vec_q(wd, K, xd)
        finally:
            release(Q)
        where = f"{M}x{K} N={N} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        assert np.array_equal(sums.cpu().numpy(), ref["sqq"]), f"{where}: S_qq differ"
        assert np.array_equal(sq.cpu().numpy(), ref["sq"]), f"{where}: S_q differ"


@pytest.mark.parametrize("M,K,N", [(512, 2048, 2), (3072, 1024, 2), (8192, 2048, 2), (11008, 2048, 2),
                                   (12288, 768, 2), (16384, 2048, 2), (32768, 768, 2), (151936, 1024, 2),
                                   (4096, 768, 3), (16384, 768, 3), (65536, 1024, 3), (8192, 768, 4),
                                   (12288, 1024, 4), (2048, 2048, 3), (8192, 2048, 4), (8960, 1536, 3)])
def test_short_nc_automatic_choice(Q, gpu, M, K, N):
    """Aligned F32 columns of such rows take the kernel by themselves (two
    columns at any rows per CU, three or four from 13), with the tile
    kernel's bits; the pre-quantised route (tile kernel or column split)
    gives the same bits."""
    g = Q.geometry(K, M, N)
    assert g["kernel"] == 5 and g["cols_per_launch"] == N, g
    wq = Q.quantize_rows_q4_K(_common.weights(M, K, 95), nthreads=16)
    x = _common.activations(N, K, 96)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        release(Q)
    assert np.array_equal(y, y_tile)
    q8d = Q.quantize_row_q8_1(xd)
    assert np.array_equal(Q.op_mul_mat_vec_q(wd, K, q8d, N).cpu().numpy(), y)


def test_short_nc_not_elsewhere(Q, gpu):
    """At up to 12 rows per CU with three or four columns of rows of 3 or 4
    blocks, at up to 4 over 5 to 8 (the column split) and over rows of 9 or
    more blocks the kernel is not chosen; rows of 9 or more blocks keep the
    column split to 4 rows per CU only."""
    assert Q.geometry(1024, 3072, 3)["cols_per_launch"] == 1
    assert Q.geometry(2304, 8192, 3)["kernel"] == 1
    assert Q.geometry(2048, 1024, 4)["cols_per_launch"] == 1
    assert Q.geometry(3584, 2048, 2)["cols_per_launch"] == 2
    assert Q.geometry(3584, 1024, 2)["cols_per_launch"] == 1


Q6 = 14
Q6_SHAPES = [(1000, 768, 2), (4096, 1024, 2), (300, 1280, 2), (37, 2048, 2), (1030, 2048, 2), (257, 1024, 3),
             (4096, 768, 4), (5, 1024, 4), (1000, 2048, 3), (257, 1280, 4)]


@pytest.mark.parametrize("M,K,N", Q6_SHAPES)
def test_q6k_short_nc_bits_equal_tile_kernel(Q, O, gpu, M, K, N):
    """The Q6_K form: every instantiated launch shape at 1, 7 and 300
    workgroups bit for bit against the Q6_K several-column tile kernel; the
    tile kernel within the parity tolerance of the oracle."""
    wq = Q.quantize_rows_q6_K(_common.weights(M, K, 110 + N), nthreads=16)
    x = _common.activations(N, K, 111 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        assert Q.geometry(K, M, N, Q6)["cols_per_launch"] == N
        y_tile = Q.mul_mat_vec_q(wd, K, xd, wtype=Q6).cpu().numpy()
    finally:
        release(Q)
    ref = O.gemv_q6K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile, ref, f"Q6_K tile {M}x{K} N={N}")
    for tr, waves, slots in variants(N, K):
        for wgs in (0, 7, 300):
            try:
                Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, workgroups=wgs, kernel=5)
                Q.set_pipeline_override(slots=slots)
                g = Q.geometry(K, M, N, Q6)  # (the Q6_K query reports rows per step as rows_per_tile)
                assert g["kernel"] == 5 and g["rows_per_tile"] == tr and g["waves_per_wg"] == waves, g
                assert g["cols_per_launch"] == N, g
                y = Q.mul_mat_vec_q(wd, K, xd, wtype=Q6).cpu().numpy()
            finally:
                release(Q)
            if not np.array_equal(y, y_tile):
                bad = np.argwhere(y != y_tile)
                raise AssertionError(f"Q6_K {M}x{K} N={N} rows/step {tr} waves {waves} slots {slots} wgs {wgs}: "
                                     f"{len(bad)} outputs differ from the tile kernel, e.g. (col, row) "
                                     f"{bad[:5].tolist()}")


@pytest.mark.parametrize("M,K,N", [(1000, 1024, 2), (300, 2048, 2), (129, 768, 4), (300, 2048, 4)])
def test_q6k_short_nc_sums_exact(Q, O, gpu, M, K, N):
    import torch
    wq = Q.quantize_rows_q6_K(_common.weights(M, K, 120 + N), nthreads=16)
    x = _common.activations(N, K, 121 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ref = O.gemv_q6K_q8_1(wq, K, O.quantize_q8_1(x))
    for tr, waves, slots in variants(N, K):
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots)
            assert Q.geometry(K, M, N, Q6)["kernel"] == 5
            y, sums, _ = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=Q6)
            y_prod = Q.mul_mat_vec_q(wd, K, xd, wtype=Q6)
        finally:
            release(Q)
        where = f"Q6_K {M}x{K} N={N} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        assert np.array_equal(sums.cpu().numpy(), ref["s16"]), f"{where}: group sums differ"


@pytest.mark.parametrize("M,K,N", [(512, 2048, 2), (8192, 2048, 2), (16384, 768, 2), (151936, 1024, 2),
                                   (4096, 768, 3), (8192, 768, 4), (40000, 1024, 4), (2048, 1536, 3),
                                   (8192, 2048, 4)])
def test_q6k_short_nc_automatic_choice(Q, gpu, M, K, N):
    """Q6_K: the same automatic range; the tile kernel's bits, also on the
    pre-quantised route."""
    g = Q.geometry(K, M, N, Q6)
    assert g["kernel"] == 5 and g["cols_per_launch"] == N, g
    wq = Q.quantize_rows_q6_K(_common.weights(M, K, 125), nthreads=16)
    x = _common.activations(N, K, 126)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd, wtype=Q6).cpu().numpy()
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd, wtype=Q6).cpu().numpy()
    finally:
        release(Q)
    assert np.array_equal(y, y_tile)
    q8d = Q.quantize_row_q8_1(xd)
    assert np.array_equal(Q.op_mul_mat_vec_q(wd, K, q8d, N, wtype=Q6).cpu().numpy(), y)
