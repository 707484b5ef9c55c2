"""GPU parity of the K-split kernels (one F32 column; the waves of a
workgroup split each row's super-blocks and quantise their own slice of the
activation: in registers for rows of 4096 or 8192 values, into per-wave LDS
slices for rows of other lengths up to 8 groups).

Bar: outputs bit for bit equal to the tile kernel's (both sum every row in
the same balanced tree over super-block positions) in every instantiated
launch shape, including uneven row splits and workgroups with fewer rows
than a wave step covers, and within the parity tolerance of the oracle;
the int32 sub-block and activation sums of its parity variant bit for bit
against the oracle.
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

# (rows per wave step, waves per workgroup, tiles in flight) of the
# instantiated variants for rows of one group; rows of two groups exist
# for 4..16 rows per step
SHAPES_G1 = [(tr, w, s) for tr in (16, 8, 4, 1) for w in (4, 8, 16) for s in (1, 2)
             if w >= tr and not (tr == 1 and w == 16)]
SHAPES_G2 = [(tr, w, s) for (tr, w, s) in SHAPES_G1 if tr >= 4]

_wcache = {}


def inputs(Q, M, K, seed):
    key = (M, K, seed)
    if key not in _wcache:
        _wcache.clear()
        _wcache[key] = Q.quantize_rows_q4_K(_common.weights(M, K, seed), nthreads=16)
    return _wcache[key], _common.activations(1, K, seed)


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def few_workgroups(M):
    """A small grid (hundreds of rows per workgroup, uneven tiles per team)
    whose (row, slice) partials still fit the LDS: at most 2048 rows each."""
    return max(7, -(-M // 2048))


def run_forced(Q, wd, K, xd, tr, waves, slots, wgs=0, prologue=-1):
    try:
        Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, workgroups=wgs, kernel=5)
        Q.set_pipeline_override(slots=slots, prologue=prologue)
        g = Q.geometry(K, wd.shape[0], 1)
        assert g["kernel"] == 5 and g["rows_per_step"] == tr and g["waves_per_wg"] == waves, g
        return Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        Q.set_geometry_override()
        Q.set_pipeline_override()


@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 4096), (1024, 4096), (3001, 4096), (37, 4096),
                                 (1, 4096), (5000, 8192), (258, 8192), (20, 8192)])
def test_ksplit_bits_equal_tile_kernel(Q, O, gpu, M, K):
    """Every instantiated launch shape, with the default one workgroup per
    CU, a few workgroups (hundreds of rows each, uneven tiles per team) and
    300 (several workgroups with fewer rows than a step), against the tile
    kernel bit for bit; the tile kernel against the oracle."""
    wq, x = inputs(Q, M, K, seed=21)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        Q.set_geometry_override()
    rows = np.arange(M) if M <= 4096 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 400, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile[:, rows], ref, f"tile {M}x{K}")
    shapes = SHAPES_G1 if K == 4096 else SHAPES_G2
    for tr, waves, slots in shapes:
        for wgs in (0, few_workgroups(M), 300):
            y = run_forced(Q, wd, K, xd, tr, waves, slots, wgs)
            if not np.array_equal(y, y_tile):
                bad = np.flatnonzero(y[0] != y_tile[0])
                raise AssertionError(f"{M}x{K} rows/step {tr} waves {waves} slots {slots} wgs {wgs}: "
                                     f"{bad.size} outputs differ from the tile kernel, e.g. rows {bad[:5]}")


@pytest.mark.parametrize("M,K", [(4096, 4096), (333, 4096), (1030, 8192)])
def test_ksplit_sums_exact(Q, O, gpu, M, K):
    """The parity variant of each launch shape: S_qq of every lane and S_q of
    the in-register quantisation bit for bit against the oracle, outputs
    equal to the product launch's."""
    import torch
    wq, x = inputs(Q, M, K, seed=22)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, 120, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    shapes = SHAPES_G1 if K == 4096 else SHAPES_G2
    for tr, waves, slots in shapes:
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots)
            y, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd)
            y_prod = Q.mul_mat_vec_q(wd, K, xd)
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        where = f"{M}x{K} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["sqq"]), f"{where}: S_qq differ"
        assert np.array_equal(sq.cpu().numpy(), ref["sq"]), f"{where}: S_q differ"


def test_ksplit_unaligned_activation_and_q8_1_route(Q, O, gpu):
    """An activation that is not 16-byte aligned, and a pre-quantised Q8_1
    activation, never reach the K-split kernel (it takes 16-byte loads of F32
    values): the override falls back to the tile kernel there, whose outputs
    are the same bits."""
    import torch
    M, K = 777, 4096
    wq, x = inputs(Q, M, K, seed=23)
    wd = to_dev(wq, gpu)
    buf = torch.zeros(K + 1, dtype=torch.float32, device=gpu)
    buf[1:] = to_dev(x[0], gpu)
    xa = buf[:K].clone()
    xa.copy_(buf[1:])
    y_al = run_forced(Q, wd, K, xa.view(1, K), 8, 16, 1)
    y_un = run_forced(Q, wd, K, buf[1:].view(1, K), 8, 16, 1)
    assert np.array_equal(y_al, y_un)
    try:
        Q.set_geometry_override(rows_per_tile=8, waves_per_wg=16, kernel=5)
        y_q8 = Q.op_mul_mat_vec_q(wd, K, Q.quantize_row_q8_1(xa.view(1, K)), 1).cpu().numpy()
    finally:
        Q.set_geometry_override()
    assert np.array_equal(y_q8, y_al)


# ------------------------------------------------------------------ Q6_K ----
# (rows per wave step, waves, tiles in flight) of the Q6_K K-split variants
Q6_SHAPES_G1 = [(tr, w, s) for tr in (16, 8, 4) for w in (4, 8, 16) for s in (1, 2) if w >= tr]
Q6_SHAPES_G2 = [(tr, w, s) for (tr, w, s) in Q6_SHAPES_G1 if not (s == 2 and w == 16)]

_w6cache = {}


def inputs6(Q, M, K, seed):
    key = (M, K, seed)
    if key not in _w6cache:
        _w6cache.clear()
        _w6cache[key] = Q.quantize_rows_q6_K(_common.weights(M, K, seed), nthreads=16)
    return _w6cache[key], _common.activations(1, K, seed)


def run_forced6(Q, wd, K, xd, tr, waves, slots, wgs=0, prologue=-1):
    t6 = Q.GGML_TYPE_Q6_K
    try:
        Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, workgroups=wgs, kernel=5)
        Q.set_pipeline_override(slots=slots, prologue=prologue)
        g = Q.geometry(K, wd.shape[0], 1, t6)
        assert g["kernel"] == 5 and g["rows_per_tile"] == tr and g["waves_per_wg"] == waves, g
        return Q.mul_mat_vec_q(wd, K, xd, wtype=t6).cpu().numpy()
    finally:
        Q.set_geometry_override()
        Q.set_pipeline_override()


@pytest.mark.parametrize("M,K", [(1024, 4096), (32768, 4096), (3001, 4096), (37, 4096), (1, 4096), (2049, 8192),
                                 (20, 8192)])
def test_q6k_ksplit_bits_equal_tile_kernel(Q, O, gpu, M, K):
    """Q6_K: every instantiated launch shape, with one workgroup per CU, a
    few and 300 workgroups, against the Q6_K tile kernel bit for bit (210-byte
    blocks: every other block's loads 2-byte aligned); the tile kernel
    against the oracle."""
    t6 = Q.GGML_TYPE_Q6_K
    wq, x = inputs6(Q, M, K, seed=31)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd, wtype=t6).cpu().numpy()
    finally:
        Q.set_geometry_override()
    rows = np.arange(M) if M <= 4096 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 400, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile[:, rows], ref, f"Q6_K tile {M}x{K}")
    for tr, waves, slots in (Q6_SHAPES_G1 if K == 4096 else Q6_SHAPES_G2):
        for wgs in (0, few_workgroups(M), 300):
            y = run_forced6(Q, wd, K, xd, tr, waves, slots, wgs)
            if not np.array_equal(y, y_tile):
                bad = np.flatnonzero(y[0] != y_tile[0])
                raise AssertionError(f"Q6_K {M}x{K} rows/step {tr} waves {waves} slots {slots} wgs {wgs}: "
                                     f"{bad.size} outputs differ from the tile kernel, e.g. rows {bad[:5]}")


@pytest.mark.parametrize("M,K", [(1024, 4096), (333, 4096), (517, 8192)])
def test_q6k_ksplit_group_sums_exact(Q, O, gpu, M, K):
    """The Q6_K parity variant of each launch shape: every lane's int32 group
    sums (q - 32) * q8, starting from the -32 * sum q8 the in-register
    quantisation hands over, bit for bit against the oracle."""
    import torch
    t6 = Q.GGML_TYPE_Q6_K
    wq, x = inputs6(Q, M, K, seed=32)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, 100, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    for tr, waves, slots in (Q6_SHAPES_G1 if K == 4096 else Q6_SHAPES_G2):
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots)
            y, s16, _ = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=t6)
            y_prod = Q.mul_mat_vec_q(wd, K, xd, wtype=t6)
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        where = f"Q6_K {M}x{K} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        got = s16[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["s16"]), f"{where}: group sums differ"


# -------------------------------------------------------- long rows ----
# (rows per wave step, waves, steps in flight) of the long-row variants: 8
# or 16 rows per step for rows of up to 8 groups, 4 for rows of up to 4;
# three or four steps in flight in workgroups of up to 8 waves
LONG_SHAPES = [(tr, w, s) for tr in (16, 8) for w in (8, 16) for s in (1, 2) if w >= tr] + [(8, 8, 3), (8, 8, 4)]
LONG_SHAPES_4 = [(4, w, s) for w in (4, 8, 16) for s in (1, 2)] + [(4, w, s) for w in (4, 8) for s in (3, 4)]


def short_team_shapes(K):
    """Rows of 9 to 14 blocks: the team sizes other than powers of two (teams
    of ceil(blocks / 2) waves at 8 rows per step, of 3 at 4 rows for up to
    12 blocks), one, two or four teams per workgroup."""
    nb = K // 256
    if not 9 <= nb <= 14:
        return []
    kt = (nb + 1) // 2
    out = [(8, kt, 1), (8, 2 * kt, 1), (8, kt, 2), (8, 2 * kt, 2)]
    if nb <= 12:
        out += [(4, 3, 1), (4, 6, 1), (4, 12, 1), (4, 6, 2)]
    return out


def long_shapes(K):
    return LONG_SHAPES + (LONG_SHAPES_4 if -(-K // 4096) <= 4 else []) + short_team_shapes(K)


@pytest.mark.parametrize("M,K", [(4096, 14336), (1000, 14336), (37, 12544), (300, 3584), (513, 2048),
                                 (96, 28672), (2000, 28672), (5, 256), (33, 20480), (700, 1024), (300, 1536),
                                 (1030, 768), (700, 2560), (300, 3072), (129, 2304)])
def test_ksplit_long_rows_bits_equal_tile_kernel(Q, O, gpu, M, K):
    """Rows of any length up to 8 groups (the last group partial: 14336 =
    3.5 groups, 12544 = 3 groups + 1 block, 3584 and 2048 under one group,
    256 = one block): every long-row launch shape, with the default grid, a
    few and 300 workgroups, against the tile kernel bit for bit; the tile
    kernel against the oracle.  Rows of 3 to 14 blocks (768 .. 3584) run
    with teams of only the waves the row needs."""
    wq, x = inputs(Q, M, K, seed=41)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        Q.set_geometry_override()
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile[:, rows], ref, f"tile {M}x{K}")
    for tr, waves, slots in long_shapes(K):
        # every group staged before the first step (prologue 2) and each just
        # before the step that first reads it (0), with the default grid
        for wgs, pro in ((0, 0), (0, 2), (few_workgroups(M), -1), (300, -1)):
            y = run_forced(Q, wd, K, xd, tr, waves, slots, wgs, pro)
            if not np.array_equal(y, y_tile):
                bad = np.flatnonzero(y[0] != y_tile[0])
                raise AssertionError(f"long {M}x{K} rows/step {tr} waves {waves} slots {slots} wgs {wgs} "
                                     f"prologue {pro}: {bad.size} outputs differ from the tile kernel, "
                                     f"e.g. rows {bad[:5]}")


@pytest.mark.parametrize("M,K", [(700, 14336), (50, 12544), (129, 2048), (77, 768), (77, 2560)])
def test_ksplit_long_rows_sums_exact(Q, O, gpu, M, K):
    """The long-row parity variants: S_qq of every lane in the row's blocks
    and S_q of the in-register quantisation (blocks of the partial group
    included) bit for bit against the oracle."""
    import torch
    wq, x = inputs(Q, M, K, seed=42)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, min(M, 100), replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    for tr, waves, slots in long_shapes(K):
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots)
            y, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd)
            y_prod = Q.mul_mat_vec_q(wd, K, xd)
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        where = f"long {M}x{K} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["sqq"]), f"{where}: S_qq differ"
        assert np.array_equal(sq.cpu().numpy(), ref["sq"]), f"{where}: S_q differ"


@pytest.mark.parametrize("M,K", [(4096, 14336), (1000, 14336), (37, 12544), (300, 3584), (96, 28672),
                                 (5, 256), (33, 20480), (513, 2048), (300, 1536), (1030, 768), (700, 2560),
                                 (129, 3072)])
def test_q6k_ksplit_long_rows_bits_equal_tile_kernel(Q, O, gpu, M, K):
    """Q6_K rows of any length up to 8 groups: every long-row launch shape,
    with the default grid, a few and 300 workgroups, against the Q6_K tile
    kernel bit for bit; the tile kernel against the oracle."""
    t6 = Q.GGML_TYPE_Q6_K
    wq, x = inputs6(Q, M, K, seed=43)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd, wtype=t6).cpu().numpy()
    finally:
        Q.set_geometry_override()
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile[:, rows], ref, f"Q6_K tile {M}x{K}")
    for tr, waves, slots in long_shapes(K):
        for wgs, pro in ((0, 0), (0, 2), (few_workgroups(M), -1), (300, -1)):
            y = run_forced6(Q, wd, K, xd, tr, waves, slots, wgs, pro)
            if not np.array_equal(y, y_tile):
                bad = np.flatnonzero(y[0] != y_tile[0])
                raise AssertionError(f"Q6_K long {M}x{K} rows/step {tr} waves {waves} slots {slots} wgs {wgs} "
                                     f"prologue {pro}: {bad.size} outputs differ from the tile kernel, "
                                     f"e.g. rows {bad[:5]}")


@pytest.mark.parametrize("M,K", [(700, 14336), (50, 12544), (129, 2048), (77, 768), (77, 3072)])
def test_q6k_ksplit_long_rows_group_sums_exact(Q, O, gpu, M, K):
    """The Q6_K long-row parity variants: every lane's int32 group sums,
    from the -32 * sum q8 starting values staged per 16 values, bit for bit
    against the oracle (the partial group's blocks included)."""
    import torch
    t6 = Q.GGML_TYPE_Q6_K
    wq, x = inputs6(Q, M, K, seed=44)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, min(M, 100), replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    for tr, waves, slots in long_shapes(K):
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots)
            y, s16, _ = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=t6)
            y_prod = Q.mul_mat_vec_q(wd, K, xd, wtype=t6)
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        where = f"Q6_K long {M}x{K} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        got = s16[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["s16"]), f"{where}: group sums differ"
