"""GPU parity of the K-split kernel for two to four F32 columns (rows of
4096 or 8192 values; each wave owns a residue class of super-blocks so that
its DPP steps and the tree over the waves form the tile kernel's
several-column reduction tree), with the activation quantised by every wave
for its own slices (in registers) or once per workgroup into LDS (staged;
pipeline override prologue 2 and 0).

Bar: outputs bit for bit equal to the tile kernel's in every instantiated
launch shape, including uneven row splits and workgroups with fewer rows
than a wave step covers, and within the parity tolerance of the oracle;
the int32 sub-block and activation sums of its parity variant bit for bit
against the oracle.
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu


def exists(nc, tr, waves, slots, G):
    """The instantiated variants (rows per step 8 = two super-blocks per
    wave, two columns only; 4 = four super-blocks; 16 waves where the
    registers fit)."""
    sbw = 16 // tr
    if not (sbw == 4 or (sbw == 2 and nc == 2)):
        return False
    if waves % (16 // sbw) or slots not in (1, 2):
        return False
    return waves < 16 or (G == 1 and (nc < 4 or slots == 1))


def shapes(nc, G):
    return [(tr, w, s) for tr in (8, 4) for w in (4, 8, 16) for s in (1, 2) if exists(nc, tr, w, s, G)]


def long_shapes(p):
    """The long-row form's variants for a p-column tree (rows per step 8:
    two super-blocks per wave, p = 2 only)."""
    return [(tr, w, s) for tr in (8, 4) for w in (4, 8, 16) for s in (1, 2)
            if 16 // tr >= p and w % tr == 0]


def tile_tree(Q, K, M, N):
    """Columns per launch of the tile kernel (whose bits the K-split forms
    reproduce), rounded up to its reduction tree's 2 or 4."""
    try:
        Q.set_geometry_override(kernel=1)
        chunk = Q.geometry(K, M, N)["cols_per_launch"]
    finally:
        Q.set_geometry_override()
    return chunk, (2 if chunk <= 2 else 4)


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


STAGING = {"registers": 2, "staged": 0}


def stagings(nc):
    """Staged variants exist for three or four columns."""
    return list(STAGING) if nc >= 3 else ["registers"]


def run_forced(Q, wd, K, xd, tr, waves, slots, wgs=0, staging="registers"):
    N = xd.shape[0]
    try:
        Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, workgroups=wgs, kernel=5)
        Q.set_pipeline_override(slots=slots, prologue=STAGING[staging])
        g = Q.geometry(K, wd.shape[0], N)
        assert g["kernel"] == 5 and g["rows_per_step"] == tr and g["waves_per_wg"] == waves, g
        assert g["cols_per_launch"] == N, g
        return Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        Q.set_geometry_override()
        Q.set_pipeline_override()


@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 4096), (1024, 4096), (3001, 4096), (37, 4096),
                                 (1, 4096), (5000, 8192), (258, 8192), (20, 8192)])
@pytest.mark.parametrize("N", [2, 3, 4])
def test_ksplit_nc_bits_equal_tile_kernel(Q, O, gpu, M, K, N):
    """Every instantiated launch shape, with one workgroup per CU, 7 (up to
    2048 rows each: uneven tiles per team) and 300 (workgroups with fewer
    rows than a step), against the tile kernel bit for bit; the tile kernel
    against the oracle."""
    wq, x = inputs(Q, M, K, N, seed=31 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        assert Q.geometry(K, M, N)["kernel"] == 1
        y_tile = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        Q.set_geometry_override()
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile[:, rows], ref, f"tile {M}x{K} N={N}")
    for tr, waves, slots in shapes(N, K // 4096):
        for wgs in (0, max(7, -(-M // 2048)), 300):
            for staging in stagings(N):
                y = run_forced(Q, wd, K, xd, tr, waves, slots, wgs, staging)
                if not np.array_equal(y, y_tile):
                    bad = np.argwhere(y != y_tile)
                    raise AssertionError(f"{M}x{K} N={N} rows/step {tr} waves {waves} slots {slots} wgs {wgs} "
                                         f"{staging}: {len(bad)} outputs differ from the tile kernel, e.g. "
                                         f"(col, row) {bad[:5].tolist()}")


@pytest.mark.parametrize("M,K", [(4096, 4096), (333, 4096), (1030, 8192)])
@pytest.mark.parametrize("N", [2, 3, 4])
def test_ksplit_nc_sums_exact(Q, O, gpu, M, K, N):
    """The parity variant of each launch shape: S_qq of every lane and
    column and S_q of the in-register quantisation bit for bit against the
    oracle, outputs equal to the product launch's."""
    import torch
    wq, x = inputs(Q, M, K, N, seed=41 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, 100, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    for (tr, waves, slots), staging in [(sh, st) for sh in shapes(N, K // 4096) for st in stagings(N)]:
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots, prologue=STAGING[staging])
            assert Q.geometry(K, M, N)["kernel"] == 5
            y, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd)
            y_prod = Q.mul_mat_vec_q(wd, K, xd)
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        where = f"{M}x{K} N={N} rows/step {tr} waves {waves} slots {slots} {staging}"
        assert torch.equal(y, y_prod), where
        got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["sqq"]), f"{where}: S_qq differ"
        assert np.array_equal(sq.cpu().numpy(), ref["sq"]), f"{where}: S_q differ"


def test_ksplit_nc_column_strides(Q, O, gpu):
    """Columns further apart than K (a 16-byte multiple) and an output with
    its own stride: the same bits as the tile kernel on the same views."""
    import torch
    M, K, N = 2000, 4096, 3
    wq, x = inputs(Q, M, K, N, seed=51)
    wd = to_dev(wq, gpu)
    xb = torch.zeros((N, K + 64), dtype=torch.float32, device=gpu)
    xb[:, :K] = to_dev(x, gpu)
    xv = xb[:, :K]
    outs = []
    for kern, pro in ((1, -1), (5, 2), (5, 0)):
        ob = torch.full((N, M + 8), -1.0, dtype=torch.float32, device=gpu)
        try:
            Q.set_geometry_override(rows_per_tile=4 if kern == 5 else 0, waves_per_wg=8 if kern == 5 else 0,
                                    kernel=kern)
            Q.set_pipeline_override(prologue=pro)
            assert Q.geometry(K, M, N)["kernel"] == kern
            Q.mul_mat_vec_q(wd, K, xv, out=ob[:, :M])
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        assert torch.all(ob[:, M:] == -1.0), "wrote past the output rows"
        outs.append(ob[:, :M].cpu().numpy())
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


@pytest.mark.parametrize("M,K,N,kernel", [(14336, 4096, 2, 5), (4096, 4096, 2, 5), (1024, 4096, 2, 5),
                                          (128256, 4096, 2, 5), (4096, 8192, 2, 5), (4096, 4096, 3, 5),
                                          (1024, 4096, 3, 5), (1024, 8192, 3, 5), (14336, 4096, 3, 1), (14336, 4096, 4, 1),
                                          (28672, 8192, 3, 5), (28672, 8192, 4, 5), (14336, 8192, 4, 1),
                                          (4096, 14336, 2, 5), (4096, 14336, 3, 5), (4096, 14336, 4, 5),
                                          (8192, 28672, 2, 5), (8192, 28672, 4, 1), (4096, 11008, 4, 5),
                                          (1000, 14336, 3, 5)])
def test_ksplit_nc_automatic_choice(Q, gpu, M, K, N, kernel):
    """The automatic geometry: the K-split kernel where it measured faster
    than the tile kernel (two columns, three columns of 8192 values up to 4
    rows per CU or of 4096 values at 5 to 16, three or four columns of 8192 values at 96 rows
    per CU or more, three or four columns of other lengths up to 16384
    values; up to 12 rows per CU, 8 for two columns, the one-column K-split
    kernel over the columns as channels), the tile kernel elsewhere; the
    pre-quantised route stays on the tile kernel (same bits)."""
    g = Q.geometry(K, M, N)
    # few rows per CU: the columns as one-column channels of one launch (one
    # column each, on the one-column K-split kernel)
    cols = 1 if (M, K, N) in {(1024, 4096, 2), (1024, 4096, 3), (1024, 8192, 3), (1000, 14336, 3)} else N
    assert g["kernel"] == kernel and g["cols_per_launch"] == cols, g
    assert Q.geometry(K, M, N, route="q8_1")["kernel"] == 1


@pytest.mark.parametrize("M,K", [(4096, 14336), (1000, 14336), (333, 28672), (777, 11008), (500, 5120),
                                 (64, 2304), (37, 256)])
@pytest.mark.parametrize("N", [2, 3, 4])
def test_ksplit_nc_long_bits_equal_tile_kernel(Q, O, gpu, M, K, N):
    """The long-row form (rows of any length up to 8 groups, the last one
    partial here except at 14336 and 28672; 256 and 2304 values: one
    partial group), every instantiated launch shape at one workgroup per CU,
    7 and 300 workgroups, against the tile kernel bit for bit (28672 values
    in four columns: the tile kernel's LDS takes two per launch, and the
    K-split form forms their two-column tree); the tile kernel against the
    oracle."""
    chunk, p = tile_tree(Q, K, M, N)
    if N % chunk:
        pytest.skip(f"the tile kernel launches {chunk} of {N} columns at a time: no K-split form")
    wq, x = inputs(Q, M, K, N, seed=61 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        Q.set_geometry_override()
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile[:, rows], ref, f"tile {M}x{K} N={N}")
    for tr, waves, slots in long_shapes(p):
        for wgs in (0, 7, 300):
            y = run_forced(Q, wd, K, xd, tr, waves, slots, wgs, "staged")
            if not np.array_equal(y, y_tile):
                bad = np.argwhere(y != y_tile)
                raise AssertionError(f"{M}x{K} N={N} rows/step {tr} waves {waves} slots {slots} wgs {wgs}: "
                                     f"{len(bad)} outputs differ from the tile kernel, e.g. (col, row) "
                                     f"{bad[:5].tolist()}")


@pytest.mark.parametrize("M,K,N", [(1000, 14336, 2), (333, 14336, 3), (300, 28672, 4), (129, 5120, 4)])
def test_ksplit_nc_long_sums_exact(Q, O, gpu, M, K, N):
    """The long-row form's parity variant: S_qq of every lane and column and
    S_q of the staging bit for bit against the oracle, outputs equal to the
    product launch's."""
    import torch
    chunk, p = tile_tree(Q, K, M, N)
    wq, x = inputs(Q, M, K, N, seed=71 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, 60, replace=False)]))
    ref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    for tr, waves, slots in long_shapes(p):
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots)
            assert Q.geometry(K, M, N)["kernel"] == 5
            y, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd)
            y_prod = Q.mul_mat_vec_q(wd, K, xd)
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        where = f"{M}x{K} N={N} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["sqq"]), f"{where}: S_qq differ"
        assert np.array_equal(sq.cpu().numpy(), ref["sq"]), f"{where}: S_q differ"


# ---------------------------------------------------------------- Q6_K ----

_w6cache = {}


def inputs_q6(Q, M, K, N, seed):
    key = (M, K, seed)
    if key not in _w6cache:
        _w6cache.clear()
        _w6cache[key] = Q.quantize_rows_q6_K(_common.weights(M, K, seed), nthreads=16)
    return _w6cache[key], _common.activations(N, K, seed)


def tile_tree_q6(Q, K, M, N):
    t6 = Q.GGML_TYPE_Q6_K
    try:
        Q.set_geometry_override(kernel=1)
        chunk = Q.geometry(K, M, N, t6)["cols_per_launch"]
    finally:
        Q.set_geometry_override()
    return chunk, (2 if chunk <= 2 else 4)


def run_forced_q6(Q, wd, K, xd, tr, waves, slots, wgs=0):
    t6 = Q.GGML_TYPE_Q6_K
    N = xd.shape[0]
    try:
        Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, workgroups=wgs, kernel=5)
        Q.set_pipeline_override(slots=slots)
        g = Q.geometry(K, wd.shape[0], N, t6)
        assert g["kernel"] == 5 and g["rows_per_tile"] == tr and g["waves_per_wg"] == waves, g
        assert g["cols_per_launch"] == N, g
        return Q.mul_mat_vec_q(wd, K, xd, wtype=t6).cpu().numpy()
    finally:
        Q.set_geometry_override()
        Q.set_pipeline_override()


@pytest.mark.parametrize("M,K", [(4096, 14336), (1000, 14336), (333, 28672), (777, 11008), (500, 5120),
                                 (64, 2304), (37, 256), (1024, 4096), (300, 8192)])
@pytest.mark.parametrize("N", [2, 3, 4])
def test_q6k_ksplit_nc_bits_equal_tile_kernel(Q, O, gpu, M, K, N):
    """Q6_K, two to four columns (the staged form for rows of any length up
    to 8 groups, partial last groups included), every instantiated launch
    shape at one workgroup per CU, 7 and 300 workgroups, against the Q6_K
    tile kernel bit for bit; the tile kernel against the oracle."""
    t6 = Q.GGML_TYPE_Q6_K
    chunk, p = tile_tree_q6(Q, K, M, N)
    if N % chunk:
        pytest.skip(f"the tile kernel launches {chunk} of {N} columns at a time: no K-split form")
    wq, x = inputs_q6(Q, M, K, N, seed=81 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        Q.set_geometry_override(kernel=1)
        y_tile = Q.mul_mat_vec_q(wd, K, xd, wtype=t6).cpu().numpy()
    finally:
        Q.set_geometry_override()
    rows = np.arange(M) if M <= 1024 else np.unique(
        np.concatenate([[0, 1, M - 2, M - 1], np.random.default_rng(M).choice(M, 300, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, y_tile[:, rows], ref, f"Q6_K tile {M}x{K} N={N}")
    for tr, waves, slots in long_shapes(p):
        for wgs in (0, 7, 300):
            y = run_forced_q6(Q, wd, K, xd, tr, waves, slots, wgs)
            if not np.array_equal(y, y_tile):
                bad = np.argwhere(y != y_tile)
                raise AssertionError(f"Q6_K {M}x{K} N={N} rows/step {tr} waves {waves} slots {slots} wgs {wgs}: "
                                     f"{len(bad)} outputs differ from the tile kernel, e.g. (col, row) "
                                     f"{bad[:5].tolist()}")


@pytest.mark.parametrize("M,K,N", [(1000, 14336, 2), (333, 14336, 3), (300, 28672, 4), (129, 5120, 4),
                                   (500, 4096, 4)])
def test_q6k_ksplit_nc_sums_exact(Q, O, gpu, M, K, N):
    """Q6_K: the parity variant's int32 group sums of every lane and column
    bit for bit against the oracle, outputs equal to the product launch's."""
    import torch
    t6 = Q.GGML_TYPE_Q6_K
    chunk, p = tile_tree_q6(Q, K, M, N)
    wq, x = inputs_q6(Q, M, K, N, seed=91 + N)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    rows = np.unique(np.concatenate([[0, M // 2, M - 1], np.random.default_rng(M).choice(M, 60, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, O.quantize_q8_1(x))
    for tr, waves, slots in long_shapes(p):
        try:
            Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, kernel=5)
            Q.set_pipeline_override(slots=slots)
            assert Q.geometry(K, M, N, t6)["kernel"] == 5
            y, s16, _ = Q.mul_mat_vec_q_sums(wd, K, xd, wtype=t6)
            y_prod = Q.mul_mat_vec_q(wd, K, xd, wtype=t6)
        finally:
            Q.set_geometry_override()
            Q.set_pipeline_override()
        where = f"Q6_K {M}x{K} N={N} rows/step {tr} waves {waves} slots {slots}"
        assert torch.equal(y, y_prod), where
        got = s16[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["s16"]), f"{where}: group sums differ"


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 2), (1000, 14336, 3), (28672, 8192, 4)])
def test_ksplit_nc_unaligned_activation_same_bits(Q, gpu, M, K, N):
    """An activation that is not 16-byte aligned cannot take the K-split
    kernels (16-byte loads): the op runs the tile kernel there, whose
    outputs are the same bits as the automatic (K-split) launch on an
    aligned copy of the same values."""
    import torch
    assert Q.geometry(K, M, N)["kernel"] == 5
    wq, x = inputs(Q, M, K, N, seed=101 + N)
    wd = to_dev(wq, gpu)
    xa = to_dev(x, gpu)
    xb = torch.zeros((N, K + 4), dtype=torch.float32, device=gpu)
    xb[:, 1:K + 1] = xa
    xu = xb[:, 1:K + 1]  # 4-byte aligned, not 16
    assert xu.data_ptr() % 16 != 0
    y_aligned = Q.mul_mat_vec_q(wd, K, xa).cpu().numpy()
    y_unaligned = Q.mul_mat_vec_q(wd, K, xu).cpu().numpy()
    assert np.array_equal(y_aligned, y_unaligned)
