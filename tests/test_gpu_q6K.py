"""GPU parity of the Q6_K GEMV (called through the C ABI) against the oracle.

Bar, as for Q4_K: the int32 sums over every 16-weight scale group bit-exact
(the probe runs the GEMV's lane map, staging and dot routine); F32 outputs
within the oracle's parity tolerance (1e-5 relative, or 4 ulp, or 8 f32
epsilons of the row's sum of |term| where terms cancel).  Shapes include odd
numbers of super-blocks per row (rows, and every other block, 2-byte
aligned), partial 16-block groups, 1..8 columns, the column-chunked path for
activations larger than the LDS, strided operands and row slices.
"""
import numpy as np
import pytest

import _common
from test_oracle_q6K import random_q6_blocks, random_q8_1

pytestmark = pytest.mark.gpu

_wcache = {}


def inputs(Q, M, K, N, seed=0):
    """Q6_K weights quantised from N(0, 0.02) (cached per shape and seed)
    and N(0, 1) activations."""
    key = (M, K, seed)
    if key not in _wcache:
        if sum(v.nbytes for v in _wcache.values()) > (1536 << 20):
            _wcache.clear()
        W = _common.weights(M, K, seed)
        _wcache[key] = Q.quantize_rows_q6_K(W, nthreads=16)
        del W
    return _wcache[key], _common.activations(N, K, seed)


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# ---------------------------------------------------------- int sums ----
@pytest.mark.parametrize("M,K,N", [(1, 256, 1), (7, 768, 2), (33, 1280, 1), (64, 4096, 3),
                                   (5, 4352, 1), (40, 14336, 2), (3, 28672, 1)])
def test_group_sums_exact(Q, O, gpu, M, K, N):
    rng = np.random.default_rng([M, K, N])
    wq = random_q6_blocks(rng, M, K)
    q8 = random_q8_1(rng, N, K)
    s16 = Q.group_sums_q6_K(to_dev(wq, gpu), K, to_dev(q8, gpu), N).cpu().numpy()
    ref = O.gemv_q6K_q8_1(wq, K, q8)
    assert ref["mismatches"] == 0
    assert np.array_equal(s16, ref["s16"])


# ------------------------------------------------------ small shapes ----
EDGE_SHAPES = [(1, 256, 1), (3, 768, 2), (5, 2304, 3), (17, 4352, 5), (64, 8192, 8),
               (129, 1024, 7), (1000, 4096, 4), (7, 2048, 6), (2, 512, 8), (1001, 4096, 1),
               (3, 12288, 1), (130, 16384, 2), (2, 14336, 8), (300, 3840, 1)]


@pytest.mark.parametrize("M,K,N", EDGE_SHAPES)
def test_gemv_edge_shapes(Q, O, gpu, M, K, N):
    wq, x = inputs(Q, M, K, N, seed=1)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q6K_q8_1(wq, K, q8, want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    _common.assert_within_tolerance(O, y, ref, f"fused {M}x{K} N={N}")
    y2 = Q.op_mul_mat_vec_q(wd, K, to_dev(q8, gpu), N, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    _common.assert_within_tolerance(O, y2, ref, f"q8_1 {M}x{K} N={N}")
    assert np.array_equal(y, y2)


def test_extreme_blocks(Q, O, gpu):
    """Every 6-bit value, scale and q8 at its extremes (through the pre-
    quantised entry, whose activation is the random Q8_1 itself)."""
    rng = np.random.default_rng(3)
    M, K, N = 50, 4352, 3
    wq = random_q6_blocks(rng, M, K)
    q8 = random_q8_1(rng, N, K)
    ref = O.gemv_q6K_q8_1(wq, K, q8, want_sums=False)
    y = Q.op_mul_mat_vec_q(to_dev(wq, gpu), K, to_dev(q8, gpu), N, wtype=Q.GGML_TYPE_Q6_K)
    _common.assert_within_tolerance(O, y.cpu().numpy(), ref, "extremes")


def test_geometry_variants_agree(Q, O, gpu):
    """8- and 16-wave workgroups and reduced grids (more steps per wave, so
    two groups in flight) all match the oracle and round identically."""
    M, K = 777, 4096
    wq, x = inputs(Q, M, K, 2, seed=4)
    ref = O.gemv_q6K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    outs = []
    try:
        for waves, wgs in ((8, 0), (16, 0), (8, 7), (16, 3), (0, 1)):
            Q.set_geometry_override(waves_per_wg=waves, workgroups=wgs)
            y = Q.mul_mat_vec_q(wd, K, xd, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
            _common.assert_within_tolerance(O, y, ref, f"waves {waves} wgs {wgs}")
            outs.append(y)
    finally:
        Q.set_geometry_override()
    for y in outs[1:]:
        assert np.array_equal(y, outs[0])


def test_strides_slices_and_descriptor(Q, O, gpu):
    """Column strides of src1/dst, a row stride above the row size, a row
    slice starting at an odd row (2-byte aligned, nb odd), and the ggml
    descriptor entry with type Q6_K."""
    import torch
    M, K, N = 45, 1280, 3                       # 5 super-blocks: 1050-byte rows
    wq, x = inputs(Q, M, K, N, seed=9)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q6K_q8_1(wq, K, q8, want_sums=False)
    # strided activation and result; padded weight rows
    xs = torch.zeros((N, K + 64), dtype=torch.float32, device=gpu)
    xs[:, :K] = to_dev(x, gpu)
    ws = torch.zeros((M, wq.shape[1] + 210), dtype=torch.uint8, device=gpu)
    ws[:, :wq.shape[1]] = to_dev(wq, gpu)
    out = torch.full((N, M + 5), 7.0, dtype=torch.float32, device=gpu)
    Q._check(Q.lib().q6k_mul_mat_vec_q(Q._ptr(ws), K, M, ws.stride(0), Q._ptr(xs), N, xs.stride(0) * 4,
                                       Q._ptr(out), out.stride(0) * 4, None, 0, Q._stream()), "strided")
    o = out.cpu().numpy()
    _common.assert_within_tolerance(O, o[:, :M], ref, "strided")
    assert (o[:, M:] == 7.0).all()
    # row slice [11, 30): the slice starts 11*1050 bytes in (2-byte aligned)
    wd = to_dev(wq, gpu)
    flat = wd.reshape(-1)
    lo, hi = 11, 30
    sl = flat[lo * wq.shape[1]:hi * wq.shape[1]].reshape(hi - lo, -1)
    assert sl.data_ptr() % 4 == 2
    y = Q.op_mul_mat_vec_q(sl, K, to_dev(q8, gpu), N, row_low=lo, row_high=hi,
                           wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    sub = {k: v[:, lo:hi] for k, v in ref.items() if k in ("y64", "l1")}
    _common.assert_within_tolerance(O, y, sub, "row slice")
    # descriptor form
    xd = to_dev(x, gpu)
    dst = torch.empty((N, M), dtype=torch.float32, device=gpu)
    s0 = Q.make_tensor(Q.GGML_TYPE_Q6_K, [K, M], [210, wq.shape[1]], wd.data_ptr())
    s1 = Q.make_tensor(Q.GGML_TYPE_F32, [K, N], [4, K * 4], xd.data_ptr())
    d = Q.make_tensor(Q.GGML_TYPE_F32, [M, N], [4, M * 4], dst.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s0, s1, d) == Q.Q4K_OK
    _common.assert_within_tolerance(O, dst.cpu().numpy(), ref, "descriptor")


def test_zero_weight_and_activation(Q, O, gpu):
    import torch
    M, K = 40, 2048
    wq = np.zeros((M, K // 256 * 210), np.uint8)
    x = _common.activations(2, K, 5)
    y = Q.mul_mat_vec_q(to_dev(wq, gpu), K, to_dev(x, gpu), wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    assert (y == 0).all()
    wq2, _ = inputs(Q, M, K, 1, seed=5)
    z = torch.zeros((1, K), dtype=torch.float32, device=gpu)
    y2 = Q.mul_mat_vec_q(to_dev(wq2, gpu), K, z, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    assert (y2 == 0).all()


def test_eight_wave_register_path_long_products(Q, O, gpu):
    """Six or more columns over >= 256 rows per workgroup run 8-wave launches
    whose registers hold every column's activation slices: the oracle on a
    row sample, and bit for bit the pre-quantised launch."""
    M, K, N = 65536, 4096, 6
    Q.set_geometry_override(kernel=1)  # the tile kernel (the automatic choice here is the matrix-core one)
    try:
        _eight_wave_long(Q, O, gpu, M, K, N)
    finally:
        Q.set_geometry_override()


def _eight_wave_long(Q, O, gpu, M, K, N):
    assert Q.geometry(K, M, N, wtype=Q.GGML_TYPE_Q6_K)["waves_per_wg"] == 8
    rng = np.random.default_rng(12)
    wq = random_q6_blocks(rng, M, K, extremes=False)
    x = _common.activations(N, K, 12)
    q8 = O.quantize_q8_1(x)
    rows = np.unique(np.concatenate([[0, 1, M - 2, M - 1], rng.choice(M, 380, replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, q8, want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    _common.assert_within_tolerance(O, y[:, rows], ref, f"8 waves {M}x{K} N={N}")
    y2 = Q.op_mul_mat_vec_q(wd, K, to_dev(q8, gpu), N, wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("M,K,waves", [(300, 12544, 8), (1000, 13568, 16), (300, 14080, 8), (1000, 14336, 16)])
def test_dense_layout_partial_groups(Q, O, gpu, M, K, waves):
    """Eight columns whose padded staging would not fit the LDS run in one
    launch with the dense layout (the last, partial 16-block group packed:
    1, 5, 7 and 8 blocks here), at 8 and 16 waves: outputs of the in-kernel
    and the pre-quantised routes against the oracle, and the launch's int32
    group sums exact."""
    N = 8
    Q.set_geometry_override(waves_per_wg=waves)  # both dense-kernel sizes
    try:
        _dense_partial(Q, O, gpu, M, K, N, waves)
    finally:
        Q.set_geometry_override()


def _dense_partial(Q, O, gpu, M, K, N, waves):
    import torch
    geo = Q.geometry(K, M, N, wtype=Q.GGML_TYPE_Q6_K)
    assert geo["cols_per_launch"] == N and geo["waves_per_wg"] == waves
    # K bytes of q8 per column, d8 and offset terms, a 256-byte ring per wave
    assert geo["lds_bytes"] == N * (K + K // 8 + K // 4) + waves * 64 * 4
    wq, x = inputs(Q, M, K, N, seed=3)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q6K_q8_1(wq, K, q8)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    for w in (None, ws):
        y, s16, _ = Q.mul_mat_vec_q_sums(wd, K, xd, workspace=w, wtype=Q.GGML_TYPE_Q6_K)
        assert np.array_equal(s16.cpu().numpy(), ref["s16"]), f"K={K}: group sums differ"
        y2 = Q.mul_mat_vec_q(wd, K, xd, workspace=w, wtype=Q.GGML_TYPE_Q6_K)
        assert torch.equal(y, y2)
        _common.assert_within_tolerance(O, y2.cpu().numpy(), ref, f"dense {M}x{K} N={N}")


# ------------------------------------------------------- workloads ----
# Q6_K tensors of a Q4_K_M model: ffn_down (4096 x 14336), attn_v
# (1024 x 4096) and the output projection (32000 x 4096, Mistral 7B).
def _q6_cases():
    out = []
    for wl, items in _common.Q6K_WORKLOADS.items():
        for M, K, ns in items:
            out += [pytest.param(M, K, N, id=f"{M}x{K}-N{N}") for N in ns]
    return out


@pytest.mark.parametrize("M,K,N", _q6_cases())
def test_workload_parity(Q, O, gpu, M, K, N):
    """Every output against the (threaded) oracle."""
    wq, x = inputs(Q, M, K, N, seed=0)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q6K_q8_1(wq, K, q8, want_sums=False)
    y = Q.mul_mat_vec_q(to_dev(wq, gpu), K, to_dev(x, gpu), wtype=Q.GGML_TYPE_Q6_K).cpu().numpy()
    st = _common.assert_within_tolerance(O, y, ref, f"{M}x{K} N={N}")
    print(f"[parity] Q6_K {M}x{K} N={N}: {st['n']} outputs, {st['n'] - st['strict_fail']} within 1e-5 rel "
          f"or 4 ulp, {st['strict_fail']} cancelling rows within {st['max_cancel_ulps']:.2f} eps32*sum|term|, "
          f"max err/tol {st['max_ratio']:.3f}", flush=True)
    # the outputs outside the strict bar are rows whose terms cancel; their
    # errors stay within one f32 epsilon of the row's sum of |term|
    # (observed at most 0.27 over every workload)
    assert st["max_cancel_ulps"] <= 1.0, st


@pytest.mark.parametrize("M,K,N", _q6_cases())
def test_production_kernel_sums(Q, O, gpu, M, K, N):
    """The int32 group sums formed inside the kernel the workload runs (the
    SUMS variant of its own launch), bit for bit against the oracle on a row
    sample; the variant's outputs equal the product launch's bit for bit."""
    import torch
    wq, x = inputs(Q, M, K, N, seed=0)
    q8 = O.quantize_q8_1(x)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    rng = np.random.default_rng(M + N)
    rows = np.unique(np.concatenate([[0, 1, M // 2, M - 1], rng.choice(M, min(M, 250), replace=False)]))
    ref = O.gemv_q6K_q8_1(wq[rows], K, q8)
    for w in (ws, None):
        if w is None and K * N <= 40960:
            continue
        y, s16, _ = Q.mul_mat_vec_q_sums(wd, K, xd, workspace=w, wtype=Q.GGML_TYPE_Q6_K)
        assert torch.equal(y, Q.mul_mat_vec_q(wd, K, xd, workspace=w, wtype=Q.GGML_TYPE_Q6_K))
        got = s16[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["s16"]), f"{M}x{K} N={N}: group sums differ"
    print(f"[sums] Q6_K {M}x{K} N={N} {Q.geometry(K, M, N, Q.GGML_TYPE_Q6_K)}: exact", flush=True)


@pytest.mark.parametrize("wtype,M,K,N", [(14, 200, 28672, 4), (14, 600, 28672, 4), (12, 600, 40960, 3)])
def test_small_result_ring_for_long_rows(Q, O, gpu, wtype, M, K, N):
    """Columns this long fit the LDS only with 64-float result rings (Q6_K:
    4 x 28672 values staged in 157,696 bytes; Q4_K: 3 x 40960 in 153,600),
    so the product runs in one launch instead of two.  With one workgroup
    (an override) each wave owns 12-38 rows, i.e. 50-150 ring entries, and
    the ring flushes mid-stream.  Outputs against the oracle, and the
    workspace (pre-quantised) route bit for bit.  (The tile kernel forced:
    at this few rows per CU the automatic launch runs the columns as
    one-column channels.)"""
    import torch
    Q.set_geometry_override(kernel=1)
    try:
        geo = Q.geometry(K, M, N, wtype=wtype)
    finally:
        Q.set_geometry_override()
    assert geo["cols_per_launch"] == N and geo["kernel"] == 1
    if wtype == Q.GGML_TYPE_Q6_K:
        wq, x = inputs(Q, M, K, N, seed=21)
        ref = O.gemv_q6K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
        act = N * (K + K // 8 + K // 4)
    else:
        wq = Q.quantize_rows_q4_K(_common.weights(M, K, 21), nthreads=16)
        x = _common.activations(N, K, 21)
        ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
        act = N * (K + K // 4)
    assert geo["lds_bytes"] == act + geo["waves_per_wg"] * 64 * 4
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    for wgs in (0, 1):
        Q.set_geometry_override(workgroups=wgs, kernel=1)
        try:
            y = Q.mul_mat_vec_q(wd, K, xd, wtype=wtype).cpu().numpy()
            y2 = Q.mul_mat_vec_q(wd, K, xd, workspace=ws, wtype=wtype).cpu().numpy()
        finally:
            Q.set_geometry_override()
        _common.assert_within_tolerance(O, y, ref, f"small ring {M}x{K} N={N} wgs={wgs}")
        assert np.array_equal(y, y2)
