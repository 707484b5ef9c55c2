"""GPU parity of the HIP path (called through the C ABI) against the oracle.

Bar: Q8_1 bytes and int32 sub-block sums bit-exact; F32 outputs within the
parity tolerance of the oracle's f64 result (1e-5 relative, or 4 ulp, or 8
f32 epsilons of the row's sum of |term| where terms cancel).  Full-size
workloads check every output against the oracle on a row sample (rows are
independent) and all outputs through size-independent properties: the fused
and pre-quantised launches agree bit for bit, and row-split calls reassemble
the full result exactly.
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

_wcache = {}


def inputs(Q, M, K, N, seed=0):
    """Q4_K weights quantised from N(0, 0.02) (cached per shape and seed:
    every workload shape fits, ~640 MB) and N(0, 1) activations."""
    key = (M, K, seed)
    if key not in _wcache:
        if sum(v.nbytes for v in _wcache.values()) > (1536 << 20):
            _wcache.clear()
        W = _common.weights(M, K, seed)
        _wcache[key] = Q.quantize_rows_q4_K(W, nthreads=16)
        del W
    return _wcache[key], _common.activations(N, K, seed)


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def oracle_rows(O, wq, K, q8, rows):
    ref = O.gemv_q4K_q8_1(wq[rows], K, q8, want_sums=False)
    return ref


# --------------------------------------------------------------- Q8_1 ----
@pytest.mark.parametrize("N,K,kpad,ld", [(1, 4096, 4096, 4096), (3, 4096, 4096, 4160),
                                         (2, 14336, 14336, 14336), (1, 300, 512, 320),
                                         (8, 8192, 8192, 8192), (2, 301, 512, 301), (3, 1000, 1024, 1003)])
def test_quantize_q8_1_bytes_exact(Q, O, gpu, N, K, kpad, ld):
    import torch
    x = np.zeros((N, ld), np.float32)
    x[:, :K] = _common.activations(N, K, seed=K)
    x[0, :32] = 0.0  # one all-zero block
    xd = to_dev(x, gpu)
    out = torch.empty((N, kpad // 32 * 36), dtype=torch.uint8, device=gpu)
    Q._check(Q.lib().q4k_quantize_row_q8_1(Q._ptr(xd), Q._ptr(out), K, ld, kpad, N, Q._stream()), "q8_1")
    ref = np.stack([O.quantize_q8_1(x[c:c + 1, :K], k_padded=kpad)[0] for c in range(N)])
    assert np.array_equal(out.cpu().numpy(), ref)


def test_quantize_q8_1_exact_ties(Q, O, gpu):
    """Values on exact ties x/d = k + 1/2 (d = 2^e) and their one-ulp
    neighbours: the standalone quantiser's bytes equal the oracle's
    (roundf: ties away from zero)."""
    import torch
    rng = np.random.default_rng(78)
    nblk = 128
    e = rng.integers(-20, 10, size=nblk)
    t = rng.integers(-127, 127, size=(nblk, 32)).astype(np.float64) + 0.5
    t[:, 0] = 127.0
    x = (t * 2.0 ** e[:, None]).astype(np.float32)
    x[1::3, 2:] = np.nextafter(x[1::3, 2:], np.float32(np.inf))
    x[2::3, 2:] = np.nextafter(x[2::3, 2:], np.float32(-np.inf))
    x = x.reshape(2, -1)
    K = x.shape[1]
    xd = to_dev(x, gpu)
    out = torch.empty((2, K // 32 * 36), dtype=torch.uint8, device=gpu)
    Q._check(Q.lib().q4k_quantize_row_q8_1(Q._ptr(xd), Q._ptr(out), K, K, K, 2, Q._stream()), "q8_1")
    assert np.array_equal(out.cpu().numpy(), O.quantize_q8_1(x, k_padded=K))


def _hip_runtime():
    """The HIP runtime this process already uses (the one torch loaded)."""
    import ctypes
    paths = sorted({ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln})
    assert len(paths) == 1, paths
    hip = ctypes.CDLL(paths[0])
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipMalloc.restype = ctypes.c_int
    hip.hipGetLastError.restype = ctypes.c_int
    hip.hipPeekAtLastError.restype = ctypes.c_int
    hip.hipGetDevice.argtypes = [ctypes.POINTER(ctypes.c_int)]
    return hip


def test_caller_error_is_left_alone(Q, O, gpu):
    """An error a caller's earlier HIP call left behind (a failed huge
    hipMalloc) is neither returned nor cleared by successful calls of the
    library: every launch checks its own status.  Covers the workspace route
    (standalone quantiser + GEMV), the in-launch route and the probes."""
    import ctypes
    import torch
    hip = _hip_runtime()
    M, K, N = 300, 14336, 4
    wq, x = inputs(Q, M, K, N, seed=8)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    dst = torch.empty((N, M), dtype=torch.float32, device=gpu)
    q8 = torch.empty((N, Q.q8_1_bytes(K, 1)), dtype=torch.uint8, device=gpu)
    sqq = torch.empty((1, M, K // 32), dtype=torch.int32, device=gpu)
    sq = torch.empty((1, K // 32), dtype=torch.int32, device=gpu)
    torch.cuda.synchronize()
    L, s = Q.lib(), Q._stream()
    hip.hipGetLastError()
    p = ctypes.c_void_p()
    err = hip.hipMalloc(ctypes.byref(p), 1 << 62)
    assert err != 0
    dev = ctypes.c_int()
    hip.hipGetDevice(ctypes.byref(dev))
    if hip.hipPeekAtLastError() != err:
        hip.hipGetLastError()
        pytest.skip("this HIP runtime resets the last error on every successful call")
    assert L.q4k_mul_mat_vec_q(Q._ptr(wd), K, M, K // 256 * 144, Q._ptr(xd), N, K * 4, Q._ptr(dst), M * 4,
                               Q._ptr(ws), ws.numel(), s) == Q.Q4K_OK
    assert L.q4k_mul_mat_vec_q(Q._ptr(wd), K, M, K // 256 * 144, Q._ptr(xd), 1, K * 4, Q._ptr(dst), M * 4,
                               None, 0, s) == Q.Q4K_OK
    assert L.q4k_quantize_row_q8_1(Q._ptr(xd), Q._ptr(q8), K, K, K, N, s) == Q.Q4K_OK
    assert L.q4k_subblock_sums(Q._ptr(wd), K, M, K // 256 * 144, Q._ptr(q8), 1, K // 32, Q._ptr(sqq),
                               Q._ptr(sq), s) == Q.Q4K_OK
    assert hip.hipGetLastError() == err
    assert hip.hipGetLastError() == 0
    torch.cuda.synchronize()
    ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, dst.cpu().numpy()[:1], {k: v[:1] for k, v in ref.items() if v is not None},
                                    "after error")


# ---------------------------------------------------------- int sums ----
@pytest.mark.parametrize("M,K,N", [(5, 256, 1), (33, 768, 2), (64, 2304, 3), (4096, 4096, 1),
                                   (96, 14336, 2), (40, 28672, 1)])
def test_subblock_sums_exact(Q, O, gpu, M, K, N):
    wq, x = inputs(Q, M, K, N)
    q8 = O.quantize_q8_1(x)
    sqq, sq = Q.subblock_sums(to_dev(wq, gpu), K, to_dev(q8, gpu), N)
    ref = O.gemv_q4K_q8_1(wq, K, q8)
    assert np.array_equal(sq.cpu().numpy(), ref["sq"])
    assert np.array_equal(sqq.cpu().numpy(), ref["sqq"])


# ------------------------------------------------------ small shapes ----
EDGE_SHAPES = [(1, 256, 1), (3, 768, 2), (5, 2304, 3), (17, 4352, 5), (64, 8192, 8),
               (129, 1024, 7), (1000, 4096, 4), (7, 2048, 6), (2, 512, 8),
               # block-per-lane kernel: 16, 32 and 33..64 super-blocks per row
               (1001, 4096, 1), (3, 8192, 1), (5, 12288, 1), (130, 16384, 1), (2, 14336, 1)]


@pytest.mark.parametrize("M,K,N", EDGE_SHAPES)
def test_gemv_edge_shapes(Q, O, gpu, M, K, N):
    wq, x = inputs(Q, M, K, N, seed=1)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q4K_q8_1(wq, K, q8, want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    _common.assert_within_tolerance(O, y, ref, f"fused {M}x{K} N={N}")
    y2 = Q.op_mul_mat_vec_q(wd, K, to_dev(q8, gpu), N).cpu().numpy()
    _common.assert_within_tolerance(O, y2, ref, f"q8_1 {M}x{K} N={N}")
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("M,K", [(999, 4096), (258, 8192), (97, 14336), (64, 16384), (3001, 4096),
                                 (5, 12288)])
def test_kernel_variants_against_oracle(Q, O, gpu, M, K):
    """Every GEMV kernel (tile, block-per-lane, block with coalesced loads) on
    shapes where each can run, forced through the geometry override."""
    wq, x = inputs(Q, M, K, 1, seed=7)
    ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    try:
        for kern in (1, 2, 3):
            Q.set_geometry_override(kernel=kern)
            assert Q.geometry(K, M, 1)["kernel"] == kern
            y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
            _common.assert_within_tolerance(O, y, ref, f"kernel {kern} {M}x{K}")
    finally:
        Q.set_geometry_override()


@pytest.mark.parametrize("M,K,N", [(2048, 2048, 8), (1024, 4096, 5), (1024, 4096, 7), (300, 3072, 8),
                                   (768, 2048, 3), (12288, 4096, 6), (28672, 4096, 3)])
def test_eight_wave_register_path(Q, O, gpu, M, K, N):
    """8-wave launches with three or more columns of one-group rows: the
    activation slices of every column held in registers, and staging rounds
    issued ahead of the weights up to the column count, of which only those
    holding values are loaded (2048- and 3072-value rows need fewer).  Checked
    against the oracle, and bit for bit against the pre-quantised launch.
    (The tile kernel forced: up to 12 rows per CU the automatic launch runs
    the columns as one-column channels.)"""
    Q.set_geometry_override(kernel=1)
    try:
        _eight_wave_register_path(Q, O, gpu, M, K, N)
    finally:
        Q.set_geometry_override()


def _eight_wave_register_path(Q, O, gpu, M, K, N):
    assert Q.geometry(K, M, N)["waves_per_wg"] == 8
    wq, x = inputs(Q, M, K, N, seed=11)
    q8 = O.quantize_q8_1(x)
    if M <= 1024:
        rows = np.arange(M)
    else:
        rng = np.random.default_rng(M)
        rows = np.unique(np.concatenate([[0, 1, M - 2, M - 1], rng.choice(M, 380, replace=False)]))
    ref = oracle_rows(O, wq, K, q8, rows)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    _common.assert_within_tolerance(O, y[:, rows], ref, f"8 waves {M}x{K} N={N}")
    y2 = Q.op_mul_mat_vec_q(wd, K, Q.quantize_row_q8_1(xd), N).cpu().numpy()
    assert np.array_equal(y, y2)


@pytest.mark.parametrize("M,K", [(1000, 2048), (37, 768), (4099, 1280), (513, 512), (3, 1024),
                                 (2047, 256), (20000, 2048)])
def test_short_rows(Q, O, gpu, M, K):
    """Rows of at most 8 super-blocks (lanes past a row's end read zeros),
    from one to thousands of rows per workgroup: against the oracle, with the
    bias epilogue, and bit for bit against the pre-quantised launch."""
    wq, x = inputs(Q, M, K, 1, seed=13)
    q8 = O.quantize_q8_1(x)
    if M <= 4099:
        rows = np.arange(M)
    else:
        rng = np.random.default_rng(M)
        rows = np.unique(np.concatenate([[0, 1, M - 2, M - 1], rng.choice(M, 380, replace=False)]))
    ref = oracle_rows(O, wq, K, q8, rows)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    _common.assert_within_tolerance(O, y[:, rows], ref, f"short rows {M}x{K}")
    y2 = Q.op_mul_mat_vec_q(wd, K, Q.quantize_row_q8_1(xd), 1).cpu().numpy()
    assert np.array_equal(y, y2)
    bias = np.random.default_rng(M + K).standard_normal(M).astype(np.float32)
    yb = Q.mul_mat_vec_q_fused(wd, K, xd, x_bias=to_dev(bias, gpu)).cpu().numpy()
    assert np.array_equal(yb, (y + bias).astype(np.float32))


def test_fused_quantisation_at_ties(Q, O, gpu):
    """Activations whose x/d falls exactly on, or one ulp beside, a half-integer:
    round-half-away (ggml's roundf) and round-half-even differ there, so the
    in-launch quantiser must take its exact path.  The fused launch must match
    the standalone quantiser (bytes checked against the oracle) bit for bit."""
    M, K, N = 64, 4096, 3
    wq, _ = inputs(Q, M, K, 1, seed=6)
    rng = np.random.default_rng(6)
    x = np.zeros((N, K), np.float32)
    blocks = x.reshape(N, -1, 32)
    blocks[:, :, 0] = 127.0                      # amax = 127 -> d = 1 exactly
    halves = (rng.integers(-127, 127, size=blocks[:, :, 1:].shape) + 0.5).astype(np.float32)
    blocks[:, :, 1:] = halves
    blocks[1, :, 1:] = np.nextafter(halves[1], np.float32(0))             # one ulp inside
    blocks[2, ::2, 0] = 100.0                    # d = 100/127: generic quotients
    blocks[2, ::2, 1:] = rng.uniform(-100, 100, size=blocks[2, ::2, 1:].shape)
    x = x.reshape(N, K)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q4K_q8_1(wq, K, q8, want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    q8d = Q.quantize_row_q8_1(xd)
    assert np.array_equal(q8d.cpu().numpy(), q8)
    y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    y2 = Q.op_mul_mat_vec_q(wd, K, q8d, N).cpu().numpy()
    assert np.array_equal(y, y2)
    _common.assert_within_tolerance(O, y, ref, "ties")


def test_concurrent_calls_from_host_threads(Q, O, gpu):
    """Four host threads, each with its own stream, calling the op at once
    (ctypes releases the GIL): shapes whose launches need the large-LDS
    attribute, the workspace route and the one-launch route.  Every result
    must equal the same call made alone."""
    import threading
    import torch
    shapes = [(300, 14336, 2), (999, 4096, 1), (64, 8192, 8), (513, 2048, 3)]
    data = []
    for M, K, N in shapes:
        wq, x = inputs(Q, M, K, N, seed=21)
        wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
        ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
        alone = Q.mul_mat_vec_q(wd, K, xd, workspace=ws).cpu().numpy()
        data.append((K, wd, xd, ws, alone))
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        K, wd, xd, ws, alone = data[t]
        st = torch.cuda.Stream(device=gpu)
        try:
            with torch.cuda.stream(st):
                outs = [Q.mul_mat_vec_q(wd, K, xd, workspace=ws, stream=st) for _ in range(20)]
            st.synchronize()
            for o in outs:
                if not np.array_equal(o.cpu().numpy(), alone):
                    errors.append(t)
                    break
        except Exception as e:  # reported below
            errors.append((t, repr(e)))

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(len(shapes))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors


def test_zero_activation_and_zero_weight(Q, O, gpu):
    M, K, N = 40, 1024, 3
    wq, x = inputs(Q, M, K, N, seed=2)
    x = x.copy()
    x[1] = 0.0
    wq = wq.copy()
    wq[5] = 0
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q4K_q8_1(wq, K, q8, want_sums=False)
    y = Q.mul_mat_vec_q(to_dev(wq, gpu), K, to_dev(x, gpu)).cpu().numpy()
    _common.assert_within_tolerance(O, y, ref, "zeros")
    assert (y[1] == 0).all() and (y[:, 5] == 0).all()


def test_strides_and_no_out_of_bounds_writes(Q, O, gpu):
    """Padded weight rows, padded activation columns and a dst column stride
    larger than M; the padding of dst must stay untouched."""
    import torch
    M, K, N = 37, 2048, 3
    wq, x = inputs(Q, M, K, N, seed=3)
    rb = wq.shape[1]
    wpad = np.full((M, rb + 144 * 2), 0xAB, np.uint8)
    wpad[:, :rb] = wq
    xpad = np.full((N, K + 64), np.nan, np.float32)
    xpad[:, :K] = x
    ld = M + 11
    dst = torch.full((N, ld), -7.0, dtype=torch.float32, device=gpu)
    wd, xd = to_dev(wpad, gpu), to_dev(xpad, gpu)
    st = Q.lib().q4k_mul_mat_vec_q(Q._ptr(wd), K, M, wpad.shape[1], Q._ptr(xd), N, (K + 64) * 4,
                                   Q._ptr(dst), ld * 4, None, 0, Q._stream())
    assert st == Q.Q4K_OK
    out = dst.cpu().numpy()
    assert (out[:, M:] == -7.0).all()
    ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    _common.assert_within_tolerance(O, out[:, :M], ref, "strided")


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("M,K,N", [(300, 14336, 4), (300, 14336, 3), (77, 28672, 2), (130, 8192, 8)])
def test_workspace_route_for_long_columns(Q, O, gpu, wtype, M, K, N):
    """With a workspace and K * N > 40960 the op quantises in a launch of its
    own and runs the GEMV on the Q8_1 buffer; without one (or with one too
    small) the GEMV quantises in-launch.  Both give the same bits, within
    the oracle's tolerance.  The activations outgrow the four staging rounds
    a 16-wave workgroup issues ahead by 1.25 (N=3), 3 (N=2, N=4) and 4 (N=8)
    rounds; from four columns on the staging loads them two rounds at a
    time."""
    import torch
    if wtype == 12:
        wq, x = inputs(Q, M, K, N, seed=8)
        ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    else:
        wq = Q.quantize_rows_q6_K(_common.weights(M, K, seed=8), nthreads=16)
        x = _common.activations(N, K, seed=9)
        ref = O.gemv_q6K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    need = Q.q8_1_bytes(K, N)
    y = Q.mul_mat_vec_q(wd, K, xd, wtype=wtype).cpu().numpy()
    _common.assert_within_tolerance(O, y, ref, f"in-launch {M}x{K} N={N}")
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    y2 = Q.mul_mat_vec_q(wd, K, xd, workspace=ws, wtype=wtype).cpu().numpy()
    assert np.array_equal(y, y2)
    small = torch.empty(need - 4, dtype=torch.uint8, device=gpu)
    y3 = Q.mul_mat_vec_q(wd, K, xd, workspace=small, wtype=wtype).cpu().numpy()
    assert np.array_equal(y, y3)


def test_unquantised_path_for_large_activation(Q, O, gpu):
    """K=28672 with 8 columns does not fit one workgroup's LDS: the op
    quantises to a Q8_1 buffer (caller workspace or stream-ordered temporary)
    and runs the GEMV in column chunks."""
    import torch
    M, K, N = 96, 28672, 8
    geo = Q.geometry(K, M, N)
    wq, x = inputs(Q, M, K, N, seed=4)
    ref = O.gemv_q4K_q8_1(wq, K, O.quantize_q8_1(x), want_sums=False)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    _common.assert_within_tolerance(O, y, ref, f"large K ({geo})")
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    y2 = Q.mul_mat_vec_q(wd, K, xd, workspace=ws).cpu().numpy()
    assert np.array_equal(y, y2)


def test_ggml_descriptor_entry(Q, O, gpu):
    import torch
    M, K, N = 300, 4096, 2
    wq, x = inputs(Q, M, K, N, seed=5)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    dst = torch.empty((N, M), dtype=torch.float32, device=gpu)
    s0 = Q.make_tensor(Q.GGML_TYPE_Q4_K, [K, M], [144, wq.shape[1]], wd.data_ptr())
    s1 = Q.make_tensor(Q.GGML_TYPE_F32, [K, N], [4, K * 4], xd.data_ptr())
    d = Q.make_tensor(Q.GGML_TYPE_F32, [M, N], [4, M * 4], dst.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s0, s1, d) == Q.Q4K_OK
    y = Q.mul_mat_vec_q(wd, K, xd)
    assert torch.equal(dst, y)
    # argument errors the reference asserts on
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, ids=s1) == Q.Q4K_EINVAL        # ids not I32
    s3 = Q.make_tensor(Q.GGML_TYPE_Q4_K, [K, M, 2], [144, wq.shape[1], wq.nbytes], wd.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s3, s1, d) == Q.Q4K_EINVAL                # 1 channel over 2 matrices
    q5 = Q.make_tensor(13, [K, M], [176, K // 256 * 176], wd.data_ptr())
    assert Q.ggml_mul_mat_vec_q(q5, s1, d) == Q.Q4K_EUNSUPPORTED          # left to the caller
    bad = Q.make_tensor(Q.GGML_TYPE_F32, [K + 256, N], [4, (K + 256) * 4], xd.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s0, bad, d) == Q.Q4K_EINVAL


def test_golden_fixture_on_gpu(Q, O, gpu):
    g = np.load(_common.GOLDEN_DIR + "/q4k_golden.npz")
    for name in sorted({k.split("/")[0] for k in g.files if k.endswith("/wq")}):
        wq, x, K = g[name + "/wq"], g[name + "/x"], int(g[name + "/K"])
        N = x.shape[0]
        ref = {"y64": g[name + "/y64"], "l1": g[name + "/l1"]}
        y = Q.mul_mat_vec_q(to_dev(wq, gpu), K, to_dev(x, gpu)).cpu().numpy()
        _common.assert_within_tolerance(O, y, ref, "golden " + name)
        q8d = Q.quantize_row_q8_1(to_dev(x, gpu))
        assert np.array_equal(q8d.cpu().numpy(), g[name + "/q8"])
        sqq, sq = Q.subblock_sums(to_dev(wq, gpu), K, q8d, N)
        assert np.array_equal(sqq.cpu().numpy(), g[name + "/sqq"])
        assert np.array_equal(sq.cpu().numpy(), g[name + "/sq"])


def test_golden_4096x4096_b1_on_gpu(Q, O, gpu):
    """The 4096x4096 b=1 workload regenerated from its seeds (digests must
    match the fixture) and run on the GPU against the fixture's result."""
    import hashlib
    g = np.load(_common.GOLDEN_DIR + "/q4k_golden.npz")
    W = _common.weights(4096, 4096, 0)
    wq = Q.quantize_rows_q4_K(W, nthreads=16)
    x = _common.activations(1, 4096, 0)
    assert hashlib.sha256(wq.tobytes()).hexdigest() == str(g["cfg_4096x4096_b1/sha256_wq"])
    assert hashlib.sha256(x.tobytes()).hexdigest() == str(g["cfg_4096x4096_b1/sha256_x_f32"])
    ref = {"y64": g["cfg_4096x4096_b1/y64"], "l1": g["cfg_4096x4096_b1/l1"]}
    y = Q.mul_mat_vec_q(to_dev(wq, gpu), 4096, to_dev(x, gpu)).cpu().numpy()
    _common.assert_within_tolerance(O, y, ref, "4096x4096 b=1")


# ---------------------------------------------------- full workloads ----
def _cases():
    out = []
    for wl, items in _common.WORKLOADS.items():
        for M, K, ns in items:
            for N in ns:
                out.append(pytest.param(M, K, N, id=f"{wl}-{M}x{K}-N{N}"))
    # de-duplicate identical shapes across workloads
    seen, uniq = set(), []
    for p in out:
        if p.values not in seen:
            seen.add(p.values)
            uniq.append(p)
    return uniq


@pytest.mark.parametrize("M,K,N", _cases())
def test_workload_parity(Q, O, gpu, M, K, N):
    """Every output of the workload against the (threaded) oracle; the
    count outside the strict bar (1e-5 relative or 4 ulp), all of them rows
    whose terms cancel, is printed."""
    wq, x = inputs(Q, M, K, N)
    q8 = O.quantize_q8_1(x)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    ref = O.gemv_q4K_q8_1(wq, K, q8, want_sums=False)
    st = _common.assert_within_tolerance(O, y, ref, f"{M}x{K} N={N}")
    print(f"[parity] Q4_K {M}x{K} N={N}: {st['n']} outputs, {st['n'] - st['strict_fail']} within 1e-5 rel "
          f"or 4 ulp, {st['strict_fail']} cancelling rows within {st['max_cancel_ulps']:.2f} eps32*sum|term|, "
          f"max err/tol {st['max_ratio']:.3f}", flush=True)
    # the outputs outside the strict bar are rows whose terms cancel; their
    # errors stay within one f32 epsilon of the row's sum of |term|
    # (observed at most 0.27 over every workload)
    assert st["max_cancel_ulps"] <= 1.0, st
    rows = np.arange(M)
    # pre-quantised launch: identical bits
    q8d = Q.quantize_row_q8_1(xd)
    y2 = Q.op_mul_mat_vec_q(wd, K, q8d, N).cpu().numpy()
    assert np.array_equal(y, y2)
    # split-mode row slices reassemble the full result: bit for bit when the
    # slices run the same kernel as the whole product (kernels differ only in
    # summation order), else each slice within tolerance of the oracle
    cut = (M // 3) // 16 * 16 + 5
    top = Q.op_mul_mat_vec_q(wd[:cut], K, q8d, N, row_low=0, row_high=cut).cpu().numpy()
    bot = Q.op_mul_mat_vec_q(wd[cut:], K, q8d, N, row_low=cut, row_high=M).cpu().numpy()
    kern = {tuple(Q.geometry(K, m, N)[f] for f in ("kernel", "cols_per_launch")) for m in (M, cut, M - cut)}
    if len(kern) == 1:
        assert np.array_equal(np.concatenate([top, bot], axis=1), y)
    else:
        both = np.concatenate([top, bot], axis=1)
        _common.assert_within_tolerance(O, both[:, rows], ref, f"split {M}x{K} N={N}")
    assert np.isfinite(y).all()


def _sum_rows(M, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, 1, M // 2, M - 2, M - 1], rng.choice(M, min(M, 250), replace=False)]))


@pytest.mark.parametrize("M,K,N", _cases())
def test_production_kernel_sums(Q, O, gpu, M, K, N):
    """The int32 sub-block sums S_qq and activation sums S_q formed inside
    the kernels the workload actually runs (the SUMS variant of its own
    launch: same route, geometry and kernel, which also stores them), bit
    for bit against the oracle on a row sample; the variant's outputs equal
    the product launch's bit for bit.  Both routes where they differ (with a
    workspace several long columns are quantised in a launch of their own)."""
    import torch
    wq, x = inputs(Q, M, K, N)
    q8 = O.quantize_q8_1(x)
    wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
    ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
    rows = _sum_rows(M, M * 7 + N)
    ref = O.gemv_q4K_q8_1(wq[rows], K, q8)
    geo = Q.geometry(K, M, N)
    for route, w in (("workspace", ws), ("in-launch", None)):
        if w is None and K * N <= 40960:
            continue  # the same route as with the workspace
        y, sums, sq = Q.mul_mat_vec_q_sums(wd, K, xd, workspace=w)
        y_prod = Q.mul_mat_vec_q(wd, K, xd, workspace=w)
        assert torch.equal(y, y_prod), f"{route}: the parity variant's outputs differ from the product's"
        got = sums[:, torch.from_numpy(rows).to(gpu)].cpu().numpy()
        assert np.array_equal(got, ref["sqq"]), f"{route} {M}x{K} N={N} {geo}: S_qq differ"
        assert np.array_equal(sq.cpu().numpy(), ref["sq"]), f"{route} {M}x{K} N={N}: S_q differ"
        del sums
    print(f"[sums] Q4_K {M}x{K} N={N} {geo}: {len(rows)} rows x {K // 32} sub-blocks x {N} exact", flush=True)


def test_parity_variants_cover_every_kernel(Q, gpu):
    """The workloads' launches, whose sums test_production_kernel_sums
    checks, include the K-split kernel (one column: 4096-value rows with the
    activation in registers, 14336- and 28672-value rows in the long-row
    variant; several columns, and the one-column kernel over the columns of
    1024 x 4096 as channels), the matrix-core kernels (128256 x 4096, eight
    columns; 4096 x 14336, eight columns, its A operand read from the Q8_1
    copy), 16-wave tile launches for several columns and both staging
    routes (the 8-wave register path: test_eight_wave_register_path).  (The block-per-lane kernel, no longer
    the automatic choice anywhere, is checked through the override in
    test_kernel_variants_against_oracle; the one-column tile kernel, which
    runs unaligned activations, the pre-quantised route and the epilogues,
    in the tests of those.)"""
    kinds = set()
    for p in _cases():
        M, K, N = p.values
        g = Q.geometry(K, M, N)
        kinds.add((g["kernel"], g["waves_per_wg"] if g["kernel"] == 1 else 0, N >= 3 and K <= 4096))
    assert Q.geometry(4096, 14336, 1)["kernel"] == 5 and Q.geometry(4096, 128256, 1)["kernel"] == 5
    assert Q.geometry(14336, 4096, 1)["kernel"] == 5 and Q.geometry(28672, 8192, 1)["kernel"] == 5
    assert (5, 0, False) in kinds                      # K-split (the headline shape, long rows)
    assert (5, 0, True) in kinds                       # several columns: K-split kernels, or one-column channels
    assert (4, 0, True) in kinds                       # matrix cores (128256 x 4096, eight columns)
    assert (6, 0, False) in kinds                      # matrix cores, A from the Q8_1 copy (4096 x 14336 N=8)
    assert (1, 16, True) in kinds                      # several columns on the tile kernel, 16 waves


@pytest.mark.parametrize("M", [8192, 14336, 20480])
def test_two_group_rows_streamed_prologue(Q, O, gpu, M):
    """Rows of two 4096-value groups with 16 waves and two slots per wave,
    on the tile kernel (forced: the automatic choice for one aligned F32
    column is the K-split kernel; the tile kernel runs this shape for
    unaligned activations and the bias epilogue): with 64 or more rows per
    workgroup (20480 rows) the one-column launch consumes its first steps
    between the quantisation rounds; with fewer it issues one early group.
    Checked against the oracle on a row sample, bit for bit against the
    pre-quantised launch (which stages the whole activation first), against
    the automatic (K-split) launch, and with the bias epilogue (same rows,
    bias added)."""
    import torch
    K = 8192
    Q.set_geometry_override(kernel=1)
    try:
        geo = Q.geometry(K, M, 1)
        assert geo["kernel"] == 1 and geo["waves_per_wg"] == 16 and geo["workgroups"] <= 256, geo
        wq, x = inputs(Q, M, K, 1, seed=9)
        wd, xd = to_dev(wq, gpu), to_dev(x, gpu)
        y = Q.mul_mat_vec_q(wd, K, xd).cpu().numpy()
    finally:
        Q.set_geometry_override()
    assert np.array_equal(Q.mul_mat_vec_q(wd, K, xd).cpu().numpy(), y)
    q8 = O.quantize_q8_1(x)
    rng = np.random.default_rng(M)
    rows = np.unique(np.concatenate([[0, 1, 31, 32, M - 2, M - 1], rng.choice(M, 250, replace=False)]))
    ref = oracle_rows(O, wq, K, q8, rows)
    _common.assert_within_tolerance(O, y[:, rows], ref, f"{M}x{K} streamed")
    y2 = Q.op_mul_mat_vec_q(wd, K, to_dev(q8, gpu), 1).cpu().numpy()
    assert np.array_equal(y, y2)
    b = rng.standard_normal(M).astype(np.float32)
    yb = Q.mul_mat_vec_q_fused(wd, K, xd, x_bias=to_dev(b, gpu)).cpu().numpy()[0]
    assert np.array_equal(yb, y[0] + b)
    # the same rows as two broadcast channels of one batched launch
    x2 = np.concatenate([x, x[:, ::-1].copy()])
    s0 = Q.make_tensor(12, [K, M, 1, 1], [144, wq.shape[1], wq.shape[1] * M, wq.shape[1] * M], wd.data_ptr())
    xd2 = to_dev(x2, gpu)
    s1 = Q.make_tensor(0, [K, 1, 2, 1], [4, 4 * K, 4 * K, 8 * K], xd2.data_ptr())
    dst = torch.empty((2, M), dtype=torch.float32, device=gpu)
    d = Q.make_tensor(0, [M, 1, 2, 1], [4, 4 * M, 4 * M, 8 * M], dst.data_ptr())
    assert Q.ggml_mul_mat_vec_q(s0, s1, d) == Q.Q4K_OK
    out = dst.cpu().numpy()
    assert np.array_equal(out[0], y[0])
    ref2 = oracle_rows(O, wq, K, O.quantize_q8_1(x2[1:2]), rows)
    _common.assert_within_tolerance(O, out[1:2, rows], ref2, f"{M}x{K} channel 1")
