"""The allocation-free entry point q4k_mul_mat_vec_q_noalloc (through the C
ABI) against q4k_mul_mat_vec_q with a caller workspace, bit for bit, on calls
in a row, each smaller than the one before, so that the scratch still holds
the previous call's Q8_1 bytes.  The shapes take the routes that use the
scratch (a quantisation launch of its own for several long columns; column
chunks when the activation does not fit the LDS) and one that does not
(quantisation inside the GEMV launch).  A request beyond the scratch is
refused with Q4K_ESCRATCH before anything is launched.  Captured into a HIP
graph, a scratch-using call records kernel nodes only (no allocation)."""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

# (M, K, N), largest first: column chunks (28672 x 8 values do not fit the
# LDS), the quantisation launch (28672 x 4 > 40960 values), then in-launch;
# 3400 rows, more per CU than the columns-as-channels launch takes (it
# quantises each column inside its own launch)
CALLS = [(3400, 28672, 8), (3400, 28672, 4), (64, 4096, 2)]


def _noalloc(Q, wd, M, K, xd, N, dst):
    return Q.lib().q4k_mul_mat_vec_q_noalloc(Q._ptr(wd), K, M, K // 256 * 144, Q._ptr(xd), N, K * 4,
                                            Q._ptr(dst), M * 4, Q._stream())


def test_noalloc_equals_workspace_route(Q, O, gpu):
    import torch
    for M, K, N in CALLS:
        print(f"[noalloc] {M}x{K} N={N}", flush=True)
        wq = Q.quantize_rows_q4_K(_common.weights(M, K, seed=M), nthreads=16)
        x = _common.activations(N, K, seed=K)
        wd = torch.from_numpy(wq).to(gpu)
        xd = torch.from_numpy(x).to(gpu)
        ws = torch.empty(Q.q8_1_bytes(K, N), dtype=torch.uint8, device=gpu)
        ref = Q.mul_mat_vec_q(wd, K, xd, workspace=ws)
        dst = torch.full((N, M), -7.0, dtype=torch.float32, device=gpu)
        assert _noalloc(Q, wd, M, K, xd, N, dst) == Q.Q4K_OK
        torch.cuda.synchronize()
        got = dst.cpu().numpy()
        assert np.array_equal(got, ref.cpu().numpy()), f"{M}x{K} N={N}"
        # and the oracle's bar, on a row sample
        rows = np.arange(0, M, 7)
        oref = O.gemv_q4K_q8_1(wq[rows], K, O.quantize_q8_1(x), want_sums=False)
        _common.assert_within_tolerance(O, got[:, rows], oref, f"noalloc {M}x{K} N={N}")


def test_noalloc_refuses_requests_beyond_the_scratch(Q, gpu):
    import torch
    M, K, N = 2, 131072, 8   # 8 x 4096 Q8_1 blocks = 1,179,648 bytes > 1 MiB
    assert Q.q8_1_bytes(K, N) > Q.NOALLOC_SCRATCH_BYTES
    wq = Q.quantize_rows_q4_K(_common.weights(M, K, seed=5), nthreads=16)
    wd = torch.from_numpy(wq).to(gpu)
    xd = torch.from_numpy(_common.activations(N, K, seed=5)).to(gpu)
    dst = torch.full((N, M), -7.0, dtype=torch.float32, device=gpu)
    assert _noalloc(Q, wd, M, K, xd, N, dst) == Q.Q4K_ESCRATCH
    torch.cuda.synchronize()
    assert (dst.cpu().numpy() == -7.0).all()
    # two columns of 65536 values (589,824 Q8_1 bytes, beyond the LDS) fit and
    # equal the allocating route (a stream-ordered temporary)
    K2, N2 = 65536, 2
    wq2 = Q.quantize_rows_q4_K(_common.weights(M, K2, seed=6), nthreads=16)
    wd2 = torch.from_numpy(wq2).to(gpu)
    xd2 = torch.from_numpy(_common.activations(N2, K2, seed=6)).to(gpu)
    dst2 = torch.full((N2, M), -7.0, dtype=torch.float32, device=gpu)
    assert _noalloc(Q, wd2, M, K2, xd2, N2, dst2) == Q.Q4K_OK
    torch.cuda.synchronize()
    assert np.array_equal(dst2.cpu().numpy(), Q.mul_mat_vec_q(wd2, K2, xd2).cpu().numpy())


def test_noalloc_graph_capture_has_kernel_nodes_only(Q, gpu):
    """A scratch-using call (eight columns of 28672 values over 3400 rows,
    more rows per CU than the columns-as-channels launch takes: column
    chunks on a Q8_1 copy in the scratch) captured into a HIP graph on a
    stream of its own holds kernel nodes only -- no memory-allocation, free
    or memset node -- and its replays, with eager work between them, equal
    the eager call bit for bit."""
    import ctypes
    import torch
    hip = ctypes.CDLL("libamdhip64.so")
    M, K, N = 3400, 28672, 8
    wq = Q.quantize_rows_q4_K(_common.weights(M, K, seed=M + 1), nthreads=16)
    wd = torch.from_numpy(wq).to(gpu)
    xd = torch.from_numpy(_common.activations(N, K, seed=K + 1)).to(gpu)
    ref = torch.full((N, M), -7.0, dtype=torch.float32, device=gpu)
    assert _noalloc(Q, wd, M, K, xd, N, ref) == Q.Q4K_OK  # eager first: resolves the device's scratch
    torch.cuda.synchronize()
    dst = torch.full((N, M), -7.0, dtype=torch.float32, device=gpu)
    stream = torch.cuda.Stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    graph, exe = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipStreamBeginCapture(sp, 1) == 0  # thread-local capture mode
    st = Q.lib().q4k_mul_mat_vec_q_noalloc(Q._ptr(wd), K, M, K // 256 * 144, Q._ptr(xd), N, K * 4, Q._ptr(dst),
                                           M * 4, sp)
    assert hip.hipStreamEndCapture(sp, ctypes.byref(graph)) == 0
    assert st == Q.Q4K_OK
    try:
        n = ctypes.c_size_t(0)
        assert hip.hipGraphGetNodes(graph, None, ctypes.byref(n)) == 0 and n.value >= 2
        nodes = (ctypes.c_void_p * n.value)()
        assert hip.hipGraphGetNodes(graph, nodes, ctypes.byref(n)) == 0
        types = []
        for nd in nodes:
            t = ctypes.c_int(-1)
            assert hip.hipGraphNodeGetType(ctypes.c_void_p(nd), ctypes.byref(t)) == 0
            types.append(t.value)
        assert all(t == 0 for t in types), f"node types {types} (0 = kernel; 10/11 = alloc/free, 2 = memset)"
        assert hip.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0) == 0
        want = ref.cpu().numpy()
        for i in range(3):
            dst.fill_(-7.0)
            torch.cuda.synchronize()
            assert hip.hipGraphLaunch(exe, sp) == 0
            stream.synchronize()
            assert np.array_equal(dst.cpu().numpy(), want), f"replay {i}"
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        hip.hipGraphDestroy(graph)
