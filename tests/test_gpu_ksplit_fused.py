"""GPU parity of the one-column Q4_K and Q6_K K-split kernels with the fused
epilogue (kernels/mmvq.cu:254-262, :309-336): the bias on the product, or
the gate weight streamed in the same launch, its bias and the GLU of the
pair.

Bar: outputs bit for bit equal to the fused tile kernel's -- both form each
product over the same balanced tree and apply the same epilogue arithmetic
-- in every instantiated launch shape (rows of 4096 and 8192 values, and
other lengths on the long-row form), with one workgroup per CU, 7 and 300
workgroups; the geometry query confirms each launch is the K-split kernel.
The fused tile kernel itself is checked against the oracle in
test_gpu_fused.py.
"""
import numpy as np
import pytest

import _common

pytestmark = pytest.mark.gpu

SHORT = [(8, 8, 1), (8, 8, 2), (8, 16, 1), (4, 4, 1), (4, 4, 2), (4, 8, 1), (4, 8, 2), (4, 16, 1)]
LONG = [(16, 16, 1), (8, 8, 1), (8, 8, 2), (8, 16, 1), (4, 4, 1), (4, 4, 2), (4, 8, 1), (4, 8, 2), (4, 16, 1)]
Q4, Q6 = 12, 14  # ggml type ids

_cache = {}


def weights(Q, M, K, seed, wtype=Q4):
    key = (M, K, seed, wtype)
    if key not in _cache:
        if len(_cache) > 4:
            _cache.clear()
        quant = Q.quantize_rows_q4_K if wtype == Q4 else Q.quantize_rows_q6_K
        _cache[key] = quant(_common.weights(M, K, seed), nthreads=16)
    return _cache[key]


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def team_shapes(K):
    """Rows of 9 to 14 blocks: teams of other sizes than powers of two."""
    nb = K // 256
    if not 9 <= nb <= 14:
        return []
    kt = (nb + 1) // 2
    return [(8, kt, 1), (8, 2 * kt, 1)] + ([(4, 3, 1), (4, 6, 1), (4, 12, 1)] if nb <= 12 else [])


def launch_shapes(K, wtype):
    if wtype == Q6:
        return LONG + team_shapes(K)  # (16 rows per step exists for rows of 4096 and 8192 values too)
    return SHORT if K in (4096, 8192) else LONG + team_shapes(K)


def fused(Q, wd, K, xd, gd, bu, bg, op, wtype=Q4):
    return Q.mul_mat_vec_q_fused(wd, K, xd, gate=gd, x_bias=bu, gate_bias=bg, glu_op=op,
                                 wtype=wtype).cpu().numpy()


@pytest.mark.parametrize("wtype", [Q4, Q6])
@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 4096), (1024, 4096), (37, 4096), (5000, 8192), (258, 8192),
                                 (4096, 14336), (1000, 11008), (300, 5120), (2048, 2048), (1030, 768),
                                 (2560, 2560), (700, 3584)])
def test_ksplit_fused_bits_equal_tile_kernel(Q, gpu, wtype, M, K):
    """Gate + GLU (SWIGLU, GEGLU, SWIGLU_OAI; with and without biases) and
    the bias-only epilogue, every K-split launch shape against the fused
    tile kernel (rows of 768 and 2048 values: teams of only the waves a row
    needs)."""
    wu, wg = weights(Q, M, K, 1, wtype), weights(Q, M, K, 2, wtype)
    x = _common.activations(1, K, seed=3)
    rng = np.random.default_rng([M, K])
    bu = to_dev(rng.standard_normal(M).astype(np.float32) * np.float32(0.1), gpu)
    bg = to_dev(rng.standard_normal(M).astype(np.float32) * np.float32(0.1), gpu)
    wud, wgd, xd = to_dev(wu, gpu), to_dev(wg, gpu), to_dev(x, gpu)
    cases = [("gate", 2, bu, bg), ("gate", 1, None, None), ("gate", 3, bu, None), ("bias", 0, bu, None)]
    for route, op, b1, b2 in cases:
        gd = wgd if route == "gate" else None
        try:
            Q.set_geometry_override(kernel=1)
            assert Q.geometry(K, M, 1, wtype, route=route)["kernel"] == 1
            y_tile = fused(Q, wud, K, xd, gd, b1, b2, op or 2, wtype)
        finally:
            Q.set_geometry_override()
        ran = 0
        for tr, waves, slots in launch_shapes(K, wtype):
            for wgs in (0, 7, 300):
                try:
                    Q.set_geometry_override(rows_per_tile=tr, waves_per_wg=waves, workgroups=wgs, kernel=5)
                    Q.set_pipeline_override(slots=slots)
                    g = Q.geometry(K, M, 1, wtype, route=route)
                    if g["kernel"] != 5:
                        continue  # no fused variant of this shape (its registers would spill)
                    if g["lds_bytes"] > 160 * 1024:
                        continue  # two weights' partials of this many rows per workgroup exceed the LDS
                    rows = g["rows_per_step"] if wtype == Q4 else g["rows_per_tile"]
                    assert rows == tr and g["waves_per_wg"] == waves, g
                    y = fused(Q, wud, K, xd, gd, b1, b2, op or 2, wtype)
                finally:
                    Q.set_geometry_override()
                    Q.set_pipeline_override()
                ran += 1
                if not np.array_equal(y, y_tile):
                    bad = np.flatnonzero(y[0] != y_tile[0])
                    raise AssertionError(f"type {wtype} {M}x{K} {route} op {op} rows/step {tr} waves {waves} "
                                         f"slots {slots} "
                                         f"wgs {wgs}: {bad.size} outputs differ from the tile kernel, e.g. rows "
                                         f"{bad[:5]}")
        assert ran >= 9, f"type {wtype} {M}x{K} {route}: only {ran} K-split launches ran"
        # the automatic choice: the same bits
        assert np.array_equal(fused(Q, wud, K, xd, gd, b1, b2, op or 2, wtype), y_tile)


@pytest.mark.parametrize("M,K", [(14336, 4096), (4096, 4096), (28672, 8192), (4096, 14336), (8192, 2048),
                                 (2048, 768), (9728, 2560)])
def test_ksplit_fused_automatic_choice(Q, gpu, M, K):
    """The fused one-column launches of the workload shapes take the K-split
    kernel automatically (Q4_K and Q6_K), and an unaligned activation the
    tile kernel (same bits)."""
    import torch
    for wtype in (Q4, Q6):
        for route in ("gate", "bias"):
            assert Q.geometry(K, M, 1, wtype, route=route)["kernel"] == 5, (wtype, route)
    if M * K > 4096 * 4096:
        return
    wu, wg = weights(Q, M, K, 1), weights(Q, M, K, 2)
    x = _common.activations(1, K, seed=4)
    wud, wgd = to_dev(wu, gpu), to_dev(wg, gpu)
    xa = to_dev(x, gpu)
    xb = torch.zeros((1, K + 4), dtype=torch.float32, device=gpu)
    xb[:, 1:K + 1] = xa
    y_a = Q.mul_mat_vec_q_fused(wud, K, xa, gate=wgd, glu_op=2).cpu().numpy()
    y_u = Q.mul_mat_vec_q_fused(wud, K, xb[:, 1:K + 1], gate=wgd, glu_op=2).cpu().numpy()
    assert np.array_equal(y_a, y_u)


def _tensor(Q, t, ne, nb, ptr):
    return Q.make_tensor(t, list(ne), list(nb), ptr)


@pytest.mark.parametrize("wtype", [Q4, Q6])
@pytest.mark.parametrize("M,K,fuse", [(14336, 4096, False), (14336, 4096, True), (4096, 14336, False),
                                      (1024, 8192, True), (3000, 11008, True), (768, 2048, True),
                                      (2048, 768, False), (1000, 1536, True), (1000, 2560, True),
                                      (2000, 3584, False)])
def test_ksplit_batched_mul_mat_id_bits_equal_tile_kernel(Q, gpu, wtype, M, K, fuse):
    """MUL_MAT_ID for one token (three experts, slots using two of them, one
    twice, and an absent id), with and without the gate weight and SWIGLU:
    the automatic launch (the batched K-split kernels; rows of 768 .. 2048
    values in short teams) and a forced 8-row, 8-wave K-split launch
    against the batched tile kernel, bit for bit; the absent expert's slot
    reads no weight."""
    import ctypes
    import torch
    BB = {Q4: 144, Q6: 210}
    nexp = 3
    ids = np.array([2, 0, 2, 7], np.int32)
    nused = len(ids)
    wu = np.stack([weights(Q, M, K, 60 + e, wtype) for e in range(nexp)])
    wg = np.stack([weights(Q, M, K, 70 + e, wtype) for e in range(nexp)]) if fuse else None
    x = _common.activations(1, K, seed=61)
    wud, xd, idd = to_dev(wu, gpu), to_dev(x, gpu), to_dev(ids, gpu)
    wgd = to_dev(wg, gpu) if fuse else None
    rb = wu.shape[-1]
    s0 = _tensor(Q, wtype, (K, M, nexp), (BB[wtype], rb, rb * M), wud.data_ptr())
    s1 = _tensor(Q, 0, (K, 1, 1), (4, 4 * K, 4 * K), xd.data_ptr())
    ti = _tensor(Q, 26, (nused, 1), (4, 4 * nused), idd.data_ptr())
    fa = None
    if fuse:
        sg = _tensor(Q, wtype, (K, M, nexp), (BB[wtype], rb, rb * M), wgd.data_ptr())
        fa = Q.q4k_fusion_args(None, ctypes.pointer(sg), None, Q.GLU_OP_SWIGLU)

    def run(**ovr):
        dst = torch.full((nused, M), 7.0, dtype=torch.float32, device=gpu)
        d = _tensor(Q, 0, (M, nused, 1), (4, 4 * M, 4 * M * nused), dst.data_ptr())
        try:
            Q.set_geometry_override(**ovr)
            assert Q.ggml_mul_mat_vec_q(s0, s1, d, ids=ti, fusion=fa) == Q.Q4K_OK
        finally:
            Q.set_geometry_override()
        return dst.cpu().numpy()

    y_tile = run(kernel=1)
    assert np.array_equal(y_tile[0], y_tile[2])
    expect_absent = 0.0  # no weight bytes: zero products (SWIGLU of 0 and 0 is 0)
    assert (y_tile[3] == expect_absent).all()
    for ovr in ({}, {"rows_per_tile": 8, "waves_per_wg": 8, "kernel": 5}):
        y = run(**ovr)
        if not np.array_equal(y, y_tile):
            bad = np.argwhere(y != y_tile)
            raise AssertionError(f"type {wtype} {M}x{K} fuse {fuse} {ovr}: {len(bad)} outputs differ from the "
                                 f"tile kernel, e.g. (slot, row) {bad[:5].tolist()}")
