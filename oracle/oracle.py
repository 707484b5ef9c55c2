"""numpy bindings of the CPU oracle (oracle/q4k_oracle.c, oracle/q6k_oracle.c).

TEST INFRASTRUCTURE ONLY: the oracle the tests compare the HIP product path
against, and the CPU baseline the benchmark times beside it.  Only tests/, the smoke entry point and
the benchmark's CPU-baseline leg may import this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq4k_oracle.so")

QK_K = 256
QK8_1 = 32
Q4K_BYTES = 144
Q6K_BYTES = 210
Q81_BYTES = 36
Q8K_BYTES = 292
MATRIX_ROW_PADDING = 512  # kernels/mmvq.cu:728 pads K to this for the Q8_1 temp

_lib = None


def build(force: bool = False) -> str:
    """Compiles the oracle with its Makefile (gcc); returns the library path."""
    if force or not os.path.exists(LIB_PATH):
        subprocess.run(["make", "-s", "-C", HERE, "-B" if force else "all"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        I = ctypes.c_int
        sig = {
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16_array": (None, [P, P, I64]),
            "orc_f16_to_f32_array": (None, [P, P, I64]),
            "orc_nearest_int": (I, [ctypes.c_float]),
            "orc_nearest_int_array": (None, [P, P, I64]),
            "orc_scale_min_k4": (None, [I, P, P, P]),
            "orc_vecdot_scale_pair": (None, [I, P, P]),
            "orc_pack_scales_k4": (None, [P, P, P]),
            "orc_selftest_scale_unpack": (I64, []),
            "orc_selftest_scale_pack": (I64, []),
            "orc_check_div127": (I64, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32]),
            "orc_quantize_q4_K": (None, [P, P, I64]),
            "orc_q4K_fit_block": (None, [P, ctypes.c_float, ctypes.c_float, I, I, P, P, P]),
            "orc_q6K_fit_block": (None, [P, ctypes.c_float, I, I, P, P]),
            "orc_quantize_q4_K_rows": (None, [P, P, I64, I64, I]),
            "orc_dequantize_q4_K": (None, [P, P, I64]),
            "orc_quantize_q8_1": (None, [P, I64, I64, P]),
            "orc_quantize_q8_1_cols": (None, [P, I64, I64, I64, I64, P]),
            "orc_gemv_q4K_q8_1": (None, [P, I64, I64, I64, P, I64, I64, P, P, P, P]),
            "orc_gemv_q4K_q8_1_mt": (None, [P, I64, I64, I64, P, I64, I64, P, P, P, P, I]),
            "orc_gemv_q6K_q8_1_mt": (I64, [P, I64, I64, I64, P, I64, I64, P, P, P, I]),
            "orc_quantize_q8_K": (None, [P, P, I64]),
            "orc_vec_dot_q4_K_q8_K_scalar": (ctypes.c_float, [I64, P, P]),
            "orc_vec_dot_q4_K_q8_K_avx2": (ctypes.c_float, [I64, P, P]),
            "orc_vec_dot_q6_K_q8_K_scalar": (ctypes.c_float, [I64, P, P]),
            "orc_vec_dot_q6_K_q8_K_avx2": (ctypes.c_float, [I64, P, P]),
            "orc_cpu_has_avx2": (I, []),
            "orc_cpu_mul_mat_q4_K": (I, [P, I64, I64, I64, P, I64, I64, P, P, I64, I, I, I]),
            "orc_cpu_mul_mat_q6_K": (I, [P, I64, I64, I64, P, I64, I64, P, P, I64, I, I, I]),
            "orc_time_cpu_mul_mat_q4_K": (None, [P, I64, I64, I64, P, I64, I64, P, P, I64, I, I, I, I, P]),
            "orc_time_cpu_mul_mat_q6_K": (None, [P, I64, I64, I64, P, I64, I64, P, P, I64, I, I, I, I, P]),
            "orc_set_pin_cpus": (None, [P, I]),
            "orc_quantize_q6_K": (None, [P, P, I64]),
            "orc_dequantize_q6_K": (None, [P, P, I64]),
            "orc_gemv_q6K_q8_1": (I64, [P, I64, I64, I64, P, I64, I64, P, P, P]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def pad_k(K: int) -> int:
    return (K + MATRIX_ROW_PADDING - 1) // MATRIX_ROW_PADDING * MATRIX_ROW_PADDING


# ---------------------------------------------------------------- fp16 ----
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_array(_p(x), _p(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_f16_to_f32_array(_p(h), _p(out), h.size)
    return out


def nearest_int(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.int32)
    lib().orc_nearest_int_array(_p(x), _p(out), x.size)
    return out


# ------------------------------------------------------------ quantisers ----
def quantize_q4_K(w: np.ndarray, nthreads: int = 1) -> np.ndarray:
    """F32 [M, K] -> Q4_K bytes [M, K/256*144] (quantize_row_q4_K_ref per row)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, K = w.shape
    assert K % QK_K == 0
    out = np.empty((M, K // QK_K * Q4K_BYTES), dtype=np.uint8)
    lib().orc_quantize_q4_K_rows(_p(w), _p(out), M, K, nthreads)
    return out


def q4K_fit(w: np.ndarray, rmin: float = -1.0, rdelta: float = 0.1, nstep: int = 20, weight_mode: int = 0):
    """Stage 1 of quantize_row_q4_K_ref on every 256-value block of w (F32,
    size a multiple of 256): the make_qkx2_quants fit of each 32-value
    sub-block.  Returns (scales [nblk, 8], mins [nblk, 8] (= -min of the fit),
    L [nblk, 256] levels 0..15).  The defaults are ggml's parameters;
    weight_mode 1 (x^2 weights) and other rmin/rdelta/nstep values are
    planted mistakes for the tests."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1, QK_K)
    n = w.shape[0]
    sc = np.empty((n, 8), np.float32)
    mn = np.empty((n, 8), np.float32)
    L = np.empty((n, QK_K), np.uint8)
    for b in range(n):
        lib().orc_q4K_fit_block(_p(w[b]), rmin, rdelta, nstep, weight_mode, _p(sc[b]), _p(mn[b]), _p(L[b]))
    return sc, mn, L


def q6K_fit(w: np.ndarray, rdelta: float = 0.1, nstep: int = 9, weight_mode: int = 0):
    """Stage 1 of quantize_row_q6_K_ref on every 256-value block of w: the
    make_qx_quants fit (nmax 32) of each 16-value group.  Returns (scales
    [nblk, 16], L [nblk, 256] as l + 32).  Defaults are ggml's parameters;
    weight_mode 1 (|x| weights) is a planted mistake for the tests."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1, QK_K)
    n = w.shape[0]
    sc = np.empty((n, 16), np.float32)
    L = np.empty((n, QK_K), np.int8)
    for b in range(n):
        lib().orc_q6K_fit_block(_p(w[b]), rdelta, nstep, weight_mode, _p(sc[b]), _p(L[b]))
    return sc, L


def dequantize_q4_K(q: np.ndarray, K: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    M = q.size // (K // QK_K * Q4K_BYTES)
    out = np.empty((M, K), dtype=np.float32)
    for r in range(M):
        lib().orc_dequantize_q4_K(_p(q[r]), _p(out[r]), K)
    return out


def quantize_q6_K(w: np.ndarray) -> np.ndarray:
    """F32 [M, K] -> Q6_K bytes [M, K/256*210] (quantize_row_q6_K_ref per row)."""
    w = np.ascontiguousarray(np.atleast_2d(w), dtype=np.float32)
    M, K = w.shape
    assert K % QK_K == 0
    out = np.empty((M, K // QK_K * Q6K_BYTES), dtype=np.uint8)
    for r in range(M):
        lib().orc_quantize_q6_K(_p(w[r]), _p(out[r]), K)
    return out


def dequantize_q6_K(q: np.ndarray, K: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    M = q.size // (K // QK_K * Q6K_BYTES)
    q = q.reshape(M, -1)
    out = np.empty((M, K), dtype=np.float32)
    for r in range(M):
        lib().orc_dequantize_q6_K(_p(q[r]), _p(out[r]), K)
    return out


def quantize_q8_1(x: np.ndarray, k_padded: int | None = None) -> np.ndarray:
    """F32 [N, K] -> Q8_1 bytes [N, K_pad/32*36] with ggml-cuda semantics."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    N, K = x.shape
    kp = pad_k(K) if k_padded is None else k_padded
    out = np.empty((N, kp // QK8_1 * Q81_BYTES), dtype=np.uint8)
    lib().orc_quantize_q8_1_cols(_p(x), K, K, N, kp, _p(out))
    return out


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    N, K = x.shape
    out = np.empty((N, K // QK_K * Q8K_BYTES), dtype=np.uint8)
    for c in range(N):
        lib().orc_quantize_q8_K(_p(x[c]), _p(out[c]), K)
    return out


# ------------------------------------------------------------------ GEMV ----
def _threads(nthreads):
    if nthreads is not None:
        return max(1, int(nthreads))
    return max(1, min(16, len(os.sched_getaffinity(0))))


def gemv_q4K_q8_1(w_q: np.ndarray, K: int, q8: np.ndarray, want_sums: bool = True, nthreads: int | None = None):
    """Q4_K [M, K/256*144] x Q8_1 [N, Kp/32*36] -> dict(y64 [N,M], l1 [N,M],
    sqq [N,M,K/32] int32, sq [N,K/32] int32); rows split over nthreads
    threads (default: the usable cores, at most 16)."""
    w_q = np.ascontiguousarray(w_q, dtype=np.uint8)
    q8 = np.ascontiguousarray(np.atleast_2d(q8), dtype=np.uint8)
    row_bytes = K // QK_K * Q4K_BYTES
    M = w_q.size // row_bytes
    N = q8.shape[0]
    stride_col_y = q8.shape[1] // Q81_BYTES
    y64 = np.empty((N, M), dtype=np.float64)
    l1 = np.empty((N, M), dtype=np.float64)
    sqq = np.empty((N, M, K // 32), dtype=np.int32) if want_sums else None
    sq = np.empty((N, K // 32), dtype=np.int32) if want_sums else None
    lib().orc_gemv_q4K_q8_1_mt(_p(w_q), M, K, row_bytes, _p(q8), N, stride_col_y, _p(y64), _p(l1),
                               _p(sqq) if want_sums else None, _p(sq) if want_sums else None, _threads(nthreads))
    return {"y64": y64, "l1": l1, "sqq": sqq, "sq": sq}


def gemv_q6K_q8_1(w_q: np.ndarray, K: int, q8: np.ndarray, want_sums: bool = True, nthreads: int | None = None):
    """Q6_K [M, K/256*210] x Q8_1 [N, Kp/32*36] -> dict(y64 [N,M], l1 [N,M],
    s16 [N,M,K/16] int32 sums of (q - 32) * q8 per 16-weight group,
    mismatches: scale-index / group-index disagreements (0 expected))."""
    w_q = np.ascontiguousarray(w_q, dtype=np.uint8)
    q8 = np.ascontiguousarray(np.atleast_2d(q8), dtype=np.uint8)
    row_bytes = K // QK_K * Q6K_BYTES
    M = w_q.size // row_bytes
    N = q8.shape[0]
    stride_col_y = q8.shape[1] // Q81_BYTES
    y64 = np.empty((N, M), dtype=np.float64)
    l1 = np.empty((N, M), dtype=np.float64)
    s16 = np.empty((N, M, K // 16), dtype=np.int32) if want_sums else None
    mism = lib().orc_gemv_q6K_q8_1_mt(_p(w_q), M, K, row_bytes, _p(q8), N, stride_col_y, _p(y64), _p(l1),
                                      _p(s16) if want_sums else None, _threads(nthreads))
    return {"y64": y64, "l1": l1, "s16": s16, "mismatches": int(mism)}


def vec_dot_q4_K_q8_K(w_row: np.ndarray, y_row: np.ndarray, K: int, isa: str = "avx2") -> float:
    f = lib().orc_vec_dot_q4_K_q8_K_avx2 if isa == "avx2" else lib().orc_vec_dot_q4_K_q8_K_scalar
    return float(f(K, _p(np.ascontiguousarray(w_row)), _p(np.ascontiguousarray(y_row))))


def vec_dot_q6_K_q8_K(w_row: np.ndarray, y_row: np.ndarray, K: int, isa: str = "avx2") -> float:
    f = lib().orc_vec_dot_q6_K_q8_K_avx2 if isa == "avx2" else lib().orc_vec_dot_q6_K_q8_K_scalar
    return float(f(K, _p(np.ascontiguousarray(w_row)), _p(np.ascontiguousarray(y_row))))


_CPU_TYPES = {"q4_K": ("orc_cpu_mul_mat_q4_K", "orc_time_cpu_mul_mat_q4_K", Q4K_BYTES),
              "q6_K": ("orc_cpu_mul_mat_q6_K", "orc_time_cpu_mul_mat_q6_K", Q6K_BYTES)}


def cpu_mul_mat_q4_K(w_q: np.ndarray, K: int, x: np.ndarray, nthreads: int = 1, isa: str = "avx2",
                     wtype: str = "q4_K"):
    """ggml CPU path: x [N, K] f32 -> Q8_K, then vec_dot per (row, column)
    (vec_dot_q4_K_q8_K, or vec_dot_q6_K_q8_K for wtype "q6_K");
    returns (dst [N, M] float32, isa_used)."""
    fn, _, bb = _CPU_TYPES[wtype]
    w_q = np.ascontiguousarray(w_q, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    N = x.shape[0]
    row_bytes = K // QK_K * bb
    M = w_q.size // row_bytes
    yq = np.empty((N, K // QK_K * Q8K_BYTES), dtype=np.uint8)
    dst = np.empty((N, M), dtype=np.float32)
    used = getattr(lib(), fn)(_p(w_q), M, K, row_bytes, _p(x), N, K, _p(yq), _p(dst), M,
                              nthreads, 1 if isa == "avx2" else 0, 1)
    return dst, ("avx2" if used else "scalar")


def set_pin_cpus(cpus):
    """Pins the threads of the CPU path: thread t runs on cpus[t % len]
    (an empty list: no pinning)."""
    a = np.ascontiguousarray(np.asarray(list(cpus), dtype=np.int32))
    lib().orc_set_pin_cpus(_p(a) if a.size else None, int(a.size))


def time_cpu_mul_mat_q4_K(w_q: np.ndarray, K: int, x: np.ndarray, nthreads: int, reps: int,
                          isa: str = "avx2", quantize: bool = True, wtype: str = "q4_K") -> np.ndarray:
    """Wall time (s) of each of `reps` calls of the threaded CPU path (Q4_K
    weights, or Q6_K for wtype "q6_K")."""
    _, fn, bb = _CPU_TYPES[wtype]
    w_q = np.ascontiguousarray(w_q, dtype=np.uint8)
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    N = x.shape[0]
    row_bytes = K // QK_K * bb
    M = w_q.size // row_bytes
    yq = quantize_q8_K(x)
    dst = np.empty((N, M), dtype=np.float32)
    t = np.empty(reps, dtype=np.float64)
    getattr(lib(), fn)(_p(w_q), M, K, row_bytes, _p(x), N, K, _p(yq), _p(dst), M,
                       nthreads, 1 if isa == "avx2" else 0, 1 if quantize else 0, reps, _p(t))
    return t


# -------------------------------------------------------------- tolerance ----
def parity_tolerance(y64: np.ndarray, l1: np.ndarray) -> np.ndarray:
    """Per-output F32 tolerance against the f64 result: 1e-5 relative, or 4 ulp
    of the result, or, where the row's terms cancel, 8 f32 epsilons of the sum
    of |term| over its per-sub-block terms (the scale of a reordered f32 sum)."""
    ulp = np.spacing(np.abs(y64).astype(np.float32)).astype(np.float64)
    return np.maximum(np.maximum(1e-5 * np.abs(y64), 4.0 * ulp), 8.0 * np.finfo(np.float32).eps * l1)


# ------------------------------------------------------ fused epilogue ----
GLU_GEGLU, GLU_SWIGLU, GLU_SWIGLU_OAI = 1, 2, 3  # ggml_glu_op values


def glu(op: int, up, g):
    """The epilogue of kernels/mmvq.cu:316-333 in f64: SWIGLU up*silu(g),
    GEGLU up*gelu(g) (tanh form, ggml's constants 0.044715 and sqrt(2/pi)),
    SWIGLU_OAI silu_1.702(min(g, 7)) * (1 + clamp(up, -7, 7)); other ops up*g."""
    up = np.asarray(up, np.float64)
    g = np.asarray(g, np.float64)
    if op == GLU_SWIGLU:
        return up * (g / (1.0 + np.exp(-g)))
    if op == GLU_GEGLU:
        return up * (0.5 * g * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * g * (1.0 + 0.044715 * g * g))))
    if op == GLU_SWIGLU_OAI:
        x = np.minimum(g, 7.0)
        u = np.clip(up, -7.0, 7.0)
        return x / (1.0 + np.exp(-1.702 * x)) * (1.0 + u)
    return up * g


def glu_tolerance(op: int, up, g, tol_up, tol_g):
    """Bound on the F32 fused result against glu(up, g) in f64 when the two
    products carry errors up to tol_up and tol_g: twice the largest change of
    glu over the corners of that box, plus 16 f32 epsilons of the epilogue's
    own magnitude (device expf/tanhf and the float operations, including the
    cancellation in 1 + tanh and 1 + up)."""
    f0 = glu(op, up, g)
    dev = np.zeros_like(f0)
    for su in (-1.0, 1.0):
        for sg in (-1.0, 1.0):
            dev = np.maximum(dev, np.abs(glu(op, up + su * tol_up, g + sg * tol_g) - f0))
    up = np.asarray(up, np.float64)
    g = np.asarray(g, np.float64)
    if op == GLU_GEGLU:
        scale = np.abs(up * g)
    elif op == GLU_SWIGLU_OAI:
        x = np.minimum(g, 7.0)
        scale = np.abs(x / (1.0 + np.exp(-1.702 * x))) * (1.0 + np.abs(np.clip(up, -7.0, 7.0)))
    else:
        scale = np.abs(f0)
    return 2.0 * dev + 16.0 * np.finfo(np.float32).eps * scale + 1e-30
