"""Python binding of libq4k_gemv.so (the C ABI in include/q4k_gemv.h).

The product is the C ABI; this module is plumbing for tests and the
benchmark: it passes torch device tensors and torch's current HIP stream to
the library and turns status codes into exceptions.  It never computes on the
CPU: if the library is missing, loading it raises.

torch is imported before the library is loaded so that the library binds to
the HIP runtime torch already loaded (one runtime per process).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libq4k_gemv.so")

Q4K_OK, Q4K_EUNSUPPORTED, Q4K_EINVAL, Q4K_EHIP, Q4K_ENOMEM, Q4K_EIO, Q4K_EFORMAT, Q4K_ESCRATCH = 0, 1, 2, 3, 4, 5, 6, 7
NOALLOC_SCRATCH_BYTES = 1 << 20
GGML_TYPE_F32, GGML_TYPE_Q8_1, GGML_TYPE_Q4_K, GGML_TYPE_Q6_K = 0, 9, 12, 14
QK_K = 256
BLOCK_Q4_K_BYTES = 144
BLOCK_Q6_K_BYTES = 210
BLOCK_Q8_1_BYTES = 36
MATRIX_ROW_PADDING = 512

class q4k_gguf_tensor_info(ctypes.Structure):
    """A GGUF tensor directory entry (include/q4k_gguf.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("type", ctypes.c_int32), ("n_dims", ctypes.c_int32),
                ("ne", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]


# Every symbol include/q4k_gemv.h and include/q4k_gguf.h declare: (restype, argtypes)
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
SIGNATURES = {
    "q4k_version": (ctypes.c_int32, []),
    "q4k_strerror": (ctypes.c_char_p, [_I]),
    "q4k_last_hip_error": (ctypes.c_int32, []),
    "q4k_q8_1_bytes": (ctypes.c_size_t, [_I64, _I64]),
    "q4k_quantize_row_q8_1": (_I, [_P, _P, _I64, _I64, _I64, _I64, _P]),
    "q4k_mul_mat_vec_q": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, ctypes.c_size_t, _P]),
    "q4k_mul_mat_vec_q_noalloc": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "q4k_mul_mat_vec_q_sums": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, ctypes.c_size_t,
                                    _P, _P, _P]),
    "q6k_mul_mat_vec_q_sums": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, ctypes.c_size_t,
                                    _P, _P]),
    "q4k_op_mul_mat_vec_q": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "q4k_ggml_mul_mat_vec_q": (_I, [_P, _P, _P, _P, _P, _P, ctypes.c_size_t, _P]),
    "q4k_subblock_sums": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _P, _P]),
    "q4k_gemv_geometry": (_I, [_I64, _I64, _I64, _P]),
    "q4k_gemv_geometry_q8_1": (_I, [_I64, _I64, _I64, _P]),
    "q4k_gemv_geometry_fused": (_I, [_I64, _I64, ctypes.c_int32, _P]),
    "q6k_gemv_geometry_fused": (_I, [_I64, _I64, ctypes.c_int32, _P]),
    "q4k_set_geometry_override": (_I, [ctypes.c_int32] * 4),
    "q4k_set_pipeline_override": (_I, [ctypes.c_int32] * 2),
    "q4k_read_probe": (_I, [_P, ctypes.c_size_t, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                            _P, _P]),
    "q4k_mul_mat_vec_q_fused": (_I, [ctypes.c_int32, _P, _I64, _I64, _I64, _P, _P, _P, _P]),
    "q4k_quantize_rows_q4_K": (_I, [_P, _P, _I64, _I64, _I]),
    "q6k_mul_mat_vec_q": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, ctypes.c_size_t, _P]),
    "q6k_op_mul_mat_vec_q": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _I64, _P]),
    "q6k_group_sums": (_I, [_P, _I64, _I64, _I64, _P, _I64, _I64, _P, _P]),
    "q6k_gemv_geometry": (_I, [_I64, _I64, _I64, _P]),
    "q6k_gemv_geometry_q8_1": (_I, [_I64, _I64, _I64, _P]),
    "q4k_quantize_rows_q6_K": (_I, [_P, _P, _I64, _I64, _I]),
    # include/q4k_gguf.h
    "q4k_gguf_open": (_I, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "q4k_gguf_close": (None, [_P]),
    "q4k_gguf_version": (ctypes.c_uint32, [_P]),
    "q4k_gguf_alignment": (ctypes.c_uint64, [_P]),
    "q4k_gguf_data_offset": (ctypes.c_uint64, [_P]),
    "q4k_gguf_tensor_count": (_I64, [_P]),
    "q4k_gguf_find_tensor": (_I64, [_P, ctypes.c_char_p]),
    "q4k_gguf_get_tensor": (_I, [_P, _I64, ctypes.POINTER(q4k_gguf_tensor_info)]),
    "q4k_ggml_row_size": (ctypes.c_uint64, [ctypes.c_int32, _I64]),
    "q4k_gguf_kv_count": (_I64, [_P]),
    "q4k_gguf_find_key": (_I64, [_P, ctypes.c_char_p]),
    "q4k_gguf_key": (ctypes.c_char_p, [_P, _I64]),
    "q4k_gguf_kv_type": (ctypes.c_int32, [_P, _I64]),
    "q4k_gguf_get_int": (_I, [_P, _I64, ctypes.POINTER(_I64)]),
    "q4k_gguf_get_float": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_double)]),
    "q4k_gguf_get_str": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_char_p)]),
    "q4k_gguf_get_arr": (_I, [_P, _I64, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(_I64),
                              ctypes.POINTER(_P)]),
    "q4k_gguf_get_arr_str": (_I, [_P, _I64, _I64, ctypes.POINTER(ctypes.c_char_p)]),
}


class q4k_tensor(ctypes.Structure):
    """The ggml_tensor subset of include/q4k_gemv.h."""
    _fields_ = [("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                ("data", ctypes.c_void_p)]


class q4k_fusion(ctypes.Structure):
    """Fused epilogue, device pointers (include/q4k_gemv.h)."""
    _fields_ = [("x_bias", ctypes.c_void_p), ("gate", ctypes.c_void_p), ("gate_bias", ctypes.c_void_p),
                ("glu_op", ctypes.c_int32)]


class q4k_fusion_args(ctypes.Structure):
    """Fused epilogue, tensor descriptors (ggml_cuda_mm_fusion_args_host)."""
    _fields_ = [("x_bias", ctypes.POINTER(q4k_tensor)), ("gate", ctypes.POINTER(q4k_tensor)),
                ("gate_bias", ctypes.POINTER(q4k_tensor)), ("glu_op", ctypes.c_int32)]


GLU_OP_GEGLU, GLU_OP_SWIGLU, GLU_OP_SWIGLU_OAI = 1, 2, 3


class Q4KError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        msg = f"{where}: {lib().q4k_strerror(status).decode()} (status {status}"
        if status == Q4K_EHIP:
            msg += f", hipError {lib().q4k_last_hip_error()}"
        super().__init__(msg + ")")


_lib = None


def lib():
    """Loads libq4k_gemv.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        import torch  # noqa: F401  -- bind to torch's HIP runtime
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with gemv-q4_k-optimization_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _check(status: int, where: str):
    if status != Q4K_OK:
        raise Q4KError(status, where)


def _stream(stream=None):
    """torch's current HIP stream (or `stream`); the null stream when no GPU
    is visible, where only the host-side argument checks can run."""
    import torch
    if stream is None:
        if not torch.cuda.is_available():
            return None
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def pad_k(K: int) -> int:
    return (K + MATRIX_ROW_PADDING - 1) // MATRIX_ROW_PADDING * MATRIX_ROW_PADDING


def q8_1_bytes(K: int, ncols: int) -> int:
    return int(lib().q4k_q8_1_bytes(K, ncols))


# ------------------------------------------------------------------ host ----
def quantize_rows_q4_K(w: np.ndarray, nthreads: int = 8) -> np.ndarray:
    """Host F32 [M, K] -> Q4_K bytes [M, K/256*144]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, K = w.shape
    out = np.empty((M, K // QK_K * BLOCK_Q4_K_BYTES), dtype=np.uint8)
    _check(lib().q4k_quantize_rows_q4_K(w.ctypes.data_as(_P), out.ctypes.data_as(_P), M, K, nthreads),
           "q4k_quantize_rows_q4_K")
    return out


def quantize_rows_q6_K(w: np.ndarray, nthreads: int = 8) -> np.ndarray:
    """Host F32 [M, K] -> Q6_K bytes [M, K/256*210]."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, K = w.shape
    out = np.empty((M, K // QK_K * BLOCK_Q6_K_BYTES), dtype=np.uint8)
    _check(lib().q4k_quantize_rows_q6_K(w.ctypes.data_as(_P), out.ctypes.data_as(_P), M, K, nthreads),
           "q4k_quantize_rows_q6_K")
    return out


# ---------------------------------------------------------------- device ----
def quantize_row_q8_1(x, K: int | None = None, out=None, stream=None):
    """x: float32 cuda [N, K] (row = one activation column) -> uint8 cuda
    [N, pad(K)/32*36] block_q8_1."""
    import torch
    N, Kx = x.shape
    K = Kx if K is None else K
    kp = pad_k(K)
    if out is None:
        out = torch.empty((N, kp // 32 * BLOCK_Q8_1_BYTES), dtype=torch.uint8, device=x.device)
    _check(lib().q4k_quantize_row_q8_1(_ptr(x), _ptr(out), K, x.stride(0), kp, N, _stream(stream)),
           "q4k_quantize_row_q8_1")
    return out


def _entry(wtype: int, q4k_name: str, q6k_name: str):
    if wtype == GGML_TYPE_Q4_K:
        return q4k_name, getattr(lib(), q4k_name)
    if wtype == GGML_TYPE_Q6_K:
        return q6k_name, getattr(lib(), q6k_name)
    raise ValueError(f"weight type {wtype} has no GEMV here")


def mul_mat_vec_q(w_q, K: int, x, out=None, workspace=None, stream=None, wtype: int = GGML_TYPE_Q4_K):
    """ggml_cuda_mul_mat_vec_q: Q4_K [M, K/256*144] or (wtype GGML_TYPE_Q6_K)
    Q6_K [M, K/256*210] (uint8 cuda) x F32 [N, K] -> F32 [N, M] (row c of the
    result = column c of ggml's dst)."""
    import torch
    M = w_q.shape[0]
    N = x.shape[0]
    if out is None:
        out = torch.empty((N, M), dtype=torch.float32, device=x.device)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    name, fn = _entry(wtype, "q4k_mul_mat_vec_q", "q6k_mul_mat_vec_q")
    _check(fn(_ptr(w_q), K, M, w_q.stride(0), _ptr(x), N, x.stride(0) * 4, _ptr(out), out.stride(0) * 4,
              _ptr(workspace), ws_bytes, _stream(stream)), name)
    return out


def mul_mat_vec_q_sums(w_q, K: int, x, workspace=None, stream=None, wtype: int = GGML_TYPE_Q4_K):
    """The parity form of mul_mat_vec_q: the production launch's SUMS
    variant.  Returns (dst F32 [N, M], sums int32, sq int32 or None): Q4_K
    sums [N, M, K/32] of q4*q8 per sub-block and sq [N, K/32] of q8; Q6_K
    sums [N, M, K/16] of (q - 32)*q8 per 16-weight group."""
    import torch
    M = w_q.shape[0]
    N = x.shape[0]
    dev = x.device
    out = torch.empty((N, M), dtype=torch.float32, device=dev)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    args = (_ptr(w_q), K, M, w_q.stride(0), _ptr(x), N, x.stride(0) * 4, _ptr(out), out.stride(0) * 4,
            _ptr(workspace), ws_bytes)
    if wtype == GGML_TYPE_Q4_K:
        sums = torch.empty((N, M, K // 32), dtype=torch.int32, device=dev)
        sq = torch.empty((N, K // 32), dtype=torch.int32, device=dev)
        _check(lib().q4k_mul_mat_vec_q_sums(*args, _ptr(sums), _ptr(sq), _stream(stream)), "q4k_mul_mat_vec_q_sums")
        return out, sums, sq
    if wtype == GGML_TYPE_Q6_K:
        sums = torch.empty((N, M, K // 16), dtype=torch.int32, device=dev)
        _check(lib().q6k_mul_mat_vec_q_sums(*args, _ptr(sums), _stream(stream)), "q6k_mul_mat_vec_q_sums")
        return out, sums, None
    raise ValueError(f"weight type {wtype} has no GEMV here")


def mul_mat_vec_q_fused(w_q, K: int, x, gate=None, x_bias=None, gate_bias=None, glu_op: int = GLU_OP_SWIGLU,
                        out=None, stream=None, wtype: int = GGML_TYPE_Q4_K):
    """One column with the fused epilogue: dst = x_bias + w_q . x, or with a
    gate weight glu(w_q . x + x_bias, gate . x + gate_bias) -> F32 [1, M]."""
    import torch
    M = w_q.shape[0]
    if out is None:
        out = torch.empty((1, M), dtype=torch.float32, device=x.device)
    f = q4k_fusion(_ptr(x_bias), _ptr(gate), _ptr(gate_bias), glu_op)
    _check(lib().q4k_mul_mat_vec_q_fused(wtype, _ptr(w_q), K, M, w_q.stride(0), _ptr(x), ctypes.byref(f),
                                         _ptr(out), _stream(stream)), "q4k_mul_mat_vec_q_fused")
    return out


def op_mul_mat_vec_q(w_q, K: int, q8, ncols: int, row_low: int = 0, row_high: int | None = None,
                     out=None, nrows_dst: int | None = None, stream=None, wtype: int = GGML_TYPE_Q4_K):
    """ggml_cuda_op_mul_mat_vec_q: rows [row_low, row_high) of a contiguous
    Q4_K (or Q6_K) weight (w_q holds exactly those rows) x pre-quantised Q8_1
    columns."""
    import torch
    if row_high is None:
        row_high = row_low + w_q.shape[0]
    rows = row_high - row_low
    nrows_dst = rows if nrows_dst is None else nrows_dst
    if out is None:
        out = torch.empty((ncols, nrows_dst), dtype=torch.float32, device=q8.device)
    padded = q8.shape[1] // BLOCK_Q8_1_BYTES * 32
    name, fn = _entry(wtype, "q4k_op_mul_mat_vec_q", "q6k_op_mul_mat_vec_q")
    _check(fn(_ptr(w_q), K, row_low, row_high, _ptr(q8), ncols, padded, _ptr(out), nrows_dst,
              _stream(stream)), name)
    return out


def make_tensor(type_id: int, ne, nb, data_ptr: int) -> q4k_tensor:
    t = q4k_tensor()
    t.type = type_id
    for i in range(4):
        t.ne[i] = ne[i] if i < len(ne) else 1
    last = nb[-1] * (ne[len(nb) - 1] if len(nb) else 1)
    for i in range(4):
        t.nb[i] = nb[i] if i < len(nb) else last
    t.data = data_ptr
    return t


def ggml_mul_mat_vec_q(src0: q4k_tensor, src1: q4k_tensor, dst: q4k_tensor, ids=None, fusion=None,
                       workspace=None, stream=None) -> int:
    """Descriptor form; returns the status (Q4K_EUNSUPPORTED means: fall back)."""
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    return int(lib().q4k_ggml_mul_mat_vec_q(ctypes.byref(src0), ctypes.byref(src1),
                                            ctypes.byref(ids) if ids is not None else None,
                                            ctypes.byref(dst),
                                            ctypes.byref(fusion) if fusion is not None else None,
                                            _ptr(workspace), ws_bytes, _stream(stream)))


def subblock_sums(w_q, K: int, q8, ncols: int, stream=None):
    """Returns (sqq int32 [N, M, K/32], sq int32 [N, K/32]) on the device."""
    import torch
    M = w_q.shape[0]
    sqq = torch.empty((ncols, M, K // 32), dtype=torch.int32, device=q8.device)
    sq = torch.empty((ncols, K // 32), dtype=torch.int32, device=q8.device)
    _check(lib().q4k_subblock_sums(_ptr(w_q), K, M, w_q.stride(0), _ptr(q8), ncols,
                                   q8.shape[1] // BLOCK_Q8_1_BYTES, _ptr(sqq), _ptr(sq),
                                   _stream(stream)), "q4k_subblock_sums")
    return sqq, sq


def group_sums_q6_K(w_q, K: int, q8, ncols: int, stream=None):
    """Q6_K parity probe: int32 [N, M, K/16] sums of (q - 32) * q8 per
    16-weight scale group, on the device."""
    import torch
    M = w_q.shape[0]
    s16 = torch.empty((ncols, M, K // 16), dtype=torch.int32, device=q8.device)
    _check(lib().q6k_group_sums(_ptr(w_q), K, M, w_q.stride(0), _ptr(q8), ncols,
                                q8.shape[1] // BLOCK_Q8_1_BYTES, _ptr(s16), _stream(stream)),
           "q6k_group_sums")
    return s16


def set_geometry_override(rows_per_tile: int = 0, waves_per_wg: int = 0, workgroups: int = 0,
                          kernel: int = 0):
    _check(lib().q4k_set_geometry_override(rows_per_tile, waves_per_wg, workgroups, kernel),
           "q4k_set_geometry_override")


def set_pipeline_override(slots: int = 0, prologue: int = -1):
    _check(lib().q4k_set_pipeline_override(slots, prologue), "q4k_set_pipeline_override")


def geometry(K: int, M: int, N: int, wtype: int = GGML_TYPE_Q4_K, route: str = "f32") -> dict:
    """The launch of an (M x K) x (K x N) product: route "f32" quantises
    the F32 activation inside the GEMV launch, "q8_1" runs on a Q8_1
    activation (op_mul_mat_vec_q, or mul_mat_vec_q with a workspace where
    it quantises separately), "gate" / "bias" the one-column launch with
    that fused epilogue (mul_mat_vec_q_fused)."""
    out = (ctypes.c_int32 * 8)()
    if route in ("gate", "bias"):
        if N != 1:
            raise ValueError("fused geometry: one column")
        name, fn = _entry(wtype, "q4k_gemv_geometry_fused", "q6k_gemv_geometry_fused")
        _check(fn(K, M, 1 if route == "gate" else 0, ctypes.cast(out, _P)), name)
    elif route == "q8_1":
        name, fn = _entry(wtype, "q4k_gemv_geometry_q8_1", "q6k_gemv_geometry_q8_1")
    else:
        name, fn = _entry(wtype, "q4k_gemv_geometry", "q6k_gemv_geometry")
    if route not in ("gate", "bias"):
        _check(fn(K, M, N, ctypes.cast(out, _P)), name)
    keys = ("rows_per_tile", "waves_per_wg", "workgroups", "lds_bytes", "cols_per_launch", "fused",
            "kernel", "rows_per_step")
    return dict(zip(keys, list(out)))


# ------------------------------------------------------------------ GGUF ----
GGUF_ARRAY, GGUF_STRING = 9, 8
_GGUF_NP = {0: np.uint8, 1: np.int8, 2: np.uint16, 3: np.int16, 4: np.uint32, 5: np.int32, 6: np.float32,
            7: np.bool_, 10: np.uint64, 11: np.int64, 12: np.float64}


class GGUFFile:
    """A GGUF file opened with the library's reader (q4k_gguf_open).
    tensors: {name: dict(type, ne, offset, nbytes)}; tensor_bytes(name) is a
    zero-copy uint8 view of the mapped data, valid until close()."""

    def __init__(self, path: str):
        self._h = ctypes.c_void_p()
        _check(lib().q4k_gguf_open(os.fsencode(path), ctypes.byref(self._h)), f"q4k_gguf_open({path})")
        L = lib()
        self.version = int(L.q4k_gguf_version(self._h))
        self.alignment = int(L.q4k_gguf_alignment(self._h))
        self.data_offset = int(L.q4k_gguf_data_offset(self._h))
        self.tensors = {}
        for i in range(L.q4k_gguf_tensor_count(self._h)):
            ti = q4k_gguf_tensor_info()
            _check(L.q4k_gguf_get_tensor(self._h, i, ctypes.byref(ti)), "q4k_gguf_get_tensor")
            self.tensors[ti.name.decode()] = {"index": i, "type": ti.type, "ne": list(ti.ne)[:ti.n_dims],
                                              "offset": int(ti.offset), "nbytes": int(ti.nbytes),
                                              "data": ti.data}

    def metadata(self) -> dict:
        L = lib()
        out = {}
        for i in range(L.q4k_gguf_kv_count(self._h)):
            key = L.q4k_gguf_key(self._h, i).decode()
            t = L.q4k_gguf_kv_type(self._h, i)
            if t == GGUF_STRING:
                sp = ctypes.c_char_p()
                _check(L.q4k_gguf_get_str(self._h, i, ctypes.byref(sp)), key)
                out[key] = sp.value.decode()
            elif t == GGUF_ARRAY:
                et, n, dp = ctypes.c_int32(), ctypes.c_int64(), ctypes.c_void_p()
                _check(L.q4k_gguf_get_arr(self._h, i, ctypes.byref(et), ctypes.byref(n), ctypes.byref(dp)), key)
                if et.value == GGUF_STRING:
                    vals = []
                    for j in range(n.value):
                        sp = ctypes.c_char_p()
                        _check(L.q4k_gguf_get_arr_str(self._h, i, j, ctypes.byref(sp)), key)
                        vals.append(sp.value.decode())
                    out[key] = vals
                else:
                    dt = np.dtype(_GGUF_NP[et.value])
                    buf = (ctypes.c_uint8 * (n.value * dt.itemsize)).from_address(dp.value) if n.value else b""
                    out[key] = np.frombuffer(bytes(buf), dtype=dt).tolist()
            elif t in (6, 12):
                v = ctypes.c_double()
                _check(L.q4k_gguf_get_float(self._h, i, ctypes.byref(v)), key)
                out[key] = v.value
            else:
                v = ctypes.c_int64()
                _check(L.q4k_gguf_get_int(self._h, i, ctypes.byref(v)), key)
                out[key] = bool(v.value) if t == 7 else v.value
        return out

    def tensor_bytes(self, name: str) -> np.ndarray:
        t = self.tensors[name]
        if not t["nbytes"]:
            raise ValueError(f"{name}: block size of ggml type {t['type']} unknown")
        buf = (ctypes.c_uint8 * t["nbytes"]).from_address(t["data"])
        return np.frombuffer(buf, dtype=np.uint8)

    def weight_rows(self, name: str) -> np.ndarray:
        """A 2-D quantised weight as [rows, row bytes] (zero-copy view)."""
        t = self.tensors[name]
        rb = int(lib().q4k_ggml_row_size(t["type"], t["ne"][0]))
        return self.tensor_bytes(name).reshape(-1, rb)

    def close(self):
        if self._h:
            lib().q4k_gguf_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
