"""The C-ABI library builds, loads and exports every entry point its header
declares; argument checks that need no GPU return the documented status."""
import ctypes
import os
import re

import pytest

import _common

HEADERS = [os.path.join(_common.ROOT, "include", h) for h in sorted(os.listdir(os.path.join(_common.ROOT, "include")))
           if h.endswith(".h")]


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(q[46]k_[A-Za-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("q4k_mul_mat_vec_q", "q4k_op_mul_mat_vec_q", "q4k_ggml_mul_mat_vec_q",
              "q4k_quantize_row_q8_1", "q4k_subblock_sums", "q4k_quantize_rows_q4_K",
              "q6k_mul_mat_vec_q", "q6k_op_mul_mat_vec_q", "q6k_group_sums", "q4k_quantize_rows_q6_K",
              "q4k_mul_mat_vec_q_fused", "q4k_gguf_open", "q4k_gguf_get_tensor"):
        assert n in names


def test_library_exports_every_declared_symbol(Q):
    L = ctypes.CDLL(Q.LIB_PATH)
    for n in declared_functions():
        assert hasattr(L, n), n
        assert n in Q.SIGNATURES, n


def test_misc_entry_points(Q):
    L = Q.lib()
    assert L.q4k_version() >= 100
    assert L.q4k_strerror(Q.Q4K_EUNSUPPORTED).decode().startswith("unsupported")
    assert L.q4k_q8_1_bytes(4096, 1) == 4096 // 32 * 36
    assert L.q4k_q8_1_bytes(4100, 2) == 2 * 4608 // 32 * 36
    assert L.q4k_q8_1_bytes(14336, 8) == 8 * 14336 // 32 * 36
    # sizes whose byte count could overflow report 0, as negative ones do
    assert L.q4k_q8_1_bytes(-1, 1) == 0
    assert L.q4k_q8_1_bytes(1 << 62, 1) == 0
    assert L.q4k_q8_1_bytes(4096, 1 << 40) == 0
    # a quantiser grid beyond 2^31 workgroups is refused before any HIP call
    assert L.q4k_quantize_row_q8_1(FAKE, FAKE, 4096, 4096, 1 << 40, 1, None) == Q.Q4K_EUNSUPPORTED


FAKE = ctypes.c_void_p(0x10000)     # never dereferenced by the host checks
FAKE_ODD = ctypes.c_void_p(0x10004)


@pytest.mark.parametrize("args,status", [
    ((FAKE, 4000, 16, 4000 // 256 * 144, FAKE, 1, 16000, FAKE, 64), 2),   # K % 256
    ((FAKE, 4096, 16, 2304, FAKE, 9, 16384, FAKE, 64), 2),                  # 9 columns
    ((FAKE, 4096, 16, 2300, FAKE, 1, 16384, FAKE, 64), 2),                  # row stride
    ((FAKE, 4096, 16, 2304, None, 1, 16384, FAKE, 64), 2),                  # null src1
    ((FAKE, 4096, 16, 2304, FAKE, 2, 1000, FAKE, 64), 2),                   # column stride
    ((FAKE_ODD, 4096, 16, 2304, FAKE, 1, 16384, FAKE, 64), 1),              # src0 alignment
    ((FAKE, 4096, 0, 2304, FAKE, 1, 16384, FAKE, 64), 0),                   # empty: no rows
    ((FAKE, 4096, 16, 2304, FAKE, 0, 16384, FAKE, 64), 0),                  # empty: no columns
])
def test_mul_mat_vec_q_argument_checks(Q, args, status):
    assert Q.lib().q4k_mul_mat_vec_q(*args, None, 0, None) == status


def test_op_and_descriptor_checks(Q):
    L = Q.lib()
    assert L.q4k_op_mul_mat_vec_q(FAKE, 4096, 10, 5, FAKE, 1, 4096, FAKE, 5, None) == Q.Q4K_EINVAL
    assert L.q4k_op_mul_mat_vec_q(FAKE, 4096, 0, 8, FAKE, 1, 4000, FAKE, 8, None) == Q.Q4K_EINVAL
    assert L.q4k_op_mul_mat_vec_q(FAKE, 4096, 0, 8, FAKE, 1, 4096, FAKE, 4, None) == Q.Q4K_EINVAL
    assert L.q4k_op_mul_mat_vec_q(FAKE, 4096, 3, 3, FAKE, 1, 4096, FAKE, 4, None) == Q.Q4K_OK
    s0 = Q.make_tensor(Q.GGML_TYPE_Q4_K, [4096, 16], [144, 2304], 0x10000)
    s1 = Q.make_tensor(Q.GGML_TYPE_F32, [4096, 1], [4, 16384], 0x20000)
    d = Q.make_tensor(Q.GGML_TYPE_F32, [16, 1], [4, 64], 0x30000)
    f16 = Q.make_tensor(1, [4096, 1], [2, 8192], 0x20000)
    assert Q.ggml_mul_mat_vec_q(s0, f16, d) == Q.Q4K_EINVAL
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, ids=s1) == Q.Q4K_EINVAL           # ids must be I32
    # fusion under the reference's checks (host-side, no device call)
    gate = Q.make_tensor(Q.GGML_TYPE_Q4_K, [4096, 16], [144, 2304], 0x50000)
    bad_bias = Q.make_tensor(1, [16], [2], 0x60000)
    fa = Q.q4k_fusion_args(None, ctypes.pointer(gate), None, 0)              # REGLU: not fused
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, fusion=fa) == Q.Q4K_EUNSUPPORTED
    fa = Q.q4k_fusion_args(ctypes.pointer(bad_bias), None, None, 2)          # F16 bias
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, fusion=fa) == Q.Q4K_EINVAL
    gate6 = Q.make_tensor(Q.GGML_TYPE_Q6_K, [4096, 16], [210, 3360], 0x50000)
    fa = Q.q4k_fusion_args(None, ctypes.pointer(gate6), None, 2)             # gate of another type
    assert Q.ggml_mul_mat_vec_q(s0, s1, d, fusion=fa) == Q.Q4K_EINVAL
    s1b = Q.make_tensor(Q.GGML_TYPE_F32, [4096, 2], [4, 16384], 0x20000)
    d2 = Q.make_tensor(Q.GGML_TYPE_F32, [16, 2], [4, 64], 0x30000)
    fa = Q.q4k_fusion_args(None, ctypes.pointer(gate), None, 2)              # fusion needs one column
    assert Q.ggml_mul_mat_vec_q(s0, s1b, d2, fusion=fa) == Q.Q4K_EINVAL
    q5 = Q.make_tensor(13, [4096, 16], [176, 2816], 0x10000)
    assert Q.ggml_mul_mat_vec_q(q5, s1, d) == Q.Q4K_EUNSUPPORTED             # other types
    q6 = Q.make_tensor(Q.GGML_TYPE_Q6_K, [4096, 16], [144, 3360], 0x10000)
    assert Q.ggml_mul_mat_vec_q(q6, s1, d) == Q.Q4K_EINVAL                   # nb00 != 210
    s3 = Q.make_tensor(Q.GGML_TYPE_F32, [4096, 1, 2], [4, 16384, 16384], 0x20000)
    assert Q.ggml_mul_mat_vec_q(s0, s3, d) == Q.Q4K_EINVAL                   # dst dims != src1's
    s03 = Q.make_tensor(Q.GGML_TYPE_Q4_K, [4096, 16, 2], [144, 2304, 2304 * 16], 0x10000)
    s13 = Q.make_tensor(Q.GGML_TYPE_F32, [4096, 1, 3], [4, 16384, 16384], 0x20000)
    d3 = Q.make_tensor(Q.GGML_TYPE_F32, [16, 1, 3], [4, 64, 64], 0x30000)
    assert Q.ggml_mul_mat_vec_q(s03, s13, d3) == Q.Q4K_EINVAL                # 3 channels over 2 matrices
    ids2 = Q.make_tensor(26, [2, 2], [4, 8], 0x40000)
    d2 = Q.make_tensor(Q.GGML_TYPE_F32, [16, 2, 2], [4, 64, 128], 0x30000)
    s12 = Q.make_tensor(Q.GGML_TYPE_F32, [4096, 1, 2], [4, 16384, 16384], 0x20000)
    assert Q.ggml_mul_mat_vec_q(s03, s12, d2, ids=ids2) == Q.Q4K_EINVAL      # MUL_MAT_ID: one token
    assert L.q4k_quantize_row_q8_1(FAKE, FAKE, 100, 100, 96, 1, None) == Q.Q4K_EINVAL
    assert L.q4k_quantize_row_q8_1(FAKE, FAKE, 100, 100, 130, 1, None) == Q.Q4K_EINVAL
    assert L.q4k_quantize_rows_q4_K(None, None, 4, 300, 1) == Q.Q4K_EINVAL


def test_host_quantiser_rejects_bad_shapes(Q):
    import numpy as np
    with pytest.raises(Q.Q4KError):
        Q.quantize_rows_q4_K(np.zeros((2, 300), np.float32))


FAKE_2 = ctypes.c_void_p(0x10002)   # 2-byte aligned: enough for Q6_K rows
FAKE_1 = ctypes.c_void_p(0x10001)


@pytest.mark.parametrize("args,status", [
    ((FAKE, 4000, 16, 4000 // 256 * 210, FAKE, 1, 16000, FAKE, 64), 2),   # K % 256
    ((FAKE, 4096, 16, 3360, FAKE, 9, 16384, FAKE, 64), 2),                  # 9 columns
    ((FAKE, 4096, 16, 3364, FAKE, 1, 16384, FAKE, 64), 2),                  # row stride % 210
    ((FAKE, 4096, 16, 3150, FAKE, 1, 16384, FAKE, 64), 2),                  # row stride < row
    ((FAKE, 4096, 16, 3360, None, 1, 16384, FAKE, 64), 2),                  # null src1
    ((FAKE_1, 4096, 16, 3360, FAKE, 1, 16384, FAKE, 64), 2),                # src0 alignment
    ((FAKE_2, 4096, 0, 3360, FAKE, 1, 16384, FAKE, 64), 0),                 # empty: no rows
    ((FAKE, 4096, 16, 3360, FAKE, 0, 16384, FAKE, 64), 0),                  # empty: no columns
])
def test_q6k_mul_mat_vec_q_argument_checks(Q, args, status):
    assert Q.lib().q6k_mul_mat_vec_q(*args, None, 0, None) == status


def test_q6k_op_and_probe_checks(Q):
    L = Q.lib()
    assert L.q6k_op_mul_mat_vec_q(FAKE, 4096, 10, 5, FAKE, 1, 4096, FAKE, 5, None) == Q.Q4K_EINVAL
    assert L.q6k_op_mul_mat_vec_q(FAKE, 4096, 0, 8, FAKE, 1, 4000, FAKE, 8, None) == Q.Q4K_EINVAL
    assert L.q6k_op_mul_mat_vec_q(FAKE, 4096, 3, 3, FAKE, 1, 4096, FAKE, 4, None) == Q.Q4K_OK
    assert L.q6k_group_sums(FAKE, 4096, 4, 3360, FAKE, 1, 100, FAKE, None) == Q.Q4K_EINVAL
    assert L.q6k_group_sums(FAKE, 4096, 0, 3360, FAKE, 1, 128, FAKE, None) == Q.Q4K_OK


def test_fused_entry_checks(Q):
    L = Q.lib()
    f = Q.q4k_fusion(None, FAKE, None, 0)
    assert L.q4k_mul_mat_vec_q_fused(13, FAKE, 4096, 16, 2304, FAKE, ctypes.byref(f), FAKE, None) == 1
    assert L.q4k_mul_mat_vec_q_fused(12, FAKE, 4096, 16, 2304, FAKE, ctypes.byref(f), FAKE, None) == 1
    f = Q.q4k_fusion(ctypes.c_void_p(0x60002), None, None, 0)               # misaligned bias
    assert L.q4k_mul_mat_vec_q_fused(12, FAKE, 4096, 16, 2304, FAKE, ctypes.byref(f), FAKE, None) == 2
    f = Q.q4k_fusion(None, FAKE_2, None, 2)                                  # Q4_K gate alignment
    assert L.q4k_mul_mat_vec_q_fused(12, FAKE, 4096, 16, 2304, FAKE, ctypes.byref(f), FAKE, None) == 1
    assert L.q4k_mul_mat_vec_q_fused(14, FAKE, 4096, 0, 3360, FAKE, ctypes.byref(f), FAKE, None) == 0
