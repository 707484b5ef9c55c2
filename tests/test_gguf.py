"""The GGUF reader (include/q4k_gguf.h) on files whose bytes the tests fix:
a hand-assembled known-answer file, files from the spec-following writer in
tests/gguf_writer.py (every metadata type, K-quant and plain tensors,
custom alignment, version 2), and malformed or truncated files, which must
be refused with a status, never read out of bounds.  No real model file is
available offline: parity of a real Q4_K_M file is unpinned here."""
import struct

import numpy as np
import pytest

import _common
import gguf_writer as W


def open_status(Q, path):
    import ctypes
    h = ctypes.c_void_p()
    st = Q.lib().q4k_gguf_open(str(path).encode(), ctypes.byref(h))
    if st == 0:
        Q.lib().q4k_gguf_close(h)
    return st


def test_known_answer_file(Q, tmp_path):
    # GGUF v3, 1 tensor, 1 metadata entry, assembled byte by byte
    raw = b"GGUF" + struct.pack("<I", 3) + struct.pack("<Q", 1) + struct.pack("<Q", 1)
    raw += struct.pack("<Q", 20) + b"general.architecture" + struct.pack("<I", 8)
    raw += struct.pack("<Q", 5) + b"llama"
    raw += struct.pack("<Q", 1) + b"t" + struct.pack("<I", 2) + struct.pack("<QQ", 4, 2)
    raw += struct.pack("<I", 0) + struct.pack("<Q", 0)
    header_len = len(raw)                       # 4+4+8+8 + 8+20+4+8+5 + 8+1+4+16+4+8 = 110
    assert header_len == 110
    raw += b"\0" * (128 - header_len)          # padding to 32
    vals = np.arange(8, dtype=np.float32) * np.float32(0.5)
    raw += vals.tobytes()
    p = tmp_path / "ka.gguf"
    p.write_bytes(raw)
    with Q.GGUFFile(str(p)) as g:
        assert g.version == 3 and g.alignment == 32 and g.data_offset == 128
        assert g.metadata() == {"general.architecture": "llama"}
        t = g.tensors["t"]
        assert t["type"] == 0 and t["ne"] == [4, 2] and t["offset"] == 128 and t["nbytes"] == 32
        assert np.array_equal(g.tensor_bytes("t").view(np.float32), vals)


def test_round_trip_every_type(Q, O, tmp_path):
    rng = np.random.default_rng(0)
    w4 = O.quantize_q4_K(rng.standard_normal((3, 512)).astype(np.float32) * np.float32(0.02))
    w6 = O.quantize_q6_K(rng.standard_normal((5, 256)).astype(np.float32) * np.float32(0.02))
    f32 = rng.standard_normal(7).astype(np.float32)
    f16 = rng.standard_normal((2, 3)).astype(np.float16)
    i32 = np.arange(-3, 3, dtype=np.int32)
    kvs = [("u8", W.UINT8, 250), ("i8", W.INT8, -7), ("u16", W.UINT16, 65000), ("i16", W.INT16, -30000),
           ("u32", W.UINT32, 4000000000), ("i32", W.INT32, -2000000000), ("f32", W.FLOAT32, 1.5),
           ("b", W.BOOL, True), ("s", W.STRING, "héllo"), ("u64", W.UINT64, 2 ** 40), ("i64", W.INT64, -2 ** 40),
           ("f64", W.FLOAT64, -2.25), ("arr_i32", W.ARRAY, (W.INT32, [1, -2, 3])),
           ("arr_s", W.ARRAY, (W.STRING, ["a", "", "xyz"])), ("arr_f32", W.ARRAY, (W.FLOAT32, [0.5, 2.0])),
           ("arr_empty", W.ARRAY, (W.UINT8, []))]
    tensors = [("blk.0.ffn_up.weight", 12, [512, 3], w4.tobytes()), ("output.weight", 14, [256, 5], w6.tobytes()),
               ("norm", 0, [7], f32.tobytes()), ("h", 1, [3, 2], f16.tobytes()), ("idx", 26, [6], i32.tobytes())]
    for align, version in ((None, 3), (64, 3), (256, 2)):
        p = tmp_path / f"rt_{align}_{version}.gguf"
        W.write_gguf(p, kvs, tensors, alignment=align, version=version)
        with Q.GGUFFile(str(p)) as g:
            assert g.version == version and g.alignment == (align or 32)
            assert g.data_offset % g.alignment == 0
            md = g.metadata()
            for key, t, v in kvs:
                got = md[key]
                if t == W.ARRAY:
                    assert got == list(v[1])
                elif t == W.FLOAT32:
                    assert got == pytest.approx(v)
                else:
                    assert got == v, key
            if align:
                assert md["general.alignment"] == align
            for name, gt, ne, data in tensors:
                t = g.tensors[name]
                assert t["type"] == gt and t["ne"] == ne and t["nbytes"] == len(data)
                assert t["offset"] % g.alignment == 0
                assert g.tensor_bytes(name).tobytes() == data
            assert np.array_equal(g.weight_rows("blk.0.ffn_up.weight"), w4)
            assert np.array_equal(g.weight_rows("output.weight"), w6)
            assert Q.lib().q4k_gguf_find_tensor(g._h, b"missing") == -1
            assert Q.lib().q4k_gguf_find_key(g._h, b"s") >= 0


def test_row_size_table(Q):
    L = Q.lib()
    assert L.q4k_ggml_row_size(12, 4096) == 16 * 144
    assert L.q4k_ggml_row_size(14, 4096) == 16 * 210
    assert L.q4k_ggml_row_size(8, 64) == 2 * 34
    assert L.q4k_ggml_row_size(0, 5) == 20
    assert L.q4k_ggml_row_size(12, 100) == 0      # not whole blocks
    assert L.q4k_ggml_row_size(99, 256) == 0      # unknown type


def _small_file():
    return W.gguf_bytes([("a", W.UINT32, 7), ("name", W.STRING, "m"), ("arr", W.ARRAY, (W.INT16, [1, 2, 3]))],
                        [("w", 12, [256, 2], bytes(288)), ("x", 0, [3], bytes(12))])


def test_every_truncation_is_refused(Q, tmp_path):
    raw = _small_file()
    p = tmp_path / "t.gguf"
    p.write_bytes(raw)
    assert open_status(Q, p) == 0
    last_meta = len(raw) - 12 - (32 - (288 % 32)) % 32 - 288   # where the tensor data starts
    for n in range(0, len(raw)):
        p.write_bytes(raw[:n])
        st = open_status(Q, p)
        assert st == Q.Q4K_EFORMAT, (n, st)


@pytest.mark.parametrize("case", ["magic", "version1", "version4", "ndims5", "ndims0", "offset_past_end",
                                  "misaligned", "dup_tensor", "dup_key", "partial_block", "bad_alignment",
                                  "alignment_type", "bad_value_type", "huge_count", "huge_string",
                                  "unknown_type", "removed_type", "offset_gap", "offset_overlap",
                                  "offset_order"])
def test_malformed_files_are_refused(Q, tmp_path, case):
    tensors = [("w", 12, [256, 2], bytes(288))]
    kvs = [("a", W.UINT32, 7)]
    if case == "magic":
        raw = b"GGUX" + _small_file()[4:]
    elif case == "version1":
        raw = W.gguf_bytes(kvs, tensors, version=1)
    elif case == "version4":
        raw = W.gguf_bytes(kvs, tensors, version=4)
    elif case == "ndims5":
        raw = W.gguf_bytes(kvs, [("w", 0, [1, 1, 1, 1, 2], bytes(8))])
    elif case == "ndims0":
        raw = W.gguf_bytes(kvs, [("w", 0, [], bytes(4))])
    elif case == "offset_past_end":
        raw = W.gguf_bytes(kvs, tensors, offsets=[4096])[:-1]
        raw = raw[:min(len(raw), 700)]
    elif case == "misaligned":
        raw = W.gguf_bytes(kvs, tensors, offsets=[4])
    elif case == "dup_tensor":
        raw = W.gguf_bytes(kvs, tensors + [("w", 0, [2], bytes(8))])
    elif case == "dup_key":
        raw = W.gguf_bytes(kvs + [("a", W.UINT32, 8)], tensors)
    elif case == "partial_block":
        raw = W.gguf_bytes(kvs, [("w", 12, [100, 2], bytes(288))])
    elif case == "bad_alignment":
        raw = W.gguf_bytes(kvs, tensors, alignment=48)
    elif case == "alignment_type":
        raw = W.gguf_bytes(kvs + [("general.alignment", W.UINT64, 64)], tensors)
    elif case == "bad_value_type":
        raw = W.gguf_bytes(kvs, tensors).replace(struct.pack("<Q", 1) + b"a" + struct.pack("<I", 4),
                                                 struct.pack("<Q", 1) + b"a" + struct.pack("<I", 13), 1)
    elif case == "unknown_type":
        raw = W.gguf_bytes(kvs, [("w", 99, [256, 2], bytes(288))])
    elif case == "removed_type":   # 4 was Q4_2, removed from ggml
        raw = W.gguf_bytes(kvs, [("w", 4, [32, 2], bytes(40))])
    elif case == "offset_gap":     # aligned, in bounds, but not where ggml expects it
        raw = W.gguf_bytes(kvs, tensors, offsets=[32]) + bytes(32)
    elif case == "offset_overlap":
        raw = W.gguf_bytes(kvs, tensors + [("x", 0, [8], bytes(32))], offsets=[0, 0])
    elif case == "offset_order":   # both tensors present, in the opposite order of the directory
        raw = W.gguf_bytes(kvs, [("x", 0, [8], bytes(32))] + tensors, offsets=[288, 0]) + bytes(32)
    elif case == "huge_count":
        raw = b"GGUF" + struct.pack("<IQQ", 3, 1 << 40, 0) + bytes(64)
    else:  # huge_string: a key length far past the end of the file
        raw = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 62) + bytes(64)
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(raw)
    assert open_status(Q, p) == Q.Q4K_EFORMAT


def test_missing_file(Q, tmp_path):
    assert open_status(Q, tmp_path / "nope.gguf") == Q.Q4K_EIO


def _read_everything(Q, path):
    """Opens the file and walks every accessor; returns the open status."""
    import ctypes
    L = Q.lib()
    h = ctypes.c_void_p()
    st = L.q4k_gguf_open(str(path).encode(), ctypes.byref(h))
    if st != 0:
        return st
    try:
        for i in range(L.q4k_gguf_kv_count(h)):
            L.q4k_gguf_key(h, i)
            t = L.q4k_gguf_kv_type(h, i)
            iv, fv, sv = ctypes.c_int64(), ctypes.c_double(), ctypes.c_char_p()
            L.q4k_gguf_get_int(h, i, ctypes.byref(iv))
            L.q4k_gguf_get_float(h, i, ctypes.byref(fv))
            L.q4k_gguf_get_str(h, i, ctypes.byref(sv))
            if t == W.ARRAY:
                et, n, data = ctypes.c_int32(), ctypes.c_int64(), ctypes.c_void_p()
                assert L.q4k_gguf_get_arr(h, i, ctypes.byref(et), ctypes.byref(n), ctypes.byref(data)) == 0
                if et.value == W.STRING:
                    for j in range(min(n.value, 64)):
                        assert L.q4k_gguf_get_arr_str(h, i, j, ctypes.byref(sv)) == 0
        info = Q.q4k_gguf_tensor_info()
        for i in range(L.q4k_gguf_tensor_count(h)):
            assert L.q4k_gguf_get_tensor(h, i, ctypes.byref(info)) == 0
            if info.nbytes:   # the mapped data is readable to its last byte
                ctypes.string_at(info.data, 1)
                ctypes.string_at(info.data + info.nbytes - 1, 1)
    finally:
        L.q4k_gguf_close(h)
    return 0


def test_mutated_files_never_crash(Q, tmp_path):
    """Seeded byte-level corruption of a valid file (flips, overwrites with
    extreme values, insertions, deletions): every open either succeeds, and
    then every accessor and the mapped tensor bytes stay readable, or is
    refused with Q4K_EFORMAT."""
    raw = bytearray(_small_file())
    rng = np.random.default_rng(1234)
    p = tmp_path / "m.gguf"
    opened = 0
    for trial in range(3000):
        b = bytearray(raw)
        for _ in range(int(rng.integers(1, 6))):
            kind = int(rng.integers(0, 4))
            pos = int(rng.integers(0, len(b)))
            if kind == 0:
                b[pos] ^= 1 << int(rng.integers(0, 8))
            elif kind == 1:
                v = [0x00, 0xFF, 0x7F, 0x80][int(rng.integers(0, 4))]
                for k in range(pos, min(len(b), pos + int(rng.integers(1, 9)))):
                    b[k] = v
            elif kind == 2:
                b[pos:pos] = bytes(rng.integers(0, 256, int(rng.integers(1, 9)), dtype=np.uint8))
            elif len(b) > 8:
                del b[pos:pos + int(rng.integers(1, 9))]
        p.write_bytes(bytes(b))
        st = _read_everything(Q, p)
        assert st in (0, Q.Q4K_EFORMAT), (trial, st)
        opened += st == 0
    assert 0 < opened < 3000   # both outcomes occur
