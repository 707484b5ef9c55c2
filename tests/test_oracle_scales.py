"""Pins the 6-bit (sc, m) unpack: ggml's get_scale_min_k4 and the GPU
vec-dot's uint16-pair form (kernels/vecdotq.cuh:796-807) must agree on every
byte pattern they read, and packing must invert unpacking."""
import ctypes

import numpy as np


def test_unpackers_agree_exhaustively(O):
    assert O.lib().orc_selftest_scale_unpack() == 0


def test_pack_unpack_identity(O):
    assert O.lib().orc_selftest_scale_pack() == 0


def test_unpack_against_bitfield_definition(O):
    # The bit layout written out field by field: sub-block s < 4 keeps its 6
    # bits in the low bits of bytes s (scale) and s+4 (min); s >= 4 keeps the
    # low 4 bits in byte s+4 (scale low nibble, min high nibble) and the top
    # 2 bits in bits 6-7 of bytes s-4 (scale) and s (min).
    rng = np.random.default_rng(11)
    b = rng.integers(0, 256, size=(20000, 12), dtype=np.uint8)
    for s in range(8):
        if s < 4:
            sc_ref = b[:, s] & 63
            m_ref = b[:, s + 4] & 63
        else:
            sc_ref = (b[:, s + 4] & 15) + ((b[:, s - 4] >> 6) << 4)
            m_ref = (b[:, s + 4] >> 4) + ((b[:, s] >> 6) << 4)
        sc = ctypes.c_uint8()
        m = ctypes.c_uint8()
        for r in range(0, 20000, 97):
            row = np.ascontiguousarray(b[r])
            O.lib().orc_scale_min_k4(s, row.ctypes.data_as(ctypes.c_void_p), ctypes.byref(sc), ctypes.byref(m))
            assert (sc.value, m.value) == (int(sc_ref[r]), int(m_ref[r]))
