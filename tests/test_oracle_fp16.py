"""Pins the oracle's fp16 conversions and nearest_int against numpy."""
import numpy as np


def test_half_to_float_exhaustive(O):
    h = np.arange(65536, dtype=np.uint16)
    got = O.f16_bits_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_float_to_half_representable_roundtrip(O):
    h = np.arange(65536, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(f)
    assert (O.f32_to_f16_bits(f[ok]) == h[ok]).all()


def test_float_to_half_ties_and_random_bits(O):
    # midpoints between consecutive finite halves: exact ties round to even
    h = np.arange(0, 0x7bff, dtype=np.uint16)
    a = h.view(np.float16).astype(np.float64)
    b = (h + 1).view(np.float16).astype(np.float64)
    mid = ((a + b) / 2).astype(np.float32)
    for v in (mid, -mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))):
        assert (O.f32_to_f16_bits(v) == v.astype(np.float16).view(np.uint16)).all()
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert (O.f32_to_f16_bits(x) == ref).all()


def test_nearest_int_is_round_half_even(O):
    rng = np.random.default_rng(3)
    x = np.concatenate([
        rng.uniform(-4e6, 4e6, 1_000_000).astype(np.float32),
        (np.arange(-2000, 2000) + 0.5).astype(np.float32),     # exact halves
        rng.normal(0, 3, 100_000).astype(np.float32),
    ])
    assert (O.nearest_int(x) == np.rint(x).astype(np.int32)).all()
