"""The committed fixtures (tests/golden/make_golden.py) are reproduced by the
oracle and, for the weight bytes, by the product's host quantiser."""
import hashlib

import numpy as np

import _common


def _load():
    return np.load(_common.GOLDEN_DIR + "/q4k_golden.npz")


def test_oracle_reproduces_fixtures(O):
    g = _load()
    names = sorted({k.split("/")[0] for k in g.files if k.endswith("/wq")})
    assert len(names) >= 5
    for name in names:
        K, x, wq = int(g[name + "/K"]), g[name + "/x"], g[name + "/wq"]
        q8 = O.quantize_q8_1(x)
        assert np.array_equal(q8, g[name + "/q8"]), name
        ref = O.gemv_q4K_q8_1(wq, K, q8)
        for k in ("sqq", "sq", "y64", "l1"):
            assert np.array_equal(ref[k], g[name + "/" + k]), (name, k)


def test_workload_digests(O, Q):
    g = _load()
    W = _common.weights(4096, 4096, 0)
    assert hashlib.sha256(W.tobytes()).hexdigest() == str(g["cfg_4096x4096_b1/sha256_w_f32"])
    wq = Q.quantize_rows_q4_K(W, nthreads=8)
    assert hashlib.sha256(wq.tobytes()).hexdigest() == str(g["cfg_4096x4096_b1/sha256_wq"])
    x = _common.activations(1, 4096, 0)
    q8 = O.quantize_q8_1(x)
    assert hashlib.sha256(q8.tobytes()).hexdigest() == str(g["cfg_4096x4096_b1/sha256_q8"])
    ref = O.gemv_q4K_q8_1(wq, 4096, q8, want_sums=False)
    assert np.array_equal(ref["y64"], g["cfg_4096x4096_b1/y64"])
