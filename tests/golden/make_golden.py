"""Writes tests/golden/q4k_golden.npz from the oracle (oracle/q4k_oracle.c).

The reference ships no golden vectors for this path, so these fixtures are the
oracle's own outputs on seeded inputs (numpy PCG64, streams (seed, 1) for
weights ~ N(0, 0.02) and (seed, 2) for activations ~ N(0, 1)), committed to pin
regressions of the oracle, the host quantiser and the GPU path alike.

Each case NAME stores NAME/{K, x, wq, q8, sqq, sq, y64, l1}; the 4096x4096
b=1 workload stores only digests of its generated inputs and its result.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import _common  # noqa: E402

O = _common.oracle()


def extreme_case():
    K, M, N = 512, 4, 2
    rng = np.random.default_rng(1234)
    wq = np.zeros((M, K // 256 * 144), np.uint8)
    b = wq.reshape(M, -1, 144)
    b[..., 0:2] = np.frombuffer(np.float16(0.0625).tobytes(), np.uint8)
    b[..., 2:4] = np.frombuffer(np.float16(0.03125).tobytes(), np.uint8)
    b[0, :, 4:16] = 0xFF                     # every 6-bit field 63
    b[1, :, 4:16] = rng.integers(0, 256, (K // 256, 12), dtype=np.uint8)
    b[2, :, 4:16] = 0x00
    b[3, :, 4:16] = rng.integers(0, 256, (K // 256, 12), dtype=np.uint8)
    b[0, :, 16:] = 0xFF                      # q4 = 15
    b[1, :, 16:] = 0x00                      # q4 = 0
    b[2, :, 16:] = 0xF0
    b[3, :, 16:] = rng.integers(0, 256, (K // 256, 128), dtype=np.uint8)
    x = np.where(rng.random((N, K)) < 0.5, 15.875, -15.875).astype(np.float32)  # q8 = +-127
    x[1, 64:96] = 0.0                        # an all-zero Q8_1 block
    return wq, x, K


def main():
    cases = {}
    for name, M, K, N, seed in [("m8_k512_n1", 8, 512, 1, 10), ("m16_k1024_n3", 16, 1024, 3, 11),
                                ("m5_k2304_n8", 5, 2304, 8, 12), ("m64_k4096_n2", 64, 4096, 2, 13),
                                ("m3_k256_n5", 3, 256, 5, 14)]:
        wq = O.quantize_q4_K(_common.weights(M, K, seed))
        cases[name] = (wq, _common.activations(N, K, seed), K)
    cases["extreme"] = extreme_case()
    out = {}
    for name, (wq, x, K) in cases.items():
        q8 = O.quantize_q8_1(x)
        ref = O.gemv_q4K_q8_1(wq, K, q8)
        out.update({f"{name}/K": np.int64(K), f"{name}/x": x, f"{name}/wq": wq, f"{name}/q8": q8,
                    f"{name}/sqq": ref["sqq"], f"{name}/sq": ref["sq"], f"{name}/y64": ref["y64"],
                    f"{name}/l1": ref["l1"]})
    # the 4096x4096 b=1 workload: digests of the generated inputs + result
    W = _common.weights(4096, 4096, 0)
    wq = O.quantize_q4_K(W, nthreads=8)
    x = _common.activations(1, 4096, 0)
    q8 = O.quantize_q8_1(x)
    ref = O.gemv_q4K_q8_1(wq, 4096, q8, want_sums=False)
    digests = {"w_f32": hashlib.sha256(W.tobytes()).hexdigest(),
               "wq": hashlib.sha256(wq.tobytes()).hexdigest(),
               "x_f32": hashlib.sha256(x.tobytes()).hexdigest(),
               "q8": hashlib.sha256(q8.tobytes()).hexdigest()}
    out["cfg_4096x4096_b1/y64"] = ref["y64"]
    out["cfg_4096x4096_b1/l1"] = ref["l1"]
    for k, v in digests.items():
        out[f"cfg_4096x4096_b1/sha256_{k}"] = np.array(v)
    np.savez_compressed(os.path.join(HERE, "q4k_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "q4k_golden.npz"))


if __name__ == "__main__":
    main()
