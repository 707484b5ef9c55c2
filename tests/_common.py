"""Shared helpers of the test suite: loaders for the product binding and the
oracle, seeded synthetic inputs and the workload table."""
from __future__ import annotations

import importlib.util
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "gemv-q4_k-optimization_amd")
ORACLE_DIR = os.path.join(ROOT, "oracle")
GOLDEN_DIR = os.path.join(ROOT, "tests", "golden")

# (name, M rows, K columns, list of ncols) -- the five workloads
MISTRAL_SHAPES = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                  ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
WORKLOADS = {
    "single_4096x4096": [(4096, 4096, [1])],
    "mistral_layer_b1": [(m, k, [1]) for _, m, k in MISTRAL_SHAPES],
    "mistral_layer_batch": [(m, k, [1, 2, 3, 4, 8]) for _, m, k in MISTRAL_SHAPES],
    "llama70b_ffn": [(28672, 8192, [1, 4]), (8192, 28672, [1, 4])],
    "lm_head_128256": [(128256, 4096, [1, 8])],
}

# Q6_K tensors of a Q4_K_M Mistral-7B (v0.3 vocabulary) / Llama-3-8B:
# ffn_down and attn_v of half the layers, and the output projection
Q6K_WORKLOADS = {
    "q4km_q6k_tensors": [(4096, 14336, [1, 2, 4, 8]), (1024, 4096, [1, 4, 8]), (32768, 4096, [1, 8]),
                         (128256, 4096, [1, 8])],
}

STREAM_W, STREAM_X = 1, 2


def pkg():
    name = "q4k_amd"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def oracle():
    if ORACLE_DIR not in sys.path:
        sys.path.insert(0, ORACLE_DIR)
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    return O


def weights(M: int, K: int, seed: int = 0) -> np.ndarray:
    """F32 [M, K] ~ N(0, 0.02): numpy PCG64 stream (seed, 1)."""
    rng = np.random.default_rng([seed, STREAM_W])
    return rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.02)


def activations(N: int, K: int, seed: int = 0) -> np.ndarray:
    """F32 [N, K] ~ N(0, 1): numpy PCG64 stream (seed, 2); row c is column c
    of ggml's src1."""
    rng = np.random.default_rng([seed, STREAM_X])
    return rng.standard_normal((N, K), dtype=np.float32)


def assert_within_tolerance(O, y, ref, where=""):
    """y (float32 [N, M]) against the oracle's f64 result within the parity
    tolerance.  Returns a dict: n outputs; max_ratio = max |err| / tol;
    strict_fail = outputs outside the strict bar (1e-5 relative or 4 ulp of
    the result), i.e. those inside the tolerance only through its
    cancellation term (8 f32 epsilons of the row's sum of |term|);
    max_cancel_ulps = the largest |err| among those in units of
    eps32 * sum |term|."""
    y = np.asarray(y, dtype=np.float64)
    tol = O.parity_tolerance(ref["y64"], ref["l1"])
    err = np.abs(y - ref["y64"])
    bad = err > tol
    if bad.any():
        idx = np.argwhere(bad)[:5]
        details = [(tuple(i), float(y[tuple(i)]), float(ref["y64"][tuple(i)]), float(tol[tuple(i)])) for i in idx]
        raise AssertionError(f"{where}: {int(bad.sum())} outputs outside tolerance, e.g. {details}")
    strict_tol = np.maximum(1e-5 * np.abs(ref["y64"]),
                            4.0 * np.spacing(np.abs(ref["y64"]).astype(np.float32)).astype(np.float64))
    loose = err > strict_tol
    eps_l1 = np.finfo(np.float32).eps * np.asarray(ref["l1"], np.float64)
    cancel = float((err[loose] / eps_l1[loose]).max()) if loose.any() else 0.0
    return {"n": int(err.size), "max_ratio": float((err / tol).max()), "strict_fail": int(loose.sum()),
            "max_cancel_ulps": cancel}
