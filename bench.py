"""Benchmark of the Q4_K GEMV op on one MI355X.

Headline workload: the Mistral-7B FFN gate/up projection, Q4_K weight
14336 x 4096 times one F32 activation column (batch 1) -- the shape the
metric is quoted on.  One step = one q4k_mul_mat_vec_q call through the C ABI
(F32 activation in, quantised to Q8_1 inside the launch, F32 out) on inputs
already resident in HBM.  The weight rotates through copies totalling more
than 1 GiB so every step streams it from HBM rather than from the 256 MB
Infinity Cache.

Timing: W untimed eager warm-up steps; the K timed steps are captured into one
HIP graph (the way ggml launches decode), which is replayed once untimed and
then once between two HIP events recorded on the stream the kernels run on.
value = algorithmic bytes per step / seconds per step (GB/s); the roofline
object prices the same bytes against the 8 TB/s HBM peak.  The CPU baseline is
the oracle's restatement of ggml's CPU path (Q8_K activations +
vec_dot_q4_K_q8_K, AVX2, a thread per core) timed on a bounded sample on the
host cores of the same machine.

--sweep prints one line per (workload, shape, ncols) of the five workloads
instead of the headline JSON; with --wtype q6_K, of the Q6_K tensors of a
Q4_K_M model (ffn_down, attn_v, output projection).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "Q4_K GEMV µs/call + achieved HBM GB/s (% of 8 TB/s), 14336x4096 b=1"
HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gemv_14336x4096_b1_traffic.txt")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


BLOCK_BYTES = {"q4_K": 144, "q6_K": 210}


def algorithmic_bytes(M: int, K: int, N: int, wtype: str = "q4_K") -> int:
    """Bytes the fused op must move: the quantised weight once, the F32
    activation once and the F32 result once."""
    return M * (K // 256) * BLOCK_BYTES[wtype] + 4 * N * K + 4 * M * N


def make_inputs(Q, M, K, N, seed=0, wtype="q4_K"):
    import _common
    W = _common.weights(M, K, seed)
    quant = Q.quantize_rows_q4_K if wtype == "q4_K" else Q.quantize_rows_q6_K
    wq = quant(W, nthreads=min(16, len(os.sched_getaffinity(0))))
    del W
    x = _common.activations(N, K, seed)
    return wq, x


class OpRunner:
    """Pre-resolved ctypes call of q4k_mul_mat_vec_q (q6k_mul_mat_vec_q for
    Q6_K) over rotating weights, with a Q8_1 workspace as ggml's pool would
    hand it (the op uses it for several long columns)."""

    def __init__(self, Q, wq, x, min_pool_bytes=1 << 30, wtype="q4_K"):
        import ctypes
        import torch
        self.Q = Q
        self.dev = torch.device("cuda:0")
        self.M, self.rb = wq.shape
        self.K = self.rb // BLOCK_BYTES[wtype] * 256
        self.N = x.shape[0]
        w0 = torch.from_numpy(wq).to(self.dev)
        self.ncopies = max(2, math.ceil(min_pool_bytes / wq.nbytes))
        self.copies = [w0] + [w0.clone() for _ in range(self.ncopies - 1)]
        self.x = torch.from_numpy(x).to(self.dev)
        self.out = torch.empty((self.N, self.M), dtype=torch.float32, device=self.dev)
        self.ws = torch.empty(Q.q8_1_bytes(self.K, self.N), dtype=torch.uint8, device=self.dev)
        self.name = "q4k_mul_mat_vec_q" if wtype == "q4_K" else "q6k_mul_mat_vec_q"
        self.fn = getattr(Q.lib(), self.name)
        self.wptr = [ctypes.c_void_p(c.data_ptr()) for c in self.copies]
        self.args = (self.K, self.M, self.rb, ctypes.c_void_p(self.x.data_ptr()), self.N, self.K * 4,
                     ctypes.c_void_p(self.out.data_ptr()), self.M * 4, ctypes.c_void_p(self.ws.data_ptr()),
                     self.ws.numel())
        self.i = 0

    def step(self, stream):
        st = self.fn(self.wptr[self.i % self.ncopies], *self.args, stream)
        self.i += 1
        if st != 0:
            raise self.Q.Q4KError(st, self.name)


class FusedRunner(OpRunner):
    """q4k_mul_mat_vec_q_fused with a gate weight and SWIGLU over rotating
    (weight, gate) pairs: one launch computes silu(gate . x) * (up . x)."""

    def __init__(self, Q, wq, gq, x, min_pool_bytes=1 << 30, wtype="q4_K", glu_op=2):
        import ctypes
        super().__init__(Q, wq, x, min_pool_bytes=min_pool_bytes // 2, wtype=wtype)
        import torch
        g0 = torch.from_numpy(gq).to(self.dev)
        self.gcopies = [g0] + [g0.clone() for _ in range(self.ncopies - 1)]
        self.fusions = [Q.q4k_fusion(None, ctypes.c_void_p(g.data_ptr()), None, glu_op) for g in self.gcopies]
        self.type_id = Q.GGML_TYPE_Q4_K if wtype == "q4_K" else Q.GGML_TYPE_Q6_K
        self.name = "q4k_mul_mat_vec_q_fused"
        self.fn = Q.lib().q4k_mul_mat_vec_q_fused
        self.fargs = (self.K, self.M, self.rb, ctypes.c_void_p(self.x.data_ptr()))
        self.outp = ctypes.c_void_p(self.out.data_ptr())

    def step(self, stream):
        import ctypes
        k = self.i % self.ncopies
        st = self.fn(self.type_id, self.wptr[k], *self.fargs, ctypes.byref(self.fusions[k]), self.outp, stream)
        self.i += 1
        if st != 0:
            raise self.Q.Q4KError(st, self.name)


def fused_sweep(args):
    """Gate+up with SWIGLU in one launch against the two plain launches, on
    the FFN shapes (batch 1, the only fused case)."""
    import _common
    import torch
    Q = _pkg()
    wt = args.wtype
    for M, K in ((14336, 4096), (4096, 4096), (28672, 8192)):
        wu, x = make_inputs(Q, M, K, 1, seed=0, wtype=wt)
        wg, _ = make_inputs(Q, M, K, 1, seed=1, wtype=wt)
        fr = FusedRunner(Q, wu, wg, x, wtype=wt)
        tf = time_gpu(fr, args.steps, args.warmup)["graph_s"]
        del fr
        torch.cuda.empty_cache()
        pr = OpRunner(Q, wu, x, wtype=wt)
        tp = time_gpu(pr, args.steps, args.warmup)["graph_s"]
        del pr
        torch.cuda.empty_cache()
        nbytes = 2 * M * (K // 256) * BLOCK_BYTES[wt] + 4 * K + 4 * M
        r = {"workload": "ffn_gate_up_swiglu_b1", "wtype": wt, "M": M, "K": K, "N": 1,
             "us_fused": round(tf * 1e6, 3), "us_two_plain": round(2 * tp * 1e6, 3),
             "GBps_fused": round(nbytes / tf / 1e9, 1), "hbm_frac": round(nbytes / tf / 1e9 / HBM_PEAK_GBS, 4)}
        print(json.dumps(r), flush=True)


class MoeRunner:
    """GGML_OP_MUL_MAT_ID for one token through q4k_ggml_mul_mat_vec_q:
    nexp expert matrices [nexp, M, K] (quantised), nused expert ids on the
    device, activation columns ne11 (1: shared, nused: one per slot),
    optionally the gate weight with SWIGLU fused.  The expert tensor rotates
    over copies totalling >= 1 GiB."""

    def __init__(self, Q, wq, nexp, M, K, ids, ne11, gq=None, wtype="q4_K", min_pool_bytes=1 << 30):
        import ctypes
        import _common
        import torch
        self.Q = Q
        dev = torch.device("cuda:0")
        gt = Q.GGML_TYPE_Q4_K if wtype == "q4_K" else Q.GGML_TYPE_Q6_K
        bb = BLOCK_BYTES[wtype]
        rb = K // 256 * bb
        per = wq.nbytes * (2 if gq is not None else 1)
        self.ncopies = max(2, math.ceil(min_pool_bytes / per))
        w0 = torch.from_numpy(wq).to(dev)
        self.w = [w0] + [w0.clone() for _ in range(self.ncopies - 1)]
        self.g = None
        if gq is not None:
            g0 = torch.from_numpy(gq).to(dev)
            self.g = [g0] + [g0.clone() for _ in range(self.ncopies - 1)]
        nused = len(ids)
        self.ids = torch.tensor(ids, dtype=torch.int32, device=dev)
        self.x = torch.from_numpy(_common.activations(ne11, K, 0)).to(dev)
        self.out = torch.empty((nused, M), dtype=torch.float32, device=dev)
        self.s0 = [Q.make_tensor(gt, [K, M, nexp], [bb, rb, rb * M], t.data_ptr()) for t in self.w]
        self.fus = []
        if self.g is not None:
            self.sg = [Q.make_tensor(gt, [K, M, nexp], [bb, rb, rb * M], t.data_ptr()) for t in self.g]
            self.fus = [Q.q4k_fusion_args(None, ctypes.pointer(t), None, 2) for t in self.sg]
        self.s1 = Q.make_tensor(0, [K, ne11, 1], [4, 4 * K, 4 * K * ne11], self.x.data_ptr())
        self.ti = Q.make_tensor(26, [nused, 1], [4, 4 * nused], self.ids.data_ptr())
        self.d = Q.make_tensor(0, [M, nused, 1], [4, 4 * M, 4 * M * nused], self.out.data_ptr())
        self.fn = Q.lib().q4k_ggml_mul_mat_vec_q
        self.i = 0

    def step(self, stream):
        import ctypes
        k = self.i % self.ncopies
        f = ctypes.byref(self.fus[k]) if self.fus else None
        st = self.fn(ctypes.byref(self.s0[k]), ctypes.byref(self.s1), ctypes.byref(self.ti), ctypes.byref(self.d),
                     f, None, 0, stream)
        self.i += 1
        if st != 0:
            raise self.Q.Q4KError(st, "q4k_ggml_mul_mat_vec_q (MUL_MAT_ID)")


# (name, experts, rows, K, ids, activation columns, weight type, fused gate)
MOE_CASES = [
    ("mixtral8x7b_ffn_gate_up_swiglu", 8, 14336, 4096, [2, 5], 1, "q4_K", True),
    ("mixtral8x7b_ffn_down", 8, 4096, 14336, [2, 5], 2, "q6_K", False),
    ("qwen3_30b_a3b_ffn_gate_up_swiglu", 128, 768, 2048, [3, 17, 40, 41, 77, 90, 100, 127], 1, "q4_K", True),
    ("qwen3_30b_a3b_ffn_down", 128, 2048, 768, [3, 17, 40, 41, 77, 90, 100, 127], 8, "q6_K", False),
]


def moe_sweep(args):
    import _common
    import torch
    Q = _pkg()
    for name, nexp, M, K, ids, ne11, wt, fused in MOE_CASES:
        quant = Q.quantize_rows_q4_K if wt == "q4_K" else Q.quantize_rows_q6_K
        nthr = min(16, len(os.sched_getaffinity(0)))
        wq = np.stack([quant(_common.weights(M, K, seed=e), nthreads=nthr) for e in range(nexp)])
        gq = np.stack([quant(_common.weights(M, K, seed=1000 + e), nthreads=nthr) for e in range(nexp)]) if fused else None
        r = MoeRunner(Q, wq, nexp, M, K, ids, ne11, gq=gq, wtype=wt)
        t = time_gpu(r, args.steps, args.warmup)["graph_s"]
        del r
        torch.cuda.empty_cache()
        nused = len(ids)
        nbytes = nused * M * (K // 256) * BLOCK_BYTES[wt] * (2 if fused else 1) + 4 * ne11 * K + 4 * M * nused
        print(json.dumps({"workload": name, "wtype": wt, "experts": nexp, "used": nused, "M": M, "K": K,
                          "ncols_y": ne11, "fused_swiglu": fused, "us_per_call": round(t * 1e6, 3),
                          "GBps": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}),
              flush=True)


def time_gpu(runner: OpRunner, steps: int, warmup: int):
    """Returns dict with graph-launched and eager seconds per step."""
    import ctypes
    import torch
    stream = torch.cuda.Stream()
    res = {}
    with torch.cuda.stream(stream):
        sp = ctypes.c_void_p(stream.cuda_stream)
        for _ in range(warmup):
            runner.step(sp)
        torch.cuda.synchronize()
        # eager: K back-to-back launches from the host
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            runner.step(sp)
        e1.record(stream)
        torch.cuda.synchronize()
        res["eager_s"] = e0.elapsed_time(e1) * 1e-3 / steps
        # graph: the same K calls captured once, replayed
        g = torch.cuda.CUDAGraph()
        runner.i = 0
        with torch.cuda.graph(g, stream=stream):
            for _ in range(steps):
                runner.step(sp)
        g.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        res["graph_s"] = e0.elapsed_time(e1) * 1e-3 / steps
    return res


def read_traffic():
    """HBM bytes per launch from the committed rocprofv3 PMC summary."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(wq, x, target_s=12.0):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    cores = min(16, len(os.sched_getaffinity(0)))
    K = wq.shape[1] // 144 * 256
    t1 = O.time_cpu_mul_mat_q4_K(wq, K, x, cores, 2)
    per = float(np.median(t1))
    reps = int(max(3, min(5000, target_s / max(per, 1e-6))))
    t = O.time_cpu_mul_mat_q4_K(wq, K, x, cores, reps)
    isa = "avx2" if O.lib().orc_cpu_has_avx2() else "scalar"
    med = float(np.median(t))
    M, N = wq.shape[0], x.shape[0]
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            model = next((ln.split(":", 1)[1].strip() for ln in fh if ln.startswith("model name")), model)
    except OSError:
        pass
    return {"value": algorithmic_bytes(M, K, N) / med / 1e9, "unit": "GB/s", "cores": cores,
            "kind": "port", "us_per_call": med * 1e6, "cpu_model": model, "isa": isa,
            "sample": f"{reps} calls of the full {M}x{K} N={N} product (Q8_K quantisation + "
                      f"vec_dot_q4_K_q8_K, {isa}, {cores} threads, row chunks of 16), "
                      f"{float(np.sum(t)):.1f} s total, median reported"}


def headline(args):
    import torch
    Q = _pkg()
    M, K, N = 14336, 4096, 1
    log(f"[bench] preparing {M}x{K} N={N} inputs")
    wq, x = make_inputs(Q, M, K, N)
    runner = OpRunner(Q, wq, x)
    log(f"[bench] {runner.ncopies} weight copies ({runner.ncopies * wq.nbytes / 2**30:.2f} GiB); "
        f"geometry {Q.geometry(K, M, N)}")
    torch.cuda.synchronize()
    t = time_gpu(runner, args.steps, args.warmup)
    sec = t["graph_s"]
    nbytes = algorithmic_bytes(M, K, N)
    achieved = nbytes / sec / 1e9
    log(f"[bench] graph {sec * 1e6:.2f} us/call ({achieved:.0f} GB/s), eager {t['eager_s'] * 1e6:.2f} us/call")
    rec = {
        "metric": METRIC, "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": sec * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_K x q8_1: int8 dot4 -> int32, f32 scale/accumulate",
        "data": "synthetic: W ~ N(0,0.02) -> Q4_K (quantize_row_q4_K_ref arithmetic), x ~ N(0,1); seed 0",
        "config": {"workload": "mistral7b_ffn_gate_14336x4096_b1", "M": M, "K": K, "ncols": N,
                   "launch": "hipGraph of the K timed calls", "weight_copies": runner.ncopies,
                   "geometry": Q.geometry(K, M, N)},
        "us_per_call": round(sec * 1e6, 3),
        "us_per_call_eager": round(t["eager_s"] * 1e6, 3),
        "hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": read_traffic(), "algorithmic_bytes_per_launch": nbytes},
    }
    if not args.no_cpu:
        log("[bench] CPU baseline (bounded sample)")
        rec["cpu_baseline"] = cpu_baseline(wq, x)
    print(json.dumps(rec), flush=True)


def sweep(args):
    import _common
    import torch
    Q = _pkg()
    rows = []
    seen = set()
    wt = args.wtype
    gtype = Q.GGML_TYPE_Q4_K if wt == "q4_K" else Q.GGML_TYPE_Q6_K
    table = _common.WORKLOADS if wt == "q4_K" else _common.Q6K_WORKLOADS
    for wl, items in table.items():
        for M, K, ns in items:
            wq = None
            for N in ns:
                if (M, K, N) in seen:
                    continue
                seen.add((M, K, N))
                if wq is None:
                    log(f"[sweep] inputs {wt} {M}x{K}")
                    wq, _ = make_inputs(Q, M, K, 1, wtype=wt)
                x = _common.activations(N, K, 0)
                runner = OpRunner(Q, wq, x, wtype=wt)
                t = time_gpu(runner, args.steps, args.warmup)
                sec = t["graph_s"]
                gbs = algorithmic_bytes(M, K, N, wt) / sec / 1e9
                r = {"workload": wl, "wtype": wt, "M": M, "K": K, "N": N, "us_per_call": round(sec * 1e6, 3),
                     "us_eager": round(t["eager_s"] * 1e6, 3), "GBps": round(gbs, 1),
                     "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "geometry": Q.geometry(K, M, N, gtype)}
                rows.append(r)
                print(json.dumps(r), flush=True)
                del runner
                torch.cuda.empty_cache()


def profile_mode(args):
    """Only the GEMV launches of the headline workload (for rocprofv3)."""
    import ctypes
    import torch
    Q = _pkg()
    M, K, N = args.shape
    wq, x = make_inputs(Q, M, K, N, wtype=args.wtype)
    if args.fused:  # gate + up with SWIGLU in one launch (one column)
        gq, _ = make_inputs(Q, M, K, 1, seed=1, wtype=args.wtype)
        runner = FusedRunner(Q, wq, gq, x[:1], wtype=args.wtype)
    else:
        runner = OpRunner(Q, wq, x, wtype=args.wtype)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(args.warmup + args.steps):
        runner.step(s)
    torch.cuda.synchronize()
    log(f"[profile] {args.warmup + args.steps} launches of {M}x{K} N={N} done")


def copy_calibration(args):
    """A plain device copy of known size (read N bytes, write N bytes) whose
    FETCH_SIZE / WRITE_SIZE readings calibrate the GEMV's counter values."""
    import torch
    n = args.copy_cal // 4
    src = torch.randn(n, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(args.warmup + args.steps):
        torch.add(src, 0.0, out=dst)
    torch.cuda.synchronize()
    log(f"[copy-cal] {args.warmup + args.steps} elementwise copies of {n * 4} bytes done")


def _pkg():
    import _common
    return _common.pkg()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--profile", action="store_true", help="plain launches only, for rocprofv3")
    ap.add_argument("--shape", type=int, nargs=3, default=[14336, 4096, 1], metavar=("M", "K", "N"))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--moe", action="store_true",
                    help="time MUL_MAT_ID (one token) on expert-FFN shapes")
    ap.add_argument("--fused", action="store_true",
                    help="time the gate+up SWIGLU launch against two plain launches")
    ap.add_argument("--wtype", choices=sorted(BLOCK_BYTES), default="q4_K",
                    help="weight format of --sweep and --profile (the headline is Q4_K)")
    ap.add_argument("--copy-cal", type=int, default=0, metavar="BYTES",
                    help="run only a plain device copy of BYTES (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the Q4_K GEMV has no multi-GPU path here "
              "(rows would shard across GPUs through q4k_op_mul_mat_vec_q); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.copy_cal:
        copy_calibration(args)
    elif args.profile:
        profile_mode(args)
    elif args.fused:
        fused_sweep(args)
    elif args.moe:
        moe_sweep(args)
    elif args.sweep:
        sweep(args)
    else:
        headline(args)


if __name__ == "__main__":
    main()
