"""Benchmark of the Q4_K GEMV op on one MI355X.

Headline workload: the Mistral-7B FFN gate/up projection, Q4_K weight
14336 x 4096 times one F32 activation column (batch 1) -- the shape the
metric is quoted on.  One step = one q4k_mul_mat_vec_q call through the C ABI
(F32 activation in, quantised to Q8_1 inside the launch, F32 out) on inputs
already resident in HBM.  The weight rotates through copies totalling more
than 1 GiB so every step streams it from HBM rather than from the 256 MB
Infinity Cache.

Timing: W untimed eager warm-up steps; then exactly K calls per trial, timed
with HIP events on the stream the kernels run on, queued behind untimed
replays of a graph of K calls: the host launches the K timed calls while the
GPU is still busy with the replays, so when the host has finished submitting
before the GPU finishes the replays (checked every trial) no timed call
waits for the host and the window holds GPU time only.  A graph launch adds
a one-off cost of ~9 us on this device (0.45 us per call at K = 20), which
this keeps out of the window.  If any trial fails the check, the figure is a
timed replay of the K-call graph itself, queued behind an untimed replay.
value is the median over the trials (min and max reported), the graph figure
is reported beside it.  value = algorithmic bytes per step / seconds per
step (GB/s); the roofline object prices the same bytes against the 8 TB/s
HBM peak, and its
traffic is the HBM bytes rocprofv3 counted for the same launch
(profiles/q4k_traffic_all_configs.txt).  The CPU baseline is the oracle's
restatement of ggml's CPU path (Q8_K activations + vec_dot_q4_K_q8_K or
vec_dot_q6_K_q8_K, AVX2) on pinned threads of this machine, timed on a bounded
sample.

Modes:
  (default)         the headline JSON line
  --sweep           one JSON line per (shape, ncols) of the five workloads
                    (--wtype q6_K: the Q6_K tensors of a Q4_K_M model), each
                    with the roofline fraction, the measured traffic and a
                    CPU baseline with and without Q8_K quantisation
  --fused, --moe    the fused gate/up launch and MUL_MAT_ID workloads
  --read-ceiling    a plain read of the headline weight's bytes (the GEMV's
                    ceiling) in several launch shapes, and the headline GEMV
  --profile         plain eager launches of one shape (for rocprofv3)
  --profile-sweep   plain eager launches of every sweep config in order, each
                    preceded by a one-block quantiser launch that marks where
                    it starts, after a device copy of known size (the counter
                    calibration); --summarize reads the rocprofv3 output of
                    such a run and prints the per-config tables
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))

METRIC = "Q4_K GEMV µs/call + achieved HBM GB/s (% of 8 TB/s), 14336x4096 b=1"
HBM_PEAK_GBS = 8000.0
PROFILES = os.path.join(ROOT, "profiles")
CPU_SHARE = 16  # CPUs a one-GPU box grants a job
CAL_BYTES = 256 << 20  # the calibration copy of --profile-sweep


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
    wq = quant(W, nthreads=min(CPU_SHARE, len(os.sched_getaffinity(0))))
    del W
    x = _common.activations(N, K, seed)
    return wq, x


def sweep_configs(wtype: str, only=None):
    """(workload, M, K, N) of the sweep, each (M, K, N) once, in table order;
    `only`: a list of "MxKxN" strings to keep."""
    import _common
    table = _common.WORKLOADS if wtype == "q4_K" else _common.Q6K_WORKLOADS
    keep = {tuple(int(v) for v in o.split("x")) for o in only} if only else None
    out, seen = [], set()
    for wl, items in table.items():
        for M, K, ns in items:
            for N in ns:
                if (M, K, N) not in seen and (keep is None or (M, K, N) in keep):
                    seen.add((M, K, N))
                    out.append((wl, M, K, N))
    return out


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
    import torch
    Q = _pkg()
    wt = args.wtype
    for M, K in ((14336, 4096), (4096, 4096), (28672, 8192)):
        wu, x = make_inputs(Q, M, K, 1, seed=0, wtype=wt)
        wg, _ = make_inputs(Q, M, K, 1, seed=1, wtype=wt)
        fr = FusedRunner(Q, wu, wg, x, wtype=wt)
        tf = time_gpu(fr, args.steps, args.warmup, args.trials)["s"]
        del fr
        torch.cuda.empty_cache()
        pr = OpRunner(Q, wu, x, wtype=wt)
        tp = time_gpu(pr, args.steps, args.warmup, args.trials)["s"]
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
        nthr = min(CPU_SHARE, len(os.sched_getaffinity(0)))
        wq = np.stack([quant(_common.weights(M, K, seed=e), nthreads=nthr) for e in range(nexp)])
        gq = np.stack([quant(_common.weights(M, K, seed=1000 + e), nthreads=nthr) for e in range(nexp)]) if fused else None
        r = MoeRunner(Q, wq, nexp, M, K, ids, ne11, gq=gq, wtype=wt)
        t = time_gpu(r, args.steps, args.warmup, args.trials)["s"]
        del r
        torch.cuda.empty_cache()
        nused = len(ids)
        nbytes = nused * M * (K // 256) * BLOCK_BYTES[wt] * (2 if fused else 1) + 4 * ne11 * K + 4 * M * nused
        print(json.dumps({"workload": name, "wtype": wt, "experts": nexp, "used": nused, "M": M, "K": K,
                          "ncols_y": ne11, "fused_swiglu": fused, "us_per_call": round(t * 1e6, 3),
                          "GBps": round(nbytes / t / 1e9, 1), "hbm_frac": round(nbytes / t / 1e9 / HBM_PEAK_GBS, 4)}),
              flush=True)


def time_gpu(runner, steps: int, warmup: int, trials: int = 7):
    """Seconds per step of exactly `steps` calls, two ways, on the stream the
    kernels run on (HIP events):
      queued: the K calls launched eagerly, queued behind untimed replays of
              a K-call graph that keep the GPU busy while the host submits
              them.  A trial is valid when the host finished submitting
              before the GPU finished those replays, i.e. no timed call
              waited for the host; then the window holds GPU time only.
      graph:  one replay of the K-call graph, queued behind an untimed
              replay (a graph launch adds a one-off cost of ~9 us on this
              device, ~0.45 us per call at K = 20).
    s / min_s / max_s: the queued figures (median over trials) when every
    trial was valid, else the graph figures; method names which.  eager_s:
    K eager calls with nothing queued ahead (host-bound when a call takes
    the host longer than the GPU)."""
    import ctypes
    import time
    import torch
    stream = torch.cuda.Stream()
    res = {}
    with torch.cuda.stream(stream):
        sp = ctypes.c_void_p(stream.cuda_stream)
        for _ in range(warmup):
            runner.step(sp)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            runner.step(sp)
        e1.record(stream)
        host_s = time.perf_counter() - t0
        torch.cuda.synchronize()
        res["eager_s"] = e0.elapsed_time(e1) * 1e-3 / steps
        g = torch.cuda.CUDAGraph()
        runner.i = 0
        with torch.cuda.graph(g, stream=stream):
            for _ in range(steps):
                runner.step(sp)
        g.replay()
        torch.cuda.synchronize()
        per = []
        for _ in range(trials):
            torch.cuda.synchronize()
            g.replay()            # untimed: keeps the GPU busy while the timed replay is queued
            e0.record(stream)
            g.replay()            # timed: exactly `steps` calls
            e1.record(stream)
            torch.cuda.synchronize()
            per.append(e0.elapsed_time(e1) * 1e-3 / steps)
        res["graph_s"] = float(np.median(per))
        res["graph_min_s"] = float(min(per))
        res["graph_max_s"] = float(max(per))
        # enough untimed replays ahead that the host (host_s per K calls)
        # stays ahead of the GPU with margin
        heads = int(min(16, max(2, math.ceil(2.0 * host_s / (steps * res["graph_s"])))))
        qper, valid = [], True
        for _ in range(trials):
            torch.cuda.synchronize()
            h0 = torch.cuda.Event(enable_timing=True)
            h0.record(stream)
            for _ in range(heads):
                g.replay()        # untimed head start
            t0 = time.perf_counter()
            e0.record(stream)
            for _ in range(steps):
                runner.step(sp)   # timed: exactly `steps` calls
            e1.record(stream)
            submit_s = time.perf_counter() - t0
            torch.cuda.synchronize()
            head_s = h0.elapsed_time(e0) * 1e-3
            valid = valid and submit_s < head_s
            qper.append(e0.elapsed_time(e1) * 1e-3 / steps)
        res["queued_s"] = float(np.median(qper))
        res["queued_min_s"] = float(min(qper))
        res["queued_max_s"] = float(max(qper))
        res["queued_valid"] = valid
        res["head_replays"] = heads
        res["trials"] = trials
        key = "queued" if valid else "graph"
        res["method"] = key
        res["s"], res["min_s"], res["max_s"] = res[f"{key}_s"], res[f"{key}_min_s"], res[f"{key}_max_s"]
    return res


def traffic_file(wtype: str) -> str:
    return os.path.join(PROFILES, f"{wtype.replace('_', '').lower()}_traffic_all_configs.txt")


def read_traffic(M: int, K: int, N: int, wtype: str = "q4_K"):
    """HBM bytes per launch of the GEMV kernel (and of the whole op) for one
    config, from the committed rocprofv3 counter summary: (kernel, op) or
    (None, None) when the config is not in it."""
    path = traffic_file(wtype)
    if not os.path.exists(path):
        return None, None
    key = f"traffic M={M} K={K} N={N} "
    for line in open(path):
        if line.startswith(key):
            kv = dict(f.split("=") for f in line.split()[1:])
            return int(kv["gemv_bytes"]), int(kv["op_bytes"])
    return None, None


def cpu_baseline(wq, x, target_s=12.0, min_reps=10, wtype="q4_K"):
    """ggml's CPU path (restated in the oracle) on this machine: Q8_K
    quantisation of x + vec_dot_q4_K_q8_K (vec_dot_q6_K_q8_K for Q6_K) per
    (row, column), AVX2, one thread per CPU of the job's share, each pinned.
    Median of >= min_reps calls with quantisation and without (Q8_K
    activation prepared beforehand)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O
    if not os.path.exists(O.LIB_PATH):
        O.build()
    cpus = sorted(os.sched_getaffinity(0))[:CPU_SHARE]
    cores = len(cpus)
    O.set_pin_cpus(cpus)
    K = wq.shape[1] // BLOCK_BYTES[wtype] * 256
    M, N = wq.shape[0], x.shape[0]
    out = {}
    for mode, quant in (("with_q8K", True), ("without_q8K", False)):
        t1 = O.time_cpu_mul_mat_q4_K(wq, K, x, cores, 2, quantize=quant, wtype=wtype)
        per = float(np.median(t1))
        reps = int(max(min_reps, min(5000, target_s / 2 / max(per, 1e-6))))
        t = O.time_cpu_mul_mat_q4_K(wq, K, x, cores, reps, quantize=quant, wtype=wtype)
        out[mode] = (float(np.median(t)), reps, float(np.sum(t)))
    O.set_pin_cpus([])
    isa = "avx2" if O.lib().orc_cpu_has_avx2() else "scalar"
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            model = next((ln.split(":", 1)[1].strip() for ln in fh if ln.startswith("model name")), model)
    except OSError:
        pass
    med, reps, tot = out["with_q8K"]
    med_nq, reps_nq, tot_nq = out["without_q8K"]
    nbytes = algorithmic_bytes(M, K, N, wtype)
    return {"value": round(nbytes / med / 1e9, 2), "unit": "GB/s", "cores": cores, "kind": "port",
            "us_per_call": round(med * 1e6, 1), "us_per_call_without_q8K": round(med_nq * 1e6, 1),
            "GBps_without_q8K": round(nbytes / med_nq / 1e9, 2), "cpu_model": model, "isa": isa,
            "host_cpus": os.cpu_count(), "pinned_cpus": f"{cpus[0]}..{cpus[-1]}" if cpus else "",
            "label": "ggml-equivalent restatement (ggml itself is not available offline)",
            "sample": f"{reps} calls of the full {M}x{K} N={N} product with Q8_K quantisation of x "
                      f"({tot:.1f} s) and {reps_nq} without ({tot_nq:.1f} s): vec_dot_{wtype}_q8_K ({isa}), "
                      f"{cores} threads pinned one per CPU (the job's CPU share of this {os.cpu_count()}-CPU "
                      f"host), ggml's row chunks of 16; medians"}


class ReadRunner:
    """One q4k_read_probe call (a plain streaming read, the GEMV's ceiling)
    over rotating copies of an nbytes buffer totalling >= 1 GiB."""

    def __init__(self, Q, nbytes, wgs, waves, per_wave, infl, min_pool_bytes=1 << 30):
        import ctypes
        import torch
        dev = torch.device("cuda:0")
        self.Q = Q
        self.ncopies = max(2, math.ceil(min_pool_bytes / nbytes))
        b0 = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
        self.copies = [b0] + [b0.clone() for _ in range(self.ncopies - 1)]
        self.sink = torch.empty(wgs * waves, dtype=torch.int32, device=dev)
        self.ptrs = [ctypes.c_void_p(c.data_ptr()) for c in self.copies]
        self.args = (nbytes, wgs, waves, per_wave, infl, ctypes.c_void_p(self.sink.data_ptr()))
        self.fn = Q.lib().q4k_read_probe
        self.i = 0

    def step(self, stream):
        st = self.fn(self.ptrs[self.i % self.ncopies], *self.args, stream)
        self.i += 1
        if st != 0:
            raise self.Q.Q4KError(st, "q4k_read_probe")


# (workgroups, waves per workgroup, 1-KB loads in flight per wave)
READ_SHAPES = [(2016, 4, 4), (2016, 4, 2), (1008, 4, 4), (4032, 4, 2), (1024, 8, 4), (512, 8, 4),
               (512, 16, 2), (256, 16, 8), (256, 16, 4), (256, 16, 2), (256, 16, 1),
               (256, 8, 2), (256, 8, 1), (256, 4, 2), (256, 4, 1)]


def read_ceiling(args):
    """A plain read of a weight's bytes (--shape M K, --wtype; default the
    headline 14336 x 4096 Q4_K: 33,030,144 B) in several launch shapes, timed
    like the headline, against that product's GEMV (one column) in the same
    process.  Shapes whose waves would read more than 1.5 times the bytes
    (the probe reads zeros past the end) are skipped."""
    import torch
    Q = _pkg()
    M, K = args.shape[0], args.shape[1]
    wt = args.wtype
    nbytes = M * (K // 256) * BLOCK_BYTES[wt]
    for wgs, waves, infl in READ_SHAPES:
        per_wave = math.ceil(nbytes / (wgs * waves) / 1024) * 1024
        if per_wave * wgs * waves > 1.5 * nbytes:
            continue
        r = ReadRunner(Q, nbytes, wgs, waves, per_wave, infl)
        t = time_gpu(r, args.steps, args.warmup, args.trials)
        del r
        torch.cuda.empty_cache()
        print(json.dumps({"kernel": "read_probe", "bytes": nbytes, "workgroups": wgs, "waves_per_wg": waves,
                          "bytes_per_wave": per_wave, "loads_in_flight": infl, "us_per_call": round(t["s"] * 1e6, 3),
                          "us_min": round(t["min_s"] * 1e6, 3), "method": t["method"],
                          "GBps": round(nbytes / t["s"] / 1e9, 1),
                          "hbm_frac": round(nbytes / t["s"] / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)
    wq, x = make_inputs(Q, M, K, 1, wtype=wt)
    r = OpRunner(Q, wq, x, wtype=wt)
    t = time_gpu(r, args.steps, args.warmup, args.trials)
    nb = algorithmic_bytes(M, K, 1, wt)
    gt = Q.GGML_TYPE_Q4_K if wt == "q4_K" else Q.GGML_TYPE_Q6_K
    print(json.dumps({"kernel": f"{wt.replace('_', '').lower()}_mul_mat_vec_q", "bytes": nb,
                      "geometry": Q.geometry(K, M, 1, gt),
                      "us_per_call": round(t["s"] * 1e6, 3), "us_min": round(t["min_s"] * 1e6, 3),
                      "method": t["method"], "GBps": round(nb / t["s"] / 1e9, 1),
                      "hbm_frac": round(nb / t["s"] / 1e9 / HBM_PEAK_GBS, 4)}), flush=True)


def launch_text(t) -> str:
    if t["method"] == "queued":
        return (f"the K timed calls launched back to back behind {t['head_replays']} untimed replays of a K-call "
                f"graph (every call queued before the GPU reached it), median of {t['trials']} trials")
    return f"hipGraph of the K timed calls, median of {t['trials']} timed replays"


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
    t = time_gpu(runner, args.steps, args.warmup, args.trials)
    sec = t["s"]
    nbytes = algorithmic_bytes(M, K, N)
    achieved = nbytes / sec / 1e9
    log(f"[bench] {t['method']} {sec * 1e6:.3f} us/call median of {t['trials']} (min {t['min_s'] * 1e6:.3f}, "
        f"max {t['max_s'] * 1e6:.3f}), {achieved:.0f} GB/s; queued {t['queued_s'] * 1e6:.3f} "
        f"(valid {t['queued_valid']}, {t['head_replays']} replays ahead), graph {t['graph_s'] * 1e6:.3f}, "
        f"eager alone {t['eager_s'] * 1e6:.2f} us/call")
    traffic, _ = read_traffic(M, K, N)
    rec = {
        "metric": METRIC, "value": round(achieved, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": sec * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_K x q8_1: int8 dot4 -> int32, f32 scale/accumulate",
        "data": "synthetic: W ~ N(0,0.02) -> Q4_K (quantize_row_q4_K_ref arithmetic), x ~ N(0,1); "
                "seed 0, numpy PCG64 streams (0, 1) for W and (0, 2) for x",
        "config": {"workload": "mistral7b_ffn_gate_14336x4096_b1", "M": M, "K": K, "ncols": N,
                   "launch": launch_text(t),
                   "weight_copies": runner.ncopies, "geometry": Q.geometry(K, M, N)},
        "us_per_call": round(sec * 1e6, 3),
        "us_per_call_min": round(t["min_s"] * 1e6, 3),
        "us_per_call_max": round(t["max_s"] * 1e6, 3),
        "us_per_call_graph": round(t["graph_s"] * 1e6, 3),
        "us_per_call_eager": round(t["eager_s"] * 1e6, 3),
        "hbm_frac": round(achieved / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "algorithmic_bytes_per_launch": nbytes},
    }
    if not args.no_cpu:
        log("[bench] CPU baseline (bounded sample)")
        rec["cpu_baseline"] = cpu_baseline(wq, x)
    print(json.dumps(rec), flush=True)


def sweep(args):
    import _common
    import torch
    Q = _pkg()
    wt = args.wtype
    gtype = Q.GGML_TYPE_Q4_K if wt == "q4_K" else Q.GGML_TYPE_Q6_K
    wq_cache = {}
    for wl, M, K, N in sweep_configs(wt, args.only):
        if (M, K) not in wq_cache:
            wq_cache.clear()
            log(f"[sweep] inputs {wt} {M}x{K}")
            wq_cache[(M, K)], _ = make_inputs(Q, M, K, 1, wtype=wt)
        wq = wq_cache[(M, K)]
        x = _common.activations(N, K, 0)
        runner = OpRunner(Q, wq, x, wtype=wt)
        t = time_gpu(runner, args.steps, args.warmup, args.trials)
        del runner
        torch.cuda.empty_cache()
        sec = t["s"]
        nbytes = algorithmic_bytes(M, K, N, wt)
        gbs = nbytes / sec / 1e9
        traffic, op_traffic = read_traffic(M, K, N, wt)
        r = {"workload": wl, "wtype": wt, "M": M, "K": K, "N": N, "us_per_call": round(sec * 1e6, 3),
             "us_min": round(t["min_s"] * 1e6, 3), "us_max": round(t["max_s"] * 1e6, 3),
             "trials": t["trials"], "method": t["method"], "us_graph": round(t["graph_s"] * 1e6, 3),
             "us_eager": round(t["eager_s"] * 1e6, 3), "GBps": round(gbs, 1),
             "hbm_frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": nbytes,
             "traffic_gemv_bytes": traffic, "traffic_op_bytes": op_traffic,
             "traffic_ratio": round(op_traffic / nbytes, 4) if op_traffic else None,
             "geometry": Q.geometry(K, M, N, gtype)}
        if not args.no_cpu:
            r["cpu_baseline"] = cpu_baseline(wq, x, target_s=args.cpu_seconds, min_reps=10, wtype=wt)
        print(json.dumps(r), flush=True)


def _launch_steps(runner, s, args):
    """warmup eager op launches, then `steps` more: eager, or (--graph)
    captured into a HIP graph and replayed once, as the timed steps of the
    benchmark run."""
    import torch
    for _ in range(args.warmup):
        runner.step(s)
    if not args.graph:
        for _ in range(args.steps):
            runner.step(s)
        return
    import ctypes
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        sp = ctypes.c_void_p(stream.cuda_stream)
        for _ in range(args.steps):
            runner.step(sp)
    g.replay()
    torch.cuda.synchronize()


def profile_mode(args):
    """Only the op launches of one shape (for rocprofv3)."""
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
    _launch_steps(runner, s, args)
    torch.cuda.synchronize()
    log(f"[profile] {args.warmup + args.steps} launches of {M}x{K} N={N} done"
        f"{' (timed steps as one graph replay)' if args.graph else ''}")


def _separator(Q, buf_x, buf_y):
    """A one-block quantiser launch (32 values): the segment marker of
    --profile-sweep (the configs' own quantiser launches have >= 4 blocks)."""
    Q._check(Q.lib().q4k_quantize_row_q8_1(Q._ptr(buf_x), Q._ptr(buf_y), 32, 32, 32, 1, Q._stream()), "separator")


def profile_sweep(args):
    """Plain eager launches of every sweep config, for rocprofv3: first a
    device copy of CAL_BYTES (counter calibration), then per config a
    separator launch followed by warmup + steps op launches."""
    import ctypes
    import _common
    import torch
    Q = _pkg()
    wt = args.wtype
    dev = torch.device("cuda:0")
    src = torch.randn(CAL_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.add(src, 0.0, out=dst)
    del src, dst
    sx = torch.zeros(32, device=dev)
    sy = torch.empty(36, dtype=torch.uint8, device=dev)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    wq = None
    for wl, M, K, N in sweep_configs(wt, args.only):
        if wq is None or wq.shape[0] != M or wq.shape[1] != K // 256 * BLOCK_BYTES[wt]:
            wq, _ = make_inputs(Q, M, K, 1, wtype=wt)
        runner = OpRunner(Q, wq, _common.activations(N, K, 0), wtype=wt, min_pool_bytes=args.pool_bytes)
        torch.cuda.synchronize()
        _separator(Q, sx, sy)
        _launch_steps(runner, s, args)
        torch.cuda.synchronize()
        del runner
        torch.cuda.empty_cache()
        log(f"[profile-sweep] {wl} {wt} {M}x{K} N={N}: {args.warmup + args.steps} launches")


def _rows(path):
    with open(path, newline="") as fh:
        return list(csv.DictReader(fh))


def _grid_threads(r):
    if "Grid_Size" in r:
        return int(r["Grid_Size"])
    return int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])


def _segments(rows, value_of):
    """Dispatches in order, split at the separator launches: [calibration
    segment, config 1, config 2, ...]; each a list of (kernel name, value)."""
    rows = sorted(rows, key=lambda r: int(r["Dispatch_Id"]))
    segs = [[]]
    for r in rows:
        name = r["Kernel_Name"]
        if "quantize_q8_1_kernel" in name and _grid_threads(r) == 256:
            segs.append([])
            continue
        if "copyBuffer" in name:  # weight copies of the runner set-up
            continue
        segs[-1].append((name, value_of(r)))
    return segs


def _short(name):
    base = name.split("(")[0]
    return base.replace("void ", "")


def _per_kernel(seg, warmup, steps):
    """{kernel: (launches per op, values of its dispatches in the timed
    launches)} for a config segment of warmup + steps op launches (a kernel
    launched n times per op keeps its last n * steps values)."""
    by = {}
    for name, v in seg:
        if "q4k::" in name:  # the library's kernels (not torch's graph-replay fill)
            by.setdefault(name, []).append(v)
    out = {}
    for name, vals in by.items():
        n = max(1, len(vals) // (warmup + steps))
        out[name] = (n, vals[-n * steps:])
    return out


SQ_NEEDED = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_INSTS_SALU", "SQ_INSTS_LDS", "SQ_INSTS_VMEM_RD", "SQ_INSTS_MFMA",
             "SQ_WAVE_CYCLES", "SQ_BUSY_CYCLES", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS", "SQ_WAIT_INST_ANY",
             "SQ_WAIT_ANY", "SQ_LDS_BANK_CONFLICT")


def _sq_table(sq):
    """Derived SQ columns per (config, kernel) with both counter sets:
    row group = one row's 16-block group (M x ceil(K/4096) per product);
    VALU busy = SQ_ACTIVE_INST_VALU x 4 cycles / 1024 SIMDs over
    SQ_BUSY_CYCLES / 32 shader engines; dependency wait = SQ_WAIT_ANY /
    SQ_WAVE_CYCLES (waves waiting at s_waitcnt or a barrier); issue wait =
    SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (waves with an instruction ready but
    not issued); wave life = SQ_WAVE_CYCLES / SQ_WAVES."""
    rows = [(key, c) for key, c in sq.items() if all(n in c for n in SQ_NEEDED)]
    if not rows:
        return
    print("| shape | N | kernel | waves | VALU instr | VALU / row group | VALU / row group / column | "
          "LDS instr / row group | VALU busy % | dependency wait % | issue wait % | wave life (SQ_WAVE_CYCLES "
          "/ wave) | LDS bank-conflict cycles / LDS active cycles | SALU instr | VMEM rd instr | MFMA instr |")
    print("|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|---|")
    for (M, K, N, k), c in rows:
        groups = M * ((K // 256 + 15) // 16)
        busy = 100 * c["SQ_ACTIVE_INST_VALU"] * 4 / 1024 / (c["SQ_BUSY_CYCLES"] / 32)
        print(f"| {M}x{K} | {N} | `{k}` | {c['SQ_WAVES']:,.0f} | {c['SQ_INSTS_VALU']:,.0f} | "
              f"{c['SQ_INSTS_VALU'] / groups:.0f} | {c['SQ_INSTS_VALU'] / groups / N:.0f} | "
              f"{c['SQ_INSTS_LDS'] / groups:.1f} | {busy:.0f} | {100 * c['SQ_WAIT_ANY'] / c['SQ_WAVE_CYCLES']:.1f} | "
              f"{100 * c['SQ_WAIT_INST_ANY'] / c['SQ_WAVE_CYCLES']:.1f} | {c['SQ_WAVE_CYCLES'] / c['SQ_WAVES']:,.0f} | "
              f"{c['SQ_LDS_BANK_CONFLICT'] / max(c['SQ_ACTIVE_INST_LDS'], 1):.2f} | {c['SQ_INSTS_SALU']:,.0f} | "
              f"{c['SQ_INSTS_VMEM_RD']:,.0f} | {c['SQ_INSTS_MFMA']:,.0f} |")


def summarize(args):
    """Per-config tables from the rocprofv3 output of a --profile-sweep run:
    kernel durations (--kernel-trace) or HBM bytes (--pmc FETCH_SIZE /
    WRITE_SIZE, scaled by the calibration copy's reading)."""
    cfgs = sweep_configs(args.wtype, args.only)
    trace, counters = [], []
    for d in args.summarize:
        trace += glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)
        counters += glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
    if trace:
        segs = _segments(_rows(trace[0]), lambda r: (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3)
        assert len(segs) == len(cfgs) + 1, (len(segs), len(cfgs))
        print("| workload | shape | N | kernel | launches/op | median us | mean us | min us | max us | "
              "op us (sum of medians) | GEMV GB/s (median) | % of 8 TB/s |")
        print("|---|---|---|---|---|---|---|---|---|---|---|---|")
        for (wl, M, K, N), seg in zip(cfgs, segs[1:]):
            ks = _per_kernel(seg, args.warmup, args.steps)
            op_us = sum(n * float(np.median(v)) for n, v in ks.values())
            gemv = [k for k in ks if "gemv" in k]
            gemv_us = sum(ks[k][0] * float(np.median(ks[k][1])) for k in gemv)
            gbs = algorithmic_bytes(M, K, N, args.wtype) / (gemv_us * 1e-6) / 1e9 if gemv_us else 0.0
            for k, (n, v) in ks.items():
                v = np.asarray(v)
                print(f"| {wl} | {M}x{K} | {N} | `{_short(k)}` | {n} | {np.median(v):.3f} | {v.mean():.3f} | "
                      f"{v.min():.3f} | {v.max():.3f} | {op_us:.3f} | {gbs:.0f} | {100 * gbs / HBM_PEAK_GBS:.1f} |")
    if counters:
        by_counter = {}
        for path in counters:
            for r in _rows(path):
                by_counter.setdefault(r["Counter_Name"], []).append(r)
        per = {}
        sq = {}
        for cname, crows in sorted(by_counter.items()):
            segs = _segments(crows, lambda r: float(r["Counter_Value"]))
            assert len(segs) == len(cfgs) + 1, (len(segs), len(cfgs))
            if cname not in ("FETCH_SIZE", "WRITE_SIZE"):  # raw counts per dispatch
                for (wl, M, K, N), seg in zip(cfgs, segs[1:]):
                    ks = _per_kernel(seg, args.warmup, args.steps)
                    for k, (n, v) in ks.items():
                        print(f"{cname} M={M} K={K} N={N} kernel={_short(k).replace(' ', '')} launches/op={n} "
                              f"median={float(np.median(v)):.0f}")
                        sq.setdefault((M, K, N, _short(k)), {})[cname] = float(np.median(v))
                continue
            # the calibration copy (the most frequent kernel before the first
            # separator) reads and writes CAL_BYTES once per dispatch
            names = [n for n, _ in segs[0]]
            copy_kernel = max(set(names), key=names.count)
            cal = [v for n, v in segs[0] if n == copy_kernel]
            factor = CAL_BYTES / (float(np.median(cal)) * 1024.0)
            print(f"# {cname}: calibration copy of {CAL_BYTES} B -> median {np.median(cal):.1f} KiB per dispatch, "
                  f"scale factor {factor:.4f}")
            for (wl, M, K, N), seg in zip(cfgs, segs[1:]):
                ks = _per_kernel(seg, args.warmup, args.steps)
                gemv = sum(n * float(np.median(v)) for k, (n, v) in ks.items() if "gemv" in k) * 1024 * factor
                op = sum(n * float(np.median(v)) for n, v in ks.values()) * 1024 * factor
                print(f"{cname} M={M} K={K} N={N} gemv_bytes={gemv:.0f} op_bytes={op:.0f}")
                per.setdefault((M, K, N), {})[cname] = (gemv, op)
        _sq_table(sq)
        if per and all({"FETCH_SIZE", "WRITE_SIZE"} <= set(v) for v in per.values()):
            print("| workload | shape | N | algorithmic B | GEMV read B | GEMV written B | op B (all kernels) | "
                  "op / algorithmic |")
            print("|---|---|---|---|---|---|---|---|")
            lines = []
            for wl, M, K, N in cfgs:
                f, w = per[(M, K, N)]["FETCH_SIZE"], per[(M, K, N)]["WRITE_SIZE"]
                alg = algorithmic_bytes(M, K, N, args.wtype)
                print(f"| {wl} | {M}x{K} | {N} | {alg:,} | {f[0]:,.0f} | {w[0]:,.0f} | {f[1] + w[1]:,.0f} | "
                      f"{(f[1] + w[1]) / alg:.4f} |")
                lines.append(f"traffic M={M} K={K} N={N} gemv_bytes={f[0] + w[0]:.0f} op_bytes={f[1] + w[1]:.0f}")
            print()
            print("\n".join(lines))


def _pkg():
    import _common
    return _common.pkg()


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--trials", type=int, default=7, help="timed replays of the K-step graph (median reported)")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--profile", action="store_true", help="plain launches only, for rocprofv3")
    ap.add_argument("--profile-sweep", action="store_true", help="plain launches of every sweep config, for rocprofv3")
    ap.add_argument("--pool-bytes", type=int, default=1 << 30, help="--profile-sweep: weight copies per config")
    ap.add_argument("--summarize", metavar="DIR", nargs="+",
                    help="per-config tables from the rocprofv3 output directories of --profile-sweep runs")
    ap.add_argument("--only", nargs="+", metavar="MxKxN",
                    help="--profile-sweep/--summarize: only these configs of the sweep")
    ap.add_argument("--graph", action="store_true",
                    help="--profile/--profile-sweep: run the timed steps as one HIP graph replay")
    ap.add_argument("--shape", type=int, nargs=3, default=[14336, 4096, 1], metavar=("M", "K", "N"))
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=2.0, help="--sweep: CPU seconds per config and mode")
    ap.add_argument("--moe", action="store_true",
                    help="time MUL_MAT_ID (one token) on expert-FFN shapes")
    ap.add_argument("--fused", action="store_true",
                    help="time the gate+up SWIGLU launch against two plain launches")
    ap.add_argument("--kernel", type=int, default=0, choices=(0, 1, 2, 3, 4, 5, 6),
                    help="--profile/--profile-sweep/--sweep: force a GEMV kernel through the geometry override "
                         "(1 tile, 2 block-per-lane, 3 coalesced block, 4 matrix-core, 5 K-split, 6 matrix-core "
                         "reading its A operand from the Q8_1 copy; 0 automatic)")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="time a plain read of a weight's bytes (--shape M K, default the headline's) in "
                         "several launch shapes")
    ap.add_argument("--wtype", choices=sorted(BLOCK_BYTES), default="q4_K",
                    help="weight format of --sweep, --profile and --profile-sweep (the headline is Q4_K)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the Q4_K GEMV has no multi-GPU path here "
              "(rows would shard across GPUs through q4k_op_mul_mat_vec_q); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.kernel:
        _pkg().set_geometry_override(kernel=args.kernel)
    if args.summarize:
        summarize(args)
    elif args.profile_sweep:
        profile_sweep(args)
    elif args.profile:
        profile_mode(args)
    elif args.fused:
        fused_sweep(args)
    elif args.moe:
        moe_sweep(args)
    elif args.sweep:
        sweep(args)
    elif args.read_ceiling:
        read_ceiling(args)
    else:
        headline(args)


if __name__ == "__main__":
    main()
