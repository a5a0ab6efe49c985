"""Benchmark of the MI355X fp32 matmul path (BASELINE.json metric: fp32 GEMM/BMM TFLOP/s and %
of the MI355X FP32 matrix peak at 4096^3).

One step = the three GEMMs of BASELINE config 4 on synthetic N(0, 1/64) data resident in HBM:
  NN  C  = A  * B      (forward)
  NT  dA = dC * B^T    (autograd gradient of A)
  TN  dB = A^T * dC    (autograd gradient of B)
each M = N = K = 4096, 2*4096^3 FLOP. `value` is the whole step's FLOP / wall time.

Prints ONE JSON line on stdout. Extra per-configuration measurements (--configs all) go to
stderr. The CPU baseline is the oracle's restatement of the reference matmul_tiled arithmetic
(oracle/oracle.c, kind "port") timed on the host cores on a bounded row sample.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense FP32 matrix peak (AMD public specification)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--configs", default="main", choices=["main", "all"],
                   help="'all' also measures every BASELINE config (reported on stderr)")
    p.add_argument("--cpu-seconds", type=float, default=12.0,
                   help="target duration of the bounded CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--pmc-target", nargs="?", const="4096", choices=["4096", "5a", "3"],
                   help="run only a profiling target for rocprofv3 --pmc passes: '4096' (the "
                        "default) the three 4096^3 forms 3x each, '5a' config 5a (1000x777x3000 "
                        "NN) 3x, '3' the config-3 gate GEMM (64x1536x4096 + bias) over 3 "
                        "timestep inputs; then a 256 MiB device copy 3x (the reference for "
                        "scaling FETCH_SIZE / WRITE_SIZE to bytes)")
    return p.parse_args()


def cpu_baseline(target_s):
    """Oracle restatement of matmul_tiled (fp32 fma chains, ascending k) on host cores, on
    a growing row sample of the 4096^3 NN GEMM until ~target_s of CPU work."""
    import oracle
    n = 4096
    threads = min(16, os.cpu_count() or 1)
    A = oracle.uniform((n, n), 3, 0)
    B = oracle.uniform((n, n), 3, 1)
    rows = max(threads, 16)
    elapsed = 0.0
    while True:
        t0 = time.perf_counter()
        oracle.matmul_rows(A, B, 0, rows, threads=threads)
        elapsed = time.perf_counter() - t0
        if elapsed >= target_s / 4 or rows >= n:
            break
        rows = min(n, int(rows * max(2.0, (target_s / 4) / max(elapsed, 1e-3))))
    # final timed sample sized to about target_s (the whole GEMM, repeated, if it is fast)
    reps = 1
    if rows >= n:
        reps = max(1, int(round(target_s / max(elapsed, 1e-3))))
    else:
        rows = min(n, max(rows, int(rows * target_s / max(elapsed, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(reps):
        oracle.matmul_rows(A, B, 0, rows, threads=threads)
    elapsed = time.perf_counter() - t0
    flop = 2.0 * rows * n * n * reps
    return {"value": round(flop / elapsed / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "kind": "port",
            "sample": f"{reps} x rows 0..{rows} of the 4096^3 NN GEMM ({flop / 1e9:.1f} GFLOP) "
                      f"with the oracle's matmul_tiled restatement (fp32 fma chains, ascending "
                      f"k; i-k-j order, AVX2), {threads} threads, {elapsed:.1f} s",
            "openmp": bool(oracle.lib().oracle_openmp_enabled())}


class Timer:
    """HIP events on torch's current stream -- the stream every migemm launch uses."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs = []

    def around(self, fn):
        s = self.torch.cuda.Event(enable_timing=True)
        e = self.torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        self.pairs.append((s, e))

    def mean_ms(self):
        self.torch.cuda.synchronize()
        return float(np.mean([s.elapsed_time(e) for s, e in self.pairs]))


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: every GPU box here has one "
                                   "MI355X, and the matmul path shards without collectives "
                                   "(see the sharding paragraph of the design notes); run "
                                   "with --gpus 1"}))
        sys.exit(2)

    import torch
    from my_pytchon_opencl_lib_amd import NnClGlob, _native

    if args.pmc_target:
        pmc_target(torch, NnClGlob("cuda:0"), args.pmc_target)
        return
    nncl = NnClGlob("cuda:0")
    dev = torch.device("cuda:0")
    n = 4096
    flop = 2.0 * n * n * n
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    std = 1.0 / 64.0
    A = torch.randn(n, n, device=dev, generator=gen) * std
    B = torch.randn(n, n, device=dev, generator=gen) * std
    dC = torch.randn(n, n, device=dev, generator=gen) * std
    C = torch.empty(n, n, device=dev)
    dA = torch.empty(n, n, device=dev)
    dB = torch.empty(n, n, device=dev)

    forms = {
        "NN": lambda: nncl.gemm(A, B, out=C),
        "NT": lambda: nncl.gemm(dC, B, transB=True, out=dA),
        "TN": lambda: nncl.gemm(A, dC, transA=True, out=dB),
    }
    timers = {k: Timer(torch) for k in forms}

    for _ in range(args.warmup):
        for f in forms.values():
            f()
    torch.cuda.synchronize()

    t0 = time.perf_counter()
    for _ in range(args.steps):
        for k, f in forms.items():
            timers[k].around(f)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    per_form = {}
    for k, t in timers.items():
        ms = t.mean_ms()
        per_form[k] = {"ms": round(ms, 4), "tflops": round(flop / (ms * 1e-3) / 1e12, 2)}
    dominant = max(per_form, key=lambda k: per_form[k]["ms"])
    dom_ms = per_form[dominant]["ms"]
    achieved = flop / (dom_ms * 1e-3) / 1e12
    value = 3 * flop / (ms_per_step * 1e-3) / 1e12

    extra = {}
    if args.configs == "all":
        extra = measure_all_configs(torch, nncl, _native)
        print(json.dumps({"configs": extra}, indent=1), file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_seconds)

    line = {
        "metric": "fp32 GEMM/BMM TFLOP/s and % of MI355X FP32 matrix peak at 4096^3",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: A, B, dC ~ N(0, 1/64) fp32 in HBM (torch generator, seed 3)",
        "config": {"workload": "BASELINE config 4: fp32 4096x4096x4096 NN forward + NT "
                               "(dA = dC*B^T) + TN (dB = A^T*dC), one step = all three",
                   "M": n, "N": n, "K": n, "forms": per_form,
                   "pct_of_fp32_matrix_peak": round(100 * value / PEAK_FP32_MFMA_TFLOPS, 2),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "kernel": f"{tiled_kernel_name()} ({dominant} form)",
                     "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": load_traffic(dominant)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def pmc_target(torch, nncl, which="4096"):
    g = torch.Generator(device="cuda:0")
    if which == "3":
        g.manual_seed(2)
        X = torch.randn(3, 64, 1536, device="cuda:0", generator=g)
        W = (torch.rand(1536, 4096, device="cuda:0", generator=g) * 2 - 1) / 32
        bias = (torch.rand(4096, device="cuda:0", generator=g) * 2 - 1) / 32
        Y = torch.empty(64, 4096, device="cuda:0")
        for i in range(3):
            nncl.gemm(X[i], W, bias=bias, out=Y)
    elif which == "5a":
        g.manual_seed(4)
        A = torch.rand(1000, 777, device="cuda:0", generator=g) * 2 - 1
        B = torch.rand(777, 3000, device="cuda:0", generator=g) * 2 - 1
        C = torch.empty(1000, 3000, device="cuda:0")
        for _ in range(3):
            nncl.gemm(A, B, out=C)
    else:
        n = 4096
        g.manual_seed(3)
        A = torch.randn(n, n, device="cuda:0", generator=g) / 64
        B = torch.randn(n, n, device="cuda:0", generator=g) / 64
        C = torch.empty(n, n, device="cuda:0")
        for _ in range(3):
            nncl.gemm(A, B, out=C)
            nncl.gemm(A, B, transB=True, out=C)
            nncl.gemm(A, B, transA=True, out=C)
    src = torch.ones(64 * 1024 * 1024, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print("pmc target done", flush=True)


def tiled_kernel_name():
    """The kernel that runs the 4096^3 forms: 256x256 tiles with operands loaded straight
    into LDS."""
    return "gemm_direct_kernel"


def load_traffic(kernel_substr):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, each
    scaled by the copy-kernel factor) for the dominant kernel, from the committed profile
    summary; None when no summary covers that kernel."""
    name = "gemm_mfma_4096_pmc.md" if tiled_kernel_name() == "gemm_mfma_kernel" else \
        "gemm_direct_4096_pmc.md"
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("TRAFFIC_BYTES_PER_LAUNCH"):
            _, form, nbytes = line.split()[:3]
            if form == kernel_substr:
                return int(nbytes)
    return None


def measure_all_configs(torch, nncl, _native, reps=20):
    """Per-config device time per call, from HIP events around a HIP graph that replays
    `reps` back-to-back calls (so host launch overhead is not measured). Inputs rotate
    where the working set must exceed the 256 MB MALL."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    out = {}

    def timed(fns):
        for f in fns:
            f()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps // len(fns)):
                for f in fns:
                    f()
        graph.replay()
        torch.cuda.synchronize()
        t = Timer(torch)
        for _ in range(5):
            t.around(graph.replay)
        return t.mean_ms() / ((reps // len(fns)) * len(fns))

    def rec(name, ms, flop, byts):
        out[name] = {"us": round(ms * 1e3, 2), "tflops": round(flop / (ms * 1e-3) / 1e12, 3),
                     "pct_mfma_peak": round(100 * flop / (ms * 1e-3) / 1e12 /
                                            PEAK_FP32_MFMA_TFLOPS, 2),
                     "GBps": round(byts / (ms * 1e-3) / 1e9, 1),
                     "pct_hbm_peak": round(100 * byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 2)}

    r = lambda *s: torch.rand(*s, device=dev, generator=g) * 2 - 1
    A, B, C = r(256, 256), r(256, 256), torch.empty(256, 256, device=dev)
    rec("1_nn_256", timed([lambda: nncl.gemm(A, B, out=C)]), 2 * 256 ** 3, 4 * 3 * 256 * 256)
    Q, Kt, P, V = r(32, 128, 64), r(32, 64, 128), r(32, 128, 128), r(32, 128, 64)
    S, O = torch.empty(32, 128, 128, device=dev), torch.empty(32, 128, 64, device=dev)
    rec("2a_bmm_qk", timed([lambda: nncl.gemm(Q, Kt, out=S)]), 2 * 32 * 128 * 128 * 64,
        4 * 32 * (128 * 64 * 2 + 128 * 128))
    rec("2b_bmm_pv", timed([lambda: nncl.gemm(P, V, out=O)]), 2 * 32 * 128 * 128 * 64,
        4 * 32 * (128 * 128 + 128 * 64 * 2))
    X = r(20, 64, 1536)
    W = r(1536, 4096) / 32
    bias = r(4096) / 32
    Y = torch.empty(64, 4096, device=dev)
    rec("3_lstm_gate_step",
        timed([lambda i=i: nncl.gemm(X[i], W, bias=bias, out=Y) for i in range(20)]),
        2 * 64 * 1536 * 4096, 4 * (64 * 1536 + 1536 * 4096 + 64 * 4096 + 4096))
    A5, B5, C5 = r(1000, 777), r(777, 3000), torch.empty(1000, 3000, device=dev)
    rec("5a_ragged", timed([lambda: nncl.gemm(A5, B5, out=C5)]), 2 * 1000 * 3000 * 777,
        4 * (1000 * 777 + 777 * 3000 + 1000 * 3000))
    x = r(1, 4096)
    copies = [r(4096, 11008) for _ in range(3)]  # 541 MB > the 256 MB MALL
    y = torch.empty(1, 11008, device=dev)
    rec("5b_gemv", timed([lambda c=c: nncl.gemm(x, c, out=y) for c in copies]),
        2 * 4096 * 11008, 4 * (4096 + 4096 * 11008 + 11008))
    return out


if __name__ == "__main__":
    main()
