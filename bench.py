"""Benchmark of the MI355X fp32 matmul path (BASELINE.json metric: fp32 GEMM/BMM TFLOP/s and %
of the MI355X FP32 matrix peak at 4096^3).

One step = the three GEMMs of BASELINE config 4 on synthetic N(0, 1/64) data resident in HBM:
  NN  C  = A  * B      (forward)
  NT  dA = dC * B^T    (autograd gradient of A)
  TN  dB = A^T * dC    (autograd gradient of B)
each M = N = K = 4096, 2*4096^3 FLOP. `value` is the whole step's FLOP / wall time.

Prints ONE JSON line on stdout. Besides the step (and, in config.torch_blas_forms, torch's
own fp32 GEMM of the three forms on the same tensors) it carries, by default:
  configs            every other BASELINE config timed on this GPU (HIP events around HIP-graph
                     replays of back-to-back calls), with its roofline fraction, the launch
                     floor (a one-element fill kernel replayed the same way), for the small
                     configs a data-movement floor (a torch kernel that reads and writes the
                     same bytes) and torch's own fp32 GEMM of the shape (torch_blas_us);
  callers            the path's callers at the reference's sizes (the Linear(500 -> 6565)
                     layer forward and backward, the LSTM GEMM stages and recurrent step);
  roofline           the dominant 4096^3 kernel, from HIP events in this run (frac) and from
                     the committed rocprofv3 kernel trace of this bench (frac_profiled);
  cpu_baseline       the oracle's restatement of the reference matmul_tiled arithmetic
                     (oracle/oracle.c, kind "port") on the host cores, a bounded row sample;
  reference_same_gpu the reference's own matmul.cl bmm_tiled, compiled from its source into
                     oracle/_ref, run through ROCm OpenCL on this GPU (there is no CPU OpenCL
                     device, PoCL, on the box).
The extra legs run after the timed region.

Profiling helpers: --pmc-target runs one workload for rocprofv3 --pmc passes, and
--summarize-trace summarises a rocprofv3 --kernel-trace CSV of this bench (the committed
profiles/*.md summaries are made with them).
"""
import argparse
import csv
import ctypes
import glob
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense FP32 matrix peak (AMD public specification)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
N4096 = 4096
FLOP_4096 = 2.0 * N4096 ** 3
EVENT_EVERY = 2  # timed steps per step whose launches carry HIP events
TRACE_SUMMARY = os.path.join(ROOT, "profiles", "gemm_direct_4096_kernel_trace.md")
PMC_SUMMARY = os.path.join(ROOT, "profiles", "gemm_direct_4096_pmc.md")
# GPU box: one GPU's share of the host is 16 threads (OMP_NUM_THREADS there)
CPU_SHARE = 16

# BASELINE configs other than the step: algorithmic FLOP and bytes per call (a broadcast
# operand counted once, bias bytes included, bias adds not counted as FLOP)
CONFIGS = {
    "1_nn_256": (2 * 256 ** 3, 4 * 3 * 256 * 256, "mfma"),
    "2a_bmm_qk": (2 * 32 * 128 * 128 * 64, 4 * 32 * (128 * 64 * 2 + 128 * 128), "hbm"),
    "2b_bmm_pv": (2 * 32 * 128 * 128 * 64, 4 * 32 * (128 * 128 + 128 * 64 * 2), "hbm"),
    "3_lstm_gate_step": (2 * 64 * 1536 * 4096,
                         4 * (64 * 1536 + 1536 * 4096 + 64 * 4096 + 4096), "mfma"),
    # config 3 in the reference's stateful form (lstm_hid_forward, lstm.cl:832-844): x_t, h_{t-1},
    # W, U as four buffers, the same FLOP and bytes as the concatenated product
    "3h_lstm_hid_step": (2 * 64 * 1536 * 4096,
                         4 * (64 * 512 + 64 * 1024 + 1536 * 4096 + 64 * 4096 + 4096), "mfma"),
    "5a_ragged": (2 * 1000 * 3000 * 777, 4 * (1000 * 777 + 777 * 3000 + 1000 * 3000), "mfma"),
    "5b_gemv": (2 * 4096 * 11008, 4 * (4096 + 4096 * 11008 + 11008), "hbm"),
    # tensor_permute (cl_kernels/permute.cl:11-50): not a BASELINE config, but the path's
    # layout row; read + write of the tensor. [1,0] of a 4096^2 operand is what BmmOp.Backward
    # materialised for config 4 (BmmOp.cs:44-60); the 4-D head split runs the generic gather.
    "a5_permute_4096_t": (0, 2 * 4 * 4096 * 4096, "hbm"),
    "a5_permute_heads_0213": (0, 2 * 4 * 32 * 128 * 16 * 64, "hbm"),
}


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    # 25 untimed steps (~70 ms): after 5 the first timed steps still ran ~1.3 % slower than
    # steady state (clocks and caches settling)
    p.add_argument("--warmup", type=int, default=25)
    p.add_argument("--configs", default="all", choices=["main", "all"],
                   help="'all' (default) also times every other BASELINE config")
    p.add_argument("--cpu-seconds", type=float, default=15.0,
                   help="target duration of the bounded CPU-baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-reference", action="store_true",
                   help="skip the reference bmm_tiled run on this GPU")
    p.add_argument("--pmc-target", nargs="?", const="4096",
                   choices=["4096", "1", "2a", "2b", "3", "3h", "5a", "5b", "a5t", "a5h",
                            "floor"],
                   help="run only one workload for rocprofv3 --pmc passes (3 launches, 21 "
                        "for the short configs): '4096' "
                        "the three 4096^3 forms, '1' / '2a' / '2b' / '3' / '5a' / '5b' that "
                        "BASELINE config, '3h' config 3 in the stateful x_t W + h_{t-1} U "
                        "form, 'a5t' / 'a5h' the 4096^2 [1,0] and the [0,2,1,3] "
                        "head-split permutes, 'floor' the one-element fill kernel; then a 256 MiB "
                        "device copy 3 times (the reference for scaling FETCH_SIZE / "
                        "WRITE_SIZE to bytes)")
    p.add_argument("--decompose", action="store_true",
                   help="only fit fixed cost + per-unit slope of the panel kernel (M = 64, "
                        "N = 4096, K = 256 .. 2048) and of 64x64 tiles (1-4 work-groups per "
                        "CU), from graph-timed sweeps; prints one JSON line")
    p.add_argument("--summarize-trace", metavar="DIR",
                   help="summarise the rocprofv3 --kernel-trace CSV under DIR, made from "
                        "'bench.py --steps S --warmup W' (pass the same --steps / --warmup)")
    return p.parse_args()


def host_cpu():
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    return {"nproc": os.cpu_count() or 1, "usable": usable, "model": model}


def cpu_baseline(target_s):
    """Oracle restatement of matmul_tiled (fp32 fma chains, ascending k) on host cores, on
    a growing row sample of the 4096^3 NN GEMM until ~target_s of CPU work."""
    import oracle
    n = N4096
    cpu = host_cpu()
    threads = max(1, min(CPU_SHARE, cpu["usable"]))
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
            "host": {"nproc": cpu["nproc"], "usable_cpus": cpu["usable"],
                     "cpu_model": cpu["model"],
                     "threads_rule": f"min({CPU_SHARE}, usable CPUs): {CPU_SHARE} is one GPU's "
                                     f"share of the GPU box's host (its OMP_NUM_THREADS)"},
            "openmp": bool(oracle.lib().oracle_openmp_enabled())}


def reference_same_gpu(step_ms_nn):
    """The reference kernel bmm_tiled (cl_kernels/matmul.cl:78-135) at 4096^3 on this GPU:
    compiled from the reference source into oracle/_ref, launched with the reference host's
    geometry (NnClGlob.cs:472-478) through ROCm OpenCL by oracle/ref_runner."""
    try:
        import oracle
        from oracle import reference_gpu as ref
        if not ref.available():
            return {"available": False, "reason": "oracle/_ref was not built"}
        A = oracle.uniform((N4096, N4096), 3, 0)
        B = oracle.uniform((N4096, N4096), 3, 1)
        _, info = ref.run("bmm_tiled", A, B, M=N4096, K=N4096, N=N4096, batch=1, reps=3)
    except Exception as e:  # noqa: BLE001 -- reported, never fatal to the bench line
        return {"available": False, "reason": f"{type(e).__name__}: {e}"}
    ms = info["median_us"] / 1e3
    tf = FLOP_4096 / (ms * 1e-3) / 1e12
    return {"kernel": "bmm_tiled (cl_kernels/matmul.cl:78-135), reference source compiled "
                      "for gfx950, ROCm OpenCL, 16x16 work-groups (NnClGlob.cs:472-478)",
            "device": info["device"], "workload": "4096x4096x4096 NN, one launch",
            "median_ms": round(ms, 3), "tflops": round(tf, 2),
            "pct_of_fp32_matrix_peak": round(100 * tf / PEAK_FP32_MFMA_TFLOPS, 2),
            "this_build_speedup": round(ms / step_ms_nn, 2), "reps": info["reps"]}


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
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.steps, args.warmup)
        return
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
    if args.decompose:
        print(json.dumps({"decompose": decompose(torch, NnClGlob("cuda:0"), _native)}),
              flush=True)
        return
    nncl = NnClGlob("cuda:0")
    dev = torch.device("cuda:0")
    n = N4096
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
    plans = {}
    for k, f in forms.items():
        f()
        plans[k] = _native.last_plan()
    timers = {k: Timer(torch) for k in forms}

    for _ in range(args.warmup):
        for f in forms.values():
            f()
    torch.cuda.synchronize()

    # Per-launch HIP events on one timed step in EVENT_EVERY only: an event pair around every
    # launch added ~0.9 % to the step's wall time (2.762 against 2.737 ms per step), on every
    # 4th step ~0.2 %, but 5 samples per form at 20 steps left the mean noisy.
    t0 = time.perf_counter()
    for i in range(args.steps):
        for k, f in forms.items():
            if i % EVENT_EVERY == 0:
                timers[k].around(f)
            else:
                f()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    per_form = {}
    for k, t in timers.items():
        ms = t.mean_ms()
        per_form[k] = {"ms": round(ms, 4), "tflops": round(FLOP_4096 / (ms * 1e-3) / 1e12, 2),
                       "kernel": plans[k]}
    dominant = max(per_form, key=lambda k: per_form[k]["ms"])
    dom_ms = per_form[dominant]["ms"]
    achieved = FLOP_4096 / (dom_ms * 1e-3) / 1e12
    value = 3 * FLOP_4096 / (ms_per_step * 1e-3) / 1e12

    # torch's own fp32 GEMM (hipBLASLt) on the same tensors and forms, for comparison only
    vendor_forms = {
        "NN": lambda: torch.mm(A, B, out=C),
        "NT": lambda: torch.mm(dC, B.t(), out=dA),
        "TN": lambda: torch.mm(A.t(), dC, out=dB),
    }
    torch_blas = {}
    for k, f in vendor_forms.items():
        for _ in range(5):
            f()
        vt = Timer(torch)
        for _ in range(10):
            vt.around(f)
        ms = vt.mean_ms()
        torch_blas[k] = {"ms": round(ms, 4),
                         "tflops": round(FLOP_4096 / (ms * 1e-3) / 1e12, 2)}

    configs = measure_all_configs(torch, nncl, _native) if args.configs == "all" else None
    callers = measure_callers(torch, nncl, _native) if args.configs == "all" else None
    ref = None if args.no_reference else reference_same_gpu(per_form["NN"]["ms"])
    cpu = None if args.no_cpu_baseline else cpu_baseline(args.cpu_seconds)

    prof = load_profiled()
    roofline = {"bound": "mfma", "kernel": f"gemm_direct_kernel ({dominant} form, 256x256 tiles)",
                "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA_TFLOPS,
                "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
                "traffic": load_traffic(dominant),
                "algorithmic_per_launch": {"flop": FLOP_4096, "bytes": 4 * 3 * n * n},
                "measured_by": f"HIP events around each launch of one timed step in "
                               f"{EVENT_EVERY}, on the launch stream, this run"}
    if dominant in prof:
        pus = prof[dominant]
        roofline["profiled_us"] = pus
        roofline["frac_profiled"] = round(FLOP_4096 / (pus * 1e-6) / 1e12 /
                                          PEAK_FP32_MFMA_TFLOPS, 4)
        roofline["profile"] = "profiles/gemm_direct_4096_kernel_trace.md (timed launches " \
                              "under rocprofv3 --kernel-trace)"
    roofline["traffic_source"] = "profiles/gemm_direct_4096_pmc.md (rocprofv3 --pmc " \
                                 "FETCH_SIZE + WRITE_SIZE, copy-kernel scaled)"

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
        "data": "synthetic: A, B, dC ~ N(0, 1/64) fp32 in HBM (torch generator, seed 3); "
                "other configs U[-1,1) / N(0,1) of their BASELINE shapes",
        "config": {"workload": "BASELINE config 4: fp32 4096x4096x4096 NN forward + NT "
                               "(dA = dC*B^T) + TN (dB = A^T*dC), one step = all three",
                   "M": n, "N": n, "K": n, "forms": per_form,
                   "torch_blas_forms": torch_blas,
                   "pct_of_fp32_matrix_peak": round(100 * value / PEAK_FP32_MFMA_TFLOPS, 2),
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "configs": configs,
        "callers": callers,
        "reference_same_gpu": ref,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def pmc_target(torch, nncl, which="4096"):
    """One workload for rocprofv3 --pmc passes, then the copy reference: 3 launches of each
    4096^3 form, of 5a, 5b (one per copy of B) and the 4096^2 permute; 21 of the short configs
    (1, 2a, 2b, 3, 3h, the head permute and the launch floor), whose per-dispatch counters
    vary more (the summary takes each counter's median over the launches)."""
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0)
    dev = torch.device("cuda:0")
    r = lambda *s: torch.rand(*s, device=dev, generator=g) * 2 - 1
    if which == "1":
        A, B, C = r(256, 256), r(256, 256), torch.empty(256, 256, device=dev)
        calls = [lambda: nncl.gemm(A, B, out=C)] * 21
    elif which in ("2a", "2b"):
        if which == "2a":
            X, Y, Z = r(32, 128, 64), r(32, 64, 128), torch.empty(32, 128, 128, device=dev)
        else:
            X, Y, Z = r(32, 128, 128), r(32, 128, 64), torch.empty(32, 128, 64, device=dev)
        calls = [lambda: nncl.gemm(X, Y, out=Z)] * 21
    elif which == "3":
        X = torch.randn(3, 64, 1536, device=dev, generator=g)
        W = r(1536, 4096) / 32
        bias = r(4096) / 32
        Y = torch.empty(64, 4096, device=dev)
        calls = [lambda i=i: nncl.gemm(X[i], W, bias=bias, out=Y) for i in range(3)] * 7
    elif which == "3h":
        Xs = torch.randn(64, 3, 512, device=dev, generator=g)
        Wx, Uh, bias = r(512, 4096) / 32, r(1024, 4096) / 32, r(4096) / 32
        Hp, Ho = r(64, 1024), r(64, 3, 1024)
        ws = torch.empty(3, 64, 4096, device=dev)
        calls = [lambda t=t: nncl.LstmHidGates(Xs, Wx, Uh, bias, Hp, Ho, ws, t)
                 for t in range(3)] * 7
    elif which == "5a":
        A, B, C = r(1000, 777), r(777, 3000), torch.empty(1000, 3000, device=dev)
        calls = [lambda: nncl.gemm(A, B, out=C)] * 3
    elif which == "5b":
        x = r(1, 4096)
        copies = [r(4096, 11008) for _ in range(3)]
        y = torch.empty(1, 11008, device=dev)
        calls = [lambda c=c: nncl.gemm(x, c, out=y) for c in copies]
    elif which == "a5t":
        T = r(4096, 4096)
        calls = [lambda: nncl.Permute(T, [1, 0])] * 3
    elif which == "a5h":
        H = r(32, 128, 16, 64)
        calls = [lambda: nncl.Permute(H, [0, 2, 1, 3])] * 21
    elif which == "floor":
        z = torch.empty(1, device=dev)
        calls = [lambda: z.fill_(1.0)] * 21
    else:
        n = N4096
        A = torch.randn(n, n, device=dev, generator=g) / 64
        B = torch.randn(n, n, device=dev, generator=g) / 64
        C = torch.empty(n, n, device=dev)
        calls = [lambda: nncl.gemm(A, B, out=C), lambda: nncl.gemm(A, B, transB=True, out=C),
                 lambda: nncl.gemm(A, B, transA=True, out=C)] * 3
    torch.cuda.synchronize()
    for f in calls:
        f()
    src = torch.ones(64 * 1024 * 1024, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"pmc target {which} done", flush=True)


def load_traffic(form):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE + WRITE_SIZE, each
    scaled by the copy-kernel factor) for the dominant form, from the committed profile
    summary; None when no summary covers it."""
    if not os.path.exists(PMC_SUMMARY):
        return None
    for line in open(PMC_SUMMARY):
        if line.startswith("TRAFFIC_BYTES_PER_LAUNCH"):
            _, f, nbytes = line.split()[:3]
            if f == form:
                return int(nbytes)
    return None


def load_profiled():
    """Timed-launch average duration (us) of each 4096^3 form under rocprofv3, from the
    committed kernel-trace summary of this bench."""
    out = {}
    if os.path.exists(TRACE_SUMMARY):
        for line in open(TRACE_SUMMARY):
            if line.startswith("PROFILED_US"):
                _, f, us = line.split()[:3]
                out[f] = float(us)
    return out


FORM_OF = {("true", "false"): "NN", ("true", "true"): "NT", ("false", "false"): "TN",
           ("false", "true"): "TT"}


def summarize_trace(directory, steps, warmup):
    """Markdown summary of a rocprofv3 --kernel-trace CSV of 'bench.py --steps S --warmup W':
    per kernel (name shortened to its template) launches and average duration, and for the
    three 4096^3 forms the average over exactly the bench's timed launches (each form runs
    once untimed to record its plan, W warm-up times, then S timed times)."""
    paths = glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
    if not paths:
        sys.exit(f"no *kernel_trace.csv under {directory}")
    rows = []
    for p in paths:
        with open(p) as f:
            rows += list(csv.DictReader(f))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    by_kernel = {}
    forms = {}
    for r in rows:
        name = r["Kernel_Name"]
        short = re.sub(r"\(.*", "", name.replace("(anonymous namespace)", "{anon}"))
        short = short.replace("void ", "")
        us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        by_kernel.setdefault(short, []).append(us)
        m = re.search(r"gemm_direct_kernel<256, 256, \d+, \d+, (true|false), (true|false)", name)
        if m:
            forms.setdefault(FORM_OF[m.groups()], []).append(us)
    print("| kernel | launches | average (us) | min (us) | max (us) |")
    print("|---|---|---|---|---|")
    for k, v in sorted(by_kernel.items(), key=lambda kv: -sum(kv[1])):
        if len(k) > 140:
            k = k[:137] + "..."
        print(f"| `{k}` | {len(v)} | {np.mean(v):.2f} | {np.min(v):.2f} | {np.max(v):.2f} |")
    print()
    print("| form | timed launches | average (us) | TFLOP/s | fraction of 157.3 |")
    print("|---|---|---|---|---|")
    lines = []
    for f in ("NN", "NT", "TN"):
        v = forms.get(f, [])
        timed = v[1 + warmup:1 + warmup + steps]
        if not timed:
            continue
        us = float(np.mean(timed))
        tf = FLOP_4096 / (us * 1e-6) / 1e12
        print(f"| {f} | {len(timed)} | {us:.1f} | {tf:.2f} | {tf / PEAK_FP32_MFMA_TFLOPS:.4f} |")
        lines.append(f"PROFILED_US {f} {us:.1f}")
    print()
    print("\n".join(lines))


def graph_timed(torch, cap, fns, per):
    """Device ms per call: HIP events around 5 replays of a HIP graph that runs the calls
    `fns` `per` times back to back, captured on stream `cap` (its own library workspace, sized
    by one eager round on it first)."""
    with torch.cuda.stream(cap):
        for f in fns:
            f()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for _ in range(per):
            for f in fns:
                f()
    # Warm replays for at least ~20 ms of device time first, so every config is timed at the
    # clocks of sustained load rather than partly during the ramp after shorter work.
    w = Timer(torch)
    w.around(graph.replay)
    for _ in range(min(200, int(20.0 / max(w.mean_ms(), 1e-3)))):
        graph.replay()
    torch.cuda.synchronize()
    t = Timer(torch)
    for _ in range(5):
        t.around(graph.replay)
    return t.mean_ms() / (per * len(fns))


def measure_all_configs(torch, nncl, _native, calls=100):
    """Per-config device time per call, from HIP events around a HIP graph that replays
    `calls` back-to-back calls (so host launch overhead is not measured, and the graph's own
    launch, ~8 us, is spread over 100 calls as for the floor), 5 replays averaged. Inputs
    rotate where BASELINE repeats a config over many inputs (config 3: 100 timesteps) or the
    working set must exceed the 256 MB MALL (config 5b: three copies of B). The launch floor
    is a one-element fill kernel replayed the same way, right before and after each config
    (x_launch_floor is taken to their mean)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    out = {}

    cap = torch.cuda.Stream()  # the capturing stream: its own library workspace

    def timed(fns, per=None):
        return graph_timed(torch, cap, fns, per or max(1, calls // len(fns)))

    z = torch.empty(1, device=dev)
    fill = [lambda: z.fill_(1.0)]
    floors = []

    def local_floor():
        us = timed(fill) * 1e3
        floors.append(us)
        return us

    def rec(name, fns, floor=None, vendor=None, per=None):
        """Times the config's calls `fns` with the launch floor right before and after it
        (the clock state of a light load can change between minutes of one run, so the ratio
        is taken to the floor of the same moment). floor = (torch op description, fns): a
        torch kernel that reads the config's input bytes and writes its output bytes, timed
        the same way (the data-movement floor)."""
        flop, byts, bound = CONFIGS[name]
        f0 = local_floor()
        ms = timed(fns, per)
        floor_us = (f0 + local_floor()) / 2
        tf = flop / (ms * 1e-3) / 1e12
        gbs = byts / (ms * 1e-3) / 1e9
        fns[0]()
        out[name] = {"us": round(ms * 1e3, 2), "tflops": round(tf, 3),
                     "pct_mfma_peak": round(100 * tf / PEAK_FP32_MFMA_TFLOPS, 2),
                     "GBps": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / PEAK_HBM_GBS, 2),
                     "bound": bound,
                     "frac": round((tf / PEAK_FP32_MFMA_TFLOPS) if bound == "mfma"
                                   else (gbs / PEAK_HBM_GBS), 4),
                     "x_launch_floor": round(ms * 1e3 / floor_us, 2),
                     "launch_floor_us": round(floor_us, 2),
                     "kernel": _native.last_plan()}
        if floor is not None:
            fl_ms = timed(floor[1])
            out[name]["data_floor"] = {"us": round(fl_ms * 1e3, 2), "kernel": floor[0]}
            out[name]["x_data_floor"] = round(ms / fl_ms, 2)
        if vendor is not None:  # torch's own fp32 GEMM of the same shape, for comparison
            vd_ms = timed(vendor)
            out[name]["torch_blas_us"] = round(vd_ms * 1e3, 2)

    r = lambda *s: torch.rand(*s, device=dev, generator=g) * 2 - 1
    A, B, C = r(256, 256), r(256, 256), torch.empty(256, 256, device=dev)
    f1 = [lambda: nncl.gemm(A, B, out=C)]
    # Data-movement floors of the small configs: one torch elementwise kernel that reads
    # the config's operands and writes its output (the same bytes, no arithmetic to speak of).
    rec("1_nn_256", f1,
        ("torch.add(A, B, out=C): reads A and B, writes C", [lambda: torch.add(A, B, out=C)]),
        [lambda: torch.mm(A, B, out=C)])
    Q, Kt, P, V = r(32, 128, 64), r(32, 64, 128), r(32, 128, 128), r(32, 128, 64)
    S, O = torch.empty(32, 128, 128, device=dev), torch.empty(32, 128, 64, device=dev)
    f2a = [lambda: nncl.gemm(Q, Kt, out=S)]
    rec("2a_bmm_qk", f2a,
        ("torch.cat([Q, K^T], out=S): reads Q and K^T, writes S (2 MB each way)",
         [lambda: torch.cat([Q.view(-1), Kt.view(-1)], out=S.view(-1))]),
        [lambda: torch.bmm(Q, Kt, out=S)])
    f2b = [lambda: nncl.gemm(P, V, out=O)]
    rec("2b_bmm_pv", f2b,
        ("torch.addcmul(V, P[..., :64], P[..., 64:], out=O): reads P and V, writes O",
         [lambda: torch.addcmul(V, P[..., :64], P[..., 64:], out=O)]),
        [lambda: torch.bmm(P, V, out=O)])
    X = torch.randn(100, 64, 1536, device=dev, generator=g)
    W = r(1536, 4096) / 32
    bias = r(4096) / 32
    Y = torch.empty(64, 4096, device=dev)
    f3 = [lambda i=i: nncl.gemm(X[i], W, bias=bias, out=Y) for i in range(100)]
    rec("3_lstm_gate_step", f3, per=1,
        vendor=[lambda i=i: torch.addmm(bias, X[i], W, out=Y) for i in range(100)])
    del X
    # the stateful form: 100 steps of one sequence chunk, step 0 from the incoming state
    Xs = torch.randn(64, 100, 512, device=dev, generator=g)
    Wx, Uh = r(512, 4096) / 32, r(1024, 4096) / 32
    Hp, Ho = r(64, 1024), r(64, 100, 1024)
    ws = torch.empty(100, 64, 4096, device=dev)
    f3h = [lambda t=t: nncl.LstmHidGates(Xs, Wx, Uh, bias, Hp, Ho, ws, t) for t in range(100)]
    rec("3h_lstm_hid_step", f3h, per=1)
    del Xs, Ho, ws
    A5, B5, C5 = r(1000, 777), r(777, 3000), torch.empty(1000, 3000, device=dev)
    f5a = [lambda: nncl.gemm(A5, B5, out=C5)]
    rec("5a_ragged", f5a, vendor=[lambda: torch.mm(A5, B5, out=C5)])
    x = r(1, 4096)
    copies = [r(4096, 11008) for _ in range(3)]  # 541 MB > the 256 MB MALL
    y = torch.empty(1, 11008, device=dev)
    f5b = [lambda c=c: nncl.gemm(x, c, out=y) for c in copies]
    # (no torch data floor here: torch's reductions may record a memset node into a graph,
    # and they read at ~3.4 TB/s; the read floor below is the library's streaming kernel)
    rec("5b_gemv", f5b, vendor=[lambda c=c: torch.mm(x, c, out=y) for c in copies])
    out["5b_gemv"]["read_floor"] = read_floor(torch, _native, timed, copies,
                                              out["5b_gemv"]["us"])
    del copies

    def permute_into(src, dst, axes):
        dims = (ctypes.c_int * src.dim())(*src.shape)
        ax = (ctypes.c_int * src.dim())(*axes)
        _native.call("migemm_tensor_permute",
                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                     ctypes.c_void_p(src.data_ptr()), ctypes.c_void_p(dst.data_ptr()), dims, ax,
                     src.dim())

    T, Tt = r(4096, 4096), torch.empty(4096, 4096, device=dev)
    fpt = [lambda: permute_into(T, Tt, [1, 0])]
    rec("a5_permute_4096_t", fpt,
        ("torch Tt.copy_(T.t()): torch's own transpose copy", [lambda: Tt.copy_(T.t())]))
    H, Hp = r(32, 128, 16, 64), torch.empty(32, 16, 128, 64, device=dev)
    fph = [lambda: permute_into(H, Hp, [0, 2, 1, 3])]
    rec("a5_permute_heads_0213", fph,
        ("torch Hp.copy_(H.permute(0, 2, 1, 3))", [lambda: Hp.copy_(H.permute(0, 2, 1, 3))]))
    # the floor of a kernel that must read its input before it writes: a torch device copy
    # of 256 KB (one 256^2 operand) replayed the same way
    c0, c1 = r(256, 256), torch.empty(256, 256, device=dev)
    out["copy_floor"] = {"us": round(timed([lambda: c1.copy_(c0)]) * 1e3, 2),
                         "kernel": "torch copy of 256 KB, graph-replayed back to back"}
    out["launch_floor"] = {"us": round(float(np.median(floors)), 2),
                           "min_us": round(min(floors), 2), "max_us": round(max(floors), 2),
                           "kernel": "torch fill of 1 element, graph-replayed back to back, "
                                     "timed before and after every config (median here)"}
    return out


def read_floor(torch, _native, timed, copies, gemv_us):
    """The streaming-read ceiling of config 5b: the library's read-only streaming kernel
    (migemm_stream_read: contiguous ranges per work-group, 16-byte non-temporal loads, one
    sum per work-group written) over the same three rotating 180 MB copies of B, timed the
    same way as the GEMV (graph replay, 100 calls), at several work-group counts; the
    fastest is the floor, and x_read_floor = the GEMV's time / the floor."""
    nbytes = copies[0].numel() * 4
    sums = torch.empty(4096, device=copies[0].device)
    st = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def call(c, blocks):
        _native.call("migemm_stream_read", st(), ctypes.c_void_p(c.data_ptr()), c.numel(),
                     ctypes.c_void_p(sums.data_ptr()), blocks)
    res = {}
    for blocks in (344, 688, 1376, 2752, 4096):
        res[blocks] = timed([lambda c=c, b=blocks: call(c, b) for c in copies]) * 1e3
    best = min(res, key=res.get)
    us = res[best]
    return {"us": round(us, 2), "kernel": f"stream_read_kernel, {best} work-groups",
            "GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
            "pct_hbm_peak": round(100 * nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 2),
            "x_read_floor": round(gemv_us / us, 3),
            "by_work_groups_us": {str(k): round(v, 2) for k, v in res.items()}}


def decompose(torch, nncl, _native):
    """Fixed cost and per-unit slope of the kernels behind configs 3 and 5a, from graph-timed
    sweeps (HIP graphs of 100 calls as for the configs, the launch floor timed beside each
    point), fitted by least squares:
      panel: C = A B + bias with M = 64, N = 4096 and K = 256 .. 2048, A rotating over 100
        inputs as in config 3 (K = 1536; the recurrent step has K = 1024): t(K) = fixed +
        K x slope. Each SIMD runs 2 of the 8 wavefronts of its tile, 8 K MFMA cycles in all,
        so 8 / slope is the clock the k loop runs at;
      tiled: 64x64 tiles at K = 768 with 1, 2, 3 and 4 co-resident work-groups per CU
        (config 5a has three): t(n) = fixed + n x slope; a work-group adds 24 576 MFMA cycles
        per SIMD, so 24 576 / slope is again a clock.
    The fixed part beside the launch floor is what a launch costs beyond the MFMA work: the
    gap between kernels, the first loads, the reduction and the epilogue."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    cap = torch.cuda.Stream()
    z = torch.empty(1, device=dev)

    def timed_us(fns, per=None):
        return graph_timed(torch, cap, fns, per or max(1, 100 // len(fns))) * 1e3

    def point(fns, per=None):
        f0 = timed_us([lambda: z.fill_(1.0)])
        us = timed_us(fns, per)
        f1 = timed_us([lambda: z.fill_(1.0)])
        return us, (f0 + f1) / 2

    def fit(xs, ys):
        slope, fixed = np.polyfit(np.asarray(xs, float), np.asarray(ys, float), 1)
        pred = fixed + slope * np.asarray(xs, float)
        resid = float(np.max(np.abs(pred - np.asarray(ys, float))))
        return float(fixed), float(slope), resid

    out = {}
    r = lambda *s: torch.rand(*s, device=dev, generator=g) * 2 - 1
    ks, ts, floors, plans = (256, 512, 768, 1024, 1280, 1536, 2048), [], [], []
    for K in ks:
        X = torch.randn(100, 64, K, device=dev, generator=g)
        W = r(K, 4096) / 32
        bias = r(4096) / 32
        Y = torch.empty(64, 4096, device=dev)
        fns = [lambda i=i: nncl.gemm(X[i], W, bias=bias, out=Y) for i in range(100)]
        fns[0]()
        plans.append(_native.last_plan().split(" M=")[0])
        us, fl = point(fns, per=1)
        ts.append(us)
        floors.append(fl)
        del X, W
    fixed, slope, resid = fit(ks, ts)
    out["panel"] = {
        "shape": "64 x K @ K x 4096 + bias, A rotating over 100 inputs",
        "points_us": {str(k): round(t, 2) for k, t in zip(ks, ts)},
        "launch_floor_us": round(float(np.mean(floors)), 2), "plans": sorted(set(plans)),
        "fixed_us": round(fixed, 2), "slope_us_per_k": round(slope, 5),
        "max_residual_us": round(resid, 3),
        "k_loop_clock_ghz": round(8 / (slope * 1e3), 3),
        "mfma_us_at_2_4_ghz": {"config3_K1536": round(8 * 1536 / 2400, 2),
                               "recurrent_K1024": round(8 * 1024 / 2400, 2)}}
    shapes = {1: (1024, 1024), 2: (1024, 2048), 3: (1536, 2048), 4: (2048, 2048)}
    ns, ts, floors, plans = [], [], [], []
    for n, (M, N) in shapes.items():
        A, B, C = r(M, 768), r(768, N), torch.empty(M, N, device=dev)
        fns = [lambda: nncl.gemm(A, B, out=C)]
        with _native.tuned(tile=64, splitk=1):
            fns[0]()
            plans.append(_native.last_plan().split(" M=")[0])
            us, fl = point(fns)
        ns.append(n)
        ts.append(us)
        floors.append(fl)
        del A, B, C
    fixed, slope, resid = fit(ns, ts)
    out["tiled64"] = {
        "shape": "M x 768 @ 768 x N in 64x64 tiles, 256 n tiles (n per CU)",
        "points_us": {str(n): round(t, 2) for n, t in zip(ns, ts)},
        "launch_floor_us": round(float(np.mean(floors)), 2), "plans": sorted(set(plans)),
        "fixed_us": round(fixed, 2), "slope_us_per_workgroup": round(slope, 3),
        "max_residual_us": round(resid, 3),
        "k_loop_clock_ghz": round(24576 / (slope * 1e3), 3),
        "slope_tflops": round(256 * 2 * 64 * 64 * 768 / (slope * 1e-6) / 1e12, 1)}
    return out


def measure_callers(torch, nncl, _native):
    """The path's callers at the sizes the reference runs them, through the host interface
    (graph replay as for the configs, device us per call):
      Linear(500 -> 6565) on [8, 1500, 500] (TestLSTMRealTrain/EncoderDecoder.cs:29,75): the
        C# forward NnClGlob.LinearForward (W [1, 500, 6565], linear.cl), the Python
        Linear.forward (W [6565, 500], core/layers.py:21-33) as one NT GEMM, LinearOp.Backward
        dX (NT), dW (one TN GEMM over 12000 rows) and db (column sum);
      the LSTM of BASELINE config 3 (batch 64 x 100 steps, input 512, hidden 1024): the three
        GEMM stages of NnClGlob.Lstm / LstmBackward and the recurrent product of one step
        (lstm.cl:80-101), rotating over the 99 steps that have one."""
    from my_pytchon_opencl_lib_amd import layers
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    cap = torch.cuda.Stream()
    r = lambda *s: torch.randn(*s, device=dev, generator=g)
    out = {}

    def rec(name, fns, per, flop=0, byts=0):
        ms = graph_timed(torch, cap, fns, per)
        fns[0]()
        e = {"us": round(ms * 1e3, 1), "kernel": _native.last_plan()}
        if flop:
            tf = flop / (ms * 1e-3) / 1e12
            e.update(tflops=round(tf, 1), frac_mfma=round(tf / PEAK_FP32_MFMA_TFLOPS, 3))
        if byts:
            gbs = byts / (ms * 1e-3) / 1e9
            e.update(GBps=round(gbs, 1), frac_hbm=round(gbs / PEAK_HBM_GBS, 3))
        out[name] = e

    B, M, K, N = 8, 1500, 500, 6565
    fl = 2 * B * M * K * N
    X, W, bias, G = r(B, M, K), r(1, K, N) / 22, r(N) / 22, r(B, M, N) / 64
    rec("linear_forward_cs 12000x500->6565 +bias", [lambda: nncl.LinearForward(X, W, bias)], 5, fl)
    lin = layers.Linear(K, N, nncl, weight=r(N, K) / 22)
    rec("linear_forward_py 12000x500->6565 (NT)", [lambda: lin(X)], 5, fl)
    rec("linear_dX 12000x6565->500 (NT)", [lambda: nncl.BmmPermute(G, W, transB=True)], 5, fl)
    rec("linear_dW 500x6565 over 12000 rows (TN)", [lambda: nncl.linear_weight_grad(X, G)], 5, fl)
    rec("linear_db column sum 12000x6565", [lambda: nncl.LinearBiasBackward(G, [N])], 20,
        byts=4 * (B * M * N + N))
    del X, G, lin
    bs, seq, F, H = 64, 100, 512, 1024
    T, Gs = bs * seq, 4 * H
    Xl, Wl, bl, Gr = r(bs, seq, F), r(F, Gs) / 32, r(Gs) / 32, r(T, Gs) / 64
    Hout, U = r(bs, seq, H), r(H, Gs) / 32
    gW, gU, gB = (torch.zeros(F, Gs, device=dev), torch.zeros(H, Gs, device=dev),
                  torch.zeros(Gs, device=dev))
    rec("lstm_gemm_xw 6400x512->4096 +bias", [lambda: nncl.LstmGemmXW(Xl, Wl, bl)], 10,
        2 * T * F * Gs)
    rec("lstm_gemm_grad_x 6400x4096->512", [lambda: nncl.LstmGemmGradX(Gr, Wl, (bs, seq, F))],
        10, 2 * T * F * Gs)
    rec("lstm_gemm_grad_weights (W, U, bias)",
        [lambda: nncl.LstmGemmGradWeights(Xl, Hout, Gr, gW, gU, gB)], 5, 2 * T * (F + H) * Gs)
    XW = r(bs, seq, Gs)
    rec("lstm_recurrent_step 64x1024->4096 (+= XW_t)",
        [lambda t=t: nncl.LstmRecurrentGates(XW, Hout, U, t) for t in range(1, seq)], 1,
        2 * bs * H * Gs)
    return out


if __name__ == "__main__":
    main()
