"""The measurement harness's host logic, on the CPU: the one-GPU contract of `bench.py
--gpus`, the timed-launch selection of `--summarize-trace` (which the committed kernel-trace
profile and `roofline.frac_profiled` rest on), the committed profiles that `roofline`
reads, and the per-config algorithmic work the roofline fractions divide by."""
import csv
import json
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def run_bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_exits_with_a_message():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


KERNEL = ("void migemm::(anonymous namespace)::gemm_direct_kernel<256, 256, 8, 2, {a}, {b}, 32, "
          "2, 2, 1, 4, 4>(migemm::TiledArgs)")
FORMS = {"NN": ("true", "false"), "NT": ("true", "true"), "TN": ("false", "false")}


def test_summarize_trace_averages_exactly_the_timed_launches(tmp_path):
    """Each form runs once to record its plan, W warm-up times, S timed times, and may run
    again later (other configs); only the S timed launches may enter PROFILED_US."""
    steps, warmup = 4, 3
    rng = np.random.default_rng(1)
    rows, t = [], 1_000_000
    expect = {}
    durations = {f: [] for f in FORMS}
    for phase, count in (("plan", 1), ("warm", warmup), ("timed", steps), ("later", 2)):
        for _ in range(count):
            for f in FORMS:
                # timed launches around 900 us, every other launch far off, so a window
                # shifted by one launch changes the average
                us = 900.0 + rng.integers(0, 20) if phase == "timed" else 5000.0
                durations[f].append((phase, us))
                rows.append({"Kernel_Name": KERNEL.format(a=FORMS[f][0], b=FORMS[f][1]),
                             "Start_Timestamp": str(t), "End_Timestamp": str(t + int(us * 1e3))})
                t += int(us * 1e3) + 5000
    # an unrelated kernel in between must not disturb the selection
    rows.append({"Kernel_Name": "void at::native::elementwise_kernel<128, 4>(int)",
                 "Start_Timestamp": str(t), "End_Timestamp": str(t + 2000)})
    for f in FORMS:
        expect[f] = np.mean([us for ph, us in durations[f] if ph == "timed"])
    d = tmp_path / "trace" / "host"
    d.mkdir(parents=True)
    rng.shuffle(rows)  # the summary orders launches by their start time itself
    with open(d / "bench_kernel_trace.csv", "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=["Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        w.writerows(rows)
    r = run_bench("--summarize-trace", str(tmp_path / "trace"), "--steps", str(steps),
                  "--warmup", str(warmup))
    assert r.returncode == 0, r.stderr
    got = {ln.split()[1]: float(ln.split()[2]) for ln in r.stdout.splitlines()
           if ln.startswith("PROFILED_US")}
    assert set(got) == set(FORMS)
    for f in FORMS:
        assert got[f] == pytest.approx(expect[f], abs=0.06), f


def test_committed_profiles_feed_the_roofline():
    """roofline.traffic and roofline.frac_profiled come from the committed profiles: every
    4096^3 form has a traffic line (HBM bytes >= the algorithmic 201 MB) and a profiled
    duration no shorter than the MFMA floor at the nominal clock (873.7 us)."""
    alg = 4 * 3 * 4096 * 4096
    prof = bench.load_profiled()
    for f in FORMS:
        traffic = bench.load_traffic(f)
        assert traffic is not None and alg <= traffic < 4 * alg, (f, traffic)
        floor_us = bench.FLOP_4096 / (bench.PEAK_FP32_MFMA_TFLOPS * 1e12) * 1e6
        assert floor_us == pytest.approx(873.7, abs=0.1)
        assert floor_us <= prof[f] < 1.2 * floor_us, (f, prof[f])


def test_algorithmic_work_per_config():
    """FLOP = 2 M N K batch; bytes = 4 (inputs + output), a broadcast operand once, the bias
    counted in bytes only."""
    c = bench.CONFIGS
    assert c["1_nn_256"][:2] == (2 * 256 ** 3, 4 * 3 * 256 ** 2)
    assert c["2a_bmm_qk"][0] == 2 * 32 * 128 * 64 * 128
    assert c["2a_bmm_qk"][1] == 4 * 32 * (128 * 64 + 64 * 128 + 128 * 128)
    assert c["2b_bmm_pv"][1] == 4 * 32 * (128 * 128 + 128 * 64 + 128 * 64)
    M, K, N = 64, 1536, 4096
    assert c["3_lstm_gate_step"][:2] == (2 * M * N * K, 4 * (M * K + K * N + M * N + N))
    # the stateful form reads x_t (512) and h_{t-1} (1024) separately: the same bytes
    assert c["3h_lstm_hid_step"][:2] == c["3_lstm_gate_step"][:2]
    assert c["5a_ragged"][:2] == (2 * 1000 * 3000 * 777,
                                  4 * (1000 * 777 + 777 * 3000 + 1000 * 3000))
    assert c["5b_gemv"][:2] == (2 * 4096 * 11008, 4 * (4096 + 4096 * 11008 + 11008))
    assert {v[2] for v in c.values()} <= {"mfma", "hbm"}
    assert c["5b_gemv"][2] == "hbm" and c["3_lstm_gate_step"][2] == "mfma"
