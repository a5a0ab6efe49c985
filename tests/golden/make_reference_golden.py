"""Writes tests/golden/reference_outputs.npz: the reference's OWN kernels' outputs on small
seeded inputs, so that the oracle's restatement stays pinned to the reference bit for bit
in the CPU test suite (tests/test_oracle.py::test_restatement_equals_reference_fixture),
also where the reference kernels cannot run.

The kernels are the reference sources compiled for gfx950 into oracle/_ref (oracle/Makefile,
target `ref`), run through the ROCm OpenCL runtime on the GPU by oracle/ref_runner.c with the
reference hosts' launch geometry (oracle/reference_gpu.py). This script therefore runs on a
GPU box:

    python tests/golden/make_reference_golden.py [out.npz]

Each case stores its inputs (from this repository's seeded generator), its launch arguments
and the reference kernel's output buffer. Nothing of the reference is imported; only data is
written.
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402
from oracle import reference_gpu as ref  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_outputs.npz")


def cases():
    """(name, kernel, inputs dict, launch arguments dict)."""
    u, n = oracle.uniform, oracle.normal
    out = []
    for (M, K, N, seed) in [(64, 128, 96, 50), (17, 33, 5, 51), (65, 129, 31, 52), (1, 1, 1, 53)]:
        out.append((f"matmul_tiled_{M}x{K}x{N}", "matmul_tiled",
                    {"A": u((M, K), seed, 0), "B": u((K, N), seed, 1)}, dict(M=M, K=K, N=N)))
    B, M, K, N = 4, 32, 64, 48
    out.append(("bmm_tiled_b4_32x64x48", "bmm_tiled",
                {"A": n((B, M, K), 54, 0), "B": n((B, K, N), 54, 1)},
                dict(M=M, K=K, N=N, batch=B, sA=M * K, sB=K * N, sC=M * N)))
    B, M, K, N = 3, 40, 24, 36  # B broadcast (batch stride 0, NnClGlob.cs:467)
    out.append(("bmm_tiled_bcast_b3_40x24x36", "bmm_tiled",
                {"A": n((B, M, K), 55, 0), "B": n((1, K, N), 55, 1)},
                dict(M=M, K=K, N=N, batch=B, sA=M * K, sB=0, sC=M * N)))
    B, M, K, N = 2, 33, 47, 29
    for ta in (0, 1):
        for tb in (0, 1):
            A = n((B, K, M) if ta else (B, M, K), 56 + 2 * ta + tb, 0)
            Bm = n((B, N, K) if tb else (B, K, N), 56 + 2 * ta + tb, 1)
            out.append((f"bmm_permute_tiled_t{ta}{tb}_b2_33x47x29", "bmm_permute_tiled",
                        {"A": A, "B": Bm},
                        dict(M=M, K=K, N=N, batch=B, sA=M * K, sB=K * N, sC=M * N, transA=ta,
                             transB=tb)))
    B, M, K, N = 2, 37, 53, 41
    out.append(("linear_forward_tiled_b2_37x53x41", "linear_forward_tiled",
                {"A": n((B, M, K), 60, 0), "B": u((K, N), 60, 1, -0.2, 0.2),
                 "bias": u((N,), 60, 2, -0.2, 0.2)},
                dict(M=M, K=K, N=N, batch=B, sA=M * K, sC=M * N)))
    for dims, axes, seed in [((3, 17, 29), (0, 2, 1), 61), ((2, 3, 5, 7), (3, 1, 0, 2), 62)]:
        meta = np.array(list(dims) + list(axes), dtype=np.int32)
        out.append((f"tensor_permute_{'x'.join(map(str, dims))}", "tensor_permute",
                    {"A": n(dims, seed, 0), "B": meta}, dict(M=len(dims))))
    T, F, H = 45, 30, 11
    G = 4 * H
    out.append(("lstm_gemm_xw_45x30x44", "lstm_gemm_xw",
                {"A": n((T, F), 63, 0), "B": u((F, G), 63, 1, -0.2, 0.2),
                 "bias": u((G,), 63, 2, -0.2, 0.2)}, dict(M=T, K=F, N=G)))
    out.append(("lstm_gemm_grad_x_45x44x30", "lstm_gemm_grad_x",
                {"A": n((T, G), 64, 0), "B": u((F, G), 64, 1, -0.2, 0.2)}, dict(M=T, K=G, N=F)))
    return out


def main(path=OUT):
    print("writing", path, flush=True)
    data, meta = {}, {}
    for name, kernel, inputs, args in cases():
        res, info = ref.run(kernel, inputs["A"], inputs.get("B"), inputs.get("bias"), reps=1,
                            **args)
        for k, v in inputs.items():
            data[f"{name}.{k}"] = v
        data[f"{name}.out"] = res
        meta[name] = {"kernel": kernel, "args": args}
        print(name, info["device"], flush=True)
    # lstm_gemm_grad_weights accumulates onto non-zero initial gradients
    batch, seq, F, H = 3, 5, 13, 7
    T, G = batch * seq, 4 * H
    X, Ho, Gr = oracle.normal((T, F), 65, 0), oracle.normal((T, H), 65, 1), oracle.normal((T, G), 65, 2)
    g0 = [oracle.normal((F, G), 65, 3), oracle.normal((H, G), 65, 4), oracle.normal((G,), 65, 5)]
    (rW, rU, rB), info = ref.lstm_gemm_grad_weights(X, Ho, Gr, *g0, batch, seq)
    name = "lstm_gemm_grad_weights_b3_s5_f13_h7"
    for k, v in {"X": X, "H_out": Ho, "G": Gr, "gW0": g0[0], "gU0": g0[1], "gB0": g0[2],
                 "gW": rW, "gU": rU, "gB": rB}.items():
        data[f"{name}.{k}"] = v
    meta[name] = {"kernel": "lstm_gemm_grad_weights",
                  "args": {"batch_size": batch, "seq_len": seq}}
    # lstm_recurrent_forward: the stored raw gates of every step
    B, S, H = 3, 4, 20
    XW, U = oracle.normal((B, S, 4 * H), 66, 0), oracle.uniform((H, 4 * H), 66, 1, -0.3, 0.3)
    Ho, gates, cells, info = ref.lstm_recurrent_forward(XW, U)
    name = "lstm_recurrent_forward_b3_s4_h20"
    for k, v in {"XW": XW, "U": U, "H_out": Ho, "gates": gates, "cells": cells}.items():
        data[f"{name}.{k}"] = v
    meta[name] = {"kernel": "lstm_recurrent_forward", "args": {"B": B, "S": S, "H": H}}
    # lstm_hid_forward: the stored raw gates of every step (bias-first chains over x_t W and
    # h_{t-1} U), with a non-zero incoming state, at two ragged sizes
    for (B, S, F, H, seed) in [(3, 4, 10, 12, 67), (2, 3, 33, 20, 68)]:
        X = oracle.normal((B, S, F), seed, 0)
        W = oracle.uniform((F, 4 * H), seed, 1, -0.3, 0.3)
        U = oracle.uniform((H, 4 * H), seed, 2, -0.3, 0.3)
        bias = oracle.uniform((4 * H,), seed, 3, -0.3, 0.3)
        Hp = oracle.uniform((B, H), seed, 4, -0.5, 0.5)
        Cp = oracle.uniform((B, H), seed, 5, -0.5, 0.5)
        Ho, gates, fH, fC, info = ref.lstm_hid_forward(X, W, U, bias, Hp, Cp)
        name = f"lstm_hid_forward_b{B}_s{S}_f{F}_h{H}"
        for k, v in {"X": X, "W": W, "U": U, "bias": bias, "H_prev": Hp, "C_prev": Cp,
                     "H_out": Ho, "gates": gates, "final_H": fH, "final_C": fC}.items():
            data[f"{name}.{k}"] = v
        meta[name] = {"kernel": "lstm_hid_forward", "args": {"B": B, "S": S, "F": F, "H": H}}
        print(name, info["device"], flush=True)
    data["_meta"] = np.frombuffer(json.dumps({"device": info["device"], "cases": meta},
                                             sort_keys=True).encode(), dtype=np.uint8)
    np.savez_compressed(path, **data)
    print("wrote", path, len(meta), "cases", flush=True)


if __name__ == "__main__":
    main(*sys.argv[1:])
