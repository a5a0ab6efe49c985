"""Writes the committed golden fixtures of the matmul path (run from the repo root):

  tests/golden/generator.json   first values of the synthetic-input generator
  tests/golden/small_cases.npz  small GEMM / BMM / NT / TN / bias cases: inputs, the
                                oracle's restatement output (the reference kernels'
                                arithmetic) and the fp64 result

Produced by this repository's own oracle (oracle/oracle.c); nothing of the reference is
imported or run. Regenerate with:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# (name, batch, M, K, N, transA, transB, bias, broadcastB)
CASES = [
    ("nn_1x1x1", 1, 1, 1, 1, 0, 0, False, False),
    ("nn_17x33x5", 1, 17, 33, 5, 0, 0, False, False),
    ("nn_64x128x96", 1, 64, 128, 96, 0, 0, False, False),
    ("bmm_b4_32x64x48", 4, 32, 64, 48, 0, 0, False, False),
    ("nt_b4_32x64x48", 4, 32, 64, 48, 0, 1, False, False),
    ("tn_b4_32x64x48", 4, 32, 64, 48, 1, 0, False, False),
    ("bias_65x129x31", 1, 65, 129, 31, 0, 0, True, False),
    ("bcast_b3_40x24x36", 3, 40, 24, 36, 0, 0, False, True),
]


def main():
    gen = {"uniform": [], "normal": []}
    for seed, tid, lo, hi in [(0, 0, -1.0, 1.0), (2, 1, -1 / 32, 1 / 32), (4, 3, -1.0, 1.0)]:
        gen["uniform"].append({"seed": seed, "tensor_id": tid, "lo": lo, "hi": hi,
                               "values": oracle.uniform((16,), seed, tid, lo, hi).tolist()})
    for seed, tid, mean, std in [(1, 0, 0.0, 1.0), (3, 2, 0.0, 1 / 64)]:
        gen["normal"].append({"seed": seed, "tensor_id": tid, "mean": mean, "std": std,
                              "values": oracle.normal((16,), seed, tid, mean, std).tolist()})
    with open(os.path.join(OUT, "generator.json"), "w") as f:
        json.dump(gen, f, indent=1)

    arrays = {}
    meta = []
    for idx, (name, batch, M, K, N, ta, tb, has_bias, bcast) in enumerate(CASES):
        A = oracle.uniform((batch, K, M) if ta else (batch, M, K), 100 + idx, 0)
        bb = 1 if bcast else batch
        B = oracle.uniform((bb, N, K) if tb else (bb, K, N), 100 + idx, 1)
        bias = oracle.uniform((N,), 100 + idx, 2) if has_bias else None
        if has_bias:
            C = oracle.linear_forward(A, B[0], bias)
        else:
            C = oracle.bmm_permute(A, B, transA=bool(ta), transB=bool(tb))
        lda = M if ta else K
        ldb = K if tb else N
        C64 = oracle.gemm_f64(A, B, ta, tb, bias, M=M, N=N, K=K, lda=lda, ldb=ldb,
                              sA=A.shape[1] * A.shape[2], sB=0 if bb == 1 else K * N,
                              batch=batch)
        arrays[f"{name}.A"] = A
        arrays[f"{name}.B"] = B
        if has_bias:
            arrays[f"{name}.bias"] = bias
        arrays[f"{name}.C_ref"] = C
        arrays[f"{name}.C64"] = C64
        meta.append({"name": name, "batch": batch, "M": M, "K": K, "N": N, "transA": ta,
                     "transB": tb, "bias": has_bias, "broadcastB": bcast})
    arrays["meta"] = np.frombuffer(json.dumps(meta).encode(), dtype=np.uint8)
    np.savez_compressed(os.path.join(OUT, "small_cases.npz"), **arrays)
    print("wrote", len(meta), "cases")


if __name__ == "__main__":
    main()
