"""Runs the reference's own OpenCL kernels on the GPU -- TEST INFRASTRUCTURE ONLY.

oracle/_ref/ holds the reference kernel sources compiled for gfx950 (oracle/Makefile, target
`ref`, built from /root/reference when it is mounted) and ref_runner, this repository's
OpenCL host for them (oracle/ref_runner.c). Each call runs one kernel in a child process
through the ROCm OpenCL runtime with the reference hosts' launch geometry and returns its
output buffer, so the oracle's restatement can be compared bit-for-bit with the reference
arithmetic as the GPU's OpenCL compiler emits it.
"""
import json
import os
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(HERE, "_ref")
RUNNER = os.path.join(REF_DIR, "ref_runner")

CODE_OBJECT = {
    "matmul_tiled": "matmul.co",
    "bmm_tiled": "matmul.co",
    "bmm_permute_tiled": "bmm_permute_tiled.co",
    "linear_forward_tiled": "linear.co",
    "tensor_permute": "permute.co",
    "lstm_gemm_xw": "lstm.co",
    "lstm_gemm_grad_x": "lstm.co",
    "lstm_gemm_grad_weights": "lstm.co",
    "lstm_recurrent_forward": "lstm.co",
    "lstm_hid_forward": "lstm.co",
}


class Unavailable(RuntimeError):
    """The reference kernels cannot run here (not built, or no OpenCL GPU device)."""


def available():
    return os.path.exists(RUNNER) and all(
        os.path.exists(os.path.join(REF_DIR, f)) for f in set(CODE_OBJECT.values()))


def run(kernel, A, B=None, bias=None, M=0, K=0, N=0, batch=1, sA=0, sB=0, sC=0, transA=0,
        transB=0, reps=3, out_elems=None, init=None):
    """Run one reference kernel; returns (flat float32 output, info dict)."""
    if not available():
        raise Unavailable("oracle/_ref is not built (needs the reference sources at build time)")
    with tempfile.TemporaryDirectory() as td:
        def dump(name, arr, dtype=np.float32):
            if arr is None:
                return "-"
            path = os.path.join(td, name)
            np.ascontiguousarray(arr, dtype=dtype).tofile(path)
            return path

        a = dump("a.bin", A)
        b = dump("b.bin", B, np.int32 if kernel == "tensor_permute" else np.float32)
        bi = dump("bias.bin", bias)
        out = os.path.join(td, "out.bin")
        if init is not None:
            np.ascontiguousarray(init, dtype=np.float32).tofile(out + ".init")
        cmd = [RUNNER, os.path.join(REF_DIR, CODE_OBJECT[kernel]), kernel, str(M), str(K),
               str(N), str(batch), str(sA), str(sB), str(sC), str(int(transA)),
               str(int(transB)), a, b, bi, out, str(reps)]
        p = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
        if p.returncode == 3:
            raise Unavailable(p.stderr.strip())
        if p.returncode != 0:
            raise RuntimeError(f"ref_runner failed ({p.returncode}): {p.stderr.strip()}")
        info = json.loads(p.stdout.strip().splitlines()[-1])
        res = np.fromfile(out, dtype=np.float32)
    if out_elems is not None:
        res = res[:out_elems]
    return res, info


def lstm_gemm_grad_weights(X, H_out, G, grad_W, grad_U, grad_bias, batch_size, seq_len,
                           reps=1):
    """Runs the reference lstm_gemm_grad_weights (cs/cl_kernels/lstm.cl:459) on the given
    initial gradients; returns (grad_W, grad_U, grad_bias) after one accumulation."""
    F = X.shape[1]
    H = H_out.shape[-1]
    init = np.concatenate([np.ravel(grad_W), np.ravel(grad_U), np.ravel(grad_bias)])
    res, info = run("lstm_gemm_grad_weights", X, H_out, G, M=batch_size, K=seq_len, N=F,
                    batch=H, reps=reps, init=init)
    nW, nU = F * 4 * H, H * 4 * H
    return (res[:nW].reshape(F, 4 * H), res[nW:nW + nU].reshape(H, 4 * H),
            res[nW + nU:].reshape(4 * H)), info


def lstm_recurrent_forward(XW, U, reps=1):
    """Runs the reference lstm_recurrent_forward (cs/cl_kernels/lstm.cl:40-127) over all
    steps of XW [B, S, 4H]; returns (H_out [B, S, H], raw gates [S, B, 4H], cell states
    [S, B, H]) -- the kernel's workspace [S, B, 5H] split into its gate and cell parts."""
    B, S, Gt = XW.shape
    H = Gt // 4
    res, info = run("lstm_recurrent_forward", XW, U, M=B, K=S, N=H, reps=reps)
    n_h = B * S * H
    ws = res[n_h:].reshape(S, B, 5 * H)
    return res[:n_h].reshape(B, S, H), ws[:, :, :4 * H], ws[:, :, 4 * H:], info


def lstm_hid_forward(X, W, U, bias, H_prev, C_prev, reps=1):
    """Runs the reference lstm_hid_forward (cs/cl_kernels/lstm.cl:788-870, one work-item per
    sequence over all steps of X [B, S, F]); returns (H_out [B, S, H], raw gates [S, B, 4H]
    -- the kernel's workspace --, final_H [B, H], final_C [B, H], info)."""
    B, S, F = X.shape
    H = U.shape[0]
    A = np.concatenate([np.ravel(X), np.ravel(H_prev), np.ravel(C_prev)]).astype(np.float32)
    Bm = np.concatenate([np.ravel(W), np.ravel(U)]).astype(np.float32)
    res, info = run("lstm_hid_forward", A, Bm, bias, M=B, K=S, N=H, batch=F, reps=reps)
    n = [B * S * H, S * B * 4 * H, B * H, B * H]
    o = np.cumsum([0] + n)
    return (res[o[0]:o[1]].reshape(B, S, H), res[o[1]:o[2]].reshape(S, B, 4 * H),
            res[o[2]:o[3]].reshape(B, H), res[o[3]:o[4]].reshape(B, H), info)
