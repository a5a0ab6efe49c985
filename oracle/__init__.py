"""CPU oracle for the matmul path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may import this
package. It is the checker, never the thing measured or shipped: the product library
(my_pytchon_opencl_lib_amd/libmigemm.so) has no CPU fallback.

Contents
  * ctypes bindings of oracle.c (the C restatement of cl_kernels/matmul.cl,
    cs/cl_kernels/bmm_permute_tiled.cl, linear.cl, lstm.cl:273-367, permute.cl,
    reduce_sum_axis.cl; "cs/" = csharp/cstorchcl/cstorchcl/ of the reference);
  * the synthetic-input generator (SplitMix64 counter-based) in C and a numpy mirror;
  * the accuracy metrics of the parity bar: normwise ||C - C64||_F / ||C64||_F and
    componentwise max |C - C64| / (|A||B|), both required <= 1e-5 * sqrt(K).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def build():
    """Compile oracle.c with gcc (no GPU needed)."""
    subprocess.run(["make", "-s", "-C", HERE, "-B", "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        f = ctypes.POINTER(ctypes.c_float)
        d = ctypes.POINTER(ctypes.c_double)
        i32 = ctypes.c_int
        i64 = ctypes.c_int64
        u64 = ctypes.c_uint64
        i = ctypes.POINTER(ctypes.c_int)
        L.oracle_fill_uniform.argtypes = [f, i64, u64, u64, ctypes.c_double, ctypes.c_double]
        L.oracle_fill_normal.argtypes = [f, i64, u64, u64, ctypes.c_double, ctypes.c_double]
        L.oracle_matmul_tiled.argtypes = [f, f, f, i32, i32, i32]
        L.oracle_bmm_tiled.argtypes = [f, f, f, i32, i32, i32, i32, i32, i32, i32]
        L.oracle_bmm_permute_tiled.argtypes = [f, f, f] + [i32] * 9
        L.oracle_linear_forward_tiled.argtypes = [f, f, f, f] + [i32] * 6
        L.oracle_lstm_gemm_xw.argtypes = [f, f, f, f, i32, i32, i32]
        L.oracle_lstm_gemm_grad_x.argtypes = [f, f, f, i32, i32, i32]
        L.oracle_lstm_gemm_grad_weights.argtypes = [f] * 6 + [i32] * 4
        L.oracle_lstm_recurrent_gates.argtypes = [f, f, f, f, i32, i32, i32, i32]
        L.oracle_lstm_hid_gates.argtypes = [f] * 7 + [i32] * 5
        L.oracle_tensor_permute.argtypes = [f, f, i, i, i32]
        L.oracle_reduce_sum_axis.argtypes = [f, f, i32, i32, i32]
        L.oracle_linear_bias_backward.argtypes = [f, f, i32, i32]
        L.oracle_gemm_f64.argtypes = [i32, i32, i32, i32, i32, f, i64, i64, f, i64, i64, f, d,
                                      i32, i32, i32]
        L.oracle_gemm_absprod.argtypes = L.oracle_gemm_f64.argtypes
        L.oracle_matmul_rows.argtypes = [f, f, f, i32, i32, i32, i32, i32, i32]
        L.oracle_openmp_enabled.restype = i32
        _lib = L
    return _lib


def _fp(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _dp(a):
    assert a.dtype == np.float64 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_double))


def _ip(a):
    a = np.ascontiguousarray(a, dtype=np.int32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


# ------------------------------------------------------------------------------------
# Generator (C) and its numpy mirror.

def uniform(shape, seed, tensor_id, lo=-1.0, hi=1.0):
    out = np.empty(shape, dtype=np.float32)
    lib().oracle_fill_uniform(_fp(out), out.size, seed, tensor_id, lo, hi)
    return out


def normal(shape, seed, tensor_id, mean=0.0, std=1.0):
    out = np.empty(shape, dtype=np.float32)
    lib().oracle_fill_normal(_fp(out), out.size, seed, tensor_id, mean, std)
    return out


_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64_np(x):
    with np.errstate(over="ignore"):
        x = x + np.uint64(0x9E3779B97F4A7C15)
        x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return x ^ (x >> np.uint64(31))


def _key_np(seed, tensor_id):
    with np.errstate(over="ignore"):
        s = _splitmix64_np(np.array([seed], dtype=np.uint64))
        t = np.array([tensor_id], dtype=np.uint64) * np.uint64(0xD1B54A32D192ED03)
        return _splitmix64_np(s ^ t)[0]


def uniform_np(shape, seed, tensor_id, lo=-1.0, hi=1.0):
    """numpy mirror of oracle_fill_uniform (identical values)."""
    n = int(np.prod(shape))
    with np.errstate(over="ignore"):
        r = _splitmix64_np(_key_np(seed, tensor_id) + np.arange(n, dtype=np.uint64))
    u = (r >> np.uint64(40)).astype(np.float64) * (1.0 / 16777216.0)
    return (lo + (hi - lo) * u).astype(np.float32).reshape(shape)


def normal_np(shape, seed, tensor_id, mean=0.0, std=1.0):
    """numpy mirror of oracle_fill_normal (identical up to libm cos/log last-bit
    differences, which the fp32 rounding absorbs except in rare ties)."""
    n = int(np.prod(shape))
    with np.errstate(over="ignore"):
        r = _splitmix64_np(_key_np(seed, tensor_id) + np.arange(n, dtype=np.uint64))
    u1 = ((r >> np.uint64(38)).astype(np.float64) + 0.5) * (1.0 / 67108864.0)
    u2 = ((r >> np.uint64(12)) & np.uint64(0x3FFFFFF)).astype(np.float64) * (1.0 / 67108864.0)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mean + std * z).astype(np.float32).reshape(shape)


# ------------------------------------------------------------------------------------
# Reference-kernel restatements.

def matmul_tiled(A, B):
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    C = np.empty((M, N), dtype=np.float32)
    lib().oracle_matmul_tiled(_fp(A), _fp(B), _fp(C), M, K, N)
    return C


def bmm_tiled(A, B, M, K, N, sA, sB, sC, batch):
    """Flat-buffer form of matmul.cl:78 (A, B flat float32 arrays)."""
    C = np.zeros(max(1, (batch - 1) * sC + M * N), dtype=np.float32)
    lib().oracle_bmm_tiled(_fp(A), _fp(B), _fp(C), M, K, N, sA, sB, sC, batch)
    return C


def bmm(A, B):
    """A [b,M,K] @ B [b or 1,K,N] with the reference's stride-0 broadcast of B."""
    b, M, K = A.shape
    bb, K2, N = B.shape
    assert K == K2 and bb in (b, 1)
    C = np.empty((b, M, N), dtype=np.float32)
    lib().oracle_bmm_tiled(_fp(A), _fp(B), _fp(C), M, K, N, M * K, 0 if bb == 1 else K * N,
                           M * N, b)
    return C


def bmm_permute(A, B, transA=False, transB=False):
    """Mirror of NnClGlob.BmmPermute shapes (cs/compiler/NnClGlob.cs:1702-1751)."""
    batch = A.shape[0]
    M = A.shape[2] if transA else A.shape[1]
    K = A.shape[1] if transA else A.shape[2]
    N = B.shape[1] if transB else B.shape[2]
    sA = 0 if A.shape[0] == 1 else A.shape[1] * A.shape[2]
    sB = 0 if B.shape[0] == 1 else B.shape[1] * B.shape[2]
    C = np.empty((batch, M, N), dtype=np.float32)
    lib().oracle_bmm_permute_tiled(_fp(A), _fp(B), _fp(C), M, K, N, sA, sB, M * N,
                                   int(transA), int(transB), batch)
    return C


def linear_forward(X, W, bias):
    batch, M, K = X.shape
    N = W.shape[-1]
    Y = np.empty((batch, M, N), dtype=np.float32)
    lib().oracle_linear_forward_tiled(_fp(X), _fp(np.ascontiguousarray(W.reshape(K, N))),
                                      _fp(bias), _fp(Y), M, K, N, M * K, M * N, batch)
    return Y


def lstm_gemm_xw(X, W, bias):
    T, F = X.shape
    G = W.shape[1]
    Y = np.empty((T, G), dtype=np.float32)
    lib().oracle_lstm_gemm_xw(_fp(X), _fp(W), _fp(bias), _fp(Y), T, F, G)
    return Y


def lstm_gemm_grad_x(G, W):
    """lstm.cl:372-457: grad_X[T, F] = G[T, 4H] * W^T, W stored [F, 4H]."""
    T, Gt = G.shape
    F = W.shape[0]
    gX = np.empty((T, F), dtype=np.float32)
    lib().oracle_lstm_gemm_grad_x(_fp(G), _fp(W), _fp(gX), T, F, Gt)
    return gX


def lstm_gemm_grad_weights(X, H_out, G, grad_W, grad_U, grad_bias, batch_size, seq_len):
    """lstm.cl:459-636: returns (grad_W + X^T G, grad_U + H_prev^T G, grad_bias + sum G)
    with the reference's per-output fp32 arithmetic; the inputs are not modified."""
    T, F = X.shape
    H = H_out.shape[-1]
    gW = np.array(grad_W, dtype=np.float32, copy=True)
    gU = np.array(grad_U, dtype=np.float32, copy=True)
    gB = np.array(grad_bias, dtype=np.float32, copy=True)
    lib().oracle_lstm_gemm_grad_weights(_fp(X), _fp(H_out), _fp(G), _fp(gW), _fp(gU), _fp(gB),
                                        batch_size, seq_len, F, H)
    return gW, gU, gB


def lstm_recurrent_gates(XW, H_out, U, t):
    """lstm.cl:80-101: the raw gates [B, 4H] of step t, XW [B, S, 4H] + h_{t-1} U with the
    reference's fp32 arithmetic (an fma chain over h ascending, starting from the XW
    value); h_{t-1} = H_out[:, t-1] (zero at t = 0)."""
    B, S, Gt = XW.shape
    H = U.shape[0]
    gates = np.empty((B, Gt), dtype=np.float32)
    lib().oracle_lstm_recurrent_gates(_fp(XW), _fp(H_out), _fp(U), _fp(gates), B, S, H, t)
    return gates


def lstm_hid_gates(X, W, U, bias, H_prev, H_out, t):
    """lstm.cl:826-844: the raw gates [B, 4H] of step t of lstm_hid_forward with the
    reference's fp32 arithmetic: bias[g] as the accumulator's start, then one fma chain over
    X[b, t, :] against W and over h_{t-1} against U; h_{t-1} = H_prev [B, H] at t = 0, else
    H_out[:, t-1] ([B, S, H])."""
    B, S, F = X.shape
    H = U.shape[0]
    gates = np.empty((B, 4 * H), dtype=np.float32)
    Hp = np.ascontiguousarray(H_prev, dtype=np.float32)
    Ho = np.ascontiguousarray(H_out, dtype=np.float32)
    lib().oracle_lstm_hid_gates(_fp(X), _fp(W), _fp(U), _fp(bias), _fp(Hp), _fp(Ho),
                                _fp(gates), B, S, F, H, t)
    return gates


def tensor_permute(x, axes):
    dims, dp = _ip(x.shape)
    ax, ap = _ip(axes)
    out = np.empty([x.shape[a] for a in axes], dtype=np.float32)
    lib().oracle_tensor_permute(_fp(x), _fp(out), dp, ap, x.ndim)
    return out


def reduce_sum_axis(x, axis):
    outer = int(np.prod(x.shape[:axis])) if axis > 0 else 1
    inner = int(np.prod(x.shape[axis + 1:])) if axis + 1 < x.ndim else 1
    out_shape = list(x.shape)
    out_shape[axis] = 1
    Y = np.empty(out_shape, dtype=np.float32)
    lib().oracle_reduce_sum_axis(_fp(x), _fp(Y), outer, x.shape[axis], inner)
    return Y


def linear_bias_backward(grad_output):
    N = grad_output.shape[-1]
    rows = grad_output.size // N
    gb = np.empty((N,), dtype=np.float32)
    lib().oracle_linear_bias_backward(_fp(grad_output), _fp(gb), rows, N)
    return gb


def gemm_f64(A, B, transA=False, transB=False, bias=None, M=None, N=None, K=None,
             lda=None, ldb=None, sA=0, sB=0, batch=1, rows=None):
    """fp64 evaluation of C_b = opA(A_b) opB(B_b) (+bias) over flat or shaped inputs.
    Returns [batch, r1-r0, N] float64 for the row range `rows` (default all)."""
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, M)
    out = np.empty((batch, r1 - r0, N), dtype=np.float64)
    bp = _fp(np.ascontiguousarray(bias, dtype=np.float32)) if bias is not None else None
    lib().oracle_gemm_f64(int(transA), int(transB), M, N, K, _fp(A), lda, sA, _fp(B), ldb, sB,
                          bp, _dp(out), batch, r0, r1)
    return out


def gemm_absprod(A, B, transA=False, transB=False, bias=None, M=None, N=None, K=None,
                 lda=None, ldb=None, sA=0, sB=0, batch=1, rows=None):
    A = np.ascontiguousarray(A, dtype=np.float32)
    B = np.ascontiguousarray(B, dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, M)
    out = np.empty((batch, r1 - r0, N), dtype=np.float64)
    bp = _fp(np.ascontiguousarray(bias, dtype=np.float32)) if bias is not None else None
    lib().oracle_gemm_absprod(int(transA), int(transB), M, N, K, _fp(A), lda, sA, _fp(B), ldb,
                              sB, bp, _dp(out), batch, r0, r1)
    return out


def matmul_rows(A, B, row0, row1, threads=1):
    """CPU-baseline evaluation of the matmul_tiled arithmetic on rows [row0, row1)."""
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((row1 - row0, N), dtype=np.float32)
    lib().oracle_matmul_rows(_fp(A), _fp(B), _fp(C), M, K, N, row0, row1, threads)
    return C


# ------------------------------------------------------------------------------------
# Parity metrics.

def tolerance(K):
    """The parity bar of the matmul path: relative error <= 1e-5 * sqrt(K)."""
    return 1e-5 * float(np.sqrt(K))


def errors(C, C64, absprod):
    """(normwise, componentwise) relative errors of C against the fp64 result C64."""
    C = np.asarray(C, dtype=np.float64)
    diff = np.abs(C - C64)
    den = np.linalg.norm(C64.ravel())
    normwise = float(np.linalg.norm(diff.ravel()) / den) if den > 0 else float(diff.max(initial=0))
    with np.errstate(divide="ignore", invalid="ignore"):
        comp = np.where(absprod > 0, diff / absprod, np.where(diff > 0, np.inf, 0.0))
    return normwise, float(comp.max(initial=0.0))
