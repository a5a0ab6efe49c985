"""The LSTM GEMM stages of the matmul path on the GPU (cs/cl_kernels/lstm.cl:273-636 via
NnClGlob.Lstm / LstmBackward, cs/compiler/NnClGlob.cs:850-1061) and the accumulating
("+=") GEMM epilogue they need, through the C ABI."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from parity import check_gemm, dev, host, sample_rows

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def small_ints(shape, seed, lo=-3, hi=3):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


def hprev(H, batch, seq):
    P = H.reshape(batch, seq, -1).copy()
    P[:, 1:] = P[:, :-1].copy()
    P[:, 0] = 0
    return P.reshape(batch * seq, -1)


def gemm_ex(A, B, C, M, N, K, transA, transB, lda, ldb, ldc, bias=None, flags=1):
    from my_pytchon_opencl_lib_amd import _native
    _native.call("migemm_gemm_strided_batched_ex",
                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), transA, transB, M, N,
                 K, ctypes.c_void_p(A.data_ptr()), lda, 0, ctypes.c_void_p(B.data_ptr()), ldb, 0,
                 None if bias is None else ctypes.c_void_p(bias.data_ptr()),
                 ctypes.c_void_p(C.data_ptr()), ldc, 0, 1, flags)


@pytest.mark.parametrize("M,K,N", [(1, 300, 257), (3, 64, 1030), (2, 300, 8200), (64, 1536, 300),
                                   (100, 70, 90),
                                   (64, 5000, 64), (300, 5000, 200), (1000, 50, 1100)])
def test_accumulate_epilogue_exact(nncl, policy, M, K, N):
    """C += A B (+ bias) with a non-zero C on every kernel family, the split-K and sliced
    GEMV paths included: exact small-integer known answers."""
    say("accumulate", policy, M, K, N)
    A = small_ints((M, K), M + K)
    B = small_ints((K, N), N + K)
    C0 = small_ints((M, N), M + N, -50, 50)
    bias = small_ints((N,), N)
    for with_bias in (False, True):
        c = dev(C0)
        gemm_ex(dev(A), dev(B), c, M, N, K, 0, 0, K, N, N, bias=dev(bias) if with_bias else None)
        expect = C0.astype(np.int64) + A.astype(np.int64) @ B.astype(np.int64)
        if with_bias:
            expect = expect + bias.astype(np.int64)
        assert np.array_equal(host(c), expect.astype(np.float32)), with_bias


def test_gemm_ex_rejects_unknown_flags(nncl):
    from my_pytchon_opencl_lib_amd import _native
    a = torch.zeros(4, 4, device="cuda:0")
    with pytest.raises(_native.MigemmArgumentError, match="flags"):
        gemm_ex(a, a.clone(), torch.zeros(4, 4, device="cuda:0"), 4, 4, 4, 0, 0, 4, 4, 4, flags=2)


@pytest.mark.parametrize("batch,seq,F,H", [(2, 5, 12, 7), (3, 1, 9, 4), (4, 50, 33, 20)])
def test_lstm_grad_weights_exact(nncl, batch, seq, F, H):
    """Accumulation onto existing gradients, the per-sequence h_{t-1} (zero at each
    sequence's first step, also for seq_len 1), exact small integers."""
    T, G = batch * seq, 4 * H
    X = small_ints((T, F), 1)
    Hout = small_ints((T, H), 2)
    Gr = small_ints((T, G), 3)
    gW0, gU0, gB0 = small_ints((F, G), 4), small_ints((H, G), 5), small_ints((G,), 6)
    tW, tU, tB = dev(gW0), dev(gU0), dev(gB0)
    say("lstm grad weights exact", batch, seq, F, H)
    nncl.LstmGemmGradWeights(dev(X.reshape(batch, seq, F)), dev(Hout.reshape(batch, seq, H)),
                             dev(Gr), tW, tU, tB)
    i64 = lambda a: a.astype(np.int64)  # noqa: E731
    assert np.array_equal(host(tW), (i64(gW0) + i64(X).T @ i64(Gr)).astype(np.float32))
    assert np.array_equal(host(tU), (i64(gU0) + i64(hprev(Hout, batch, seq)).T @ i64(Gr))
                          .astype(np.float32))
    assert np.array_equal(host(tB), (i64(gB0) + i64(Gr).sum(axis=0)).astype(np.float32))
    oW, oU, oB = oracle.lstm_gemm_grad_weights(X, Hout, Gr, gW0, gU0, gB0, batch, seq)
    assert np.array_equal(host(tW), oW) and np.array_equal(host(tU), oU)


def test_lstm_grad_weights_rejects_overlap(nncl):
    from my_pytchon_opencl_lib_amd import _native
    x = torch.zeros(2, 3, 4, device="cuda:0")
    h = torch.zeros(2, 3, 5, device="cuda:0")
    g = torch.zeros(6, 20, device="cuda:0")
    gw = torch.zeros(4, 20, device="cuda:0")
    gu = torch.zeros(5, 20, device="cuda:0")
    with pytest.raises(_native.MigemmArgumentError, match="overlap"):
        nncl.LstmGemmGradWeights(x, h, g, gw, gu, gw[0])
    with pytest.raises(_native.MigemmArgumentError, match="overlap"):
        nncl.LstmGemmGradWeights(x, h, g, gw, gu, g[0])


def test_lstm_gemms_at_baseline_size(nncl):
    """The LSTM of BASELINE config 3 (input 512, hidden 1024, 4096 gates) over a batch of 64
    sequences of 100 steps: XW, grad_X and the weight gradients against fp64 on sampled
    rows."""
    batch, seq, F, H = 64, 100, 512, 1024
    T, G = batch * seq, 4 * H
    X = oracle.normal((T, F), 32, 0)
    W = oracle.uniform((F, G), 32, 1, -1 / 32, 1 / 32)
    bias = oracle.uniform((G,), 32, 2, -1 / 32, 1 / 32)
    Hout = oracle.uniform((T, H), 32, 3, -1.0, 1.0)
    Gr = oracle.normal((T, G), 32, 4, 0.0, 1.0 / 64)
    say("lstm XW 6400x512 -> 4096")
    XW = host(nncl.LstmGemmXW(dev(X.reshape(batch, seq, F)), dev(W), dev(bias)))
    check_gemm(XW, X, W, 0, 0, bias=bias, M=T, N=G, K=F, lda=F, ldb=G, rows=sample_rows(T, 12))
    say("lstm grad_X")
    gX = host(nncl.LstmGemmGradX(dev(Gr), dev(W), (batch, seq, F))).reshape(T, F)
    check_gemm(gX, Gr, W, 0, 1, M=T, N=F, K=G, lda=G, ldb=G, rows=sample_rows(T, 12))
    say("lstm grad weights")
    z = torch.zeros
    tW, tU, tB = z(F, G, device="cuda:0"), z(H, G, device="cuda:0"), z(G, device="cuda:0")
    nncl.LstmGemmGradWeights(dev(X.reshape(batch, seq, F)), dev(Hout.reshape(batch, seq, H)),
                             dev(Gr), tW, tU, tB)
    check_gemm(host(tW), X, Gr, 1, 0, M=F, N=G, K=T, lda=F, ldb=G, rows=sample_rows(F, 10))
    P = hprev(Hout, batch, seq)
    check_gemm(host(tU), P, Gr, 1, 0, M=H, N=G, K=T, lda=H, ldb=G, rows=sample_rows(H, 10))
    ref = Gr.astype(np.float64).sum(axis=0)
    bound = (256 - 1 + 25 - 1) * 2.0 ** -24 * np.abs(Gr.astype(np.float64)).sum(axis=0)
    assert np.all(np.abs(host(tB) - ref) <= bound)


def test_lstm_recurrent_gates_over_steps(nncl):
    """The per-step recurrent product of lstm_recurrent_forward (lstm.cl:80-101) at the LSTM of
    BASELINE config 3 (batch 64, hidden 1024): XW[:, t] += h_{t-1} U in place, one GEMM per
    step. Each step is within 1e-5*sqrt(H) of fp64 (denominator |XW| + |h||U|) and of the
    restated reference arithmetic; the other steps' slices are untouched, step 0 is a no-op."""
    B, S, H = 64, 5, 1024
    XW = oracle.normal((B, S, 4 * H), 41, 0)
    U = oracle.uniform((H, 4 * H), 41, 1, -1 / 32, 1 / 32)
    Ho = oracle.uniform((B, S, H), 41, 2)
    xw, ho, u = dev(XW), dev(Ho), dev(U)
    for t in range(S):
        say("lstm recurrent gates step", t)
        before = host(xw).copy()
        nncl.LstmRecurrentGates(xw, ho, u, t)
        got = host(xw)
        others = [s for s in range(S) if s != t]
        assert np.array_equal(got[:, others], before[:, others]), f"step {t}: other steps changed"
        g = got[:, t].astype(np.float64)
        restated = oracle.lstm_recurrent_gates(XW, Ho, U, t).astype(np.float64)
        prev = Ho[:, t - 1].astype(np.float64) if t > 0 else np.zeros((B, H))
        exact = XW[:, t].astype(np.float64) + prev @ U.astype(np.float64)
        den = np.abs(XW[:, t]).astype(np.float64) + np.abs(prev) @ np.abs(U.astype(np.float64))
        tol = oracle.tolerance(H)
        assert np.max(np.abs(g - exact) / den) <= tol, t
        assert np.max(np.abs(g - restated) / den) <= 2 * tol, t
        nw = np.linalg.norm(g - exact) / np.linalg.norm(exact)
        assert nw <= tol, t
        if t == 0:
            assert np.array_equal(got[:, 0], XW[:, 0])


def test_lstm_recurrent_gates_small_ints_exact(nncl):
    """Ragged sizes (batch 5, hidden 33) with small integers: exact at every step."""
    B, S, H = 5, 4, 33
    XW = small_ints((B, S, 4 * H), 42)
    U = small_ints((H, 4 * H), 43)
    Ho = small_ints((B, S, H), 44)
    xw = dev(XW)
    for t in range(S):
        nncl.LstmRecurrentGates(xw, dev(Ho), dev(U), t)
        assert np.array_equal(host(xw)[:, t], oracle.lstm_recurrent_gates(XW, Ho, U, t)), t
