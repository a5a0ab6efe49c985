"""The reference's own OpenCL kernels, run on the GPU, against the oracle and the HIP path.

oracle/_ref holds cl_kernels/matmul.cl, cl_kernels/permute.cl and the C# tree's
bmm_permute_tiled.cl / linear.cl compiled for gfx950 (oracle/Makefile target `ref`), run by
oracle/ref_runner.c through the ROCm OpenCL runtime with the reference hosts' launch
geometry. Two claims are checked on identical seeded inputs:
  1. the oracle's C restatement reproduces the reference kernels bit-for-bit (this pins the
     restatement's fp32 fma-chain arithmetic against the reference itself);
  2. the HIP path is within 1e-5*sqrt(K) (relative, componentwise |A||B|) of the
     reference's output, and of fp64.
A GPU run without oracle/_ref fails: the prebuilt reference kernels travel with the tree
(built where the reference sources are mounted). Skipped (with the reason) only when the box
has no OpenCL GPU device; tests/golden/reference_outputs.npz keeps the restatement pinned to
these kernels' outputs on the CPU either way (tests/test_oracle.py).
"""
import numpy as np
import pytest

import oracle
from oracle import reference_gpu as ref
from parity import check_full, check_gemm, dev, host, sample_rows

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def run_ref(*args, **kw):
    if not ref.available():
        pytest.fail("oracle/_ref is missing: build it where the reference sources are mounted "
                    "(__graft_entry__.build()) so the reference kernels travel with the tree")
    try:
        return ref.run(*args, **kw)
    except ref.Unavailable as e:
        pytest.skip(f"reference OpenCL kernels unavailable: {e}")


def require_ref():
    if not ref.available():
        pytest.fail("oracle/_ref is missing: build it where the reference sources are mounted")


def ulp_report(a, b):
    ai = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return int(np.max(np.abs(ai - bi))) if ai.size else 0


def rel_distance(C, R, absprod):
    d = np.abs(np.asarray(C, np.float64) - np.asarray(R, np.float64))
    with np.errstate(divide="ignore", invalid="ignore"):
        return float(np.max(np.where(absprod > 0, d / absprod, np.where(d > 0, np.inf, 0.0))))


@pytest.mark.parametrize("M,K,N,seed", [(256, 256, 256, 0), (64, 128, 96, 10), (65, 129, 31, 6),
                                        (17, 33, 5, 7)])
def test_matmul_tiled_reference(nncl, M, K, N, seed):
    A = oracle.uniform((M, K), seed, 0)
    B = oracle.uniform((K, N), seed, 1)
    say("reference matmul_tiled", M, K, N)
    R, info = run_ref("matmul_tiled", A, B, M=M, K=K, N=N)
    R = R.reshape(M, N)
    say(info)
    ours = oracle.matmul_tiled(A, B)
    assert np.array_equal(ours, R), f"restatement differs by {ulp_report(ours, R)} ulp"
    C = host(nncl.gemm(dev(A), dev(B)))
    ap = oracle.gemm_absprod(A, B, 0, 0, None, M=M, N=N, K=K, lda=K, ldb=N)[0]
    assert rel_distance(C, R, ap) <= oracle.tolerance(K)
    check_gemm(C, A, B, 0, 0, M=M, N=N, K=K, lda=K, ldb=N)


@pytest.mark.parametrize("batch,M,K,N,bcast", [(4, 32, 64, 48, False), (3, 40, 24, 36, True),
                                               (32, 128, 64, 128, False)])
def test_bmm_tiled_reference(nncl, batch, M, K, N, bcast):
    A = oracle.normal((batch, M, K), 777, 0)
    B = oracle.normal((1 if bcast else batch, K, N), 777, 1)
    sB = 0 if bcast else K * N
    say("reference bmm_tiled", batch, M, K, N, "broadcast" if bcast else "")
    R, info = run_ref("bmm_tiled", A, B, M=M, K=K, N=N, batch=batch, sA=M * K, sB=sB, sC=M * N)
    R = R.reshape(batch, M, N)
    say(info)
    ours = oracle.bmm(A, B)
    assert np.array_equal(ours, R), f"restatement differs by {ulp_report(ours, R)} ulp"
    C = host(nncl.Bmm(dev(A), dev(B)))
    ap = oracle.gemm_absprod(A, B, 0, 0, None, M=M, N=N, K=K, lda=K, ldb=N, sA=M * K, sB=sB,
                             batch=batch)
    assert rel_distance(C, R, ap) <= oracle.tolerance(K)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bmm_permute_tiled_reference(nncl, ta, tb):
    batch, M, K, N = 4, 32, 64, 48
    A = oracle.normal((batch, K, M) if ta else (batch, M, K), 778, 0)
    B = oracle.normal((batch, N, K) if tb else (batch, K, N), 778, 1)
    say("reference bmm_permute_tiled", ta, tb)
    R, info = run_ref("bmm_permute_tiled", A, B, M=M, K=K, N=N, batch=batch, sA=M * K,
                      sB=K * N, sC=M * N, transA=ta, transB=tb)
    R = R.reshape(batch, M, N)
    say(info)
    ours = oracle.bmm_permute(A, B, transA=bool(ta), transB=bool(tb))
    assert np.array_equal(ours, R), f"restatement differs by {ulp_report(ours, R)} ulp"
    C = host(nncl.BmmPermute(dev(A), dev(B), transA=bool(ta), transB=bool(tb)))
    ap = oracle.gemm_absprod(A, B, ta, tb, None, M=M, N=N, K=K, lda=M if ta else K,
                             ldb=K if tb else N, sA=M * K, sB=K * N, batch=batch)
    assert rel_distance(C, R, ap) <= oracle.tolerance(K)


@pytest.mark.parametrize("batch,M,K,N", [(2, 33, 40, 70), (1, 64, 1536, 4096)])
def test_linear_forward_tiled_reference(nncl, batch, M, K, N):
    X = oracle.normal((batch, M, K), 2, 0)
    W = oracle.uniform((K, N), 2, 1, -1 / 32, 1 / 32)
    bias = oracle.uniform((N,), 2, 2, -1 / 32, 1 / 32)
    say("reference linear_forward_tiled", batch, M, K, N)
    R, info = run_ref("linear_forward_tiled", X, W, bias, M=M, K=K, N=N, batch=batch,
                      sA=M * K, sC=M * N)
    R = R.reshape(batch, M, N)
    say(info)
    ours = oracle.linear_forward(X, W, bias)
    assert np.array_equal(ours, R), f"restatement differs by {ulp_report(ours, R)} ulp"
    C = host(nncl.LinearForward(dev(X), dev(W[None]), dev(bias)))
    ap = oracle.gemm_absprod(X, W, 0, 0, bias, M=M, N=N, K=K, lda=K, ldb=N, sA=M * K, sB=0,
                             batch=batch)
    assert rel_distance(C, R, ap) <= oracle.tolerance(K)


def test_tensor_permute_reference(nncl):
    rng = np.random.default_rng(3)
    for shape, axes in [((4, 32, 48), [0, 2, 1]), ((3, 5), [1, 0]),
                        ((2, 3, 4, 5, 6), [3, 0, 4, 2, 1])]:
        x = rng.standard_normal(shape).astype(np.float32)
        meta = np.array(list(shape) + list(axes), dtype=np.int32)
        say("reference tensor_permute", shape, axes)
        R, _ = run_ref("tensor_permute", x, meta, M=len(shape))
        assert np.array_equal(oracle.tensor_permute(x, axes).ravel(), R)
        assert np.array_equal(host(nncl.Permute(dev(x), axes)).ravel(), R)


def test_config4_nn_4096_reference(nncl):
    """BASELINE config 4 forward through the reference bmm_tiled on the GPU: the oracle's
    restatement matches it bit-for-bit on sampled rows; the HIP path is within tolerance of
    fp64 and of the reference's output on every one of the 4096^2 elements."""
    n = 4096
    A = oracle.normal((n, n), 3, 0, 0.0, 1.0 / 64)
    B = oracle.normal((n, n), 3, 1, 0.0, 1.0 / 64)
    say("reference bmm_tiled 4096^3")
    R, info = run_ref("bmm_tiled", A, B, M=n, K=n, N=n, batch=1, sA=n * n, sB=0, sC=n * n,
                      reps=2)
    R = R.reshape(n, n)
    say(info)
    rows = sample_rows(n, 12)
    for r in rows:
        ours = oracle.matmul_rows(A, B, r, r + 1, threads=8)[0]
        assert np.array_equal(ours, R[r]), f"row {r}: restatement differs"
    C = host(nncl.gemm(dev(A), dev(B)))
    nw, cw, vs_ref = check_full(C, A, B, 0, 0, ref=R)
    say("whole output: normwise", nw, "componentwise", cw, "to the reference", vs_ref)
    # the reference kernel's own output meets the same fp64 bound everywhere
    check_full(R, A, B, 0, 0)


def test_lstm_gemm_kernels_reference(nncl):
    """lstm.cl's three GEMM kernels (lstm_gemm_xw, lstm_gemm_grad_x, lstm_gemm_grad_weights)
    run by the reference geometry: the restatement is bit-identical to them, the HIP path
    within tolerance. grad_weights accumulates onto non-zero initial gradients."""
    import torch
    batch, seq, F, H = 3, 37, 70, 33  # T = 111 tokens, 132 gates: ragged everywhere
    T, G = batch * seq, 4 * H
    X = oracle.normal((T, F), 31, 0)
    W = oracle.uniform((F, G), 31, 1, -0.2, 0.2)
    bias = oracle.uniform((G,), 31, 2, -0.2, 0.2)
    say("reference lstm_gemm_xw")
    R, _ = run_ref("lstm_gemm_xw", X, W, bias, M=T, K=F, N=G)
    assert np.array_equal(oracle.lstm_gemm_xw(X, W, bias).ravel(), R)
    XW = host(nncl.LstmGemmXW(dev(X.reshape(batch, seq, F)), dev(W), dev(bias)))
    ap = oracle.gemm_absprod(X, W, 0, 0, bias, M=T, N=G, K=F, lda=F, ldb=G)[0]
    assert rel_distance(XW, R.reshape(T, G), ap) <= oracle.tolerance(F)

    Gr = oracle.normal((T, G), 31, 3)
    say("reference lstm_gemm_grad_x")
    R, _ = run_ref("lstm_gemm_grad_x", Gr, W, M=T, K=G, N=F)
    assert np.array_equal(oracle.lstm_gemm_grad_x(Gr, W).ravel(), R)
    gX = host(nncl.LstmGemmGradX(dev(Gr), dev(W), (batch, seq, F))).reshape(T, F)
    ap = oracle.gemm_absprod(Gr, W, 0, 1, None, M=T, N=F, K=G, lda=G, ldb=G)[0]
    assert rel_distance(gX, R.reshape(T, F), ap) <= oracle.tolerance(G)

    Hout = oracle.normal((T, H), 31, 4)
    gW0 = oracle.normal((F, G), 31, 5)
    gU0 = oracle.normal((H, G), 31, 6)
    gB0 = oracle.normal((G,), 31, 7)
    say("reference lstm_gemm_grad_weights")
    require_ref()
    try:
        (rW, rU, rB), _ = ref.lstm_gemm_grad_weights(X, Hout, Gr, gW0, gU0, gB0, batch, seq)
    except ref.Unavailable as e:
        pytest.skip(f"reference OpenCL kernels unavailable: {e}")
    oW, oU, oB = oracle.lstm_gemm_grad_weights(X, Hout, Gr, gW0, gU0, gB0, batch, seq)
    assert np.array_equal(oW, rW) and np.array_equal(oU, rU) and np.array_equal(oB, rB)
    tW, tU, tB = dev(gW0), dev(gU0), dev(gB0)
    nncl.LstmGemmGradWeights(dev(X.reshape(batch, seq, F)), dev(Hout.reshape(batch, seq, H)),
                             dev(Gr), tW, tU, tB)
    torch.cuda.synchronize()
    P = Hout.reshape(batch, seq, H).copy()
    P[:, 1:] = P[:, :-1].copy()
    P[:, 0] = 0
    P = P.reshape(T, H)
    for got, ref_, A_, K_ in [(host(tW), rW, X, F), (host(tU), rU, P, H)]:
        den = np.abs(A_.astype(np.float64)).T @ np.abs(Gr.astype(np.float64)) + np.abs(ref_)
        assert rel_distance(got, ref_, den) <= oracle.tolerance(T), K_
    denb = np.abs(Gr.astype(np.float64)).sum(axis=0) + np.abs(gB0)
    assert rel_distance(host(tB), rB, denb) <= oracle.tolerance(T)


def test_lstm_gemm_kernels_reference_at_baseline_size(nncl):
    """lstm.cl's GEMM kernels at the LSTM of BASELINE config 3 (input 512, hidden 1024) over
    64 sequences of 100 steps: the restatement reproduces sampled rows of lstm_gemm_xw and
    lstm_gemm_grad_x bit for bit (matmul_rows is the same fma chain); the HIP path is within
    tolerance of the reference. Prints the reference kernels' times on this GPU."""
    batch, seq, F, H = 64, 100, 512, 1024
    T, G = batch * seq, 4 * H
    X = oracle.normal((T, F), 32, 0)
    W = oracle.uniform((F, G), 32, 1, -1 / 32, 1 / 32)
    bias = oracle.uniform((G,), 32, 2, -1 / 32, 1 / 32)
    Gr = oracle.normal((T, G), 32, 4, 0.0, 1.0 / 64)
    rows = sample_rows(T, 8)
    say("reference lstm_gemm_xw", T, F, G)
    R, info = run_ref("lstm_gemm_xw", X, W, bias, M=T, K=F, N=G)
    say(info)
    R = R.reshape(T, G)
    for r in rows:
        ours = oracle.matmul_rows(X, W, r, r + 1, threads=8)[0] + bias
        assert np.array_equal(ours, R[r]), f"row {r}"
    C = host(nncl.LstmGemmXW(dev(X.reshape(batch, seq, F)), dev(W), dev(bias)))
    check_gemm(C, X, W, 0, 0, bias=bias, M=T, N=G, K=F, lda=F, ldb=G, rows=rows, ref=R)
    say("reference lstm_gemm_grad_x", T, F, G)
    R, info = run_ref("lstm_gemm_grad_x", Gr, W, M=T, K=G, N=F)
    say(info)
    R = R.reshape(T, F)
    Wt = np.ascontiguousarray(W.T)
    for r in rows:
        assert np.array_equal(oracle.matmul_rows(Gr, Wt, r, r + 1, threads=8)[0], R[r]), r
    C = host(nncl.LstmGemmGradX(dev(Gr), dev(W), (T, F)))
    check_gemm(C, Gr, W, 0, 1, M=T, N=F, K=G, lda=G, ldb=G, rows=rows, ref=R)
    Hout = oracle.uniform((T, H), 32, 3, -1.0, 1.0)
    say("reference lstm_gemm_grad_weights", batch, seq, F, H)
    z = np.zeros
    require_ref()
    try:
        (rW, rU, rB), info = ref.lstm_gemm_grad_weights(
            X, Hout, Gr, z((F, G), np.float32), z((H, G), np.float32), z(G, np.float32), batch,
            seq, reps=3)
    except ref.Unavailable as e:
        pytest.skip(f"reference OpenCL kernels unavailable: {e}")
    say(info)
    check_gemm(rW, X, Gr, 1, 0, M=F, N=G, K=T, lda=F, ldb=G, rows=sample_rows(F, 6))


def test_lstm_recurrent_forward_reference(nncl):
    """The reference lstm_recurrent_forward (lstm.cl:40-127) over several steps at batch 64
    with hidden 64, where its work-group is one wavefront: its stored raw gates
    (workspace[t, b, :4H], lstm.cl:103-106) are reproduced bit for bit by the restatement
    given its H_out as h_{t-1}, and the HIP per-step product (migemm_lstm_recurrent_gates)
    on the same H_out is within 1e-5*sqrt(H) of them and of fp64."""
    B, S, H = 64, 5, 64
    XW = oracle.normal((B, S, 4 * H), 45, 0)
    U = oracle.uniform((H, 4 * H), 45, 1, -1 / 8, 1 / 8)
    say("reference lstm_recurrent_forward", B, S, H)
    require_ref()
    try:
        Ho, gates, cells, info = ref.lstm_recurrent_forward(XW, U)
    except ref.Unavailable as e:
        pytest.skip(f"reference OpenCL kernels unavailable: {e}")
    say(info)
    assert np.all(np.abs(Ho) < 1) and np.any(Ho != 0)
    xw, ho, u = dev(XW), dev(Ho), dev(U)
    for t in range(S):
        restated = oracle.lstm_recurrent_gates(XW, Ho, U, t)
        assert np.array_equal(restated, gates[t]), \
            f"step {t}: restatement differs by {ulp_report(restated, gates[t])} ulp"
        nncl.LstmRecurrentGates(xw, ho, u, t)
        got = host(xw)[:, t].astype(np.float64)
        prev = Ho[:, t - 1].astype(np.float64) if t > 0 else np.zeros((B, H))
        den = np.abs(XW[:, t]).astype(np.float64) + np.abs(prev) @ np.abs(U.astype(np.float64))
        exact = XW[:, t].astype(np.float64) + prev @ U.astype(np.float64)
        assert rel_distance(got, gates[t], den) <= oracle.tolerance(H), t
        assert rel_distance(got, exact, den) <= oracle.tolerance(H), t


def test_lstm_recurrent_forward_reference_races_beyond_one_wavefront(nncl):
    """A defect of the reference kernel, kept visible: lstm_recurrent_forward writes
    h_local[hid] (the new h_t) inside the step (lstm.cl:122) with no barrier before the same
    thread's next hidden unit, and the other wavefronts, read h_local[h] as h_{t-1} (:91).
    With hidden 1024 (BASELINE config 3's LSTM) its work-group holds several wavefronts and
    each thread several hidden units, so its stored gates are not XW + h_{t-1} U: at step 0,
    where h_{-1} = 0 and the gates must equal XW exactly, the units after each thread's first
    read h_0 values and deviate. The HIP product follows the mathematics (XW exactly at step
    0, fp64 within tolerance at step 1 given the reference's own H_out)."""
    B, S, H = 64, 2, 1024
    XW = oracle.normal((B, S, 4 * H), 46, 0)
    U = oracle.uniform((H, 4 * H), 46, 1, -1 / 32, 1 / 32)
    say("reference lstm_recurrent_forward (race)", B, S, H)
    require_ref()
    try:
        Ho, gates, cells, info = ref.lstm_recurrent_forward(XW, U)
    except ref.Unavailable as e:
        pytest.skip(f"reference OpenCL kernels unavailable: {e}")
    say(info)
    dev_ = np.abs(gates[0].astype(np.float64) - XW[:, 0]) / (
        np.abs(XW[:, 0]).astype(np.float64) + np.abs(U).sum(axis=0)[None, :])
    worst = float(np.max(dev_))
    say("reference step-0 gates: worst deviation from XW", worst)
    assert worst > 10 * oracle.tolerance(H)  # rounding alone stays below 1x
    xw, ho, u = dev(XW), dev(Ho), dev(U)
    nncl.LstmRecurrentGates(xw, ho, u, 0)
    assert np.array_equal(host(xw)[:, 0], XW[:, 0])
    nncl.LstmRecurrentGates(xw, ho, u, 1)
    got = host(xw)[:, 1].astype(np.float64)
    prev = Ho[:, 0].astype(np.float64)
    den = np.abs(XW[:, 1]).astype(np.float64) + np.abs(prev) @ np.abs(U.astype(np.float64))
    exact = XW[:, 1].astype(np.float64) + prev @ U.astype(np.float64)
    assert rel_distance(got, exact, den) <= oracle.tolerance(H)


@pytest.mark.parametrize("B,S,F,H,seed", [(5, 4, 40, 24, 47), (64, 3, 512, 1024, 48)])
def test_lstm_hid_forward_reference(nncl, B, S, F, H, seed):
    """The reference lstm_hid_forward (lstm.cl:788-870: one work-item per sequence, the gates
    of every step stored in its workspace [S, B, 4H], :843) with a non-zero incoming state,
    at a ragged size and at BASELINE config 3's LSTM (input 512, hidden 1024, 64 sequences):
    the restatement (bias first, then one fma chain over x_t W and h_{t-1} U, :833-841)
    reproduces every stored gate bit for bit given the kernel's own H_out as h_{t-1}, and
    the HIP product (migemm_lstm_hid_gates) on the same inputs is within 1e-5*sqrt(F + H) of
    those gates and of fp64."""
    G = 4 * H
    X = oracle.normal((B, S, F), seed, 0)
    W = oracle.uniform((F, G), seed, 1, -1 / 32, 1 / 32)
    U = oracle.uniform((H, G), seed, 2, -1 / 32, 1 / 32)
    bias = oracle.uniform((G,), seed, 3, -1 / 32, 1 / 32)
    Hp = oracle.uniform((B, H), seed, 4, -0.5, 0.5)
    Cp = oracle.uniform((B, H), seed, 5, -0.5, 0.5)
    say("reference lstm_hid_forward", B, S, F, H)
    require_ref()
    try:
        Ho, gates, fH, fC, info = ref.lstm_hid_forward(X, W, U, bias, Hp, Cp)
    except ref.Unavailable as e:
        pytest.skip(f"reference OpenCL kernels unavailable: {e}")
    say(info)
    assert np.all(np.abs(Ho) < 1) and np.any(Ho != 0)
    assert np.array_equal(fH, Ho[:, -1])
    x, w, u, b, hp, ho = dev(X), dev(W), dev(U), dev(bias), dev(Hp), dev(Ho)
    ws = dev(np.zeros((S, B, G), np.float32))
    WU = np.concatenate([W, U]).astype(np.float64)
    for t in range(S):
        restated = oracle.lstm_hid_gates(X, W, U, bias, Hp, Ho, t)
        assert np.array_equal(restated, gates[t]), \
            f"step {t}: restatement differs by {ulp_report(restated, gates[t])} ulp"
        nncl.LstmHidGates(x, w, u, b, hp, ho, ws, t)
        got = host(ws)[t].astype(np.float64)
        prev = Hp if t == 0 else Ho[:, t - 1]
        xh = np.concatenate([X[:, t], prev], axis=1).astype(np.float64)
        den = np.abs(xh) @ np.abs(WU) + np.abs(bias)
        exact = xh @ WU + bias
        assert rel_distance(got, gates[t], den) <= oracle.tolerance(F + H), t
        assert rel_distance(got, exact, den) <= oracle.tolerance(F + H), t
