"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

The reference holds no golden vectors for the matmul path (its tests compare against live
PyTorch at rtol=atol=1e-4: tests/test_matrix_ops.py:130, tests/test_bmm.py:70,
tests/test_nncl_glob.py:165-173). The oracle is therefore pinned by what the mathematics
fixes: exact known answers (every partial sum exactly representable), identities between
the reference's forms, brute force against fp64 on tiny shapes, and library routines
(numpy float64 matmul / transpose / cumulative sums). A planted-mistake test shows the
known-answer tests catch a transposed operand, a dropped k term and a wrong bias.
"""
import itertools
import json
import os

import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

import oracle

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def small_ints(shape, seed, lo=-4, hi=4):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


# ------------------------------------------------------------------------------ generator
def test_generator_c_matches_numpy_mirror():
    for seed, tid, n in [(0, 0, 1000), (3, 2, 4097), (12345, 7, 333)]:
        c = oracle.uniform((n,), seed, tid)
        p = oracle.uniform_np((n,), seed, tid)
        assert np.array_equal(c, p)
        assert c.min() >= -1.0 and c.max() < 1.0
        cn = oracle.normal((n,), seed, tid)
        pn = oracle.normal_np((n,), seed, tid)
        # libm vs numpy cos/log may differ in the last double bit; fp32 rounding absorbs it
        assert np.max(np.abs(cn.astype(np.float64) - pn)) <= 1e-6 * max(1.0, np.abs(cn).max())


def test_generator_golden_values():
    with open(os.path.join(GOLDEN, "generator.json")) as f:
        g = json.load(f)
    for case in g["uniform"]:
        v = oracle.uniform((len(case["values"]),), case["seed"], case["tensor_id"],
                           case["lo"], case["hi"])
        assert v.tolist() == case["values"]
    for case in g["normal"]:
        v = oracle.normal((len(case["values"]),), case["seed"], case["tensor_id"],
                          case["mean"], case["std"])
        np.testing.assert_allclose(v, np.array(case["values"], dtype=np.float32), rtol=1e-6,
                                   atol=1e-6)


def test_generator_statistics():
    u = oracle.uniform((1 << 18,), 4, 1)
    assert abs(u.mean()) < 0.01 and abs(u.var() - 1.0 / 3.0) < 0.01
    z = oracle.normal((1 << 18,), 1, 1)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    w = oracle.uniform((1 << 16,), 2, 3, -1.0 / 32, 1.0 / 32)
    assert w.min() >= -1.0 / 32 and w.max() < 1.0 / 32


# ------------------------------------------------------------------- known-answer tests
@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (17, 33, 5), (64, 128, 96), (31, 300, 47)])
def test_matmul_tiled_small_int_exact(M, K, N):
    A = small_ints((M, K), 1)
    B = small_ints((K, N), 2)
    expect = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)
    assert np.array_equal(oracle.matmul_tiled(A, B), expect)


def test_matmul_tiled_identity_ones_rank1():
    rng = np.random.default_rng(5)
    A = rng.standard_normal((37, 37)).astype(np.float32)
    eye = np.eye(37, dtype=np.float32)
    assert np.array_equal(oracle.matmul_tiled(A, eye), A)
    assert np.array_equal(oracle.matmul_tiled(eye, A), A)
    ones_a = np.ones((9, 777), np.float32)
    ones_b = np.ones((777, 13), np.float32)
    assert np.all(oracle.matmul_tiled(ones_a, ones_b) == 777.0)
    u = small_ints((23, 1), 3)
    v = small_ints((1, 29), 4)
    assert np.array_equal(oracle.matmul_tiled(u, v), u @ v)


def probe_case(M, K, N, i, k, j):
    A = np.zeros((M, K), np.float32)
    B = np.zeros((K, N), np.float32)
    A[i, k] = 3.0
    B[k, j] = 5.0
    C = np.zeros((M, N), np.float32)
    C[i, j] = 15.0
    return A, B, C


def test_matmul_tiled_probes_every_edge():
    M, K, N = 19, 35, 21  # no dimension a multiple of the 16-wide tile
    for i, k, j in itertools.product([0, 15, 16, 18], [0, 15, 16, 31, 32, 34], [0, 15, 16, 20]):
        A, B, C = probe_case(M, K, N, i, k, j)
        assert np.array_equal(oracle.matmul_tiled(A, B), C), (i, k, j)


# --------------------------------------------------------- brute force vs fp64 / numpy
@settings(max_examples=60, deadline=None)
@given(st.integers(1, 33), st.integers(1, 33), st.integers(1, 33), st.integers(0, 2**31 - 1))
def test_matmul_tiled_vs_fp64_brute_force(M, K, N, seed):
    A = oracle.uniform((M, K), seed, 0)
    B = oracle.uniform((K, N), seed, 1)
    C = oracle.matmul_tiled(A, B)
    ref = np.zeros((M, N))
    for k in range(K):  # explicit fp64 triple loop over k
        ref += np.outer(A[:, k].astype(np.float64), B[k, :].astype(np.float64))
    absprod = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
    nw, cw = oracle.errors(C, ref, absprod)
    assert nw <= oracle.tolerance(K) and cw <= oracle.tolerance(K)


def test_gemm_f64_matches_numpy():
    rng = np.random.default_rng(9)
    for ta, tb in itertools.product([0, 1], [0, 1]):
        M, N, K = 13, 17, 19
        A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        B = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        bias = rng.standard_normal(N).astype(np.float32)
        got = oracle.gemm_f64(A, B, ta, tb, bias, M=M, N=N, K=K, lda=A.shape[1],
                              ldb=B.shape[1])[0]
        a64 = A.astype(np.float64).T if ta else A.astype(np.float64)
        b64 = B.astype(np.float64).T if tb else B.astype(np.float64)
        np.testing.assert_allclose(got, a64 @ b64 + bias, rtol=1e-12, atol=1e-12)
        ap = oracle.gemm_absprod(A, B, ta, tb, None, M=M, N=N, K=K, lda=A.shape[1],
                                 ldb=B.shape[1])[0]
        np.testing.assert_allclose(ap, np.abs(a64) @ np.abs(b64), rtol=1e-12)


# ----------------------------------------------------- identities between the forms
def test_bmm_broadcast_equals_per_batch_loop():
    A = oracle.uniform((4, 32, 64), 7, 0)
    B1 = oracle.uniform((1, 64, 48), 7, 1)
    C = oracle.bmm(A, B1)
    for z in range(4):
        assert np.array_equal(C[z], oracle.matmul_tiled(A[z], B1[0]))


def test_permute_forms_equal_materialised_transposes():
    A = oracle.uniform((3, 20, 37), 8, 0)   # [b, M, K]
    B = oracle.uniform((3, 37, 26), 8, 1)   # [b, K, N]
    nn = oracle.bmm(A, B)
    assert np.array_equal(oracle.bmm_permute(A, B), nn)  # same fma chain as bmm_tiled
    Bt = np.ascontiguousarray(B.transpose(0, 2, 1))
    At = np.ascontiguousarray(A.transpose(0, 2, 1))
    assert np.array_equal(oracle.bmm_permute(A, Bt, transB=True), nn)
    assert np.array_equal(oracle.bmm_permute(At, B, transA=True), nn)
    assert np.array_equal(oracle.bmm_permute(At, Bt, transA=True, transB=True), nn)


def test_linear_forward_is_bmm_plus_bias():
    X = oracle.uniform((2, 33, 40), 2, 0)
    W = oracle.uniform((40, 70), 2, 1, -1 / 32, 1 / 32)
    b = oracle.uniform((70,), 2, 2, -1 / 32, 1 / 32)
    Y = oracle.linear_forward(X, W, b)
    assert np.array_equal(Y, oracle.bmm(X, W[None]) + b)
    assert np.array_equal(oracle.lstm_gemm_xw(X[0], W, b), Y[0])


def test_tensor_permute_matches_numpy():
    rng = np.random.default_rng(11)
    for nd in range(1, 11):
        shape = tuple(int(s) for s in rng.integers(1, 4, size=nd))
        x = rng.standard_normal(shape).astype(np.float32)
        axes = list(rng.permutation(nd))
        assert np.array_equal(oracle.tensor_permute(x, axes), np.transpose(x, axes))


def test_reduce_sum_axis_sequential():
    x = small_ints((3, 50, 7), 4).astype(np.float32)
    np.testing.assert_array_equal(oracle.reduce_sum_axis(x, 1)[:, 0, :], x.sum(axis=1))
    y = oracle.normal((3, 1001, 5), 1, 2)
    seq = np.add.accumulate(y, axis=1, dtype=np.float32)[:, -1, :]  # float32, ascending
    assert np.array_equal(oracle.reduce_sum_axis(y, 1)[:, 0, :], seq)
    g = oracle.normal((2, 9, 6), 3, 3)
    assert np.array_equal(oracle.linear_bias_backward(g),
                          np.add.accumulate(g.reshape(-1, 6), axis=0, dtype=np.float32)[-1])


# ---------------------------------------- the reference's own test shapes
@pytest.mark.parametrize("batch,M,K,N", [(1, 64, 128, 96), (4, 32, 64, 32), (4, 32, 64, 48),
                                         (1, 8, 16, 8), (1, 4, 8, 8)])
def test_reference_test_shapes_within_tolerance(batch, M, K, N):
    A = oracle.normal((batch, M, K), 777, 0)
    B = oracle.normal((batch, K, N), 777, 1)
    C = oracle.bmm(A, B)
    ref = np.einsum("bmk,bkn->bmn", A.astype(np.float64), B.astype(np.float64))
    ap = np.einsum("bmk,bkn->bmn", np.abs(A.astype(np.float64)), np.abs(B.astype(np.float64)))
    nw, cw = oracle.errors(C, ref, ap)
    assert nw <= oracle.tolerance(K) and cw <= oracle.tolerance(K)
    # the reference tests' own bar
    np.testing.assert_allclose(C, ref, rtol=1e-4, atol=1e-4)


def test_matmul_rows_bit_identical_to_matmul_tiled():
    A = oracle.uniform((40, 777), 4, 0)
    B = oracle.uniform((777, 50), 4, 1)
    full = oracle.matmul_tiled(A, B)
    assert np.array_equal(oracle.matmul_rows(A, B, 0, 40, threads=2), full)
    assert np.array_equal(oracle.matmul_rows(A, B, 7, 19, threads=1), full[7:19])


# ------------------------------------------------------------------- planted mistakes
def test_known_answer_tests_catch_planted_mistakes():
    """Mutated copies of the restatement (a transposed operand, a dropped last k term, a
    bias added twice) must each fail at least one known-answer check."""
    A = small_ints((19, 35), 1)
    B = small_ints((35, 21), 2)
    exact = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.float32)

    def transposed_b(a, b):
        # B(k, n) read at B[n*K + k] instead of B[k*N + n]: a transposed index formula
        wrong = np.ascontiguousarray(b).reshape(1, b.shape[1], b.shape[0])
        return oracle.bmm_permute(a[None], wrong, transB=True)[0]

    def dropped_last_k(a, b):
        return oracle.matmul_tiled(np.ascontiguousarray(a[:, :-1]),
                                   np.ascontiguousarray(b[:-1, :]))

    for bad in (transposed_b, dropped_last_k):
        caught = not np.array_equal(bad(A, B), exact)
        for (i, k, j) in [(0, 34, 0), (18, 0, 20), (5, 16, 7)]:
            pa, pb, pc = probe_case(19, 35, 21, i, k, j)
            caught |= not np.array_equal(bad(pa, pb), pc)
        assert caught, bad.__name__

    X = small_ints((1, 5, 6), 3)
    W = small_ints((6, 4), 4)
    bias = small_ints((4,), 5)
    twice = oracle.linear_forward(X, W, bias) + bias
    assert not np.array_equal(twice[0], (X[0] @ W) + bias)
    assert np.array_equal(oracle.linear_forward(X, W, bias)[0], (X[0] @ W) + bias)


# ------------------------------------------------------------- LSTM gradient GEMMs
def hprev_numpy(H, batch, seq):
    """Independent construction of the grad_U operand: within each sequence the previous
    step's hidden state, zero at the first step."""
    Hs = H.reshape(batch, seq, -1)
    P = np.zeros_like(Hs)
    P[:, 1:] = Hs[:, :-1]
    return P.reshape(batch * seq, -1)


def test_lstm_gemm_grad_x_exact_and_identity():
    G = small_ints((37, 20), 40)
    W = small_ints((19, 20), 41)
    exact = (G.astype(np.int64) @ W.T.astype(np.int64)).astype(np.float32)
    assert np.array_equal(oracle.lstm_gemm_grad_x(G, W), exact)
    Gn = oracle.normal((37, 20), 42, 0)
    Wn = oracle.normal((19, 20), 42, 1)
    assert np.array_equal(oracle.lstm_gemm_grad_x(Gn, Wn),
                          oracle.bmm_permute(Gn[None], Wn[None], transB=True)[0])


@pytest.mark.parametrize("batch,seq,F,H", [(3, 7, 10, 5), (2, 1, 4, 3), (1, 33, 17, 9)])
def test_lstm_gemm_grad_weights_exact(batch, seq, F, H):
    """Exact small-integer known answers: grad_W += X^T G, grad_U += H_prev^T G with the
    per-sequence shift, grad_bias += sum G, each added onto a non-zero old value."""
    T, Gt = batch * seq, 4 * H
    X = small_ints((T, F), 43)
    Hout = small_ints((T, H), 44)
    G = small_ints((T, Gt), 45)
    gW0, gU0, gB0 = small_ints((F, Gt), 46), small_ints((H, Gt), 47), small_ints((Gt,), 48)
    gW, gU, gB = oracle.lstm_gemm_grad_weights(X, Hout, G, gW0, gU0, gB0, batch, seq)
    i64 = lambda a: a.astype(np.int64)  # noqa: E731
    assert np.array_equal(gW, (i64(gW0) + i64(X).T @ i64(G)).astype(np.float32))
    P = hprev_numpy(Hout, batch, seq)
    assert np.array_equal(gU, (i64(gU0) + i64(P).T @ i64(G)).astype(np.float32))
    assert np.array_equal(gB, (i64(gB0) + i64(G).sum(axis=0)).astype(np.float32))
    # planted mistakes the known answers tell apart: a shift that crosses sequences, and
    # overwriting instead of accumulating
    if batch > 1 and seq > 1:
        crossing = np.zeros_like(Hout)
        crossing[1:] = Hout[:-1]
        assert not np.array_equal(gU, (i64(gU0) + i64(crossing).T @ i64(G)).astype(np.float32))
    assert not np.array_equal(gW, (i64(X).T @ i64(G)).astype(np.float32))
    assert not np.array_equal(gB, i64(G).sum(axis=0).astype(np.float32))


def test_lstm_gemm_grad_weights_vs_fp64():
    batch, seq, F, H = 4, 9, 24, 8
    T, Gt = batch * seq, 4 * H
    X = oracle.normal((T, F), 49, 0)
    Hout = oracle.normal((T, H), 49, 1)
    G = oracle.normal((T, Gt), 49, 2)
    z = np.zeros
    gW, gU, gB = oracle.lstm_gemm_grad_weights(X, Hout, G, z((F, Gt), np.float32),
                                               z((H, Gt), np.float32), z(Gt, np.float32),
                                               batch, seq)
    P = hprev_numpy(Hout, batch, seq).astype(np.float64)
    G64 = G.astype(np.float64)
    tol = oracle.tolerance(T)
    X64 = X.astype(np.float64)
    for got, ref, den in [(gW, X64.T @ G64, np.abs(X64).T @ np.abs(G64)),
                          (gU, P.T @ G64, np.abs(P).T @ np.abs(G64))]:
        assert np.max(np.abs(got - ref) / np.maximum(den, 1e-30)) <= tol
    assert np.max(np.abs(gB - G64.sum(axis=0)) / np.abs(G64).sum(axis=0)) <= tol


# ------------------------------------------------------------ LSTM recurrent step
@pytest.mark.parametrize("B,S,H", [(3, 4, 5), (2, 7, 17), (4, 3, 33)])
def test_lstm_recurrent_gates_exact(B, S, H):
    """lstm.cl:80-101: the gates of step t are XW[:, t] + h_{t-1} U with h_{-1} = 0. Small
    integers keep every partial sum exact, so the restatement must equal an independent
    numpy construction bit for bit at every step."""
    XW = small_ints((B, S, 4 * H), 70 + H)
    U = small_ints((H, 4 * H), 71 + H)
    Ho = small_ints((B, S, H), 72 + H)
    for t in range(S):
        prev = Ho[:, t - 1].astype(np.int64) if t > 0 else np.zeros((B, H), np.int64)
        expect = (XW[:, t].astype(np.int64) + prev @ U.astype(np.int64)).astype(np.float32)
        assert np.array_equal(oracle.lstm_recurrent_gates(XW, Ho, U, t), expect), t


def test_lstm_recurrent_gates_catch_planted_mistakes():
    """A restatement that used the current step's hidden state (h_t instead of h_{t-1}), or
    started the chain from zero instead of the XW value, fails the known answers."""
    B, S, H = 2, 5, 6
    XW = small_ints((B, S, 4 * H), 80)
    U = small_ints((H, 4 * H), 81)
    Ho = small_ints((B, S, H), 82)

    def expect(t):
        prev = Ho[:, t - 1].astype(np.int64) if t > 0 else np.zeros((B, H), np.int64)
        return (XW[:, t].astype(np.int64) + prev @ U.astype(np.int64)).astype(np.float32)

    def current_h(t):  # h_t instead of h_{t-1}
        shifted = np.ascontiguousarray(np.concatenate([Ho[:, 1:], Ho[:, :1]], axis=1))
        return oracle.lstm_recurrent_gates(XW, shifted, U, t)

    def from_zero(t):  # bias / input projection dropped
        return oracle.lstm_recurrent_gates(np.zeros_like(XW), Ho, U, t)

    for bad in (current_h, from_zero):
        assert any(not np.array_equal(bad(t), expect(t)) for t in range(S)), bad.__name__
    assert all(np.array_equal(oracle.lstm_recurrent_gates(XW, Ho, U, t), expect(t))
               for t in range(S))


def test_lstm_recurrent_gates_vs_fp64():
    """N(0,1) gates at hidden 256: the fp32 chain stays within 1e-5*sqrt(H) of fp64."""
    B, S, H = 4, 3, 256
    XW = oracle.normal((B, S, 4 * H), 83, 0)
    U = oracle.uniform((H, 4 * H), 83, 1, -1 / 16, 1 / 16)
    Ho = oracle.uniform((B, S, H), 83, 2)
    for t in range(S):
        g = oracle.lstm_recurrent_gates(XW, Ho, U, t).astype(np.float64)
        prev = Ho[:, t - 1].astype(np.float64) if t > 0 else np.zeros((B, H))
        ref = XW[:, t].astype(np.float64) + prev @ U.astype(np.float64)
        den = np.abs(XW[:, t]).astype(np.float64) + np.abs(prev) @ np.abs(U.astype(np.float64))
        assert np.max(np.abs(g - ref) / den) <= oracle.tolerance(H)


# ------------------------------------------------- the reference kernels' own outputs
REF_FIXTURE = os.path.join(os.path.dirname(__file__), "golden", "reference_outputs.npz")


def _restate(kernel, inp, a):
    """The oracle's restatement of one reference kernel, on a fixture's inputs."""
    if kernel == "matmul_tiled":
        return oracle.matmul_tiled(inp["A"], inp["B"])
    if kernel == "bmm_tiled":
        return oracle.bmm_tiled(inp["A"], inp["B"], a["M"], a["K"], a["N"], a["sA"], a["sB"],
                                a["sC"], a["batch"])
    if kernel == "bmm_permute_tiled":
        return oracle.bmm_permute(inp["A"], inp["B"], bool(a["transA"]), bool(a["transB"]))
    if kernel == "linear_forward_tiled":
        return oracle.linear_forward(inp["A"], inp["B"], inp["bias"])
    if kernel == "tensor_permute":
        nd = a["M"]
        return oracle.tensor_permute(inp["A"], [int(v) for v in inp["B"][nd:]])
    if kernel == "lstm_gemm_xw":
        return oracle.lstm_gemm_xw(inp["A"], inp["B"], inp["bias"])
    if kernel == "lstm_gemm_grad_x":
        return oracle.lstm_gemm_grad_x(inp["A"], inp["B"])
    raise KeyError(kernel)


def test_restatement_equals_reference_fixture():
    """tests/golden/reference_outputs.npz holds the outputs of the reference's own kernels
    (its OpenCL sources compiled for gfx950, run on the GPU by
    tests/golden/make_reference_golden.py): matmul_tiled, bmm_tiled (with a broadcast B),
    bmm_permute_tiled in all four layouts, linear_forward_tiled, tensor_permute, the three
    lstm.cl GEMMs, lstm_recurrent_forward's and lstm_hid_forward's stored gates. The
    restatement reproduces every
    one of them bit for bit, here on the CPU."""
    import json
    d = np.load(REF_FIXTURE, allow_pickle=False)
    meta = json.loads(bytes(d["_meta"]).decode())
    assert meta["device"].startswith("gfx950")
    kernels = set()
    for name, m in meta["cases"].items():
        kernel, a = m["kernel"], m["args"]
        kernels.add(kernel)
        if kernel == "lstm_gemm_grad_weights":
            g = {k: d[f"{name}.{k}"] for k in ("X", "H_out", "G", "gW0", "gU0", "gB0")}
            oW, oU, oB = oracle.lstm_gemm_grad_weights(g["X"], g["H_out"], g["G"], g["gW0"],
                                                       g["gU0"], g["gB0"], a["batch_size"],
                                                       a["seq_len"])
            for ours, key in ((oW, "gW"), (oU, "gU"), (oB, "gB")):
                assert np.array_equal(ours, d[f"{name}.{key}"]), (name, key)
        elif kernel == "lstm_recurrent_forward":
            XW, U, Ho, gates = (d[f"{name}.{k}"] for k in ("XW", "U", "H_out", "gates"))
            for t in range(a["S"]):
                assert np.array_equal(oracle.lstm_recurrent_gates(XW, Ho, U, t), gates[t]), \
                    (name, t)
        elif kernel == "lstm_hid_forward":
            X, W, U, bias, Hp, Ho, gates = (d[f"{name}.{k}"] for k in (
                "X", "W", "U", "bias", "H_prev", "H_out", "gates"))
            for t in range(a["S"]):
                assert np.array_equal(oracle.lstm_hid_gates(X, W, U, bias, Hp, Ho, t),
                                      gates[t]), (name, t)
        else:
            inp = {k: d[f"{name}.{k}"] for k in ("A", "B", "bias") if f"{name}.{k}" in d}
            out = d[f"{name}.out"]
            ours = np.ravel(_restate(kernel, inp, a))
            assert ours.shape == out.shape and np.array_equal(ours, out), name
    assert kernels == {"matmul_tiled", "bmm_tiled", "bmm_permute_tiled", "linear_forward_tiled",
                       "tensor_permute", "lstm_gemm_xw", "lstm_gemm_grad_x",
                       "lstm_gemm_grad_weights", "lstm_recurrent_forward", "lstm_hid_forward"}


def test_reference_fixture_catches_planted_mistakes():
    """The fixture tells a faithful restatement from plausible mistakes: the same ascending
    chain without the fused multiply-add (product and sum rounded separately, as a compiler
    that does not contract `acc += a*b` would give), the sum in pairwise order, and a
    transposed operand."""
    d = np.load(REF_FIXTURE, allow_pickle=False)
    name = "matmul_tiled_64x128x96"
    A, B, out = d[f"{name}.A"], d[f"{name}.B"], d[f"{name}.out"]
    assert np.array_equal(np.ravel(oracle.matmul_tiled(A, B)), out)
    unfused = np.zeros((A.shape[0], B.shape[1]), np.float32)
    for k in range(A.shape[1]):
        unfused = unfused + A[:, k, None] * B[None, k, :]  # float32 product, then float32 add
    assert not np.array_equal(np.ravel(unfused), out)
    pairwise = np.sum(A[:, :, None] * B[None, :, :], axis=1, dtype=np.float32)
    assert not np.array_equal(np.ravel(pairwise), out)
    name = "bmm_permute_tiled_t01_b2_33x47x29"
    A, B, out = d[f"{name}.A"], d[f"{name}.B"], d[f"{name}.out"]
    wrong = oracle.bmm_permute(A, np.ascontiguousarray(B.reshape(2, 47, 29)), False, False)
    assert not np.array_equal(np.ravel(wrong), out)


def _hid_case(name):
    d = np.load(REF_FIXTURE, allow_pickle=False)
    return {k: d[f"{name}.{k}"] for k in ("X", "W", "U", "bias", "H_prev", "H_out", "gates")}


def test_hid_gates_small_integer_answers():
    """oracle_lstm_hid_gates with small-integer operands (every partial sum exact) equals
    the integer answer bias + x_t W + h_{t-1} U, built here with int64 numpy, at every step:
    h_{t-1} is the incoming state at t = 0 and the previous step's output after. A mistake
    of index (the step's own output h_t, x of another step, a transposed weight) changes
    the answer."""
    rng = np.random.default_rng(5)
    B, S, F, H = 3, 4, 7, 5
    G = 4 * H
    ints = lambda *s: rng.integers(-3, 4, size=s).astype(np.float32)
    X, W, U, bias, Hp, Ho = ints(B, S, F), ints(F, G), ints(H, G), ints(G), ints(B, H), ints(B, S, H)
    i64 = lambda a: a.astype(np.int64)
    for t in range(S):
        prev = Hp if t == 0 else Ho[:, t - 1]
        expect = i64(bias) + i64(X[:, t]) @ i64(W) + i64(prev) @ i64(U)
        got = oracle.lstm_hid_gates(X, W, U, bias, Hp, Ho, t)
        assert np.array_equal(got, expect.astype(np.float32)), t
        wrong = i64(bias) + i64(X[:, t]) @ i64(W) + i64(Ho[:, t]) @ i64(U)
        assert not np.array_equal(got, wrong.astype(np.float32)), t


def test_hid_fixture_catches_planted_mistakes():
    """The reference's stored lstm_hid_forward gates reject plausible restatement mistakes:
    the bias added after the products (as linear.cl / lstm_gemm_xw do, not lstm.cl:833),
    the U chain before the W chain, a chain without fused multiply-adds, and h_t in place
    of h_{t-1}. Each would be a single plausible slip in the restatement."""
    c = _hid_case("lstm_hid_forward_b2_s3_f33_h20")
    X, W, U, bias, Hp, Ho, gates = (c[k] for k in ("X", "W", "U", "bias", "H_prev", "H_out",
                                                   "gates"))
    B, S, F = X.shape
    H = U.shape[0]
    z = np.zeros_like(bias)
    for t in range(S):
        prev = Hp if t == 0 else Ho[:, t - 1]
        assert np.array_equal(oracle.lstm_hid_gates(X, W, U, bias, Hp, Ho, t), gates[t])
        # bias last: the chain from 0, then one add
        bias_last = oracle.lstm_hid_gates(X, W, U, z, Hp, Ho, t) + bias
        assert not np.array_equal(bias_last, gates[t]), t
        # U chain first: one chain over [h_{t-1} || x_t] against [U; W] (the h part of the
        # restatement fed zeros, whose fmas leave the accumulator unchanged)
        xh = np.concatenate([prev, X[:, t]], axis=1)[:, None, :].copy()
        UW = np.concatenate([U, W])
        zU, zH = np.zeros_like(U), np.zeros((B, H), np.float32)
        swapped = oracle.lstm_hid_gates(xh, UW, zU, bias, zH, zH[:, None, :].copy(), 0)
        assert not np.array_equal(swapped, gates[t]), t
        same_order = np.concatenate([X[:, t], prev], axis=1)[:, None, :].copy()
        kept = oracle.lstm_hid_gates(same_order, np.concatenate([W, U]), zU, bias, zH,
                                     zH[:, None, :].copy(), 0)
        assert np.array_equal(kept, gates[t]), t  # the construction itself is faithful
        # unfused chain in the kernel's own order
        unfused = np.empty_like(gates[t])
        for b in range(B):
            acc = bias.copy()
            for i in range(F):
                acc = (acc + X[b, t, i] * W[i]).astype(np.float32)
            for h in range(H):
                acc = (acc + prev[b, h] * U[h]).astype(np.float32)
            unfused[b] = acc
        assert not np.array_equal(unfused, gates[t]), t
        if t > 0:
            own = np.ascontiguousarray(Ho[:, 1:])  # h_t in place of h_{t-1}: shift by one
            Ho_shift = np.concatenate([own, Ho[:, -1:]], axis=1)
            assert not np.array_equal(oracle.lstm_hid_gates(X, W, U, bias, Hp, Ho_shift, t),
                                      gates[t]), t
