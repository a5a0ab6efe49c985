"""GPU parity of the HIP matmul path against the oracle, through the C ABI.

Each case prints what it runs before the GPU call, so a failure names its shape.
Exactness: small-integer operands make every partial sum exactly representable, so the
MFMA result must equal the reference arithmetic bit-for-bit; random operands are held to
the 1e-5*sqrt(K) relative bar against fp64."""
import ctypes
import itertools
import json
import os

import numpy as np
import pytest
import torch

import dispatch_cases
import oracle
from parity import Tuner, check_full, check_gemm, dev, host, sample_rows

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "small_cases.npz")


def small_ints(shape, seed, lo=-4, hi=4):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


def say(*a):
    print(*a, flush=True)


def gemm_gpu(nncl, A, B, transA=False, transB=False, bias=None):
    out = nncl.gemm(dev(A), dev(B), transA=transA, transB=transB,
                    bias=dev(bias) if bias is not None else None)
    return host(out)


# ------------------------------------------------------------------------ golden fixtures
def test_golden_fixtures(nncl):
    z = np.load(GOLDEN, allow_pickle=False)
    meta = json.loads(bytes(z["meta"]).decode())
    for m in meta:
        name = m["name"]
        say("golden", name)
        A, B, C64, Cref = z[f"{name}.A"], z[f"{name}.B"], z[f"{name}.C64"], z[f"{name}.C_ref"]
        M, K, N, ta, tb, batch = m["M"], m["K"], m["N"], m["transA"], m["transB"], m["batch"]
        if m["bias"]:
            bias = z[f"{name}.bias"]
            got = host(nncl.LinearForward(dev(A), dev(B), dev(bias)))
        else:
            bias = None
            got = host(nncl.BmmPermute(dev(A), dev(B), transA=bool(ta), transB=bool(tb)))
        ap = oracle.gemm_absprod(A, B, ta, tb, bias, M=M, N=N, K=K, lda=M if ta else K,
                                 ldb=K if tb else N, sA=A.shape[1] * A.shape[2],
                                 sB=0 if B.shape[0] == 1 else K * N, batch=batch)
        nw, cw = oracle.errors(got, C64, ap)
        assert nw <= oracle.tolerance(K) and cw <= oracle.tolerance(K), (name, nw, cw)
        nw2, cw2 = oracle.errors(got, Cref.astype(np.float64), ap)
        assert cw2 <= 2 * oracle.tolerance(K), (name, cw2)


# ------------------------------------------------------------------- exact known answers
SHAPES = [(1, 1, 1), (5, 7, 3), (17, 33, 5), (64, 128, 96), (127, 129, 65), (128, 128, 128),
          (200, 40, 300), (1000, 777, 3000), (2, 300, 1000), (4, 4096, 600), (300, 9, 257)]


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_small_int_exact_all_layouts(nncl, policy, M, K, N, ta, tb):
    say("exact", policy, M, K, N, "transA", ta, "transB", tb)
    A = small_ints((K, M) if ta else (M, K), M * 7 + K)
    B = small_ints((N, K) if tb else (K, N), N * 3 + K)
    Aop = A.T if ta else A
    Bop = B.T if tb else B
    expect = (Aop.astype(np.int64) @ Bop.astype(np.int64)).astype(np.float32)
    got = gemm_gpu(nncl, A, B, bool(ta), bool(tb))
    assert np.array_equal(got, expect)


def test_probe_matrices_hit_every_edge(nncl, policy):
    """Single non-zero probes at tile boundaries of every tile size the dispatcher uses."""
    for (M, K, N) in [(1000, 777, 3000), (100, 70, 90), (33, 65, 130)]:
        for ta, tb in [(0, 0), (0, 1), (1, 0)]:
            say("probe", policy, M, K, N, ta, tb)
            cases = list(itertools.product(
                sorted({0, 31, 32, 63, 64, 127, 128, M - 1} & set(range(M))),
                sorted({0, 7, 8, 31, 32, K - 1} & set(range(K))),
                sorted({0, 31, 32, 127, 128, N - 1} & set(range(N)))))
            rng = np.random.default_rng(M + K + N)
            for idx in rng.choice(len(cases), size=min(12, len(cases)), replace=False):
                i, k, j = cases[idx]
                A = np.zeros((M, K), np.float32)
                B = np.zeros((K, N), np.float32)
                A[i, k] = 3.0
                B[k, j] = 5.0
                An = np.ascontiguousarray(A.T) if ta else A
                Bn = np.ascontiguousarray(B.T) if tb else B
                got = gemm_gpu(nncl, An, Bn, bool(ta), bool(tb))
                nz = np.argwhere(got != 0)
                assert nz.tolist() == [[i, j]] and got[i, j] == 15.0, ((M, K, N), (i, k, j))


# --------------------------------------------------------------- output-boundary canary
def test_writes_stay_inside_m_by_n(nncl, policy):
    """Pooled buffers may be larger than M*N (OpenCLBufferManager.cs:29-40): nothing
    outside C's [M x N] per batch entry may change."""
    M, K, N, batch = 70, 33, 45, 3
    A = oracle.uniform((batch, M, K), 5, 0)
    B = oracle.uniform((batch, K, N), 5, 1)
    ldc = N + 7
    strideC = M * ldc + 11
    buf = torch.full((batch * strideC + 64,), float("nan"), device="cuda:0")
    from my_pytchon_opencl_lib_amd import _native
    import ctypes
    a, b = dev(A), dev(B)
    _native.call("migemm_gemm_strided_batched",
                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), 0, 0, M, N, K,
                 ctypes.c_void_p(a.data_ptr()), K, M * K, ctypes.c_void_p(b.data_ptr()), N,
                 K * N, None, ctypes.c_void_p(buf.data_ptr()), ldc, strideC, batch)
    out = host(buf)
    mask = np.zeros(out.shape, bool)
    for z in range(batch):
        for r in range(M):
            s = z * strideC + r * ldc
            mask[s:s + N] = True
    assert np.all(np.isnan(out[~mask])), "write outside [M x N]"
    C = np.stack([out[z * strideC:z * strideC + M * ldc].reshape(M, ldc)[:, :N]
                  for z in range(batch)])
    check_gemm(C, A, B, 0, 0, M=M, N=N, K=K, lda=K, ldb=N, sA=M * K, sB=K * N, batch=batch)


# -------------------------------------------------------------- properties between forms
def test_nt_tn_equal_nn_on_materialised_transposes(nncl):
    M, K, N = 300, 260, 200
    A = oracle.normal((M, K), 3, 0)
    B = oracle.normal((K, N), 3, 1)
    say("forms", M, K, N)
    nn = gemm_gpu(nncl, A, B)
    nt = gemm_gpu(nncl, A, np.ascontiguousarray(B.T), transB=True)
    tn = gemm_gpu(nncl, np.ascontiguousarray(A.T), B, transA=True)
    # same MFMA operands in the same k order whatever the storage layout: bit-identical
    assert np.array_equal(nn, nt)
    assert np.array_equal(nn, tn)


def test_broadcast_equals_per_batch_loop(nncl):
    A = oracle.normal((6, 77, 50), 9, 0)
    B = oracle.normal((1, 50, 90), 9, 1)
    say("broadcast")
    got = host(nncl.Bmm(dev(A), dev(B)))
    for z in range(6):
        assert np.array_equal(got[z], gemm_gpu(nncl, A[z], B[0]))


def test_bias_epilogue_is_gemm_plus_row_add(nncl, policy):
    X = oracle.normal((2, 64, 1536), 2, 0)
    W = oracle.uniform((1, 1536, 4096), 2, 1, -1 / 32, 1 / 32)
    bias = oracle.uniform((4096,), 2, 2, -1 / 32, 1 / 32)
    say("bias epilogue", policy)
    y = host(nncl.LinearForward(dev(X), dev(W), dev(bias)))
    plain = host(nncl.Bmm(dev(X), dev(W)))
    assert np.array_equal(y, (plain + bias).astype(np.float32))


# ---------------------------------------------------------- BASELINE.json configurations
def test_config1_nn_256(nncl):
    A = oracle.uniform((256, 256), 0, 0)
    B = oracle.uniform((256, 256), 0, 1)
    say("config1 256^3")
    C = gemm_gpu(nncl, A, B)
    check_gemm(C, A, B, 0, 0, M=256, N=256, K=256, lda=256, ldb=256,
               ref=oracle.matmul_tiled(A, B))


def test_config2_attention_bmm(nncl):
    Q = oracle.normal((32, 128, 64), 1, 0)
    Kt = oracle.normal((32, 64, 128), 1, 1)
    say("config2 QK^T")
    S = host(nncl.Bmm(dev(Q), dev(Kt)))
    check_gemm(S, Q, Kt, 0, 0, M=128, N=128, K=64, lda=64, ldb=128, sA=128 * 64, sB=64 * 128,
               batch=32, ref=oracle.bmm(Q, Kt))
    logits = oracle.normal((32, 128, 128), 1, 2).astype(np.float64)
    e = np.exp(logits - logits.max(axis=-1, keepdims=True))
    P = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    V = oracle.normal((32, 128, 64), 1, 3)
    say("config2 PV")
    O = host(nncl.Bmm(dev(P), dev(V)))
    check_gemm(O, P, V, 0, 0, M=128, N=64, K=128, lda=128, ldb=64, sA=128 * 128, sB=128 * 64,
               batch=32, ref=oracle.bmm(P, V))


def test_config3_lstm_gate_gemm(nncl):
    X = oracle.normal((64, 1536), 2, 0)
    W = oracle.uniform((1536, 4096), 2, 1, -1 / 32, 1 / 32)
    bias = oracle.uniform((4096,), 2, 2, -1 / 32, 1 / 32)
    say("config3 lstm gate")
    from my_pytchon_opencl_lib_amd import _native
    import ctypes
    x, w, b = dev(X), dev(W), dev(bias)
    out = torch.empty((64, 4096), device="cuda:0")
    _native.call("migemm_lstm_gemm_xw", ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                 ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(w.data_ptr()),
                 ctypes.c_void_p(b.data_ptr()), ctypes.c_void_p(out.data_ptr()), 64, 1536, 4096)
    check_gemm(host(out), X, W, 0, 0, bias=bias, M=64, N=4096, K=1536, lda=1536, ldb=4096,
               ref=oracle.lstm_gemm_xw(X, W, bias))


def test_config3_all_100_timesteps_and_graph_replay(nncl):
    """BASELINE config 3 as the bench runs it: 100 timestep inputs x[t] (64 x 1536) through
    gemm + bias with one W [1536, 4096]. Every step is checked against fp64 (every element of
    the stacked 6400 x 4096 output, tolerance 1e-5 sqrt(K)); then the 100 calls are captured
    in a HIP graph and each of three replays must reproduce the eager outputs bit for bit
    (the kernels are deterministic, and the graph path must not change the plan)."""
    steps = 100
    X = oracle.normal((steps * 64, 1536), 22, 0)
    W = oracle.uniform((1536, 4096), 22, 1, -1 / 32, 1 / 32)
    bias = oracle.uniform((4096,), 22, 2, -1 / 32, 1 / 32)
    say("config3 100 timesteps")
    x, w, b = dev(X).view(steps, 64, 1536), dev(W), dev(bias)
    eager = torch.empty((steps, 64, 4096), device="cuda:0")
    for t in range(steps):
        nncl.gemm(x[t], w, bias=b, out=eager[t])
    Y = host(eager).reshape(steps * 64, 4096)
    check_full(Y, X, W, 0, 0, bias=bias)
    out = torch.full((steps, 64, 4096), float("nan"), device="cuda:0")
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):
        for t in range(steps):
            nncl.gemm(x[t], w, bias=b, out=out[t])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        for t in range(steps):
            nncl.gemm(x[t], w, bias=b, out=out[t])
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep} differs from the eager steps"


@pytest.mark.parametrize("form", ["NN", "NT", "TN"])
def test_config4_4096_cube(nncl, form):
    n = 4096
    A = oracle.normal((n, n), 3, 0, 0.0, 1.0 / 64)
    B = oracle.normal((n, n), 3, 1, 0.0, 1.0 / 64)
    ta, tb = {"NN": (0, 0), "NT": (0, 1), "TN": (1, 0)}[form]
    say("config4", form)
    C = gemm_gpu(nncl, A, B, bool(ta), bool(tb))
    # every one of the 4096^2 outputs against fp64 (numpy float64 matmul, a few seconds)
    nw, cw, _ = check_full(C, A, B, ta, tb)
    say("config4", form, "whole output: normwise", nw, "componentwise", cw)


def test_config5a_ragged(nncl):
    A = oracle.uniform((1000, 777), 4, 0)
    B = oracle.uniform((777, 3000), 4, 1)
    say("config5a ragged")
    C = gemm_gpu(nncl, A, B)
    ref = oracle.matmul_rows(A, B, 0, 1000, threads=8)
    check_full(C, A, B, 0, 0, ref=ref)


def test_config5b_gemv(nncl):
    A = oracle.uniform((1, 4096), 4, 2)
    B = oracle.uniform((4096, 11008), 4, 3)
    say("config5b gemv")
    C = gemm_gpu(nncl, A, B)
    check_gemm(C, A, B, 0, 0, M=1, N=11008, K=4096, lda=4096, ldb=11008,
               ref=oracle.matmul_rows(A, B, 0, 1, threads=8))
    # a repeated call (same plan, same workspace) gives the same bits
    C2 = gemm_gpu(nncl, A, B)
    assert np.array_equal(C, C2)


@pytest.mark.parametrize("n,blocks", [(4, 1), (4096, 7), (1 << 20, 688), (180 * 256, 4096)])
def test_stream_read_sums_its_ranges(nncl, n, blocks):
    """migemm_stream_read (the streaming-read reference of the GEMV's roofline) reads every
    element once: each work-group's sum is the sum of its contiguous range."""
    from my_pytchon_opencl_lib_amd import _native
    rng = np.random.default_rng(n + blocks)
    x = rng.integers(-3, 4, size=n).astype(np.float32)
    sums = torch.full((blocks,), float("nan"), device="cuda:0")
    xd = dev(x)
    _native.call("migemm_stream_read", ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                 ctypes.c_void_p(xd.data_ptr()), n, ctypes.c_void_p(sums.data_ptr()), blocks)
    n4 = n // 4
    per = -(-n4 // blocks)
    expect = [x[4 * b * per:4 * min(n4, (b + 1) * per)].astype(np.int64).sum()
              for b in range(blocks)]
    assert np.array_equal(host(sums), np.array(expect, dtype=np.float32))


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_skinny_rows_and_bias(nncl, policy, M):
    K, N = 1000, 1030  # N not a multiple of 4 -> scalar loads; K not a slice multiple
    A = oracle.uniform((M, K), 6, M)
    B = oracle.uniform((K, N), 6, 10 + M)
    bias = oracle.uniform((N,), 6, 20 + M)
    say("skinny", policy, M)
    C = gemm_gpu(nncl, A, B, bias=bias)
    check_gemm(C, A, B, 0, 0, bias=bias, M=M, N=N, K=K, lda=K, ldb=N)
    At = np.ascontiguousarray(A.T)
    C2 = gemm_gpu(nncl, At, B, transA=True, bias=bias)
    assert np.array_equal(C, C2)


@pytest.mark.parametrize("M,K,N,batch", [(1, 1001, 777, 1), (1, 4096, 2048, 1), (1, 206, 228, 8),
                                         (2, 1001, 777, 1), (3, 2050, 300, 2), (4, 1027, 513, 1)])
def test_rows_gemv_transposed_a(nncl, M, K, N, batch):
    """B stored [N, K] and A stored transposed and dense ([K, M], lda = M): one row is read
    as a contiguous row, 2-4 rows as 4 M contiguous floats per 4 values of k. Small-integer
    operands make the result exact in any summation order."""
    from my_pytchon_opencl_lib_amd import _native
    say("rows gemv, A transposed", M, K, N, batch)
    A = small_ints((batch, K, M), K + N + M)
    B = small_ints((batch, N, K), K * 3 + N)
    bias = small_ints((N,), N)
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_SKINNY)
    try:
        C = gemm_gpu(nncl, A, B, transA=True, transB=True, bias=bias)
        assert _native.last_plan().startswith("skinny-rows"), _native.last_plan()
    finally:
        _native.set_gemm_policy(prev)
    expect = np.einsum("bkm,bnk->bmn", A.astype(np.int64), B.astype(np.int64)) + bias
    assert np.array_equal(C.reshape(batch, M, N), expect.astype(np.float32))


def test_graph_capture_replays_match_eager(nncl):
    """Callers may capture the GEMMs in a HIP graph. The capturing stream's workspace is
    sized by running the same calls on it first; replays are interleaved with eager work and
    synchronisations, and every replay is compared with the eager result."""
    dev_ = torch.device("cuda:0")
    A = dev(oracle.normal((64, 1536), 21, 0))
    W = dev(oracle.uniform((1536, 4096), 21, 1, -1 / 32, 1 / 32))
    bias = dev(oracle.uniform((4096,), 21, 2, -1 / 32, 1 / 32))
    x = dev(oracle.uniform((1, 4096), 21, 3))
    Bv = dev(oracle.uniform((4096, 11008), 21, 4))
    say("graph capture: split-K gate GEMM + split GEMV")
    y1 = torch.empty(64, 4096, device=dev_)
    y2 = torch.empty(1, 11008, device=dev_)
    eager1 = host(nncl.gemm(A, W, bias=bias)).copy()
    eager2 = host(nncl.gemm(x, Bv)).copy()
    cap = torch.cuda.Stream()
    with torch.cuda.stream(cap):  # sizes the capturing stream's own workspace
        nncl.gemm(A, W, bias=bias, out=y1)
        nncl.gemm(x, Bv, out=y2)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        nncl.gemm(A, W, bias=bias, out=y1)
        nncl.gemm(x, Bv, out=y2)
    for i in range(3):
        y1.fill_(float("nan"))
        y2.fill_(float("nan"))
        noise = nncl.gemm(Bv[:64, :4096].contiguous(), W[:4096 // 4].T.contiguous())  # eager work
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(host(y1), eager1), f"replay {i}: gate GEMM differs"
        assert np.array_equal(host(y2), eager2), f"replay {i}: GEMV differs"
        del noise


def test_graph_capture_needs_its_own_workspace(nncl):
    """A split-K GEMM captured on a stream whose workspace was never sized fails with
    MIGEMM_ERR_WORKSPACE (it does not borrow another stream's buffer); after
    migemm_workspace_reserve on that stream the same capture succeeds."""
    from my_pytchon_opencl_lib_amd import _native
    W = dev(small_ints((8192, 1536), 91, -2, 2))
    X = dev(small_ints((64, 8192), 92, -2, 2))
    Y = torch.empty(64, 1536, device="cuda:0")
    nncl.gemm(X, W, out=Y)  # sizes the default stream's workspace only
    torch.cuda.synchronize()
    say("graph capture without a sized workspace")
    cap = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(_native.MigemmRuntimeError, match="WORKSPACE"):
        with torch.cuda.graph(g, stream=cap):
            nncl.gemm(X, W, out=Y)
    torch.cuda.synchronize()
    nncl.reserve_workspace(cap, 64 << 20)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        nncl.gemm(X, W, out=Y)
    Y.fill_(float("nan"))
    g.replay()
    expect = (host(X).astype(np.float64) @ host(W).astype(np.float64)).astype(np.float32)
    assert np.array_equal(host(Y), expect)


def test_graph_replay_overlaps_eager_split_k(nncl):
    """A graph replay on one stream runs at the same time as eager split-K GEMMs of the
    same shape on another stream, with no synchronisation between the two: each stream has
    its own partial sums, so both results are exact."""
    say("graph replay overlapping eager split-K on another stream")
    W = dev(small_ints((8192, 1536), 93, -2, 2))
    xs = [dev(small_ints((64, 8192), 94 + i, -2, 2)) for i in range(4)]
    expect = [(host(x).astype(np.float64) @ host(W).astype(np.float64)).astype(np.float32)
              for x in xs]
    cap, other = torch.cuda.Stream(), torch.cuda.Stream()
    y_graph = torch.empty(64, 1536, device="cuda:0")
    with torch.cuda.stream(cap):
        nncl.gemm(xs[0], W, out=y_graph)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        for _ in range(8):
            nncl.gemm(xs[0], W, out=y_graph)
    ys = [torch.empty(64, 1536, device="cuda:0") for _ in range(3)]
    torch.cuda.synchronize()
    for rep in range(3):
        y_graph.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(cap):
            g.replay()
        with torch.cuda.stream(other):
            for i in range(3):
                for _ in range(4):
                    nncl.gemm(xs[1 + i], W, out=ys[i])
        torch.cuda.synchronize()
        assert np.array_equal(host(y_graph), expect[0]), f"replay {rep} differs"
        for i in range(3):
            assert np.array_equal(host(ys[i]), expect[1 + i]), f"eager {rep}/{i} differs"


def test_graph_replay_elsewhere_while_eager_runs_on_the_capture_stream(nncl):
    """A graph captured on stream S is replayed on another stream while eager split-K GEMMs
    run on S itself, with no synchronisation between them. The captured partial-sum buffer
    belongs to the graph once the capture has ended: the eager calls on S get a buffer of
    their own, so neither result is corrupted."""
    say("graph replay on another stream, eager split-K on the capture stream")
    W = dev(small_ints((8192, 1536), 97, -2, 2))
    xs = [dev(small_ints((64, 8192), 98 + i, -2, 2)) for i in range(4)]
    expect = [(host(x).astype(np.float64) @ host(W).astype(np.float64)).astype(np.float32)
              for x in xs]
    cap, other = torch.cuda.Stream(), torch.cuda.Stream()
    y_graph = torch.empty(64, 1536, device="cuda:0")
    with torch.cuda.stream(cap):
        nncl.gemm(xs[0], W, out=y_graph)  # sizes cap's workspace before the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        for _ in range(8):
            nncl.gemm(xs[0], W, out=y_graph)
    ys = [torch.empty(64, 1536, device="cuda:0") for _ in range(3)]
    torch.cuda.synchronize()
    for rep in range(3):
        y_graph.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(other):
            g.replay()
        with torch.cuda.stream(cap):
            for i in range(3):
                for _ in range(4):
                    nncl.gemm(xs[1 + i], W, out=ys[i])
        torch.cuda.synchronize()
        assert np.array_equal(host(y_graph), expect[0]), f"replay {rep} differs"
        for i in range(3):
            assert np.array_equal(host(ys[i]), expect[1 + i]), f"eager {rep}/{i} differs"


def test_stream_destroy_frees_its_workspace(nncl):
    """migemm_stream_destroy waits for the stream's work and frees the workspace the
    library held for it; migemm_workspace_release does the same for a caller's stream."""
    from my_pytchon_opencl_lib_amd import _native
    L = _native.load()
    W = dev(small_ints((8192, 1536), 95, -2, 2))
    X = dev(small_ints((64, 8192), 96, -2, 2))
    Y = torch.empty(64, 1536, device="cuda:0")
    expect = (host(X).astype(np.float64) @ host(W).astype(np.float64)).astype(np.float32)
    torch.cuda.synchronize()
    for release in (False, True):
        s = ctypes.c_void_p()
        _native.call("migemm_stream_create", ctypes.byref(s))
        say("workspace freed with the stream" if not release else "workspace release")
        _native.call("migemm_gemm_strided_batched", s, 0, 0, 64, 1536, 8192,
                     ctypes.c_void_p(X.data_ptr()), 8192, 0, ctypes.c_void_p(W.data_ptr()),
                     1536, 0, None, ctypes.c_void_p(Y.data_ptr()), 1536, 0, 1)
        assert "splits=" in _native.last_plan() and "splits=1 " not in _native.last_plan()
        size = ctypes.c_size_t(0)
        _native.call("migemm_workspace_size", s, ctypes.byref(size))
        assert size.value >= 64 * 1536 * 4 * 2
        if release:
            _native.call("migemm_workspace_release", s)
            _native.call("migemm_workspace_size", s, ctypes.byref(size))
            assert size.value == 0
            assert np.array_equal(host(Y), expect)
            _native.call("migemm_stream_destroy", s)
        else:
            _native.call("migemm_stream_destroy", s)
            _native.call("migemm_workspace_size", s, ctypes.byref(size))
            assert size.value == 0
            assert np.array_equal(host(Y), expect)
        assert L.migemm_last_error() == b""


def test_split_k_on_two_streams_concurrently(nncl):
    """The reference host keeps one command queue per thread (DeviceQueueRegistry.cs:14).
    GEMMs that keep partial sums in the library workspace (split-K, sliced GEMV, chunked
    column sum) run on two streams at once, with no synchronisation between the streams,
    and each result must be exact."""
    say("two streams: split-K 64x8192x1536, GEMV 1x4096x11008, column sum 12000x300")
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    W = small_ints((8192, 1536), 61, -2, 2)
    Bv = small_ints((4096, 11008), 62, -2, 2)
    G = small_ints((12000, 300), 63, -2, 2)
    xs = [small_ints((64, 8192), 70 + i, -2, 2) for i in range(6)]
    vs = [small_ints((1, 4096), 80 + i, -2, 2) for i in range(6)]
    w, bv, g = dev(W), dev(Bv), dev(G)
    dxs, dvs = [dev(x) for x in xs], [dev(v) for v in vs]
    torch.cuda.synchronize()
    outs = []
    for i in range(6):
        with torch.cuda.stream(s1 if i % 2 == 0 else s2):
            outs.append(("gemm", i, nncl.gemm(dxs[i], w)))
        with torch.cuda.stream(s2 if i % 2 == 0 else s1):
            outs.append(("gemv", i, nncl.gemm(dvs[i], bv)))
            outs.append(("sum", i, nncl.Sum(g, 0)))
    torch.cuda.synchronize()
    colsum = G.astype(np.float64).sum(axis=0).astype(np.float32)
    for kind, i, t in outs:
        got = host(t)
        if kind == "gemm":
            expect = (xs[i].astype(np.float64) @ W.astype(np.float64)).astype(np.float32)
        elif kind == "gemv":
            expect = (vs[i].astype(np.float64) @ Bv.astype(np.float64)).astype(np.float32)
        else:
            expect = colsum
        assert np.array_equal(got.reshape(expect.shape), expect), (kind, i)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_unaligned_bases_and_leading_dims(nncl, policy, ta, tb):
    """Operands that start 4 bytes past a 16-byte boundary with leading dimensions that
    are not multiples of 4 (128-bit loads from dword-aligned addresses)."""
    import ctypes
    from my_pytchon_opencl_lib_amd import _native
    M, K, N = 260, 300, 196
    A = small_ints((K, M) if ta else (M, K), 31)
    B = small_ints((N, K) if tb else (K, N), 32)
    lda, ldb = A.shape[1] + 1, B.shape[1] + 3
    abuf = np.zeros(1 + A.shape[0] * lda, np.float32)
    bbuf = np.zeros(3 + B.shape[0] * ldb, np.float32)
    abuf[1:].reshape(A.shape[0], lda)[:, :A.shape[1]] = A
    bbuf[3:].reshape(B.shape[0], ldb)[:, :B.shape[1]] = B
    a, b = dev(abuf), dev(bbuf)
    c = torch.full((M, N), float("nan"), device="cuda:0")
    say("unaligned", policy, ta, tb)
    _native.call("migemm_gemm_strided_batched",
                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), ta, tb, M, N, K,
                 ctypes.c_void_p(a.data_ptr() + 4), lda, 0, ctypes.c_void_p(b.data_ptr() + 12),
                 ldb, 0, None, ctypes.c_void_p(c.data_ptr()), N, 0, 1)
    Aop = A.T if ta else A
    Bop = B.T if tb else B
    expect = (Aop.astype(np.int64) @ Bop.astype(np.int64)).astype(np.float32)
    assert np.array_equal(host(c), expect)


@pytest.fixture
def forced_tile(request):
    """Forces one macro-tile of the tiled kernel (the library's tile tuning override) under
    the TILED policy, restoring both afterwards."""
    from my_pytchon_opencl_lib_amd import _native
    tuner = Tuner()
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_TILED)
    tuner.set(tile=request.param)
    yield request.param
    tuner.restore()
    _native.set_gemm_policy(prev)


@pytest.mark.parametrize("forced_tile", ["128", "128x256", "256"], indirect=True)
@pytest.mark.parametrize("M,K,N", [(2000, 50, 3980), (3000, 70, 2900), (1000, 300, 1100),
                                   (1001, 301, 1103)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_large_tile_shapes_exact(nncl, forced_tile, M, K, N, ta, tb):
    """Ragged shapes through each large macro-tile (128x128, 128x256, 256x256), with a
    zero-filled K tail; exact small-integer products."""
    say("large tiles exact", forced_tile, M, K, N, ta, tb)
    A = small_ints((K, M) if ta else (M, K), M + K)
    B = small_ints((N, K) if tb else (K, N), N + K)
    Aop = (A.T if ta else A).astype(np.float64)
    Bop = (B.T if tb else B).astype(np.float64)
    expect = (Aop @ Bop).astype(np.float32)  # exact: |sums| <= 16*K << 2^24
    got = gemm_gpu(nncl, A, B, bool(ta), bool(tb))
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("M,K,N", [(300, 5000, 200), (129, 4099, 131), (500, 12000, 700),
                                   (512, 4100, 4096), (1024, 4108, 2048), (768, 4096, 3072)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_long_k_split_tiles_exact(nncl, M, K, N, ta, tb):
    """Long K with few tiles, split into k ranges: 64x64 tiles (ragged M, N and a K tail in
    the last range), 256x256 tiles with one work-group per CU (512 x 4100 x 4096, 1024 x
    4108 x 2048) and 128x128 tiles (768 x 4096 x 3072); exact small-integer products."""
    say("long-K split exact", M, K, N, ta, tb)
    A = small_ints((K, M) if ta else (M, K), M + 2 * K, -2, 2)
    B = small_ints((N, K) if tb else (K, N), N + 2 * K, -2, 2)
    Aop = (A.T if ta else A).astype(np.float64)
    Bop = (B.T if tb else B).astype(np.float64)
    expect = (Aop @ Bop).astype(np.float32)  # exact: |sums| <= 4*K << 2^24
    got = gemm_gpu(nncl, A, B, bool(ta), bool(tb))
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(333, 8195), (4096, 11008), (7, 8192)])
def test_gemv_wide_exact(nncl, M, K, N):
    """M <= 4 on wide outputs (the sliced kernel with its ordered reduce): exact
    small-integer products with and without bias, A in both layouts; N % 4 != 0 reads
    columns one by one."""
    say("gemv wide", M, K, N)
    A = small_ints((M, K), M * 5 + K)
    B = small_ints((K, N), N + K)
    bias = small_ints((N,), N)
    expect = A.astype(np.int64) @ B.astype(np.int64)
    assert np.array_equal(gemm_gpu(nncl, A, B), expect.astype(np.float32))
    assert np.array_equal(gemm_gpu(nncl, A, B, bias=bias),
                          (expect + bias.astype(np.int64)).astype(np.float32))
    At = np.ascontiguousarray(A.T)
    assert np.array_equal(gemm_gpu(nncl, At, B, transA=True), expect.astype(np.float32))


# ------------------------------------------------------------- seeded random strided cases
def _random_case(rng):
    """One strided-batched request: shape class, layouts, padded leading dimensions, batch
    strides (stride 0 = broadcast), bias and the accumulate flag."""
    cls = int(rng.integers(0, 4))
    if cls == 0:    # tiny: every dimension below one 16-wide tile
        M, N, K = (int(v) for v in rng.integers(1, 41, 3))
    elif cls == 1:  # skinny rows, wide and long (the GEMV family)
        M, N, K = int(rng.integers(1, 5)), int(rng.integers(1, 5000)), int(rng.integers(1, 3000))
    elif cls == 2:  # medium ragged
        M, N = (int(v) for v in rng.integers(40, 600, 2))
        K = int(rng.integers(1, 900))
    else:           # long K (split over work-groups)
        M, N = (int(v) for v in rng.integers(1, 200, 2))
        K = int(rng.integers(2000, 6000))
    ta, tb = (int(v) for v in rng.integers(0, 2, 2))
    batch = int(rng.integers(1, 4)) if M * N * K < 30_000_000 else 1
    c = dict(M=M, N=N, K=K, ta=ta, tb=tb, batch=batch,
             bias=bool(rng.random() < 0.4), acc=bool(rng.random() < 0.3))
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    c["lda"] = a_cols + int(rng.integers(0, 4)) * int(rng.random() < 0.5)
    c["ldb"] = b_cols + int(rng.integers(0, 4)) * int(rng.random() < 0.5)
    c["ldc"] = N + int(rng.integers(0, 4)) * int(rng.random() < 0.5)
    bcast_a = batch > 1 and rng.random() < 0.25
    bcast_b = batch > 1 and not bcast_a and rng.random() < 0.25
    c["sA"] = 0 if bcast_a else a_rows * c["lda"] + int(rng.integers(0, 6))
    c["sB"] = 0 if bcast_b else b_rows * c["ldb"] + int(rng.integers(0, 6))
    c["sC"] = M * c["ldc"] + int(rng.integers(0, 6))
    c["a_shape"], c["b_shape"] = (a_rows, a_cols), (b_rows, b_cols)
    return c


def _strided(rows, cols, ld, stride, batch, rng, lo, hi):
    """A flat buffer holding `batch` windows of [rows x cols] (leading dimension ld, batch
    stride `stride`, 0 = one shared window) of small integers; everything else is NaN."""
    count = 1 if stride == 0 else batch
    size = (count - 1) * stride + rows * ld
    buf = np.full(size, np.nan, np.float32)
    wins = []
    for z in range(count):
        w = rng.integers(lo, hi + 1, size=(rows, cols)).astype(np.float32)
        buf[z * stride:z * stride + rows * ld].reshape(rows, ld)[:, :cols] = w
        wins.append(w)
    return buf, [wins[0 if stride == 0 else z] for z in range(batch)]


def test_random_strided_batched_exact(nncl, policy):
    """180 seeded requests through migemm_gemm_strided_batched_ex over every kernel family:
    random shapes (tiny, skinny, medium ragged, long K), all four layouts, padded leading
    dimensions, batch strides with gaps and stride-0 broadcast, bias and the accumulating
    epilogue. Small-integer operands make the answer exact in any summation order, so each
    result must equal the float64 product bit-for-bit. The padding of A and B is NaN, so a
    kernel that multiplies anything outside the [rows x cols] windows poisons its output;
    C's padding is NaN as well and must stay NaN (no write outside [M x N])."""
    import ctypes
    from my_pytchon_opencl_lib_amd import _native
    seeds = {"auto": 0, "small": 1, "tiled": 2, "skinny": 3, "panel": 4, "tiny": 5}
    rng = np.random.default_rng(20260 + seeds[policy])
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i in range(60):
        c = _random_case(rng)
        M, N, K, batch = c["M"], c["N"], c["K"], c["batch"]
        say("random", policy, i, {k: v for k, v in c.items() if not k.endswith("shape")})
        lo, hi = (-2, 2) if K > 2000 else (-4, 4)
        abuf, As = _strided(*c["a_shape"], c["lda"], c["sA"], batch, rng, lo, hi)
        bbuf, Bs = _strided(*c["b_shape"], c["ldb"], c["sB"], batch, rng, lo, hi)
        bias = rng.integers(-20, 21, size=N).astype(np.float32) if c["bias"] else None
        cbuf = np.full((batch - 1) * c["sC"] + M * c["ldc"] + 16, np.nan, np.float32)
        C0 = [rng.integers(-50, 51, size=(M, N)).astype(np.float32) for _ in range(batch)]
        if c["acc"]:
            for z in range(batch):
                cbuf[z * c["sC"]:z * c["sC"] + M * c["ldc"]].reshape(M, c["ldc"])[:, :N] = C0[z]
        a, b, cc = dev(abuf), dev(bbuf), dev(cbuf)
        bt = dev(bias) if bias is not None else None
        _native.call("migemm_gemm_strided_batched_ex", stream, c["ta"], c["tb"], M, N, K,
                     ctypes.c_void_p(a.data_ptr()), c["lda"], c["sA"],
                     ctypes.c_void_p(b.data_ptr()), c["ldb"], c["sB"],
                     None if bt is None else ctypes.c_void_p(bt.data_ptr()),
                     ctypes.c_void_p(cc.data_ptr()), c["ldc"], c["sC"], batch, int(c["acc"]))
        out = host(cc)
        inside = np.zeros(out.shape, bool)
        for z in range(batch):
            Aop = As[z].T if c["ta"] else As[z]
            Bop = Bs[z].T if c["tb"] else Bs[z]
            expect = Aop.astype(np.float64) @ Bop.astype(np.float64)
            if bias is not None:
                expect = expect + bias
            if c["acc"]:
                expect = expect + C0[z]
            s = z * c["sC"]
            got = out[s:s + M * c["ldc"]].reshape(M, c["ldc"])[:, :N]
            assert np.array_equal(got, expect.astype(np.float32)), (i, z, c)
            inside[s:s + M * c["ldc"]].reshape(M, c["ldc"])[:, :N] = True
        assert np.all(np.isnan(out[~inside])), (i, "write outside [M x N]", c)


# ------------------------------------------------------------------- non-finite inputs
def _special_pattern(A, B):
    """IEEE classes of C = A B for small-integer A, B holding a few +-Inf / NaN entries:
    (nan, +inf, -inf) masks and the exact finite values. A product is NaN when a factor is
    NaN or an infinity meets a zero; a sum is NaN when it holds a NaN product or infinities
    of both signs. The zero padding of partial tiles is 0 x 0 and changes nothing."""
    M, K = A.shape
    N = B.shape[1]
    specA = ~np.isfinite(A)
    specB = ~np.isfinite(B)
    fin = (np.where(specA, 0, A).astype(np.float64) @ np.where(specB, 0, B).astype(np.float64))
    nan = np.zeros((M, N), bool)
    pos = np.zeros((M, N), bool)
    neg = np.zeros((M, N), bool)

    def add(i, j, a, b):  # a * b with at least one non-finite factor
        if np.isnan(a) or np.isnan(b) or (np.isinf(a) and b == 0) or (np.isinf(b) and a == 0):
            nan[i, j] = True
        elif np.sign(a) * np.sign(b) > 0:
            pos[i, j] = True
        else:
            neg[i, j] = True

    for i, k in zip(*np.nonzero(specA)):
        for j in range(N):
            add(i, j, A[i, k], B[k, j])
    for k, j in zip(*np.nonzero(specB)):
        for i in range(M):
            if not specA[i, k]:
                add(i, j, A[i, k], B[k, j])
    nan |= pos & neg
    return nan, pos & ~nan, neg & ~nan, fin


@pytest.mark.parametrize("M,K,N", [(3, 300, 40), (37, 45, 29), (200, 300, 260), (129, 4099, 131)])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_nonfinite_inputs_propagate(nncl, policy, M, K, N, ta, tb):
    """+-Inf and NaN in A and B reach exactly the outputs IEEE arithmetic says they reach,
    with the right class, on every kernel family (edge tiles, zero-filled k tails, k
    splits); every other output is the exact small-integer product."""
    say("nonfinite", policy, M, K, N, ta, tb)
    rng = np.random.default_rng(M * 1000 + K + N)
    A = rng.integers(-3, 4, size=(M, K)).astype(np.float32)
    B = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
    for X, count in ((A, 3), (B, 3)):
        idx = rng.choice(X.size, size=count, replace=False)
        X.flat[idx] = np.array([np.inf, -np.inf, np.nan], np.float32)[:count]
    nan, pos, neg, fin = _special_pattern(A, B)
    An = np.ascontiguousarray(A.T) if ta else A
    Bn = np.ascontiguousarray(B.T) if tb else B
    got = gemm_gpu(nncl, An, Bn, bool(ta), bool(tb))
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(np.isposinf(got), pos)
    assert np.array_equal(np.isneginf(got), neg)
    ok = ~(nan | pos | neg)
    assert np.array_equal(got[ok], fin[ok].astype(np.float32))


# Shapes the dispatcher sends to particular kernels under AUTO (the regimes a random-shape audit
# of the dispatcher found): each is checked against fp64 with the kernel it must run.
AUTO_REGIMES = dispatch_cases.AUTO_REGIMES  # shared with the CPU plan test


@pytest.mark.parametrize("spec,plan", AUTO_REGIMES)
def test_auto_regimes(nncl, spec, plan):
    from my_pytchon_opencl_lib_amd import _native
    b, M, K, N, ta, tb = (spec[k] for k in ("batch", "M", "K", "N", "ta", "tb"))
    say("auto regime", spec, plan)
    rng = np.random.default_rng(M * 7 + K + N)
    A = rng.uniform(-1, 1, (b, K, M) if ta else (b, M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (b, N, K) if tb else (b, K, N)).astype(np.float32)
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_AUTO)
    try:
        C = host(nncl.gemm(dev(A), dev(B), transA=bool(ta), transB=bool(tb)))
        assert _native.last_plan().startswith(plan), _native.last_plan()
    finally:
        _native.set_gemm_policy(prev)
    check_gemm(C.reshape(b, M, N), A, B, ta, tb, M=M, N=N, K=K, lda=M if ta else K,
               ldb=K if tb else N, sA=M * K, sB=K * N, batch=b, rows=sample_rows(M, 32))


def _extent(batch, stride, rows, ld, cols):
    return (batch - 1) * stride + (rows - 1) * ld + cols


PINNED = [(n, s, p, False) for n, s, p in dispatch_cases.BASELINE + dispatch_cases.CALLERS] + \
    [(str(s), s, p, True) for s, p in AUTO_REGIMES]


@pytest.mark.parametrize("name,spec,plan,regime", PINNED, ids=[c[0] for c in PINNED])
def test_dry_run_plans_match_real_calls(nncl, name, spec, plan, regime):
    """The plan the dry-run entry point migemm_gemm_plan reports for a call (the CPU test
    tests/test_plans.py pins those) is the plan the real call runs, for every pinned shape."""
    dc = dispatch_cases
    from my_pytchon_opencl_lib_amd import _native
    a = list(dc.regime_args(spec) if regime else dc.args(**spec))
    ta, tb, M, N, K, _, lda, sA, _, ldb, sB, _, _, ldc, sC, batch, flags = a
    offA = (a[5] - dc.BASES["A"]) // 4
    offC = (a[12] - dc.BASES["C"]) // 4
    say("dry run vs real call", name)
    bufs = {
        "A": torch.zeros(offA + _extent(batch, sA, K if ta else M, lda, M if ta else K),
                         device="cuda:0"),
        "B": torch.zeros(_extent(batch, sB, N if tb else K, ldb, K if tb else N),
                         device="cuda:0"),
        "C": torch.zeros(offC + _extent(batch, sC, M, ldc, N), device="cuda:0"),
        "bias": torch.zeros(N, device="cuda:0"),
    }
    real = list(a)
    real[5] = bufs["A"].data_ptr() + 4 * offA
    real[8] = bufs["B"].data_ptr()
    real[11] = bufs["bias"].data_ptr() if a[11] is not None else None
    real[12] = bufs["C"].data_ptr() + 4 * offC
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_AUTO)
    try:
        dry = _native.gemm_plan(*real)
        _native.call("migemm_gemm_strided_batched_ex",
                     ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                     *[ctypes.c_void_p(v) if i in (5, 8, 11, 12) and v is not None else v
                       for i, v in enumerate(real)])
        ran = _native.last_plan()
        torch.cuda.synchronize()
    finally:
        _native.set_gemm_policy(prev)
    assert dry == ran, (dry, ran)
    assert ran.startswith(plan) if regime else ran == plan, (ran, plan)
