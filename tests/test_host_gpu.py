"""The reference's own hot-path tests, re-run through the host API (NnClGlob mirror) on the
HIP kernels. Shapes follow the reference tests; inputs come from this repository's seeded
generator (the reference's are unseeded numpy draws). Each test also applies the reference
tests' own bar (np.testing.assert_allclose rtol=atol=1e-4 against PyTorch CPU) next to the
fp64 bar of the matmul path."""
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


def test_matmul_tiled_reference_shape(nncl):
    """tests/test_matrix_ops.py:87-131 (Test 2): M,K,N = 64,128,96."""
    A = oracle.normal((64, 128), 10, 0)
    B = oracle.normal((128, 96), 10, 1)
    say("test_matrix_ops matmul 64x128x96")
    import ctypes
    from my_pytchon_opencl_lib_amd import _native
    a, b = dev(A), dev(B)
    c = torch.empty((64, 96), device="cuda:0")
    _native.call("migemm_matmul_tiled", ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                 ctypes.c_void_p(a.data_ptr()), ctypes.c_void_p(b.data_ptr()),
                 ctypes.c_void_p(c.data_ptr()), 64, 128, 96)
    C = host(c)
    np.testing.assert_allclose(C, torch.matmul(torch.from_numpy(A), torch.from_numpy(B)).numpy(),
                               rtol=1e-4, atol=1e-4)
    check_gemm(C, A, B, 0, 0, M=64, N=96, K=128, lda=128, ldb=96, ref=oracle.matmul_tiled(A, B))


def test_bmm_tiled_reference_shape(nncl):
    """tests/test_bmm.py:6-74: BATCH=4, M,K,N = 32,64,32 (the reference swallows failures
    there, test_bmm.py:69-74; here they fail)."""
    A = oracle.normal((4, 32, 64), 11, 0)
    B = oracle.normal((4, 64, 32), 11, 1)
    say("test_bmm 4x32x64x32")
    C = host(nncl.bmm(dev(A), dev(B)))
    np.testing.assert_allclose(C, torch.bmm(torch.from_numpy(A), torch.from_numpy(B)).numpy(),
                               rtol=1e-4, atol=1e-4)
    check_gemm(C, A, B, 0, 0, M=32, N=32, K=64, lda=64, ldb=32, sA=32 * 64, sB=64 * 32,
               batch=4, ref=oracle.bmm(A, B))


def test_bmm_glob_pipeline(nncl):
    """tests/test_nncl_glob.py:118-177: BATCH,M,K,N = 4,32,64,48; forward, then
    bmm_backward(grad_output, A, B) checked against PyTorch autograd."""
    A = oracle.normal((4, 32, 64), 777, 0)
    B = oracle.normal((4, 64, 48), 777, 1)
    G = oracle.normal((4, 32, 48), 777, 2)
    say("test_bmm_glob_pipeline")
    C = host(nncl.bmm(dev(A), dev(B)))
    gA, gB = nncl.bmm_backward(dev(G), dev(A), dev(B))
    gA, gB = host(gA), host(gB)
    tA = torch.tensor(A, requires_grad=True)
    tB = torch.tensor(B, requires_grad=True)
    tC = torch.bmm(tA, tB)
    tC.backward(torch.tensor(G))
    np.testing.assert_allclose(C, tC.detach().numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(gA, tA.grad.numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(gB, tB.grad.numpy(), rtol=1e-4, atol=1e-4)
    # fp64 bar: dA = dC B^T (NT over N=48), dB = A^T dC (TN over M=32)
    check_gemm(gA, G, B, 0, 1, M=32, N=64, K=48, lda=48, ldb=48, sA=32 * 48, sB=64 * 48,
               batch=4)
    check_gemm(gB, A, G, 1, 0, M=64, N=48, K=32, lda=64, ldb=48, sA=32 * 64, sB=32 * 48,
               batch=4)
    # grad_A is a separate tensor: the reference's "bmm_c" aliasing (BmmOp.cs:47,60) is gone
    assert gA.shape == (4, 32, 64) and gB.shape == (4, 64, 48)


def test_linear_via_permute_and_bmm(nncl):
    """tests/test_layers.py:88-112 with core/layers.py:21-33: Linear(16 -> 8) on 8 tokens,
    weight [out, in] transposed by permute([1, 0]) then bmm."""
    x = oracle.normal((2, 4, 16), 42, 0)
    bound = 1.0 / np.sqrt(16)
    w = oracle.uniform((8, 16), 42, 1, -bound, bound)
    say("test_layers Linear")
    wt = nncl.permute(dev(w), [1, 0])
    assert np.array_equal(host(wt), w.T)
    y = host(nncl.bmm(dev(x.reshape(1, 8, 16)), wt.unsqueeze(0).contiguous()))
    ref = torch.nn.functional.linear(torch.from_numpy(x), torch.from_numpy(w)).numpy()
    np.testing.assert_allclose(y.reshape(-1, 8), ref.reshape(-1, 8), rtol=1e-4, atol=1e-4)


def test_linear_layer_runs_nt_without_permute(nncl, monkeypatch):
    """core/layers.py:21-33 at the tests/test_layers.py:88-112 shape (Linear(16 -> 8) on 2x4
    tokens) through layers.Linear: one NT GEMM on the [out, in] weight, no tensor_permute
    launch. Within 1e-5*sqrt(K) of fp64 and of the reference's permute + bmm path; exact on
    small integers. Also the Linear(500 -> 6565) shape of the reference's largest caller."""
    from my_pytchon_opencl_lib_amd import NnClGlob, _native, layers
    x = oracle.normal((2, 4, 16), 42, 0)
    bound = 1.0 / np.sqrt(16)
    w = oracle.uniform((8, 16), 42, 1, -bound, bound)
    ref_path = host(nncl.bmm(dev(x.reshape(1, 8, 16)),
                             nncl.permute(dev(w), [1, 0]).unsqueeze(0).contiguous()))

    def no_permute(*a, **k):
        raise AssertionError("Linear.forward must not materialise the weight transpose")
    monkeypatch.setattr(NnClGlob, "Permute", no_permute)
    monkeypatch.setattr(NnClGlob, "permute", no_permute)
    say("layers.Linear 16 -> 8")
    lin = layers.Linear(16, 8, nncl, weight=w)
    y = host(lin.forward(dev(x)))
    assert y.shape == (2, 4, 8)
    plan = _native.last_plan()
    assert plan.endswith(" NT") and "K=16" in plan and "N=8" in plan, plan
    check_gemm(y.reshape(8, 8), x.reshape(8, 16), w, 0, 1, M=8, N=8, K=16, lda=16, ldb=16)
    ap = oracle.gemm_absprod(x.reshape(8, 16), w, 0, 1, None, M=8, N=8, K=16, lda=16,
                             ldb=16)[0]
    d = np.abs(y.reshape(8, 8).astype(np.float64) - ref_path.reshape(8, 8)) / ap
    assert np.max(d) <= oracle.tolerance(16)
    ref = torch.nn.functional.linear(torch.from_numpy(x), torch.from_numpy(w)).numpy()
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4)  # the reference test's bar
    xi = small_ints((3, 7, 33), 5)
    wi = small_ints((20, 33), 6)
    yi = host(layers.Linear(33, 20, nncl, weight=wi)(dev(xi)))
    assert np.array_equal(yi, (xi.astype(np.int64) @ wi.T.astype(np.int64)).astype(np.float32))
    say("layers.Linear 500 -> 6565 on [8, 1500, 500]")
    xb = oracle.normal((8, 1500, 500), 43, 0)
    wb = oracle.uniform((6565, 500), 43, 1, -1 / np.sqrt(500), 1 / np.sqrt(500))
    yb = host(layers.Linear(500, 6565, nncl, weight=wb)(dev(xb))).reshape(12000, 6565)
    check_gemm(yb, xb.reshape(12000, 500), wb, 0, 1, M=12000, N=6565, K=500, lda=500, ldb=500,
               rows=sample_rows(12000, 12))


def test_linear_op_backward(nncl):
    """cs/core/LinearOp.cs:16-49 (dX NT, dW TN + batch sum, db column sum) against
    PyTorch autograd and fp64, on the TestLSTMRealTrain-style ragged N."""
    from my_pytchon_opencl_lib_amd.autograd import LinearOp
    batch, M, K, N = 3, 50, 40, 6565 // 50  # 131 columns: N not a multiple of 4
    X = oracle.normal((batch, M, K), 12, 0)
    W = oracle.uniform((1, K, N), 12, 1, -0.1, 0.1)
    bias = oracle.uniform((N,), 12, 2, -0.1, 0.1)
    G = oracle.normal((batch, M, N), 12, 3)
    say("LinearOp backward")
    y = nncl.LinearForward(dev(X), dev(W), dev(bias))
    node = LinearOp(dev(X), dev(W), dev(bias), y, nncl)
    gX, gW, gb = [host(t) for t in node.Backward(dev(G))]
    tX = torch.tensor(X, requires_grad=True)
    tW = torch.tensor(W, requires_grad=True)
    tb = torch.tensor(bias, requires_grad=True)
    ty = torch.matmul(tX, tW) + tb
    ty.backward(torch.tensor(G))
    np.testing.assert_allclose(host(y), ty.detach().numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(gX, tX.grad.numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(gW, tW.grad.numpy(), rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(gb, tb.grad.numpy(), rtol=1e-4, atol=1e-4)
    assert np.array_equal(gb, oracle.linear_bias_backward(G))  # same sequential order
    check_gemm(gX, G, W, 0, 1, M=M, N=K, K=N, lda=N, ldb=N, sA=M * N, sB=0, batch=batch)
    Xf = X.reshape(batch * M, K)
    Gf = G.reshape(batch * M, N)
    check_gemm(gW.reshape(K, N), Xf, Gf, 1, 0, M=K, N=N, K=batch * M, lda=K, ldb=N)


def test_autograd_functions_match_torch(nncl):
    from my_pytchon_opencl_lib_amd import autograd as ag
    A = dev(oracle.normal((3, 20, 30), 13, 0)).requires_grad_()
    B = dev(oracle.normal((1, 30, 25), 13, 1)).requires_grad_()
    say("autograd bmm (broadcast B)")
    out = ag.bmm(A, B)
    g = dev(oracle.normal((3, 20, 25), 13, 2))
    out.backward(g)
    tA = A.detach().cpu().requires_grad_()
    tB = B.detach().cpu().requires_grad_()
    tout = torch.matmul(tA, tB)
    tout.backward(g.cpu())
    np.testing.assert_allclose(host(out), tout.detach().numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(host(A.grad), tA.grad.numpy(), rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(host(B.grad), tB.grad.numpy(), rtol=1e-4, atol=1e-4)


def test_permute_generic_and_transpose(nncl):
    rng = np.random.default_rng(14)
    for nd in range(1, 11):
        shape = tuple(int(s) for s in rng.integers(1, 5, size=nd))
        x = rng.standard_normal(shape).astype(np.float32)
        axes = [int(a) for a in rng.permutation(nd)]
        say("permute", shape, axes)
        assert np.array_equal(host(nncl.Permute(dev(x), axes)), oracle.tensor_permute(x, axes))
    x = oracle.normal((5, 70, 33), 14, 1)
    assert np.array_equal(host(nncl.Permute(dev(x), [0, 2, 1])), x.transpose(0, 2, 1))


def test_permute_canonical_forms(nncl):
    """Size-1 axes, runs of axes that stay adjacent (merged into one), identity permutations,
    batched transposes that only appear after merging, the 16-byte path (innermost axis
    contiguous in both layouts, a multiple of 4 long) and a source 4 bytes off 16-byte
    alignment (which must take the 4-byte path): each equals numpy exactly."""
    cases = [((32, 128, 16, 64), (0, 2, 1, 3)), ((4, 1, 5), (0, 2, 1)), ((1, 1, 1), (2, 0, 1)),
             ((6, 7, 8), (0, 1, 2)), ((2, 3, 4, 5), (0, 1, 3, 2)), ((2, 3, 4, 5), (2, 3, 0, 1)),
             ((3, 1, 4, 1, 8), (4, 2, 0, 3, 1)), ((5, 6, 7, 8), (1, 0, 2, 3)),
             ((2, 2, 3, 3, 4), (3, 4, 0, 1, 2)), ((9, 12), (1, 0)), ((7, 5, 12), (1, 0, 2))]
    for shape, axes in cases:
        x = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape)
        say("permute canonical", shape, axes)
        assert np.array_equal(host(nncl.Permute(dev(x), list(axes))), x.transpose(axes))
        base = torch.empty(x.size + 1, dtype=torch.float32, device="cuda:0")
        xs = base[1:].view(shape)  # data pointer 4 bytes past a 16-byte boundary
        xs.copy_(torch.from_numpy(x))
        assert np.array_equal(host(nncl.Permute(xs, list(axes))), x.transpose(axes))


@pytest.mark.parametrize("shape,axes", [((3, 100003, 2), (1, 2, 0)),
                                        ((70001, 3, 5), (2, 0, 1)),
                                        ((2, 3, 65537, 4), (2, 3, 1, 0)),
                                        ((1, 2097153), (1, 0)),
                                        ((7, 1, 1, 131071), (3, 0, 2, 1))])
def test_permute_large_axes(nncl, shape, axes):
    """Axes of 65537-2097153 (odd, prime, 2^k + 1 sizes) through the generic gather: its
    invariant-divisor index unpacking must equal numpy's transpose exactly."""
    x = np.arange(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    say("permute large", shape, axes)
    assert np.array_equal(host(nncl.Permute(dev(x), list(axes))), x.transpose(axes))


def test_sum_and_bias_backward_bit_exact(nncl):
    """Up to 256 summed rows the library adds in the reference's order (one ascending
    chain from +0.0f, reduce_sum_axis.cl:3-27, linear.cl:149-168): bit-identical."""
    x = oracle.normal((4, 200, 37), 15, 0)
    say("sum / bias backward, one chunk")
    for axis in (0, 1, 2):
        got = host(nncl.Sum(dev(x), axis, keepDims=True))
        assert np.array_equal(got, oracle.reduce_sum_axis(x, axis))
    gb = host(nncl.LinearBiasBackward(dev(x[:1]), [37]))
    assert np.array_equal(gb, oracle.linear_bias_backward(x[:1]))


def blocked_sum_bound(x2d, rows=256):
    """Error bound of the chunked sum over axis 0 of x2d: (rows - 1 + chunks - 1) * u * sum|x|
    (recursive summation within a chunk, then over the chunk sums; u = 2^-24)."""
    n = x2d.shape[0]
    chunks = -(-n // rows)
    steps = min(n, rows) - 1 + chunks - 1
    return steps * 2.0 ** -24 * np.abs(x2d.astype(np.float64)).sum(axis=0)


@pytest.mark.parametrize("rows,N", [(12000, 6565), (1000, 37), (257, 512), (70000, 3)])
def test_chunked_column_sum(nncl, rows, N):
    """Longer axes are summed in 256-row chunks, combined in chunk order. Small integers make
    every order exact (bit-identical to the reference's chain); random data stays within
    the blocked-summation bound of the fp64 sum."""
    say("chunked column sum", rows, N)
    xi = small_int_matrix(rows, N, 17)
    gb = host(nncl.LinearBiasBackward(dev(xi), [N]))
    assert np.array_equal(gb, oracle.linear_bias_backward(xi))
    x = oracle.normal((rows, N), 17, 1)
    gb = host(nncl.LinearBiasBackward(dev(x), [N])).astype(np.float64)
    ref = x.astype(np.float64).sum(axis=0)
    assert np.all(np.abs(gb - ref) <= blocked_sum_bound(x))
    got = host(nncl.Sum(dev(x.reshape(1, rows, N)), 1, keepDims=True)).reshape(N)
    assert np.array_equal(got.astype(np.float64), gb)  # same kernel, same order


def small_int_matrix(rows, N, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(-8, 9, size=(rows, N)).astype(np.float32)


def test_linear_500_to_6565_end_to_end(nncl):
    """The largest real caller of the path: Linear(500 -> 6565) on [8, 1500, 500]
    (cs/TestLSTMRealTrain/EncoderDecoder.cs:29,75): forward with the bias epilogue, then
    LinearOp.Backward (cs/core/LinearOp.cs:16-49): dX = dY W^T (NT), dW = sum_b X_b^T dY_b
    (one TN GEMM over 12000 rows), db = column sum of dY."""
    from my_pytchon_opencl_lib_amd.autograd import LinearOp
    batch, M, K, N = 8, 1500, 500, 6565
    X = oracle.normal((batch, M, K), 18, 0)
    W = oracle.uniform((1, K, N), 18, 1, -1 / 22, 1 / 22)
    bias = oracle.uniform((N,), 18, 2, -1 / 22, 1 / 22)
    G = oracle.normal((batch, M, N), 18, 3, 0.0, 1.0 / 64)
    say("Linear(500->6565) forward")
    y = nncl.LinearForward(dev(X), dev(W), dev(bias))
    rows = sample_rows(M, 16)
    check_gemm(host(y), X, W, 0, 0, bias=bias, M=M, N=N, K=K, lda=K, ldb=N, sA=M * K, sB=0,
               batch=batch, rows=rows)
    say("Linear(500->6565) backward")
    node = LinearOp(dev(X), dev(W), dev(bias), y, nncl)
    gX, gW, gb = [host(t) for t in node.Backward(dev(G))]
    check_gemm(gX, G, W, 0, 1, M=M, N=K, K=N, lda=N, ldb=N, sA=M * N, sB=0, batch=batch,
               rows=rows)
    Xf = X.reshape(batch * M, K)
    Gf = G.reshape(batch * M, N)
    check_gemm(gW.reshape(K, N), Xf, Gf, 1, 0, M=K, N=N, K=batch * M, lda=K, ldb=N,
               rows=sample_rows(K, 16))
    ref = Gf.astype(np.float64).sum(axis=0)
    assert np.all(np.abs(gb.astype(np.float64) - ref) <= blocked_sum_bound(Gf))


def test_shape_errors_before_launch(nncl):
    from my_pytchon_opencl_lib_amd import ShapeError
    a = dev(np.zeros((2, 3, 4), np.float32))
    with pytest.raises(ShapeError):
        nncl.Bmm(a, dev(np.zeros((3, 4, 5), np.float32)))  # batch 2 vs 3
    with pytest.raises(ShapeError):
        nncl.Bmm(a, dev(np.zeros((2, 5, 5), np.float32)))  # K 4 vs 5
    with pytest.raises(ShapeError):
        nncl.BmmPermute(a, dev(np.zeros((2, 5, 3), np.float32)), transB=True)
    with pytest.raises(ShapeError):
        nncl.Permute(a, [0, 1])


def test_c_caller_on_the_gpu():
    """A plain C99 program (no torch, no Python: the way the C# host would call the library)
    allocates, copies, runs the GEMM entry points on GPU 0 and checks them exactly
    (tests/c_abi_check.c). It runs as a child process."""
    import c_abi
    say("c_abi_check gpu")
    r = c_abi.run("gpu")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c_abi_check gpu: ok" in r.stdout


def test_shared_weight_batches_run_as_one_gemm(nncl):
    """Under the AUTO policy a batch that shares B (stride 0) with contiguous A and C entries
    runs as one GEMM of batch * M rows: LinearForward on [8, 300, 52] -> 260 equals the
    flattened [2400, 52] GEMM + bias bit for bit, and the NT form (dX = dY W^T) likewise."""
    X = oracle.normal((8, 300, 52), 41, 0)
    W = oracle.uniform((1, 52, 260), 41, 1)
    bias = oracle.uniform((260,), 41, 2)
    say("shared weight batches")
    y = host(nncl.LinearForward(dev(X), dev(W), dev(bias)))
    flat = host(nncl.gemm(dev(X.reshape(2400, 52)), dev(W[0]), bias=dev(bias)))
    assert np.array_equal(y.reshape(2400, 260), flat)
    G = oracle.normal((8, 300, 260), 41, 3)
    gx = host(nncl.BmmPermute(dev(G), dev(W), transB=True))
    flat = host(nncl.gemm(dev(G.reshape(2400, 260)), dev(W[0]), transB=True))
    assert np.array_equal(gx.reshape(2400, 52), flat)
    check_gemm(gx.reshape(2400, 52), G.reshape(2400, 260), W[0], 0, 1, M=2400, N=52, K=260,
               lda=260, ldb=260)
