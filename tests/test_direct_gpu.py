"""GPU parity of the tiled kernel whose operands are loaded straight into LDS
(gemm_direct_kernel: 256x256, 128x256, 128x128 and 64x64 tiles), through the C ABI.

The kernel runs a three-stage LDS pipeline over 16-wide k-tiles: a prologue of one or two
tiles, a main loop of three tiles per pass, a remainder of one or two, and a zero-filled K
tail fetched through registers. The shapes below reach each of those paths (K below one
tile, 1-5 full tiles, K tails) with ragged M and N, in every operand layout, with batch
strides, bias, the accumulating epilogue and split-K ranges. Small-integer operands make the
exact answer known in any summation order. On random operands the kernel must equal the
register-staged 256x256 kernel bit for bit: both sum each output over k in the same order.
"""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from parity import Tuner, check_gemm, dev, host

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def small_ints(shape, seed, lo=-4, hi=4):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


@pytest.fixture(params=["256", "128x256", "128", "64"])
def tiled256(request):
    """The TILED policy with one macro-tile forced (tuning key tile: 256x256, 128x256,
    128x128, 64x64), direct loads forced wherever they apply (direct=2: also for split-K
    ranges of 128x256 tiles, which the library's own choice runs register-staged)."""
    from my_pytchon_opencl_lib_amd import _native
    env = Tuner()
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_TILED)
    env.set(tile=request.param, direct=2, splitk=None)
    yield env
    env.restore()
    _native.set_gemm_policy(prev)


def gemm_ex(ta, tb, M, N, K, a, lda, sA, b, ldb, sB, bias, c, ldc, sC, batch, acc=False):
    from my_pytchon_opencl_lib_amd import _native
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _native.call("migemm_gemm_strided_batched_ex", stream, int(ta), int(tb), M, N, K,
                 ctypes.c_void_p(a.data_ptr()), lda, sA, ctypes.c_void_p(b.data_ptr()), ldb, sB,
                 None if bias is None else ctypes.c_void_p(bias.data_ptr()),
                 ctypes.c_void_p(c.data_ptr()), ldc, sC, batch, int(acc))


def run_exact(M, K, N, ta, tb, batch=1, bias=False, acc=False, seed=0):
    """One strided-batched request on small integers; returns (got, expect)."""
    rng = np.random.default_rng(seed)
    lo, hi = (-2, 2) if K > 2000 else (-4, 4)
    a_rows, a_cols = (K, M) if ta else (M, K)
    b_rows, b_cols = (N, K) if tb else (K, N)
    A = rng.integers(lo, hi + 1, size=(batch, a_rows, a_cols)).astype(np.float32)
    B = rng.integers(lo, hi + 1, size=(batch, b_rows, b_cols)).astype(np.float32)
    bv = rng.integers(-20, 21, size=N).astype(np.float32) if bias else None
    C0 = rng.integers(-50, 51, size=(batch, M, N)).astype(np.float32)
    a, b = dev(A), dev(B)
    c = dev(C0) if acc else torch.full((batch, M, N), float("nan"), device="cuda")
    gemm_ex(ta, tb, M, N, K, a, a_cols, a_rows * a_cols, b, b_cols, b_rows * b_cols,
            None if bv is None else dev(bv), c, N, M * N, batch, acc)
    Aop = np.swapaxes(A, 1, 2) if ta else A
    Bop = np.swapaxes(B, 1, 2) if tb else B
    expect = Aop.astype(np.float64) @ Bop.astype(np.float64)
    if bv is not None:
        expect = expect + bv
    if acc:
        expect = expect + C0
    return host(c), expect.astype(np.float32)


LAYOUTS = [(0, 0), (0, 1), (1, 0), (1, 1)]
# (M, K, N): every extent a multiple of 4 (the direct path's condition). K = 4, 8, 12: the
# tail tile alone; 16, 32, 48: one to three full tiles (prologue and remainder only); 64 and
# 80: a main-loop pass plus a remainder of one and two; 300 and 1036: long loops with tails.
SHAPES = [(256, 4, 256), (260, 8, 516), (300, 12, 300), (256, 16, 260), (516, 32, 260),
          (1000, 48, 1100), (256, 64, 512), (512, 80, 256), (1000, 300, 1100),
          (520, 1036, 264)]


@pytest.mark.parametrize("M,K,N", SHAPES)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_exact(tiled256, M, K, N, ta, tb):
    say("direct exact", M, K, N, ta, tb)
    got, expect = run_exact(M, K, N, ta, tb, seed=M + 3 * K + 7 * N + ta + 2 * tb)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_batched_bias_accumulate(tiled256, ta, tb):
    """Batch strides, bias after the k loop and C += result."""
    for M, K, N, bias, acc in [(300, 100, 520, True, False), (260, 68, 256, False, True),
                               (512, 36, 300, True, True)]:
        say("direct batched", M, K, N, ta, tb, "bias", bias, "acc", acc)
        got, expect = run_exact(M, K, N, ta, tb, batch=3, bias=bias, acc=acc, seed=K)
        assert np.array_equal(got, expect)


@pytest.mark.parametrize("splits", [2, 3, 7])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_split_ranges(tiled256, splits, ta, tb):
    """Forced split-K: ranges that start past k-tile 0, ranges of 1-2 tiles, the K tail in
    the last range; partial sums through the ordered reduce, with bias and accumulate."""
    tiled256.set(splitk=splits)
    for M, K, N, bias, acc in [(516, 1036, 260, False, False), (256, 100, 512, True, True),
                               (300, 4100, 256, True, False)]:
        say("direct split", splits, M, K, N, ta, tb)
        got, expect = run_exact(M, K, N, ta, tb, bias=bias, acc=acc, seed=splits + K)
        assert np.array_equal(got, expect)


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_equals_staged_kernel(tiled256, ta, tb):
    """N(0,1) operands: the direct kernel and the register-staged kernel of the same tile
    (the same MFMA sequence per output) give identical bits. K is not split (the staged NT kernel
    counts ranges in 32-wide k-tiles, the direct kernel in 16-wide ones)."""
    tiled256.set(splitk=1)
    g = torch.Generator(device="cpu").manual_seed(77 + ta + 2 * tb)
    for M, K, N in [(768, 528, 1024), (1028, 1000, 516), (256, 4100, 768)]:
        say("direct vs staged", M, K, N, ta, tb)
        A = torch.randn((K, M) if ta else (M, K), generator=g).cuda()
        B = torch.randn((N, K) if tb else (K, N), generator=g).cuda()
        bias = torch.randn(N, generator=g).cuda()
        outs = []
        for direct in (2, 1):  # direct loads forced, then never
            tiled256.set(direct=direct)
            c = torch.empty((M, N), device="cuda")
            gemm_ex(ta, tb, M, N, K, A, A.shape[1], 0, B, B.shape[1], 0, bias, c, N, 0, 1)
            outs.append(host(c))
        assert np.array_equal(outs[0], outs[1])


def test_unaligned_rows(tiled256):
    """Leading dimensions that are not multiples of 4 (rows off 16-byte boundaries) and an
    operand starting 4 bytes into its buffer: 4-byte loads into LDS; exact."""
    M, K, N = 300, 100, 260
    for lda, ldb, off in [(K + 1, N, 0), (K, N + 2, 0), (K, N, 1)]:
        say("direct unaligned", lda, ldb, off)
        A = small_ints((M, lda), lda)
        B = small_ints((K, ldb), ldb)
        a = dev(np.concatenate([np.zeros(off, np.float32), A.ravel()]))
        b = dev(B)
        c = torch.empty((M, N), device="cuda")
        av = a[off:]
        gemm_ex(0, 0, M, N, K, av, lda, 0, b, ldb, 0, None, c, N, 0, 1)
        expect = A[:, :K].astype(np.float64) @ B[:, :N].astype(np.float64)
        assert np.array_equal(host(c), expect.astype(np.float32))


UNALIGNED = [(67, 5, 129), (130, 33, 70), (257, 131, 259), (1000, 777, 300), (64, 777, 64)]


@pytest.mark.parametrize("M,K,N", UNALIGNED)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_unaligned_operands_exact(tiled256, M, K, N, ta, tb):
    """Odd K, M and N (contiguous extents not multiples of 4, rows off 16-byte boundaries):
    such operands are loaded 4 bytes per lane (global_load_lds_dword). Exact small-integer
    products, batch 2 with bias."""
    say("direct unaligned exact", M, K, N, ta, tb)
    got, expect = run_exact(M, K, N, ta, tb, batch=2, bias=True, seed=M * 3 + K + N + ta)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_direct_unaligned_equals_staged_kernel(tiled256, ta, tb):
    """N(0,1) operands with odd K / M / N (4-byte loads into LDS) give the same bits as the
    register-staged kernel of the same tile (one split range)."""
    tiled256.set(splitk=1)
    g = torch.Generator(device="cpu").manual_seed(99 + ta + 2 * tb)
    for M, K, N in [(1000, 777, 3000), (131, 1001, 257)]:
        say("direct unaligned vs staged", M, K, N, ta, tb)
        A = torch.randn((K, M) if ta else (M, K), generator=g).cuda()
        B = torch.randn((N, K) if tb else (K, N), generator=g).cuda()
        outs = []
        for direct in (2, 1):  # direct loads forced, then never
            tiled256.set(direct=direct)
            c = torch.empty((M, N), device="cuda")
            gemm_ex(ta, tb, M, N, K, A, A.shape[1], 0, B, B.shape[1], 0, None, c, N, 0, 1)
            outs.append(host(c))
        assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_small_kernel_32x32_tiles_exact(ta, tb):
    """The small-output kernel with 32x32 work-group tiles (2 x 2 blocks of 16x16; forced
    with the tuning key small_tiles=2 in every layout): ragged M and N, K tails, k ranges split over
    work-groups, batch strides, bias and the accumulating epilogue, exact."""
    from my_pytchon_opencl_lib_amd import _native
    env = Tuner()
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_SMALL)
    try:
        env.set(small_tiles=2, small_splitk=None)
        for M, K, N, batch, bias, acc, splits in [
                (64, 1536, 4096, 1, True, False, None), (100, 777, 300, 2, True, True, None),
                (65, 4100, 33, 1, False, True, 5), (130, 40, 70, 3, True, False, None),
                (64, 300, 50, 2, False, False, 3)]:
            env.set(small_splitk=splits)
            say("small 32x32", M, K, N, batch, bias, acc, splits, ta, tb)
            got, expect = run_exact(M, K, N, ta, tb, batch=batch, bias=bias, acc=acc,
                                    seed=M + K + N + ta + 2 * tb)
            assert np.array_equal(got, expect)
    finally:
        env.restore()
        _native.set_gemm_policy(prev)


# The panel kernel (gemm_panel_kernel: 32x32 tiles, K % 32 == 0, N % 4 == 0, M % 4 == 0 when
# A is transposed), in every operand layout: ragged M (1, 17, 33, 63, 65; rounded up to a
# multiple of 4 for a transposed A) and N (4, 36, 260), K with 1, 2, 4, 8 and more k-groups
# (so 1, 2, 4 and 8 wavefronts, uneven shares), batches with bias and the accumulating
# epilogue (whose C group is loaded at kernel start with 4 or more wavefronts, in the
# epilogue with 1 or 2).
PANEL_SHAPES = [(1, 32, 4, 1, False, False), (17, 64, 36, 2, True, False),
                (5, 32, 8, 2, True, True), (20, 64, 68, 2, False, True),
                (33, 128, 260, 3, False, True), (63, 256, 100, 1, True, True),
                (65, 1536, 4096, 1, True, False), (64, 800, 516, 2, False, False),
                (128, 2048, 260, 1, True, True), (40, 4096, 68, 1, False, False)]


@pytest.mark.parametrize("M,K,N,batch,bias,acc", PANEL_SHAPES)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_panel_kernel_exact(M, K, N, batch, bias, acc, ta, tb):
    from my_pytchon_opencl_lib_amd import _native
    if ta:
        M = (M + 3) // 4 * 4
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_PANEL)
    try:
        say("panel exact", M, K, N, batch, bias, acc, ta, tb)
        got, expect = run_exact(M, K, N, ta, tb, batch=batch, bias=bias, acc=acc,
                                seed=M + 3 * K + 7 * N + ta + 2 * tb)
        assert _native.last_plan().startswith("panel"), _native.last_plan()
        assert np.array_equal(got, expect)
    finally:
        _native.set_gemm_policy(prev)


def test_panel_layouts_give_identical_bits():
    """The panel kernel sums each output over k in the same order whatever the operand
    layout: NN, NT, TN and TT of the same random operands give the same bits, within
    1e-5 sqrt(K) of fp64."""
    from my_pytchon_opencl_lib_amd import _native
    M, K, N, batch = 96, 1536, 520, 2
    rng = np.random.default_rng(1536)
    A = rng.standard_normal((batch, M, K)).astype(np.float32)
    B = rng.standard_normal((batch, K, N)).astype(np.float32)
    At = np.ascontiguousarray(np.swapaxes(A, 1, 2))
    Bt = np.ascontiguousarray(np.swapaxes(B, 1, 2))
    outs = []
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_PANEL)
    try:
        for ta, tb in LAYOUTS:
            say("panel layouts", ta, tb)
            a, lda = (At, M) if ta else (A, K)
            b, ldb = (Bt, K) if tb else (B, N)
            c = torch.full((batch, M, N), float("nan"), device="cuda")
            gemm_ex(ta, tb, M, N, K, dev(a), lda, M * K, dev(b), ldb, K * N, None, c, N,
                    M * N, batch)
            assert _native.last_plan().startswith("panel"), _native.last_plan()
            outs.append(host(c))
    finally:
        _native.set_gemm_policy(prev)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    check_gemm(outs[0], A, B, 0, 0, M=M, N=N, K=K, lda=K, ldb=N, sA=M * K, sB=K * N,
               batch=batch)


@pytest.mark.parametrize("acc", [False, True])
def test_panel_kernel_unaligned_output_and_bias(acc):
    """The panel epilogue stores 4 columns at a time and reads the bias 4 at a time: C and
    the bias may start at any float (here one float past a 16-byte boundary, with an odd
    ldc and batch stride); the elements between the rows of C stay untouched."""
    from my_pytchon_opencl_lib_amd import _native
    M, K, N, batch = 65, 256, 260, 2
    ldc, sC = N + 3, (N + 3) * M + 5
    rng = np.random.default_rng(11 + acc)
    A = rng.integers(-4, 5, size=(batch, M, K)).astype(np.float32)
    B = rng.integers(-4, 5, size=(batch, K, N)).astype(np.float32)
    bv = rng.integers(-20, 21, size=N + 1).astype(np.float32)
    buf = np.full(1 + batch * sC, np.nan, dtype=np.float32)
    C0 = rng.integers(-50, 51, size=(batch, M, N)).astype(np.float32)
    for b in range(batch):
        for m in range(M):
            s = 1 + b * sC + m * ldc
            buf[s:s + N] = C0[b, m] if acc else np.nan
    c = dev(buf)
    bias = dev(bv)
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_PANEL)
    try:
        gemm_ex(0, 0, M, N, K, dev(A), K, M * K, dev(B), N, K * N, bias[1:], c[1:], ldc, sC,
                batch, acc)
        assert _native.last_plan().startswith("panel"), _native.last_plan()
    finally:
        _native.set_gemm_policy(prev)
    got = host(c)
    expect = A.astype(np.float64) @ B.astype(np.float64) + bv[1:]
    if acc:
        expect = expect + C0
    written = np.zeros(buf.shape, dtype=bool)
    for b in range(batch):
        for m in range(M):
            s = 1 + b * sC + m * ldc
            written[s:s + N] = True
            assert np.array_equal(got[s:s + N], expect[b, m].astype(np.float32)), (b, m)
    assert np.isnan(got[~written]).all()


def test_panel_kernel_falls_back_outside_its_shapes():
    """K % 32 != 0, N % 4 != 0 or, with A transposed, M % 4 != 0 (whose rows are then not
    16-byte aligned either): the PANEL policy runs the dispatcher's own choice instead, with
    the same result."""
    from my_pytchon_opencl_lib_amd import _native
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_PANEL)
    try:
        for M, K, N, ta, tb in [(64, 100, 256, 0, 0), (64, 128, 258, 0, 0), (66, 128, 256, 1, 0),
                                (64, 100, 256, 0, 1), (65, 128, 256, 1, 1)]:
            got, expect = run_exact(M, K, N, ta, tb, seed=K + N + ta)
            assert not _native.last_plan().startswith("panel"), (M, K, N, ta, tb)
            assert np.array_equal(got, expect)
    finally:
        _native.set_gemm_policy(prev)


# (M, K, N, batch, bias, accumulate) for the short-K kernel: K = 1, 15, 16, 17 (no full
# k-group, one, one plus a partial), 33, 64 (config 2a), 79 and 80 (the longest for one
# wavefront per tile); K = 96, 160 (two wavefronts per tile) and 128 (config 2b), 192, 256,
# 320 (four), with ragged M and N around the 16-wide tiles, batches and both epilogues.
TINY_SHAPES = [(1, 1, 1, 1, False, False), (17, 15, 33, 2, True, False),
               (16, 16, 16, 1, False, True), (33, 17, 47, 3, True, True),
               (128, 64, 128, 32, False, False), (100, 33, 70, 8, True, False),
               (255, 79, 129, 1, False, True), (64, 80, 1000, 2, True, True),
               (47, 96, 65, 3, True, False), (128, 128, 64, 32, False, False),
               (33, 160, 100, 2, False, True), (1, 192, 17, 1, True, True),
               (130, 256, 31, 2, True, False), (64, 320, 64, 5, False, False)]


@pytest.mark.parametrize("M,K,N,batch,bias,acc", TINY_SHAPES)
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_tiny_kernel_exact(M, K, N, batch, bias, acc, ta, tb):
    from my_pytchon_opencl_lib_amd import _native
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_TINY)
    try:
        say("tiny exact", M, K, N, batch, bias, acc, ta, tb)
        got, expect = run_exact(M, K, N, ta, tb, batch=batch, bias=bias, acc=acc,
                                seed=M + 3 * K + 7 * N + ta + 2 * tb)
        assert _native.last_plan().startswith("tiny"), _native.last_plan()
        assert np.array_equal(got, expect)
    finally:
        _native.set_gemm_policy(prev)


def test_tiny_kernel_falls_back_outside_its_k():
    """K = 81, 112 (not a multiple of 32), 288 (not of 64) and 384: the TINY policy runs the
    dispatcher's own choice, with the same result."""
    from my_pytchon_opencl_lib_amd import _native
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_TINY)
    try:
        for K in (81, 112, 288, 384):
            got, expect = run_exact(64, K, 64, 0, 0, seed=K)
            assert not _native.last_plan().startswith("tiny"), (K, _native.last_plan())
            assert np.array_equal(got, expect)
    finally:
        _native.set_gemm_policy(prev)


@pytest.mark.parametrize("K,parts", [(96, 2), (128, 4)])
def test_tiny_split_reduction_is_the_single_wavefront_sum_in_k_order(K, parts):
    """K = 96 on two wavefronts per tile and K = 128 on four: the partial tiles are added in
    k order, so the result is identical on every call (and for the same operands in any
    layout)."""
    from my_pytchon_opencl_lib_amd import _native
    rng = np.random.default_rng(K)
    A = rng.standard_normal((4, 100, K)).astype(np.float32)
    B = rng.standard_normal((4, K, 90)).astype(np.float32)
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_TINY)
    try:
        outs = []
        for rep in range(3):
            c = torch.full((4, 100, 90), float("nan"), device="cuda")
            gemm_ex(0, 0, 100, 90, K, dev(A), K, 100 * K, dev(B), 90, K * 90, None, c,
                    90, 100 * 90, 4)
            assert f"splits={parts}" in _native.last_plan(), _native.last_plan()
            outs.append(host(c))
        bt = np.ascontiguousarray(np.swapaxes(B, 1, 2))
        c = torch.full((4, 100, 90), float("nan"), device="cuda")
        gemm_ex(0, 1, 100, 90, K, dev(A), K, 100 * K, dev(bt), K, 90 * K, None, c,
                90, 100 * 90, 4)
        outs.append(host(c))
    finally:
        _native.set_gemm_policy(prev)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    check_gemm(outs[0], A, B, 0, 0, M=100, N=90, K=K, lda=K, ldb=90, sA=100 * K,
               sB=K * 90, batch=4)


def test_tiny_is_the_config2a_choice():
    """BASELINE config 2a (32 x 128x64 @ 64x128) runs on the short-K kernel under AUTO, and
    its result is within 1e-5 sqrt(K) of fp64."""
    from my_pytchon_opencl_lib_amd import _native
    Q = oracle.normal((32, 128, 64), 1, 0)
    Kt = oracle.normal((32, 64, 128), 1, 1)
    say("config 2a plan")
    c = torch.empty((32, 128, 128), device="cuda")
    gemm_ex(0, 0, 128, 128, 64, dev(Q), 64, 128 * 64, dev(Kt), 128, 64 * 128, None, c, 128,
            128 * 128, 32, 0)
    assert _native.last_plan().startswith("tiny"), _native.last_plan()
    check_gemm(host(c), Q, Kt, 0, 0, M=128, N=128, K=64, lda=64, ldb=128, sA=128 * 64,
               sB=64 * 128, batch=32)


# The rows kernel of the skinny family (gemv_rows_kernel: M <= 4, B stored [N, K], each
# wavefront streaming 1, 2 or 4 whole rows of B): K with no whole batch of loads (3, 200),
# one batch and a vector tail (2304 = 2048 + 256), batches with a partial last chunk
# (2051, 4099: k beyond K in the last 16 bytes), N not a multiple of the rows per wavefront,
# A in both layouts, batches with bias and the accumulating epilogue.
ROWS_SHAPES = [(1, 3, 5, 1, False, False), (2, 200, 37, 2, True, False),
               (3, 2304, 1030, 1, False, True), (4, 2051, 1026, 2, True, True),
               (1, 4099, 2050, 1, True, False), (2, 1027, 3, 3, False, False)]


@pytest.mark.parametrize("M,K,N,batch,bias,acc", ROWS_SHAPES)
@pytest.mark.parametrize("ta", [0, 1])
def test_rows_kernel_exact(M, K, N, batch, bias, acc, ta):
    from my_pytchon_opencl_lib_amd import _native
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_SKINNY)
    try:
        say("rows exact", M, K, N, batch, bias, acc, ta)
        got, expect = run_exact(M, K, N, ta, 1, batch=batch, bias=bias, acc=acc,
                                seed=M + 3 * K + 7 * N + ta)
        assert _native.last_plan().startswith("skinny-rows"), _native.last_plan()
        assert np.array_equal(got, expect)
    finally:
        _native.set_gemm_policy(prev)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_rows_kernel_random_and_dispatch(M):
    """Random operands within 1e-5 sqrt(K) of fp64, the same bits for either layout of A, and
    the GEMV the dispatcher sends to the rows kernel under AUTO (M = 1, any width; M = 2-4
    with many rows of long K)."""
    from my_pytchon_opencl_lib_amd import _native
    K, N = 4099, 11008
    rng = np.random.default_rng(4099 + M)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    Bt = rng.uniform(-1, 1, (N, K)).astype(np.float32)
    bias = rng.uniform(-1, 1, N).astype(np.float32)
    say("rows random", M, K, N)
    outs = []
    for ta in (0, 1):
        a = np.ascontiguousarray(A.T) if ta else A
        c = torch.full((M, N), float("nan"), device="cuda")
        gemm_ex(ta, 1, M, N, K, dev(a), M if ta else K, 0, dev(Bt), K, 0, dev(bias), c, N, 0, 1)
        assert _native.last_plan().startswith("skinny-rows"), (ta, _native.last_plan())
        outs.append(host(c))
    assert np.array_equal(outs[0], outs[1])
    check_gemm(outs[0], A, Bt, 0, 1, bias=bias, M=M, N=N, K=K, lda=K, ldb=K)
