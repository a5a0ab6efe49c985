"""GPU parity at element offsets beyond 2^31 and leading dimensions beyond 2^21, through the
C ABI, for every kernel family.

An MI355X holds 288 GB, so a batch entry, a row or a column of an operand can start more
than 2^31 floats (8 GiB) into its buffer. Every kernel forms those addresses in 64 bits;
the tiled kernel that loads straight into LDS adds a 32-bit per-lane offset to a 64-bit
tile base, which it uses only while a 256-row panel spans less than 4 GiB (leading
dimension <= 2^21 floats), and the dispatcher sends longer rows to the register-staged
kernel. The cases below place batch entries 2^31 + 1024 floats apart, use leading
dimensions of exactly 2^21 (the largest the direct loads take, with tile rows 2^31 floats
in) and 2^21 + 4, in every operand layout, with bias, split-K ranges and the accumulating
epilogue. Small-integer operands make the exact answer known, so results must be equal.
The three pools take ~29 GB of device memory and are freed at the end.
"""
import ctypes

import numpy as np
import pytest
import torch

from parity import Tuner, dev, host

pytestmark = pytest.mark.gpu

BIG = (1 << 31) + 1024          # batch stride, floats (16-byte multiple)
POOL = 2_400_000_000            # floats per operand pool (9.6 GB)
LD_DIRECT = 1 << 21             # largest leading dimension of the direct loads
LD_WIDE = (1 << 21) + 4


def say(*a):
    print(*a, flush=True)


@pytest.fixture(scope="module")
def pools():
    p = {k: torch.empty(POOL, dtype=torch.float32, device="cuda") for k in "ABC"}
    yield p
    del p
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


@pytest.fixture
def policy():
    from my_pytchon_opencl_lib_amd import _native
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_AUTO)
    tuner = Tuner()

    def use(name, **tune):
        _native.set_gemm_policy(getattr(_native, "MIGEMM_POLICY_" + name))
        tuner.set(tile=None, splitk=None, direct=None)
        tuner.set(**tune)

    yield use
    _native.set_gemm_policy(prev)
    tuner.restore()


def place(pool, X, stride, ld):
    """Writes X[batch, rows, cols] into `pool` with batch stride `stride` and row pitch
    `ld`; returns the strided view."""
    b, r, c = X.shape
    view = pool.as_strided((b, r, c), (stride, ld, 1))
    view.copy_(dev(X))
    return view


def run(pools, ta, tb, M, K, N, batch, sA, sB, sC, lda, ldb, ldc, bias=False, acc=False,
        seed=0, lo=-4, hi=4):
    from my_pytchon_opencl_lib_amd import _native
    rng = np.random.default_rng(seed)
    a_shape = (batch, K, M) if ta else (batch, M, K)
    b_shape = (batch, N, K) if tb else (batch, K, N)
    A = rng.integers(lo, hi + 1, size=a_shape).astype(np.float32)
    B = rng.integers(lo, hi + 1, size=b_shape).astype(np.float32)
    C0 = rng.integers(-50, 51, size=(batch, M, N)).astype(np.float32)
    bv = rng.integers(-20, 21, size=N).astype(np.float32) if bias else None
    place(pools["A"], A, sA, lda)
    place(pools["B"], B, sB, ldb)
    cview = pools["C"].as_strided((batch, M, N), (sC, ldc, 1))
    if acc:
        cview.copy_(dev(C0))
    else:
        cview.fill_(float("nan"))
    bias_t = dev(bv) if bias else None
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _native.call("migemm_gemm_strided_batched_ex", stream, int(ta), int(tb), M, N, K,
                 ctypes.c_void_p(pools["A"].data_ptr()), lda, sA,
                 ctypes.c_void_p(pools["B"].data_ptr()), ldb, sB,
                 None if bias_t is None else ctypes.c_void_p(bias_t.data_ptr()),
                 ctypes.c_void_p(pools["C"].data_ptr()), ldc, sC, batch, int(acc))
    got = host(cview)
    Aop = np.swapaxes(A, 1, 2) if ta else A
    Bop = np.swapaxes(B, 1, 2) if tb else B
    expect = Aop.astype(np.float64) @ Bop.astype(np.float64)
    if bias:
        expect = expect + bv
    if acc:
        expect = expect + C0
    return got, expect.astype(np.float32)


LAYOUTS = [(0, 0), (0, 1), (1, 0), (1, 1)]
# Kernel families, each forced: the direct kernel in 64x64 and 256x256 tiles (tuning key tile; the
# dispatcher would take 32x32 tiles at these sizes), the register-staged kernel in 128x128
# tiles and the small-output kernel.
FAMILIES = [("TILED", {"tile": 64}), ("TILED", {"tile": 256}),
            ("TILED", {"tile": 128, "direct": 1}), ("SMALL", {})]


@pytest.mark.parametrize("fam", range(len(FAMILIES)))
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_batch_entries_beyond_2_31(pools, policy, fam, ta, tb):
    """Batch entry 1 of A, B and C starts 2^31 + 1024 floats into its buffer."""
    name, env = FAMILIES[fam]
    policy(name, **env)
    M, K, N = 300, 100, 520
    lda = M if ta else K
    ldb = K if tb else N
    say("large offsets batch", name, env, ta, tb)
    got, expect = run(pools, ta, tb, M, K, N, 2, BIG, BIG, BIG, lda, ldb, N, bias=True,
                      seed=ta + 2 * tb + 4 * fam)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("tile", ["128", "256"])
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_split_ranges_beyond_2_31(pools, policy, tile, ta, tb):
    """Split-K partial sums reduced into batch entries 2^31 + 1024 floats apart, C += result
    (direct loads into LDS, also for 128x128 ranges)."""
    policy("TILED", splitk=3, tile=tile, direct=2)
    M, K, N = 260, 1036, 300
    lda = M if ta else K
    ldb = K if tb else N
    say("large offsets split", tile, ta, tb)
    got, expect = run(pools, ta, tb, M, K, N, 2, BIG, BIG, BIG, lda, ldb, N, acc=True,
                      seed=11 + ta + 2 * tb)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("ta", [0, 1])
def test_skinny_batch_entries_beyond_2_31(pools, policy, ta):
    """The M <= 4 streaming kernel: B entries of 64 MB, the second 2^31 + 1024 floats in."""
    policy("SKINNY")
    M, K, N = 3, 4096, 4096
    say("large offsets skinny", ta)
    got, expect = run(pools, ta, 0, M, K, N, 2, BIG, BIG, BIG, M if ta else K, N, N,
                      bias=True, seed=21 + ta, lo=-2, hi=2)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("fam", range(len(FAMILIES)))
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_rows_beyond_2_31(pools, policy, fam, ta, tb):
    """A's rows (or k-rows, transposed) 2^21 floats apart, the direct loads' limit. Not
    transposed, 1100 rows: the last tiles start 2^31 floats in, and a 256-row tile's lanes
    reach 255 * 2^21 floats past its base."""
    name, env = FAMILIES[fam]
    policy(name, **env)
    M, K, N = 1100, 64, 260
    ldb = K if tb else N
    say("large offsets rows", name, env, ta, tb)
    got, expect = run(pools, ta, tb, M, K, N, 1, 0, 0, 0, LD_DIRECT, ldb, N, bias=True,
                      seed=31 + ta + 2 * tb + 4 * fam)
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("fam", range(len(FAMILIES)))
@pytest.mark.parametrize("ta,tb", LAYOUTS)
def test_leading_dimensions_beyond_2_21(pools, policy, fam, ta, tb):
    """lda, ldb and ldc of 2^21 + 4 floats: beyond the direct loads' 32-bit offsets, so the
    tiled dispatcher takes the register-staged kernel."""
    name, env = FAMILIES[fam]
    policy(name, **env)
    M, K, N = 300, 100, 260
    say("wide leading dimensions", name, env, ta, tb)
    got, expect = run(pools, ta, tb, M, K, N, 1, 0, 0, 0, LD_WIDE, LD_WIDE, LD_WIDE,
                      bias=True, seed=41 + ta + 2 * tb + 4 * fam)
    assert np.array_equal(got, expect)
