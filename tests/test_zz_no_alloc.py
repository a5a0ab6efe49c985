"""The no-allocation GEMM entry point (migemm_gemm_strided_batched_noalloc), through the C ABI.

It runs the kernels of migemm_gemm_strided_batched_ex with their partial sums in the
library's static device scratch array instead of the stream's workspace, so it calls no
hipMalloc. Each case runs two calls in a row, the second with a smaller input (so the
scratch still holds the first call's partial sums), and compares both with the existing
entry point's output bit for bit: the same kernels in the same order, so the same bits.
"""
import ctypes

import numpy as np
import pytest
import torch

from parity import Tuner, dev, host

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20  # MIGEMM_NOALLOC_SCRATCH_BYTES


def say(*a):
    print(*a, flush=True)


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def run(entry, stream, ta, tb, M, N, K, A, B, bias, C, batch, sA, sB, sC, flags):
    from my_pytchon_opencl_lib_amd import _native
    L = _native.load()
    lda = A.shape[-1]
    ldb = B.shape[-1]
    return getattr(L, entry)(stream, ta, tb, M, N, K, _p(A), lda, sA, _p(B), ldb, sB, _p(bias),
                             _p(C), N, sC, batch, flags)


def case(seed, ta, tb, M, N, K, batch=1, bias=False, acc=False, broadcast_b=False):
    g = torch.Generator(device="cpu").manual_seed(seed)
    A = torch.randn((batch,) + ((K, M) if ta else (M, K)), generator=g).cuda()
    nb = 1 if broadcast_b else batch
    B = torch.randn((nb,) + ((N, K) if tb else (K, N)), generator=g).cuda()
    b = torch.randn(N, generator=g).cuda() if bias else None
    C0 = torch.randn(batch, M, N, generator=g).cuda()
    sA = M * K if batch > 1 else 0
    sB = 0 if broadcast_b else (K * N if batch > 1 else 0)
    sC = M * N if batch > 1 else 0
    return dict(ta=ta, tb=tb, M=M, N=N, K=K, A=A, B=B, bias=b, C0=C0, batch=batch, sA=sA,
                sB=sB, sC=sC, flags=1 if acc else 0)


def both(stream, c):
    """(existing entry's output, no-allocation entry's output) of one case."""
    from my_pytchon_opencl_lib_amd import _native
    outs = []
    for entry in ("migemm_gemm_strided_batched_ex", "migemm_gemm_strided_batched_noalloc"):
        C = c["C0"].clone()
        torch.cuda.synchronize()
        rc = run(entry, stream, c["ta"], c["tb"], c["M"], c["N"], c["K"], c["A"], c["B"],
                 c["bias"], C, c["batch"], c["sA"], c["sB"], c["sC"], c["flags"])
        assert rc == 0, (entry, rc, _native.last_error())
        plan = _native.last_plan()
        torch.cuda.synchronize()
        outs.append((host(C), plan))
    return outs


# (first call, second smaller call): each pair keeps partial sums in the scratch.
PAIRS = [
    # tiled split-K (64 x 8192 x 1536: 64x64 tiles in 27 k ranges), then a shorter one
    (dict(seed=1, ta=0, tb=0, M=64, N=1536, K=8192),
     dict(seed=2, ta=0, tb=0, M=64, N=512, K=4096)),
    # the sliced GEMV (config 5b's kernel), then a narrower one with bias, accumulating
    (dict(seed=3, ta=0, tb=0, M=1, N=11008, K=4096),
     dict(seed=4, ta=0, tb=0, M=1, N=4096, K=2048, bias=True, acc=True)),
    # small-output kernel with its k range split over work-groups, NT then TN, batched
    (dict(seed=5, ta=0, tb=1, M=64, N=64, K=2048, batch=3),
     dict(seed=6, ta=1, tb=0, M=48, N=40, K=1024, batch=2, bias=True)),
    # long-K split of a large output, then a ragged one with a broadcast B
    (dict(seed=7, ta=1, tb=0, M=512, N=1024, K=8192),
     dict(seed=8, ta=0, tb=0, M=100, N=300, K=3000, batch=2, broadcast_b=True, acc=True)),
]


@pytest.mark.parametrize("pair", range(len(PAIRS)))
def test_noalloc_matches_existing_entry(pair):
    from my_pytchon_opencl_lib_amd import _native
    _native.load()
    s = ctypes.c_void_p()
    _native.call("migemm_stream_create", ctypes.byref(s))
    try:
        for i, spec in enumerate(PAIRS[pair]):
            c = case(**spec)
            say("noalloc", pair, i, {k: v for k, v in spec.items() if k != "seed"})
            (ref, ref_plan), (got, plan) = both(s, c)
            assert plan == ref_plan, (plan, ref_plan)
            assert np.array_equal(got, ref), f"call {i} differs from the existing entry point"
        # a stream that only the no-allocation entry point used has no library workspace
        size = ctypes.c_size_t(1)
        c = case(**PAIRS[pair][0])
        s2 = ctypes.c_void_p()
        _native.call("migemm_stream_create", ctypes.byref(s2))
        rc = run("migemm_gemm_strided_batched_noalloc", s2, c["ta"], c["tb"], c["M"], c["N"],
                 c["K"], c["A"], c["B"], c["bias"], c["C0"].clone(), c["batch"], c["sA"],
                 c["sB"], c["sC"], c["flags"])
        assert rc == 0, _native.last_error()
        assert "splits=1 " not in _native.last_plan(), "the case must use the scratch"
        _native.call("migemm_workspace_size", s2, ctypes.byref(size))
        assert size.value == 0
        _native.call("migemm_stream_destroy", s2)
    finally:
        _native.call("migemm_stream_destroy", s)


def test_noalloc_rejects_more_than_its_scratch():
    """64 k ranges of a 1024 x 1024 output keep 256 MiB of partial sums: more than the
    scratch holds, so the call fails with MIGEMM_ERR_WORKSPACE before any launch."""
    from my_pytchon_opencl_lib_amd import _native
    L = _native.load()
    c = case(seed=9, ta=0, tb=0, M=1024, N=1024, K=4096)
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_TILED)
    tuner = Tuner()
    try:
        tuner.set(tile=64, splitk=64)
        C = torch.full((1024, 1024), float("nan"), device="cuda:0")
        torch.cuda.synchronize()
        rc = run("migemm_gemm_strided_batched_noalloc", None, 0, 0, 1024, 1024, 4096, c["A"],
                 c["B"], None, C, 1, 0, 0, 0, 0)
        assert rc == _native.MIGEMM_ERR_WORKSPACE
        msg = _native.last_error()
        assert str(64 * 1024 * 1024 * 4) in msg and str(SCRATCH_BYTES) in msg, msg
        torch.cuda.synchronize()
        assert torch.isnan(C).all(), "a rejected call must not write its output"
    finally:
        tuner.restore()
        _native.set_gemm_policy(prev)
    assert L.migemm_gemm_strided_batched_noalloc(None, 0, 0, 0, 4, 4, None, 4, 0, None, 4, 0,
                                                 None, None, 4, 0, 1, 0) == \
        _native.MIGEMM_ERR_INVALID_ARG


def test_noalloc_under_graph_capture():
    """Callers that cannot allocate include code under HIP graph capture: the no-allocation
    entry point's split-K GEMM and sliced GEMV are captured on a stream that was never used
    before, the graph is replayed three times with eager work between the replays, and each
    replay's outputs equal the existing entry point's eager outputs bit for bit."""
    from my_pytchon_opencl_lib_amd import _native
    _native.load()
    cases = [case(**PAIRS[0][0]), case(**PAIRS[1][0])]
    s = ctypes.c_void_p()
    _native.call("migemm_stream_create", ctypes.byref(s))
    try:
        eager = []
        for c in cases:
            (ref, _), _ = both(s, c)
            eager.append(ref)
        say("noalloc under capture")
        cap = torch.cuda.Stream()
        outs = [c["C0"].clone() for c in cases]
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap):
            st = ctypes.c_void_p(cap.cuda_stream)
            for c, C in zip(cases, outs):
                rc = run("migemm_gemm_strided_batched_noalloc", st, c["ta"], c["tb"], c["M"],
                         c["N"], c["K"], c["A"], c["B"], c["bias"], C, c["batch"], c["sA"],
                         c["sB"], c["sC"], c["flags"])
                assert rc == 0, _native.last_error()
        size = ctypes.c_size_t(1)
        _native.call("migemm_workspace_size", ctypes.c_void_p(cap.cuda_stream),
                     ctypes.byref(size))
        assert size.value == 0, "the capture allocated a workspace"
        for rep in range(3):
            for c, C in zip(cases, outs):
                C.copy_(c["C0"])
            noise = torch.mm(cases[0]["A"][0], cases[0]["B"][0])  # eager work between replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for i, C in enumerate(outs):
                assert np.array_equal(host(C), eager[i]), f"replay {rep}, case {i}"
            del noise
    finally:
        _native.call("migemm_stream_destroy", s)
