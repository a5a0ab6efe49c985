"""The reference host's runtime objects on HIP, through the C ABI ("cs/" =
csharp/cstorchcl/cstorchcl/):
  * the device context (cs/core/ComputeContext.cs:35-170),
  * the name-keyed buffer pool (cs/compiler/OpenCLBufferManager.cs:22-91): reuse while large
    enough, replacement when it grows or the context differs, release,
  * the per-thread current queue (cs/core/DeviceQueueRegistry.cs:14-46),
  * Tensor.DataBuffer (cs/core/Tensor.cs:41) as migemm_tensor_buffer,
  * the Bmm -> BmmOp.Backward sequence on pooled buffers: with the reference's shared "bmm_c"
    name gradB overwrites gradA (BmmOp.cs:47,60); with a fresh name per output both survive.
"""
import ctypes
import threading

import numpy as np
import pytest
import torch

from parity import host

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


@pytest.fixture
def rt():
    from my_pytchon_opencl_lib_amd import _native, runtime
    _native.load()
    yield runtime
    runtime.OpenCLBufferManager.DisposeAll()
    runtime.DeviceQueueRegistry.Clear()


def test_context_reports_the_device(rt):
    say("runtime context")
    with rt.ComputeContext() as ctx:
        assert ctx.arch.startswith("gfx950")
        assert 0 <= ctx.Device < torch.cuda.device_count()
        assert ctx.warp_size == 64
        assert ctx.compute_units >= 200
        assert ctx.MAX_WORK_GROUP_SIZE == 1024
        # the reference's derivation (ComputeContext.cs:148-152): Y = warp / 8, X = MAX / Y
        assert (ctx.MAX_WORK_GPOUP_SIZE_X, ctx.MAX_WORK_GPOUP_SIZE_Y) == (128, 8)
        assert ctx.global_mem_bytes > (200 << 30)
    from my_pytchon_opencl_lib_amd import _native
    with pytest.raises(_native.MigemmArgumentError):
        rt.ComputeContext(device=999)


def test_pool_reuses_grows_and_replaces(rt):
    from my_pytchon_opencl_lib_amd import _native
    say("runtime pool")
    M = rt.OpenCLBufferManager
    with rt.ComputeContext() as ctx, rt.ComputeContext() as other:
        a = M.GetOrCreateBuffer(ctx, "t0", 4096)
        assert M.GetOrCreateBuffer(ctx, "t0", 4096).ptr == a.ptr          # same size: reused
        assert M.GetOrCreateBuffer(ctx, "t0", 100).ptr == a.ptr           # smaller: reused
        b = M.GetOrCreateBuffer(ctx, "t1", 4096)
        assert b.ptr != a.ptr
        assert M.Count() == (2, 8192)
        # the buffer holds data across lookups
        v = a.as_tensor((1024,))
        v.copy_(torch.arange(1024, dtype=torch.float32, device=v.device))
        assert np.array_equal(host(M.GetOrCreateBuffer(ctx, "t0", 4096).as_tensor((1024,))),
                              np.arange(1024, dtype=np.float32))
        # larger: freed and replaced by one of exactly the new size
        c = M.GetOrCreateBuffer(ctx, "t0", 1 << 20)
        assert M.Count() == (2, (1 << 20) + 4096)
        assert M.GetOrCreateBuffer(ctx, "t0", 1 << 20).ptr == c.ptr
        # another context: replaced (OpenCLBufferManager.cs:48-55)
        d = M.GetOrCreateBuffer(other, "t0", 1 << 20)
        assert M.GetOrCreateBuffer(other, "t0", 16).ptr == d.ptr
        assert M.Count()[0] == 2
        M.ReleaseBuffer("t1")
        assert M.Count() == (1, 1 << 20)
        M.ReleaseBuffer("t1")  # unknown: no error
        # destroying a context frees its buffers
        other.Dispose()
        assert M.Count() == (0, 0)
        with pytest.raises(_native.MigemmArgumentError, match="unknown context"):
            M.GetOrCreateBuffer(other, "t9", 16)
        M.GetOrCreateBuffer(ctx, "t2", 64)
        M.DisposeAll()
        assert M.Count() == (0, 0)


def test_queue_registry_is_per_thread(rt):
    from my_pytchon_opencl_lib_amd import _native
    say("runtime per-thread queues")
    with rt.ComputeContext() as ctx:
        queues = [ctx.CreateCommandQueue() for _ in range(3)]
        seen = {}
        errors = []
        barrier = threading.Barrier(4, timeout=60)

        def worker(i):
            try:
                rt.DeviceQueueRegistry.RegisterCurrent(queues[i])
                barrier.wait()  # every thread has registered before any reads
                c, s = ctypes.c_void_p(), ctypes.c_void_p()
                _native.call("migemm_queue_get_current", ctypes.byref(c), ctypes.byref(s))
                seen[i] = (s.value, rt.DeviceQueueRegistry.GetCurrent() is queues[i],
                           c.value == ctx.handle.value)
                # Tensor.DataBuffer in this thread's context
                t = rt.tensor_buffer(f"thread{i}", (16,))
                t.fill_(float(i))
                rt.DeviceQueueRegistry.Clear()
                try:
                    rt.DeviceQueueRegistry.GetCurrent()
                    errors.append(f"{i}: cleared queue still current")
                except _native.MigemmRuntimeError as e:
                    assert e.status == _native.MIGEMM_ERR_NO_QUEUE
            except Exception as e:  # noqa: BLE001
                errors.append(f"{i}: {e!r}")

        threads = [threading.Thread(target=worker, args=(i,)) for i in range(3)]
        for th in threads:
            th.start()
        barrier.wait()
        # the main thread registered nothing
        with pytest.raises(_native.MigemmRuntimeError, match="NO_QUEUE"):
            rt.DeviceQueueRegistry.GetCurrent()
        for th in threads:
            th.join()
        assert not errors, errors
        for i, q in enumerate(queues):
            assert seen[i] == (q.handle.value, True, True), (i, seen[i])
        torch.cuda.synchronize()
        for i in range(3):
            buf = rt.OpenCLBufferManager.GetOrCreateBuffer(ctx, f"thread{i}", 64)
            assert np.all(host(buf.as_tensor((16,))) == i)
        for q in queues:
            q.Dispose()


def _bmm(stream, a, b, c, batch, m, k, n, ta=0, tb=0):
    from my_pytchon_opencl_lib_amd import _native
    _native.call("migemm_bmm_permute_tiled", stream, ctypes.c_void_p(a), ctypes.c_void_p(b),
                 ctypes.c_void_p(c), m, k, n, m * k, k * n, m * n, ta, tb, batch)


def test_bmm_backward_on_pooled_buffers(rt):
    """NnClGlob.Bmm then BmmOp.Backward on pooled device buffers, the way the C# host runs
    them: inputs and outputs are pool buffers named by TensorID on the registered queue, and
    every output is read back through its name (Tensor.DataBuffer, Tensor.cs:41). M = K = N,
    so the three outputs have one size and a shared name never makes the pool replace (free)
    a buffer."""
    from my_pytchon_opencl_lib_amd import _native
    say("runtime Bmm -> BmmOp.Backward")
    rng = np.random.default_rng(5)
    B, M, K, N = 4, 48, 48, 48
    A = rng.integers(-3, 4, (B, M, K)).astype(np.float32)
    Bm = rng.integers(-3, 4, (B, K, N)).astype(np.float32)
    dC = rng.integers(-3, 4, (B, M, N)).astype(np.float32)
    exp_c = np.einsum("bmk,bkn->bmn", A.astype(np.int64), Bm.astype(np.int64)).astype(np.float32)
    exp_ga = np.einsum("bmn,bkn->bmk", dC.astype(np.int64), Bm.astype(np.int64)).astype(np.float32)
    exp_gb = np.einsum("bmk,bmn->bkn", A.astype(np.int64), dC.astype(np.int64)).astype(np.float32)

    def buf(name, shape):  # Tensor.DataBuffer
        p = ctypes.c_void_p()
        _native.call("migemm_tensor_buffer", name.encode(), 4 * int(np.prod(shape)),
                     ctypes.byref(p))
        return p.value

    def read(name, shape):
        return host(rt.tensor_buffer(name, shape))

    with rt.ComputeContext() as ctx:
        q = ctx.CreateCommandQueue()
        rt.DeviceQueueRegistry.RegisterCurrent(q)
        with torch.cuda.stream(q.torch_stream()):
            rt.tensor_buffer("a", (B, M, K)).copy_(torch.from_numpy(A))
            rt.tensor_buffer("b", (B, K, N)).copy_(torch.from_numpy(Bm))
            rt.tensor_buffer("grad_c", (B, M, N)).copy_(torch.from_numpy(dC))
        q.Finish()
        s = q.handle
        pa, pb, pg = buf("a", (B, M, K)), buf("b", (B, K, N)), buf("grad_c", (B, M, N))
        for shared in (True, False):
            # the reference names every Bmm output "bmm_c" (NnClGlob.cs:460)
            names = ("bmm_c",) * 3 if shared else ("bmm_c#1", "bmm_c#2", "bmm_c#3")
            pc = buf(names[0], (B, M, N))
            _bmm(s, pa, pb, pc, B, M, K, N)
            q.Finish()  # Bmm is synchronous (NnClGlob.cs:498)
            assert np.array_equal(read(names[0], (B, M, N)), exp_c)
            pga = buf(names[1], (B, M, K))
            _bmm(s, pg, pb, pga, B, M, N, K, 0, 1)   # gradA = dC B^T (BmmOp.cs:44-47)
            pgb = buf(names[2], (B, K, N))
            _bmm(s, pa, pg, pgb, B, K, M, N, 1, 0)   # gradB = A^T dC (BmmOp.cs:57-60)
            q.Finish()
            ga, gb = read(names[1], (B, M, K)), read(names[2], (B, K, N))
            assert np.array_equal(gb, exp_gb)
            if shared:
                # one buffer for all three: gradA was overwritten by gradB (BmmOp.cs:47,60)
                assert pga == pgb == pc
                assert np.array_equal(ga, exp_gb) and not np.array_equal(ga, exp_ga)
            else:
                assert len({pc, pga, pgb}) == 3
                assert np.array_equal(ga, exp_ga)
                assert np.array_equal(read(names[0], (B, M, N)), exp_c)
        rt.DeviceQueueRegistry.Clear()
        q.Dispose()


def test_c_caller_runtime_on_the_gpu():
    """The same runtime sequence from a plain C99 program with POSIX threads (no torch):
    tests/c_abi_check.c, mode runtime."""
    import c_abi
    say("c_abi_check runtime")
    r = c_abi.run("runtime")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c_abi_check runtime: ok" in r.stdout


def _fill_ints(t, seed, lo=-2, hi=2):
    g = torch.Generator(device=t.device)
    g.manual_seed(seed)
    t.copy_(torch.randint(lo, hi + 1, t.shape, device=t.device, generator=g).float())


def test_pool_release_never_waits_for_other_queues(rt, nncl):
    """Thread B queues ~30 ms of GEMMs on its queue over pooled operands; meanwhile thread A
    grows a buffer of its own (the pool replaces and frees the old one) and releases it. A
    returns while B's GEMMs are still running (the free is ordered after them on the device,
    not waited for on the host), B's buffer lookups run meanwhile, and B's product is exact.
    Then B's own operand is replaced while its GEMM still reads it, and the memory of the
    old operand is not handed out (and overwritten) before that GEMM has finished."""
    import time
    say("runtime pool: release without waiting")
    n = 8192
    M = rt.OpenCLBufferManager
    with rt.ComputeContext() as ctx:
        qa, qb = ctx.CreateCommandQueue(), ctx.CreateCommandQueue()
        sb = qb.torch_stream()
        bufs = {k: M.GetOrCreateBuffer(ctx, f"b_{k}", 4 * n * n) for k in "ABC"}
        with torch.cuda.stream(sb):
            _fill_ints(bufs["A"].as_tensor((n, n)), 1)
            _fill_ints(bufs["B"].as_tensor((n, n)), 2)
        qb.Finish()
        with torch.cuda.stream(sb):
            expect = torch.mm(bufs["A"].as_tensor((n, n)), bufs["B"].as_tensor((n, n)))
        qb.Finish()
        res, errors = {}, []
        queued = threading.Event()

        def thread_b():
            try:
                rt.DeviceQueueRegistry.RegisterCurrent(qb)
                with torch.cuda.stream(sb):
                    a, b, c = (bufs[k].as_tensor((n, n)) for k in "ABC")
                    for _ in range(4):
                        nncl.gemm(a, b, out=c)
                queued.set()
                t0 = time.perf_counter()
                for _ in range(200):
                    rt.tensor_buffer("b_C", (n, n))
                res["lookups_s"] = time.perf_counter() - t0
                res["b_busy_after_lookups"] = not sb.query()
                rt.DeviceQueueRegistry.Clear()
            except Exception as e:  # noqa: BLE001
                errors.append(repr(e))
                queued.set()

        def thread_a():
            try:
                rt.DeviceQueueRegistry.RegisterCurrent(qa)
                M.GetOrCreateBuffer(ctx, "a_grow", 1 << 20)
                queued.wait(60)
                t0 = time.perf_counter()
                M.GetOrCreateBuffer(ctx, "a_grow", 64 << 20)  # replaces (frees) the 1 MB one
                M.ReleaseBuffer("a_grow")
                res["grow_s"] = time.perf_counter() - t0
                res["b_busy_after_grow"] = not sb.query()
                rt.DeviceQueueRegistry.Clear()
            except Exception as e:  # noqa: BLE001
                errors.append(repr(e))

        ta, tb = threading.Thread(target=thread_a), threading.Thread(target=thread_b)
        tb.start()
        ta.start()
        ta.join()
        tb.join()
        assert not errors, errors
        say("grow", res["grow_s"], "lookups", res["lookups_s"])
        assert res["b_busy_after_grow"], "A's grow and release waited for B's GEMMs"
        assert res["grow_s"] < 0.01
        qb.Finish()
        assert torch.equal(bufs["C"].as_tensor((n, n)), expect)
        # B's operand replaced while its GEMM reads it; the old memory must outlive the GEMM
        rt.DeviceQueueRegistry.RegisterCurrent(qb)
        with torch.cuda.stream(sb):
            a, b, c = (bufs[k].as_tensor((n, n)) for k in "ABC")
            c.zero_()
            nncl.gemm(a, b, out=c)
            nncl.gemm(a, b, out=c)
        M.GetOrCreateBuffer(ctx, "b_A", 8 * n * n)  # a larger "b_A": the old one is released
        junk = M.GetOrCreateBuffer(ctx, "junk", 4 * n * n)
        with torch.cuda.stream(qa.torch_stream()):
            junk.as_tensor((n, n)).fill_(float("nan"))
        assert not sb.query(), "B's GEMMs finished before the replacement: test too short"
        qb.Finish()
        qa.Finish()
        assert torch.equal(bufs["C"].as_tensor((n, n)), expect)
        rt.DeviceQueueRegistry.Clear()
        del a, b, c, expect
        for q in (qa, qb):
            q.Dispose()


def test_destroyed_context_is_rejected_on_every_thread(rt):
    """A context destroyed on one thread is rejected on another whose current queue names it
    (its handle is an id that is never reused): buffer lookups, Tensor.DataBuffer and
    GetCurrent fail instead of using freed state, and a new context gets another handle."""
    from my_pytchon_opencl_lib_amd import _native
    say("runtime: destroyed context")
    ctx = rt.ComputeContext()
    q = ctx.CreateCommandQueue()
    stage, out = threading.Barrier(2, timeout=60), {}

    def other():
        try:
            rt.DeviceQueueRegistry.RegisterCurrent(q)
            out["before"] = rt.tensor_buffer("x", (4,)).numel()
            stage.wait()   # main destroys the context now
            stage.wait()
            p = ctypes.c_void_p()
            out["tensor_buffer"] = _native.load().migemm_tensor_buffer(b"x", 16, ctypes.byref(p))
            out["get_current"] = _native.load().migemm_queue_get_current(None, None)
            out["get_or_create"] = _native.load().migemm_buffer_get_or_create(
                ctx.handle, b"y", 16, ctypes.byref(p))
            rt.DeviceQueueRegistry.Clear()
        except Exception as e:  # noqa: BLE001
            out["error"] = repr(e)
            stage.abort()

    th = threading.Thread(target=other)
    th.start()
    stage.wait()
    old = ctx.handle.value
    ctx.Dispose()
    fresh = rt.ComputeContext()
    stage.wait()
    th.join()
    assert "error" not in out, out
    assert out["before"] == 4
    assert out["tensor_buffer"] == _native.MIGEMM_ERR_INVALID_ARG
    assert out["get_current"] == _native.MIGEMM_ERR_INVALID_ARG
    assert out["get_or_create"] == _native.MIGEMM_ERR_INVALID_ARG
    assert fresh.handle.value != old
    fresh.Dispose()
    q.Dispose()
