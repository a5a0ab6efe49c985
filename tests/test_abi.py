"""CPU checks of the drop-in boundary: libmigemm.so loads without a GPU, exports every
function include/migemm.h declares, and rejects bad arguments before touching HIP (the
reference's ArgumentException paths, csharp/cstorchcl/cstorchcl/compiler/NnClGlob.cs:443-452,
:1704-1714, and Tensor.cs:191-192 for non-positive dimensions)."""
import ctypes
import os
import re

import pytest

from my_pytchon_opencl_lib_amd import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "migemm.h")

INVALID = _native.MIGEMM_ERR_INVALID_ARG
ALIAS = _native.MIGEMM_ERR_ALIAS

# Fake, never dereferenced device addresses: validation must fail before any access.
P = [ctypes.c_void_p(0x100000 * (i + 1)) for i in range(6)]
NULL = None


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(migemm_\w+)\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    return _native.load()


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = header_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(names)


def _arg_count(params):
    params = " ".join(params.split())
    return 0 if params in ("", "void") else params.count(",") + 1


def test_pinvoke_block_binds_every_declared_function():
    """The C# P/Invoke block of the integration notes declares every function of
    include/migemm.h with the header's argument count, so a maintainer can paste it as the
    host's binding."""
    header = open(HEADER).read()
    decl = {m.group(1): _arg_count(m.group(2)) for m in
            re.finditer(r"^(?:int|const char \*)\s*(migemm_\w+)\(([^)]*)\);", header, re.M)}
    doc = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    bound = {m.group(1): _arg_count(m.group(2)) for m in
             re.finditer(r"static extern \w+\s+(migemm_\w+)\(([^)]*)\);", doc)}
    assert set(decl) == set(header_functions())
    assert bound == decl


def test_version_and_empty_last_error(lib):
    assert lib.migemm_version().decode() == "0.1.0"
    assert isinstance(lib.migemm_last_error(), bytes)


def expect(status, code, fragment):
    assert status == code, (status, _native.last_error())
    assert fragment in _native.last_error()


@pytest.mark.parametrize("M,N,K,batch", [(0, 4, 4, 1), (4, 0, 4, 1), (4, 4, 0, 1),
                                         (4, 4, 4, 0), (-1, 4, 4, 1)])
def test_gemm_rejects_non_positive_sizes(lib, M, N, K, batch):
    st = lib.migemm_gemm_strided_batched(NULL, 0, 0, M, N, K, P[0], max(K, 1), 0, P[1],
                                         max(N, 1), 0, NULL, P[2], max(N, 1), 0, batch)
    expect(st, INVALID, "sizes must be >= 1")


def test_gemm_rejects_null_pointers_and_flags(lib):
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, NULL, 4, 0, P[1], 4, 0, NULL,
                                           P[2], 4, 0, 1), INVALID, "non-null")
    expect(lib.migemm_gemm_strided_batched(NULL, 2, 0, 4, 4, 4, P[0], 4, 0, P[1], 4, 0, NULL,
                                           P[2], 4, 0, 1), INVALID, "transA")


def test_gemm_rejects_bad_leading_dims_and_strides(lib):
    # A not transposed needs lda >= K
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 8, P[0], 7, 0, P[1], 4, 0, NULL,
                                           P[2], 4, 0, 1), INVALID, "lda")
    # A transposed is stored [K, M]: lda >= M
    expect(lib.migemm_gemm_strided_batched(NULL, 1, 0, 9, 4, 8, P[0], 8, 0, P[1], 4, 0, NULL,
                                           P[2], 4, 0, 1), INVALID, "lda")
    # B transposed is stored [N, K]: ldb >= K
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 1, 4, 4, 8, P[0], 8, 0, P[1], 4, 0, NULL,
                                           P[2], 4, 0, 1), INVALID, "ldb")
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 0, 4, 6, 4, P[0], 4, 0, P[1], 6, 0, NULL,
                                           P[2], 5, 0, 1), INVALID, "ldc")
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, P[0], 4, -1, P[1], 4, 0, NULL,
                                           P[2], 4, 16, 2), INVALID, "strides")
    # two batch entries writing the same C elements
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, P[0], 4, 16, P[1], 4, 16, NULL,
                                           P[2], 4, 8, 2), INVALID, "overlap")


def test_gemm_rejects_aliased_output(lib):
    a = 0x200000
    c = ctypes.c_void_p(a + 8)  # overlaps A's 16 floats
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, ctypes.c_void_p(a), 4, 0, P[1],
                                           4, 0, NULL, c, 4, 0, 1), ALIAS, "overlaps")


def test_gemm_rejects_overflowing_extent(lib):
    expect(lib.migemm_gemm_strided_batched(NULL, 0, 0, 2**30, 4, 4, P[0], 2**40, 0, P[1], 4, 0,
                                           NULL, P[2], 4, 0, 1), INVALID, "overflow")


def test_reference_shaped_entry_points_validate(lib):
    expect(lib.migemm_bmm_tiled(NULL, P[0], P[1], P[2], 4, 4, 4, -16, 16, 16, 2), INVALID,
           "strides")
    expect(lib.migemm_bmm_tiled(NULL, P[0], P[1], P[2], 4, 0, 4, 16, 16, 16, 1), INVALID,
           "sizes")
    expect(lib.migemm_matmul_tiled(NULL, P[0], P[1], NULL, 4, 4, 4), INVALID, "non-null")
    expect(lib.migemm_bmm_permute_tiled(NULL, P[0], P[1], P[2], 0, 4, 4, 0, 0, 0, 1, 0, 1),
           INVALID, "sizes")
    expect(lib.migemm_linear_forward(NULL, P[0], P[1], NULL, P[3], 4, 4, 4, 16, 16, 1), INVALID,
           "bias")
    expect(lib.migemm_lstm_gemm_xw(NULL, P[0], P[1], NULL, P[3], 4, 4, 4), INVALID, "bias")
    expect(lib.migemm_linear_weight_grad(NULL, P[0], P[1], P[2], 0, 4, 4, 1), INVALID, "sizes")
    expect(lib.migemm_linear_bias_backward(NULL, P[0], P[1], 0, 4), INVALID, "sizes")
    expect(lib.migemm_reduce_sum_axis(NULL, P[0], P[1], 1, 0, 4), INVALID, "sizes")


def test_permute_validates_axes_and_dims(lib):
    dims = (ctypes.c_int * 3)(2, 3, 4)
    bad = (ctypes.c_int * 3)(0, 2, 2)
    expect(lib.migemm_tensor_permute(NULL, P[0], P[1], dims, bad, 3), INVALID, "permutation")
    good = (ctypes.c_int * 3)(0, 2, 1)
    expect(lib.migemm_tensor_permute(NULL, P[0], P[1], dims, good, 11), INVALID, "num_dims")
    zero = (ctypes.c_int * 3)(2, 0, 4)
    expect(lib.migemm_tensor_permute(NULL, P[0], P[1], zero, good, 3), INVALID, "dim 1")
    expect(lib.migemm_tensor_permute(NULL, P[0], ctypes.c_void_p(0x100000 + 4), dims, good, 3),
           ALIAS, "overlaps")


def test_services_validate_without_device(lib):
    expect(lib.migemm_malloc(None, 16), INVALID, "null")
    expect(lib.migemm_set_device(-1), INVALID, "device")
    expect(lib.migemm_memcpy_h2d(NULL, NULL, P[0], 4), INVALID, "null")
    assert lib.migemm_free(None) == 0


def test_gemm_policy_set_and_rejected(lib):
    prev = ctypes.c_int(-7)
    assert lib.migemm_set_gemm_policy(2, ctypes.byref(prev)) == 0
    assert prev.value == 0
    assert lib.migemm_set_gemm_policy(0, ctypes.byref(prev)) == 0
    assert prev.value == 2
    expect(lib.migemm_set_gemm_policy(6, None), INVALID, "policy")
    expect(lib.migemm_set_gemm_policy(-1, None), INVALID, "policy")
    assert lib.migemm_set_gemm_policy(0, None) == 0


def test_python_wrapper_maps_status_to_exceptions():
    with pytest.raises(_native.MigemmArgumentError):
        _native.call("migemm_bmm_tiled", NULL, P[0], P[1], P[2], 4, 0, 4, 16, 16, 16, 1)
    with pytest.raises(ValueError):
        _native.check(_native.MIGEMM_ERR_ALIAS)
    with pytest.raises(RuntimeError):
        _native.check(_native.MIGEMM_ERR_HIP)


def test_host_api_rejects_cpu_tensors_loudly():
    import torch
    from my_pytchon_opencl_lib_amd import NnClGlob, ShapeError
    g = NnClGlob("cuda:0")
    a = torch.zeros(2, 3, 4)
    b = torch.zeros(2, 4, 5)
    with pytest.raises(ShapeError, match="no CPU fallback"):
        g.Bmm(a, b)
    with pytest.raises(AssertionError):  # the Python reference asserts
        g.bmm(a, b)


def test_c_caller_compiles_and_validates_without_gpu():
    """include/migemm.h compiles as strict C99 and a C program linked against libmigemm.so
    gets the argument errors, with messages, without a GPU (tests/c_abi_check.c)."""
    import c_abi
    r = c_abi.run("validate")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "c_abi_check validate: ok" in r.stdout


def test_runtime_services_validate_without_gpu(lib):
    """The runtime objects' argument checks (the reference's ArgumentNullException /
    ArgumentException / InvalidOperationException paths, OpenCLBufferManager.cs:24-26,
    DeviceQueueRegistry.cs:21,30-36) run before any HIP call."""
    import threading
    NO_QUEUE = _native.MIGEMM_ERR_NO_QUEUE
    out = ctypes.c_void_p()
    expect(lib.migemm_buffer_get_or_create(NULL, b"x", 16, ctypes.byref(out)), INVALID,
           "null context")
    expect(lib.migemm_buffer_get_or_create(P[0], b"", 16, ctypes.byref(out)), INVALID,
           "empty buffer name")
    expect(lib.migemm_buffer_get_or_create(P[0], b"x", 0, ctypes.byref(out)), INVALID,
           "size must be > 0")
    expect(lib.migemm_buffer_get_or_create(P[0], b"x", 16, ctypes.byref(out)), INVALID,
           "unknown context")
    expect(lib.migemm_queue_register_current(P[0], NULL), INVALID, "must not be null")
    expect(lib.migemm_queue_register_current(P[0], P[1]), INVALID, "unknown context")
    expect(lib.migemm_context_create(-2, ctypes.byref(out)), INVALID, "device -2")
    expect(lib.migemm_context_info(P[0], None, None, 0, None, None, None, None, None, None),
           INVALID, "unknown context")

    results = {}

    def fresh_thread():  # a thread that registered nothing
        results["get"] = lib.migemm_queue_get_current(None, None)
        results["get_msg"] = _native.last_error()
        results["buf"] = lib.migemm_tensor_buffer(b"t0", 64, ctypes.byref(ctypes.c_void_p()))
    def other_thread():  # handles that are not live contexts fail on any thread
        results["other"] = lib.migemm_buffer_get_or_create(P[0], b"x", 16,
                                                           ctypes.byref(ctypes.c_void_p()))
        results["other_msg"] = _native.last_error()
        results["other_reg"] = lib.migemm_queue_register_current(ctypes.c_void_p(1), P[1])
    th = threading.Thread(target=fresh_thread)
    th.start()
    th.join()
    th = threading.Thread(target=other_thread)
    th.start()
    th.join()
    assert results["get"] == NO_QUEUE and "no queue is registered" in results["get_msg"]
    assert results["buf"] == NO_QUEUE
    assert results["other"] == INVALID and "unknown context" in results["other_msg"]
    assert results["other_reg"] == INVALID
    assert lib.migemm_queue_clear_current() == 0
    n, b = ctypes.c_size_t(9), ctypes.c_size_t(9)
    assert lib.migemm_buffer_count(ctypes.byref(n), ctypes.byref(b)) == 0 and n.value == 0
    assert lib.migemm_buffer_release(b"never-created") == 0


def test_runtime_mirror_maps_no_queue_to_runtime_error():
    from my_pytchon_opencl_lib_amd import runtime
    import threading
    err = {}

    def t():
        try:
            runtime.DeviceQueueRegistry.GetCurrent()
        except Exception as e:  # noqa: BLE001
            err["e"] = e
    th = threading.Thread(target=t)
    th.start()
    th.join()
    assert isinstance(err["e"], _native.MigemmRuntimeError)
    assert err["e"].status == _native.MIGEMM_ERR_NO_QUEUE
    with pytest.raises(_native.MigemmArgumentError):
        runtime.ComputeContext(preferAccelerator=False)


def test_lstm_recurrent_gates_rejects_bad_arguments(lib):
    f = lib.migemm_lstm_recurrent_gates
    expect(f(NULL, NULL, P[1], P[2], 2, 3, 4, 1), INVALID, "null pointer")
    expect(f(NULL, P[0], P[1], P[2], 0, 3, 4, 1), INVALID, "sizes must be >= 1")
    expect(f(NULL, P[0], P[1], P[2], 2, 3, 4, 3), INVALID, "step 3 not in [0, 3)")
    expect(f(NULL, P[0], P[1], P[2], 2, 3, 4, -1), INVALID, "step -1")
    assert f(NULL, P[0], P[1], P[2], 2, 3, 4, 0) == 0  # step 0: no work, no HIP call
