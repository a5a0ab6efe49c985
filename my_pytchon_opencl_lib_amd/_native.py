"""ctypes binding of libmigemm.so, the HIP/gfx950 C ABI declared in include/migemm.h.

The shared library is built in-tree by build_native.py. There is no fallback: if the
library is missing or cannot be loaded, every operator raises, so a silent CPU or
PyTorch path can never stand in for the HIP kernels.
"""
import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmigemm.so")

MIGEMM_OK = 0
MIGEMM_ERR_INVALID_ARG = 1
MIGEMM_ERR_ALIAS = 2
MIGEMM_ERR_HIP = 3
MIGEMM_ERR_NO_DEVICE = 4
MIGEMM_ERR_WORKSPACE = 5
MIGEMM_ERR_UNSUPPORTED = 6
MIGEMM_ERR_NO_QUEUE = 7

MIGEMM_GEMM_ACCUMULATE = 1  # migemm_gemm_strided_batched_ex flag: C += result

# Kernel-family policies (migemm_set_gemm_policy)
MIGEMM_POLICY_AUTO = 0
MIGEMM_POLICY_TILED = 1
MIGEMM_POLICY_SMALL = 2
MIGEMM_POLICY_SKINNY = 3
MIGEMM_POLICY_PANEL = 4
MIGEMM_POLICY_TINY = 5

# Tuning keys (migemm_set_tuning); 0 = the dispatcher's choice
MIGEMM_TUNE_TILE = 1
MIGEMM_TUNE_SPLITK = 2
MIGEMM_TUNE_DIRECT = 3
MIGEMM_TUNE_SMALL_TILES = 4
MIGEMM_TUNE_SMALL_SPLITK = 5
MIGEMM_TILE_128x256 = 128256
TUNE_KEYS = {"tile": MIGEMM_TUNE_TILE, "splitk": MIGEMM_TUNE_SPLITK,
             "direct": MIGEMM_TUNE_DIRECT, "small_tiles": MIGEMM_TUNE_SMALL_TILES,
             "small_splitk": MIGEMM_TUNE_SMALL_SPLITK}

STATUS_NAMES = {
    MIGEMM_OK: "MIGEMM_OK",
    MIGEMM_ERR_INVALID_ARG: "MIGEMM_ERR_INVALID_ARG",
    MIGEMM_ERR_ALIAS: "MIGEMM_ERR_ALIAS",
    MIGEMM_ERR_HIP: "MIGEMM_ERR_HIP",
    MIGEMM_ERR_NO_DEVICE: "MIGEMM_ERR_NO_DEVICE",
    MIGEMM_ERR_WORKSPACE: "MIGEMM_ERR_WORKSPACE",
    MIGEMM_ERR_UNSUPPORTED: "MIGEMM_ERR_UNSUPPORTED",
    MIGEMM_ERR_NO_QUEUE: "MIGEMM_ERR_NO_QUEUE",
}


class MigemmArgumentError(ValueError):
    """Argument / shape error (the reference throws ArgumentException,
    csharp/cstorchcl/cstorchcl/compiler/NnClGlob.cs:443-452)."""

    def __init__(self, status, message):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


class MigemmRuntimeError(RuntimeError):
    """Device / runtime error (the reference throws InvalidOperationException,
    csharp/cstorchcl/cstorchcl/compiler/JITProgramCache.cs:40-43)."""

    def __init__(self, status, message):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


# Every exported symbol with its C signature (argument types, return type). The CPU test
# suite checks this table against include/migemm.h.
_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_sz = ctypes.c_size_t
_ip = ctypes.POINTER(ctypes.c_int)
SIGNATURES = {
    "migemm_gemm_strided_batched": ([_vp, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _vp,
                                     _i64, _i64, _vp, _vp, _i64, _i64, _i32], _i32),
    "migemm_gemm_strided_batched_ex": ([_vp, _i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64,
                                        _vp, _i64, _i64, _vp, _vp, _i64, _i64, _i32, _i32],
                                       _i32),
    "migemm_gemm_strided_batched_noalloc": ([_vp, _i32, _i32, _i32, _i32, _i32, _vp, _i64,
                                             _i64, _vp, _i64, _i64, _vp, _vp, _i64, _i64,
                                             _i32, _i32], _i32),
    "migemm_matmul_tiled": ([_vp, _vp, _vp, _vp, _i32, _i32, _i32], _i32),
    "migemm_bmm_tiled": ([_vp, _vp, _vp, _vp] + [_i32] * 7, _i32),
    "migemm_bmm_permute_tiled": ([_vp, _vp, _vp, _vp] + [_i32] * 9, _i32),
    "migemm_linear_forward": ([_vp, _vp, _vp, _vp, _vp] + [_i32] * 6, _i32),
    "migemm_lstm_gemm_xw": ([_vp, _vp, _vp, _vp, _vp, _i32, _i32, _i32], _i32),
    "migemm_lstm_gemm_grad_x": ([_vp, _vp, _vp, _vp, _i32, _i32, _i32], _i32),
    "migemm_lstm_gemm_grad_weights": ([_vp] * 7 + [_i32] * 4, _i32),
    "migemm_lstm_recurrent_gates": ([_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32], _i32),
    "migemm_lstm_hid_gates": ([_vp] * 8 + [_i32] * 5, _i32),
    "migemm_tensor_permute": ([_vp, _vp, _vp, _ip, _ip, _i32], _i32),
    "migemm_linear_bias_backward": ([_vp, _vp, _vp, _i32, _i32], _i32),
    "migemm_reduce_sum_axis": ([_vp, _vp, _vp, _i32, _i32, _i32], _i32),
    "migemm_linear_weight_grad": ([_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32], _i32),
    "migemm_device_count": ([_ip], _i32),
    "migemm_set_device": ([_i32], _i32),
    "migemm_device_info": ([_i32, ctypes.c_char_p, _sz, _ip, ctypes.POINTER(_sz)], _i32),
    "migemm_malloc": ([ctypes.POINTER(_vp), _sz], _i32),
    "migemm_free": ([_vp], _i32),
    "migemm_memcpy_h2d": ([_vp, _vp, _vp, _sz], _i32),
    "migemm_memcpy_d2h": ([_vp, _vp, _vp, _sz], _i32),
    "migemm_memset": ([_vp, _vp, _i32, _sz], _i32),
    "migemm_stream_create": ([ctypes.POINTER(_vp)], _i32),
    "migemm_stream_destroy": ([_vp], _i32),
    "migemm_stream_synchronize": ([_vp], _i32),
    "migemm_workspace_reserve": ([_vp, _sz], _i32),
    "migemm_workspace_release": ([_vp], _i32),
    "migemm_workspace_size": ([_vp, ctypes.POINTER(_sz)], _i32),
    "migemm_last_error": ([], ctypes.c_char_p),
    "migemm_version": ([], ctypes.c_char_p),
    "migemm_context_create": ([_i32, ctypes.POINTER(_vp)], _i32),
    "migemm_context_destroy": ([_vp], _i32),
    "migemm_context_info": ([_vp, _ip, ctypes.c_char_p, _sz, _ip, _ip, _ip, _ip, _ip,
                             ctypes.POINTER(_sz)], _i32),
    "migemm_buffer_get_or_create": ([_vp, ctypes.c_char_p, _sz, ctypes.POINTER(_vp)], _i32),
    "migemm_buffer_release": ([ctypes.c_char_p], _i32),
    "migemm_buffer_release_all": ([], _i32),
    "migemm_buffer_count": ([ctypes.POINTER(_sz), ctypes.POINTER(_sz)], _i32),
    "migemm_queue_register_current": ([_vp, _vp], _i32),
    "migemm_queue_get_current": ([ctypes.POINTER(_vp), ctypes.POINTER(_vp)], _i32),
    "migemm_queue_clear_current": ([], _i32),
    "migemm_tensor_buffer": ([ctypes.c_char_p, _sz, ctypes.POINTER(_vp)], _i32),
    "migemm_set_gemm_policy": ([_i32, _ip], _i32),
    "migemm_set_tuning": ([_i32, _i32, _ip], _i32),
    "migemm_last_plan": ([ctypes.c_char_p, _sz], _i32),
    "migemm_stream_read": ([_vp, _vp, _sz, _vp, _i32], _i32),
    "migemm_gemm_plan": ([_i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _vp, _i64, _i64, _vp,
                          _vp, _i64, _i64, _i32, _i32, ctypes.c_char_p, _sz], _i32),
}

_lib = None
_lock = threading.Lock()


def load():
    """Load libmigemm.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"libmigemm.so not found at {LIB_PATH}: build it first "
                    "(python -c 'import __graft_entry__ as g; g.build()' or "
                    "python my_pytchon_opencl_lib_amd/build_native.py)")
            # torch ships its own libamdhip64.so.7 (same soname as /opt/rocm's). Loading
            # torch first makes the dynamic linker bind libmigemm.so to that runtime, so the
            # process holds one HIP runtime and tensors from torch are valid here. Loaded
            # first, libmigemm.so would pull in /opt/rocm's copy and torch would then load a
            # second runtime beside it.
            import torch  # noqa: F401
            L = ctypes.CDLL(LIB_PATH)
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = res
            _lib = L
    return _lib


def last_error():
    return load().migemm_last_error().decode(errors="replace")


def check(status):
    """Raise the exception type that matches a migemm status code."""
    if status == MIGEMM_OK:
        return
    msg = last_error()
    if status in (MIGEMM_ERR_INVALID_ARG, MIGEMM_ERR_ALIAS, MIGEMM_ERR_UNSUPPORTED):
        raise MigemmArgumentError(status, msg)
    raise MigemmRuntimeError(status, msg)


def call(name, *args):
    """Call an exported function and raise on a non-zero status."""
    check(getattr(load(), name)(*args))


def set_gemm_policy(policy):
    """Select the kernel family for later GEMM calls; returns the previous policy."""
    prev = ctypes.c_int(0)
    call("migemm_set_gemm_policy", int(policy), ctypes.byref(prev))
    return prev.value


def set_tuning(key, value):
    """Set one dispatcher tuning override (a TUNE_KEYS name or MIGEMM_TUNE_* value; 0 = the
    dispatcher's choice); returns the previous value."""
    prev = ctypes.c_int(0)
    call("migemm_set_tuning", TUNE_KEYS.get(key, key), int(value), ctypes.byref(prev))
    return prev.value


class tuned:
    """Context manager: tuning overrides for a block (tile=, splitk=, direct=, small_tiles=,
    small_splitk=), the previous values restored on exit."""

    def __init__(self, **overrides):
        self.overrides = overrides
        self.saved = {}

    def __enter__(self):
        for k, v in self.overrides.items():
            self.saved[k] = set_tuning(k, 0 if v is None else v)
        return self

    def __exit__(self, *exc):
        for k, v in self.saved.items():
            set_tuning(k, v)
        return False


def last_plan():
    """What the last GEMM / permute / column-sum call of this thread ran."""
    buf = ctypes.create_string_buffer(256)
    call("migemm_last_plan", buf, len(buf))
    return buf.value.decode()


def gemm_plan(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, bias, C, ldc, strideC,
              batch=1, flags=0):
    """The plan string migemm_gemm_strided_batched_ex would run for these arguments, without
    running it (no GPU needed). A, B, bias and C are integer addresses (None for no bias)."""
    buf = ctypes.create_string_buffer(256)
    call("migemm_gemm_plan", int(transA), int(transB), M, N, K, A, lda, strideA, B, ldb,
         strideB, bias, C, ldc, strideC, batch, flags, buf, len(buf))
    return buf.value.decode()
