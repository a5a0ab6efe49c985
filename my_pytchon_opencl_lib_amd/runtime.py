"""The reference host's runtime objects on HIP, over the C ABI's runtime services.

Mirrors ("cs/" = csharp/cstorchcl/cstorchcl/):
  ComputeContext(preferAccelerator)       cs/core/ComputeContext.cs:11-171
  DeviceQueueRegistry                     cs/core/DeviceQueueRegistry.cs:10-47
                                          (and the Python core/queue_registry.py:3-20)
  OpenCLBufferManager                     cs/compiler/OpenCLBufferManager.cs:11-92
  Tensor.DataBuffer                       cs/core/Tensor.cs:41   -> tensor_buffer()

A queue is a HIP stream created by the library (migemm_stream_create); a buffer is HIP device
memory owned by the library's name-keyed pool. Buffers can be viewed as torch tensors
(DeviceBuffer.as_tensor) and queues used as torch streams (CommandQueue.torch_stream), so the
GEMM operators can run on pooled memory; the compute entry points take the raw pointers.
As in the reference, a pooled buffer that is replaced (a larger request under the same name)
or released is freed: views of it must not be used afterwards.
"""
import ctypes
import threading

from . import _native


class ComputeContext:
    """A device context (cs/core/ComputeContext.cs:35-159). preferAccelerator=False asks the
    reference for the CPU device (:85-89); the HIP path has none, so it is rejected."""

    def __init__(self, preferAccelerator=True, device=-1):
        if not preferAccelerator:
            raise _native.MigemmArgumentError(
                _native.MIGEMM_ERR_UNSUPPORTED, "the HIP matmul path has no CPU device")
        h = ctypes.c_void_p()
        _native.call("migemm_context_create", int(device), ctypes.byref(h))
        self.handle = h
        dev, cu, wave, mwg, wx, wy = (ctypes.c_int() for _ in range(6))
        mem = ctypes.c_size_t()
        arch = ctypes.create_string_buffer(64)
        _native.call("migemm_context_info", h, ctypes.byref(dev), arch, len(arch),
                     ctypes.byref(cu), ctypes.byref(wave), ctypes.byref(mwg), ctypes.byref(wx),
                     ctypes.byref(wy), ctypes.byref(mem))
        self.Device = dev.value
        self.arch = arch.value.decode()
        self.compute_units = cu.value
        self.warp_size = wave.value
        self.MAX_WORK_GROUP_SIZE = mwg.value
        # the reference's property names, spelling included (ComputeContext.cs:24-25)
        self.MAX_WORK_GPOUP_SIZE_X = wx.value
        self.MAX_WORK_GPOUP_SIZE_Y = wy.value
        self.global_mem_bytes = mem.value
        self._disposed = False

    def CreateCommandQueue(self):
        return CommandQueue(self)

    def Dispose(self):
        """ComputeContext.Dispose (:161-170); frees the context's pooled buffers."""
        if not self._disposed:
            _native.call("migemm_context_destroy", self.handle)
            self._disposed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.Dispose()
        return False


class CommandQueue:
    """An in-order queue of a context: a HIP stream owned by the library."""

    def __init__(self, context):
        self.Context = context
        s = ctypes.c_void_p()
        _native.call("migemm_stream_create", ctypes.byref(s))
        self.handle = s

    def Finish(self):
        _native.call("migemm_stream_synchronize", self.handle)

    def torch_stream(self):
        """The queue as a torch stream, to run the NnClGlob operators on it."""
        import torch
        return torch.cuda.ExternalStream(self.handle.value,
                                         device=torch.device("cuda", self.Context.Device))

    def Dispose(self):
        if self.handle is not None:
            _native.call("migemm_stream_destroy", self.handle)
            self.handle = None


class DeviceQueueRegistry:
    """The calling thread's current queue (cs/core/DeviceQueueRegistry.cs:14-46): the
    library keeps the (context, stream) pair per host thread, this class the Python queue
    object that goes with it."""

    _local = threading.local()

    @classmethod
    def RegisterCurrent(cls, queue):
        if queue is None:
            raise _native.MigemmArgumentError(_native.MIGEMM_ERR_INVALID_ARG,
                                              "the command queue must not be None")
        _native.call("migemm_queue_register_current", queue.Context.handle, queue.handle)
        cls._local.queue = queue

    @classmethod
    def GetCurrent(cls):
        """Raises MigemmRuntimeError (MIGEMM_ERR_NO_QUEUE) when this thread has none."""
        _native.call("migemm_queue_get_current", None, None)
        return cls._local.queue

    @classmethod
    def Clear(cls):
        _native.call("migemm_queue_clear_current")
        cls._local.queue = None

    # the Python reference's names (core/queue_registry.py:10-20)
    set_current = RegisterCurrent
    get_current = GetCurrent


class DeviceBuffer:
    """A pooled device buffer: its pointer and size."""

    def __init__(self, name, ptr, nbytes, device):
        self.name = name
        self.ptr = ptr
        self.nbytes = nbytes
        self.device = device

    def as_tensor(self, shape):
        """A float32 torch view of the buffer's first prod(shape) elements."""
        import torch
        n = 1
        for s in shape:
            n *= int(s)
        if 4 * n > self.nbytes:
            raise _native.MigemmArgumentError(
                _native.MIGEMM_ERR_INVALID_ARG,
                f"shape {list(shape)} needs {4 * n} bytes, buffer {self.name!r} holds "
                f"{self.nbytes}")
        view = _CudaArray(self.ptr, tuple(int(s) for s in shape))
        return torch.as_tensor(view, device=torch.device("cuda", self.device))


class _CudaArray:
    def __init__(self, ptr, shape):
        self.__cuda_array_interface__ = {"shape": shape, "typestr": "<f4",
                                         "data": (int(ptr), False), "version": 2,
                                         "strides": None}


class OpenCLBufferManager:
    """The name-keyed device-buffer pool (cs/compiler/OpenCLBufferManager.cs:11-92)."""

    @staticmethod
    def GetOrCreateBuffer(context, bufName, bufSize):
        if context is None:
            raise _native.MigemmArgumentError(_native.MIGEMM_ERR_INVALID_ARG,
                                              "context must not be None")
        p = ctypes.c_void_p()
        _native.call("migemm_buffer_get_or_create", context.handle,
                     str(bufName).encode(), int(bufSize), ctypes.byref(p))
        return DeviceBuffer(bufName, p.value, int(bufSize), context.Device)

    @staticmethod
    def ReleaseBuffer(bufName):
        _native.call("migemm_buffer_release", str(bufName).encode())

    @staticmethod
    def DisposeAll():
        _native.call("migemm_buffer_release_all")

    @staticmethod
    def Count():
        """(number of pooled buffers, their total bytes)."""
        n, b = ctypes.c_size_t(), ctypes.c_size_t()
        _native.call("migemm_buffer_count", ctypes.byref(n), ctypes.byref(b))
        return n.value, b.value


def tensor_buffer(tensor_id, shape):
    """Tensor.DataBuffer (cs/core/Tensor.cs:41): the pooled buffer named tensor_id in the
    current queue's context, sized 4 * prod(shape) bytes, as a torch view of that shape."""
    n = 1
    for s in shape:
        n *= int(s)
    p = ctypes.c_void_p()
    _native.call("migemm_tensor_buffer", str(tensor_id).encode(), 4 * n, ctypes.byref(p))
    q = DeviceQueueRegistry.GetCurrent()
    return DeviceBuffer(tensor_id, p.value, 4 * n, q.Context.Device).as_tensor(shape)
