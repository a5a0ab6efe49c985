// Runtime services of the reference's C# host, on HIP: the device context, the name-keyed
// device-buffer pool and the per-thread current queue ("cs/" = csharp/cstorchcl/cstorchcl/).
//
//   reference                                            here
//   new ComputeContext(preferAccelerator)                migemm_context_create
//     cs/core/ComputeContext.cs:35-159
//   ComputeContext.Dispose  cs/core/ComputeContext.cs:161-170
//                                                        migemm_context_destroy
//   OpenCLBufferManager.GetOrCreateBuffer                migemm_buffer_get_or_create
//     cs/compiler/OpenCLBufferManager.cs:22-61
//   OpenCLBufferManager.ReleaseBuffer / DisposeAll       migemm_buffer_release / _release_all
//     cs/compiler/OpenCLBufferManager.cs:66-91
//   DeviceQueueRegistry.RegisterCurrent / GetCurrent / Clear
//     cs/core/DeviceQueueRegistry.cs:14-46              migemm_queue_register_current / ...
//   Tensor.DataBuffer  cs/core/Tensor.cs:41             migemm_tensor_buffer
//
// A buffer is plain HIP device memory (hipMalloc) on the context's device; its pointer is
// what the compute entry points take. The pool follows the reference's rule: a name maps to
// one buffer, which is returned when it belongs to the same context and is at least as large
// as requested, and is otherwise freed and replaced by one of exactly the requested size. An
// OpenCL buffer released while kernels still use it stays alive until they finish; a HIP
// buffer does not, so a replaced or released buffer is freed only after its device has
// finished the work queued so far.
#include <string.h>

#include <mutex>
#include <set>
#include <string>
#include <unordered_map>

#include "migemm_internal.h"

namespace migemm {
namespace {

struct Context {
    int device;
    int compute_units;
    int wavefront_size;
    int max_work_group_size;
    int wg_x, wg_y;
    size_t global_mem;
    char arch[64];
};

struct PoolEntry {
    size_t bytes;
    void *ptr;
    Context *ctx;
};

std::mutex g_rt_mutex;                              // guards the three tables below
std::set<Context *> g_contexts;                     // live contexts (handles are validated)
std::unordered_map<std::string, PoolEntry> g_pool;  // buffer name -> buffer

thread_local Context *t_queue_ctx = nullptr;  // DeviceQueueRegistry._currentQueue
thread_local void *t_queue_stream = nullptr;
thread_local bool t_queue_set = false;

// Makes `device` current for the scope and restores the caller's device after it.
struct DeviceScope {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceScope(int device) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != device) err = hipSetDevice(device);
    }
    ~DeviceScope() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Frees a pooled buffer once its device has finished the work queued so far (kernels may
// still read or write it, as an OpenCL buffer outlives its release until they finish).
int free_entry(const PoolEntry &e) {
    DeviceScope scope(e.ctx->device);
    MIGEMM_HIP(scope.err);
    MIGEMM_HIP(hipDeviceSynchronize());
    MIGEMM_HIP(hipFree(e.ptr));
    return MIGEMM_OK;
}

// Work-group limits as the reference derives them from the warp size
// (cs/core/ComputeContext.cs:108-156).
void work_group_limits(Context *c) {
    const int w = c->wavefront_size, m = c->max_work_group_size;
    if (m < w) {
        if (m < 4) {
            c->wg_x = c->wg_y = 1;
        } else if (m < 16) {
            c->wg_x = c->wg_y = 2;
        } else if (m < 32) {
            c->wg_x = c->wg_y = 4;
        } else {
            c->wg_x = 8;
            c->wg_y = 4;
        }
    } else {
        c->wg_y = w / 8;
        c->wg_x = m / c->wg_y;
    }
}

int get_or_create_locked(Context *ctx, const char *name, size_t bytes, void **ptr) {
    auto it = g_pool.find(name);
    if (it != g_pool.end()) {
        if (it->second.ctx == ctx && it->second.bytes >= bytes) {
            *ptr = it->second.ptr;
            return MIGEMM_OK;
        }
        // too small, or from another context: free it (OpenCLBufferManager.cs:53-55)
        const PoolEntry old = it->second;
        g_pool.erase(it);
        int rc = free_entry(old);
        if (rc != MIGEMM_OK) return rc;
    }
    DeviceScope scope(ctx->device);
    MIGEMM_HIP(scope.err);
    void *p = nullptr;
    MIGEMM_HIP(hipMalloc(&p, bytes));
    g_pool.emplace(name, PoolEntry{bytes, p, ctx});
    *ptr = p;
    return MIGEMM_OK;
}

bool live(Context *c) { return c != nullptr && g_contexts.count(c) != 0; }

}  // namespace
}  // namespace migemm

using namespace migemm;

extern "C" {

int migemm_context_create(int device, void **ctx) {
    clear_error();
    if (ctx == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "context_create: null pointer");
    *ctx = nullptr;
    if (device < -1)
        return set_error(MIGEMM_ERR_INVALID_ARG, "context_create: device %d < -1", device);
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice || (e == hipSuccess && n == 0))
        return set_error(MIGEMM_ERR_NO_DEVICE, "context_create: no HIP device is visible");
    MIGEMM_HIP(e);
    // The reference takes the first accelerator / GPU (ComputeContext.cs:53-96); this library's
    // kernels are built for gfx950 only, so the first gfx950 device, unless one is named.
    int pick = -1;
    hipDeviceProp_t prop;
    for (int d = (device >= 0 ? device : 0); d < n && pick < 0; ++d) {
        MIGEMM_HIP(hipGetDeviceProperties(&prop, d));
        if (strncmp(prop.gcnArchName, "gfx950", 6) == 0) pick = d;
        if (device >= 0) break;
    }
    if (pick < 0) {
        if (device >= n)
            return set_error(MIGEMM_ERR_INVALID_ARG, "context_create: device %d of %d", device,
                             n);
        return set_error(MIGEMM_ERR_NO_DEVICE,
                         device >= 0 ? "context_create: device %d is not a gfx950 GPU"
                                     : "context_create: none of the %d devices is a gfx950 GPU",
                         device >= 0 ? device : n);
    }
    MIGEMM_HIP(hipGetDeviceProperties(&prop, pick));
    Context *c = new Context();
    c->device = pick;
    c->compute_units = prop.multiProcessorCount;
    c->wavefront_size = prop.warpSize;
    c->max_work_group_size = prop.maxThreadsPerBlock;
    c->global_mem = prop.totalGlobalMem;
    strncpy(c->arch, prop.gcnArchName, sizeof(c->arch) - 1);
    c->arch[sizeof(c->arch) - 1] = '\0';
    work_group_limits(c);
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    g_contexts.insert(c);
    *ctx = c;
    return MIGEMM_OK;
}

int migemm_context_destroy(void *ctx) {
    clear_error();
    Context *c = static_cast<Context *>(ctx);
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    if (c == nullptr) return MIGEMM_OK;
    if (!live(c)) return set_error(MIGEMM_ERR_INVALID_ARG, "context_destroy: unknown context");
    // its buffers go with it (an OpenCL context's buffers are invalid once it is released)
    int rc = MIGEMM_OK;
    for (auto it = g_pool.begin(); it != g_pool.end();) {
        if (it->second.ctx == c) {
            const int r = free_entry(it->second);
            if (rc == MIGEMM_OK) rc = r;
            it = g_pool.erase(it);
        } else {
            ++it;
        }
    }
    if (t_queue_ctx == c) {
        t_queue_ctx = nullptr;
        t_queue_stream = nullptr;
        t_queue_set = false;
    }
    g_contexts.erase(c);
    delete c;
    return rc;
}

int migemm_context_info(void *ctx, int *device, char *arch_name, size_t arch_name_len,
                        int *compute_units, int *wavefront_size, int *max_work_group_size,
                        int *work_group_x, int *work_group_y, size_t *global_mem_bytes) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    Context *c = static_cast<Context *>(ctx);
    if (!live(c)) return set_error(MIGEMM_ERR_INVALID_ARG, "context_info: unknown context");
    if (device) *device = c->device;
    if (arch_name && arch_name_len > 0) {
        strncpy(arch_name, c->arch, arch_name_len - 1);
        arch_name[arch_name_len - 1] = '\0';
    }
    if (compute_units) *compute_units = c->compute_units;
    if (wavefront_size) *wavefront_size = c->wavefront_size;
    if (max_work_group_size) *max_work_group_size = c->max_work_group_size;
    if (work_group_x) *work_group_x = c->wg_x;
    if (work_group_y) *work_group_y = c->wg_y;
    if (global_mem_bytes) *global_mem_bytes = c->global_mem;
    return MIGEMM_OK;
}

int migemm_buffer_get_or_create(void *ctx, const char *name, size_t bytes, void **ptr) {
    clear_error();
    if (ptr == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_get_or_create: null ptr");
    *ptr = nullptr;
    if (ctx == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_get_or_create: null context");
    if (name == nullptr || name[0] == '\0')
        return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_get_or_create: empty buffer name");
    if (bytes == 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_get_or_create: size must be > 0");
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    Context *c = static_cast<Context *>(ctx);
    if (!live(c)) return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_get_or_create: unknown context");
    return get_or_create_locked(c, name, bytes, ptr);
}

int migemm_buffer_release(const char *name) {
    clear_error();
    if (name == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_release: null name");
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    auto it = g_pool.find(name);
    if (it == g_pool.end()) return MIGEMM_OK;
    const PoolEntry e = it->second;
    g_pool.erase(it);
    return free_entry(e);
}

int migemm_buffer_release_all(void) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    int rc = MIGEMM_OK;
    for (auto &kv : g_pool) {
        const int r = free_entry(kv.second);
        if (rc == MIGEMM_OK) rc = r;
    }
    g_pool.clear();
    return rc;
}

int migemm_buffer_count(size_t *count, size_t *total_bytes) {
    clear_error();
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    size_t total = 0;
    for (auto &kv : g_pool) total += kv.second.bytes;
    if (count) *count = g_pool.size();
    if (total_bytes) *total_bytes = total;
    return MIGEMM_OK;
}

int migemm_queue_register_current(void *ctx, void *stream) {
    clear_error();
    if (stream == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "queue_register_current: the queue (stream) must not be null");
    std::lock_guard<std::mutex> lock(g_rt_mutex);
    Context *c = static_cast<Context *>(ctx);
    if (!live(c))
        return set_error(MIGEMM_ERR_INVALID_ARG, "queue_register_current: unknown context");
    t_queue_ctx = c;
    t_queue_stream = stream;
    t_queue_set = true;
    return MIGEMM_OK;
}

int migemm_queue_get_current(void **ctx, void **stream) {
    clear_error();
    if (!t_queue_set)
        return set_error(MIGEMM_ERR_NO_QUEUE,
                         "no queue is registered on this thread: call "
                         "migemm_queue_register_current(ctx, stream) before computing");
    if (ctx) *ctx = t_queue_ctx;
    if (stream) *stream = t_queue_stream;
    return MIGEMM_OK;
}

int migemm_queue_clear_current(void) {
    clear_error();
    t_queue_ctx = nullptr;
    t_queue_stream = nullptr;
    t_queue_set = false;
    return MIGEMM_OK;
}

int migemm_tensor_buffer(const char *tensor_id, size_t bytes, void **ptr) {
    clear_error();
    if (ptr == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "tensor_buffer: null ptr");
    *ptr = nullptr;
    if (!t_queue_set)
        return set_error(MIGEMM_ERR_NO_QUEUE,
                         "tensor_buffer: no queue is registered on this thread");
    return migemm_buffer_get_or_create(t_queue_ctx, tensor_id, bytes, ptr);
}

}  // extern "C"
