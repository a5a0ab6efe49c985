// Runtime services of the reference's C# host, on HIP: the device context, the name-keyed
// device-buffer pool and the per-thread current queue ("cs/" = csharp/cstorchcl/cstorchcl/),
// and the library's device-memory service they and the stream workspaces share.
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
// The pool follows the reference's rule: a name maps to one buffer, which is returned when
// it belongs to the same context and is at least as large as requested, and is otherwise
// replaced by one of exactly the requested size.
//
// Freeing without waiting. An OpenCL buffer released while kernels still use it stays alive
// until they finish, and the releasing thread does not wait for them. hipFree cannot do
// that: it synchronizes the whole device, so one thread replacing a buffer would wait for
// every other thread's queued work. Pool buffers therefore come from a memory pool the
// library owns (one per device). At release, an event is recorded on every queue registered
// on the buffer's device (by any thread) and on the null stream, and the buffer is parked
// with those events; later library calls poll them (hipEventQuery) and return the memory to
// the pool (hipFreeAsync, which does not wait) only once all have passed. Nothing on the host
// waits, and the pool never holds memory that queued work may still use: its own
// cross-stream reuse rules are not relied on (a free ordered after an event wait on another
// stream was seen handed out again before the event had passed). The pool keeps freed memory
// for reuse (no release threshold), so an allocation does not wait either.
//
// Locking: one reader-writer lock guards the tables. Lookups that find their buffer (the
// Tensor.DataBuffer path) take it shared, in parallel with each other; inserting, replacing
// and releasing take it exclusively, and only for asynchronous HIP calls. Device memory is
// allocated outside the lock.
//
// Context handles are ids that are never reused, so a destroyed context's handle is rejected
// on every thread, including threads whose current queue still names it.
#include <string.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <shared_mutex>
#include <string>
#include <unordered_map>
#include <vector>

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
    uint64_t ctx;  // id of the owning context
    int device;
};

std::shared_mutex g_rt_mutex;  // guards the tables below
std::unordered_map<uint64_t, std::unique_ptr<Context>> g_contexts;  // live contexts by id
std::unordered_map<std::string, PoolEntry> g_pool;                  // buffer name -> buffer
// queues registered as some thread's current queue: (device, stream) -> number of threads
std::map<std::pair<int, void *>, int> g_registered;
std::atomic<uint64_t> g_next_ctx{1};

// DeviceQueueRegistry._currentQueue of this thread; unregistered when the thread ends
struct ThreadQueue {
    uint64_t ctx = 0;
    void *stream = nullptr;
    int device = -1;
    bool set = false;
    ~ThreadQueue();
};
thread_local ThreadQueue t_queue;

void unregister_locked(ThreadQueue &q) {
    if (!q.set) return;
    auto it = g_registered.find({q.device, q.stream});
    if (it != g_registered.end() && --it->second == 0) g_registered.erase(it);
    q = ThreadQueue{};
}

ThreadQueue::~ThreadQueue() {
    if (!set) return;
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    unregister_locked(*this);
}

void *handle_of(uint64_t id) { return reinterpret_cast<void *>(static_cast<uintptr_t>(id)); }
uint64_t id_of(void *h) { return static_cast<uint64_t>(reinterpret_cast<uintptr_t>(h)); }

Context *find_locked(void *h) {
    auto it = g_contexts.find(id_of(h));
    return it == g_contexts.end() ? nullptr : it->second.get();
}

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

// ---- device memory service ----
constexpr int kMaxDevices = 64;
struct DevMem {
    bool ready = false;
    hipMemPool_t pool = nullptr;
    // allocations, and frees of memory no queued work uses any more: synchronizing it waits
    // for nothing else
    hipStream_t alloc_stream = nullptr;
};
std::mutex g_devmem_mutex;
DevMem g_devmem[kMaxDevices];

int devmem(int device, DevMem **out) {
    if (device < 0 || device >= kMaxDevices)
        return set_error(MIGEMM_ERR_UNSUPPORTED, "device %d: devices 0..%d are supported", device,
                         kMaxDevices - 1);
    std::lock_guard<std::mutex> lock(g_devmem_mutex);
    DevMem &m = g_devmem[device];
    if (!m.ready) {
        DeviceScope scope(device);
        MIGEMM_HIP(scope.err);
        int supported = 0;
        MIGEMM_HIP(hipDeviceGetAttribute(&supported, hipDeviceAttributeMemoryPoolsSupported,
                                         device));
        if (!supported)
            return set_error(MIGEMM_ERR_UNSUPPORTED,
                             "device %d has no stream-ordered memory allocator", device);
        hipMemPoolProps props;
        memset(&props, 0, sizeof(props));
        props.allocType = hipMemAllocationTypePinned;
        props.handleTypes = hipMemHandleTypeNone;
        props.location.type = hipMemLocationTypeDevice;
        props.location.id = device;
        MIGEMM_HIP(hipMemPoolCreate(&m.pool, &props));
        uint64_t keep = UINT64_MAX;  // freed memory stays in the pool for reuse
        MIGEMM_HIP(hipMemPoolSetAttribute(m.pool, hipMemPoolAttrReleaseThreshold, &keep));
        int off = 0;  // never hand out memory whose free has not run yet
        MIGEMM_HIP(hipMemPoolSetAttribute(m.pool, hipMemPoolReuseAllowInternalDependencies, &off));
        MIGEMM_HIP(hipStreamCreateWithFlags(&m.alloc_stream, hipStreamNonBlocking));
        m.ready = true;
    }
    *out = &m;
    return MIGEMM_OK;
}

// Released pool memory waits here until every event recorded at its release has passed
// (hipEventQuery, never a host wait); only then is it returned to the pool, so the pool
// never holds memory that queued work may still touch, whatever its own reuse rules.
struct Grave {
    int device;
    void *ptr;
    std::vector<hipEvent_t> events;
};
std::mutex g_grave_mutex;
std::vector<Grave> g_graves;

// Returns the memory of every grave whose events have all passed to its pool (with `wait`,
// of every grave, after waiting for its events).
int reap(bool wait) {
    std::lock_guard<std::mutex> lock(g_grave_mutex);
    int rc = MIGEMM_OK;
    for (size_t i = 0; i < g_graves.size();) {
        Grave &g = g_graves[i];
        bool done = true;
        for (hipEvent_t ev : g.events) {
            const hipError_t e = wait ? hipEventSynchronize(ev) : hipEventQuery(ev);
            if (e == hipErrorNotReady) {
                done = false;
                break;
            }
            if (e != hipSuccess && rc == MIGEMM_OK) rc = hip_check(e, "hipEventQuery");
        }
        if (!done) {
            ++i;
            continue;
        }
        DevMem *m = nullptr;
        int r = devmem(g.device, &m);
        if (r == MIGEMM_OK) {
            DeviceScope scope(g.device);
            r = hip_check(scope.err, "hipSetDevice");
            if (r == MIGEMM_OK) r = hip_check(hipFreeAsync(g.ptr, m->alloc_stream), "hipFreeAsync");
        }
        if (r != MIGEMM_OK && rc == MIGEMM_OK) rc = r;
        for (hipEvent_t ev : g.events) (void)hipEventDestroy(ev);
        g_graves[i] = std::move(g_graves.back());
        g_graves.pop_back();
    }
    return rc;
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

// Frees a pooled buffer once the work queued so far on every registered queue of its device
// (and on the null stream) has passed; never waits on the host. Called with the lock held.
int retire_locked(const PoolEntry &e) {
    std::vector<void *> streams;
    for (auto &kv : g_registered)
        if (kv.first.first == e.device) streams.push_back(kv.first.second);
    streams.push_back(nullptr);
    return devmem_free_after(e.device, e.ptr, streams.data(), (int)streams.size());
}

}  // namespace

int devmem_alloc(int device, size_t bytes, void **ptr) {
    DevMem *m = nullptr;
    int rc = devmem(device, &m);
    if (rc != MIGEMM_OK) return rc;
    rc = reap(false);
    if (rc != MIGEMM_OK) return rc;
    DeviceScope scope(device);
    MIGEMM_HIP(scope.err);
    void *p = nullptr;
    hipError_t e = hipMallocFromPoolAsync(&p, bytes, m->pool, m->alloc_stream);
    if (e == hipErrorOutOfMemory)
        return set_error(MIGEMM_ERR_HIP, "allocation of %zu bytes: out of device memory", bytes);
    MIGEMM_HIP(e);
    MIGEMM_HIP(hipStreamSynchronize(m->alloc_stream));
    *ptr = p;
    return MIGEMM_OK;
}

int devmem_alloc_on(hipStream_t stream, int device, size_t bytes, void **ptr) {
    DevMem *m = nullptr;
    int rc = devmem(device, &m);
    if (rc != MIGEMM_OK) return rc;
    rc = reap(false);
    if (rc != MIGEMM_OK) return rc;
    void *p = nullptr;
    hipError_t e = hipMallocFromPoolAsync(&p, bytes, m->pool, stream);
    if (e == hipErrorOutOfMemory)
        return set_error(MIGEMM_ERR_WORKSPACE, "workspace of %zu bytes: out of device memory",
                         bytes);
    MIGEMM_HIP(e);
    *ptr = p;
    return MIGEMM_OK;
}

int devmem_free_after(int device, void *ptr, void *const *streams, int n) {
    if (ptr == nullptr) return MIGEMM_OK;
    Grave g;
    g.device = device;
    g.ptr = ptr;
    {
        DeviceScope scope(device);
        MIGEMM_HIP(scope.err);
        for (int i = 0; i < n; ++i) {
            hipEvent_t ev;
            MIGEMM_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
            g.events.push_back(ev);
            MIGEMM_HIP(hipEventRecord(ev, static_cast<hipStream_t>(streams[i])));
        }
    }
    {
        std::lock_guard<std::mutex> lock(g_grave_mutex);
        g_graves.push_back(std::move(g));
    }
    return reap(false);
}

int devmem_free_on(hipStream_t stream, void *ptr) {
    if (ptr == nullptr) return MIGEMM_OK;
    int device = 0;
    int rc = stream_device(stream, &device);
    if (rc != MIGEMM_OK) return rc;
    void *s = stream;
    return devmem_free_after(device, ptr, &s, 1);
}

int devmem_trim(int device) {
    DevMem *m = nullptr;
    int rc = devmem(device, &m);
    if (rc != MIGEMM_OK) return rc;
    rc = reap(true);
    if (rc != MIGEMM_OK) return rc;
    DeviceScope scope(device);
    MIGEMM_HIP(scope.err);
    MIGEMM_HIP(hipStreamSynchronize(m->alloc_stream));
    MIGEMM_HIP(hipMemPoolTrimTo(m->pool, 0));
    return MIGEMM_OK;
}

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
    auto c = std::make_unique<Context>();
    c->device = pick;
    c->compute_units = prop.multiProcessorCount;
    c->wavefront_size = prop.warpSize;
    c->max_work_group_size = prop.maxThreadsPerBlock;
    c->global_mem = prop.totalGlobalMem;
    strncpy(c->arch, prop.gcnArchName, sizeof(c->arch) - 1);
    c->arch[sizeof(c->arch) - 1] = '\0';
    work_group_limits(c.get());
    const uint64_t id = g_next_ctx.fetch_add(1);
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    g_contexts.emplace(id, std::move(c));
    *ctx = handle_of(id);
    return MIGEMM_OK;
}

int migemm_context_destroy(void *ctx) {
    clear_error();
    if (ctx == nullptr) return MIGEMM_OK;
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    if (find_locked(ctx) == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "context_destroy: unknown context");
    // its buffers go with it (an OpenCL context's buffers are invalid once it is released)
    int rc = MIGEMM_OK;
    for (auto it = g_pool.begin(); it != g_pool.end();) {
        if (it->second.ctx == id_of(ctx)) {
            const int r = retire_locked(it->second);
            if (rc == MIGEMM_OK) rc = r;
            it = g_pool.erase(it);
        } else {
            ++it;
        }
    }
    if (t_queue.set && t_queue.ctx == id_of(ctx)) unregister_locked(t_queue);
    g_contexts.erase(id_of(ctx));
    return rc;
}

int migemm_context_info(void *ctx, int *device, char *arch_name, size_t arch_name_len,
                        int *compute_units, int *wavefront_size, int *max_work_group_size,
                        int *work_group_x, int *work_group_y, size_t *global_mem_bytes) {
    clear_error();
    std::shared_lock<std::shared_mutex> lock(g_rt_mutex);
    const Context *c = find_locked(ctx);
    if (c == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "context_info: unknown context");
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
    int device = -1;
    {
        // the fast path (OpenCLBufferManager.cs:28-41): a shared lookup
        std::shared_lock<std::shared_mutex> lock(g_rt_mutex);
        const Context *c = find_locked(ctx);
        if (c == nullptr)
            return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_get_or_create: unknown context");
        device = c->device;
        auto it = g_pool.find(name);
        if (it != g_pool.end() && it->second.ctx == id_of(ctx) && it->second.bytes >= bytes) {
            *ptr = it->second.ptr;
            return MIGEMM_OK;
        }
    }
    // a new buffer of exactly `bytes` (OpenCLBufferManager.cs:53-59), allocated unlocked
    void *fresh = nullptr;
    int rc = devmem_alloc(device, bytes, &fresh);
    if (rc != MIGEMM_OK) return rc;
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    if (find_locked(ctx) == nullptr) {  // destroyed meanwhile
        (void)devmem_free_after(device, fresh, nullptr, 0);
        return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_get_or_create: unknown context");
    }
    auto it = g_pool.find(name);
    if (it != g_pool.end()) {
        if (it->second.ctx == id_of(ctx) && it->second.bytes >= bytes) {
            // another thread created a large enough one meanwhile: use it, drop ours
            *ptr = it->second.ptr;
            return devmem_free_after(device, fresh, nullptr, 0);
        }
        // too small, or from another context: replaced (OpenCLBufferManager.cs:48-55)
        rc = retire_locked(it->second);
        g_pool.erase(it);
        if (rc != MIGEMM_OK) {
            (void)devmem_free_after(device, fresh, nullptr, 0);
            return rc;
        }
    }
    g_pool.emplace(name, PoolEntry{bytes, fresh, id_of(ctx), device});
    *ptr = fresh;
    return MIGEMM_OK;
}

int migemm_buffer_release(const char *name) {
    clear_error();
    if (name == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "buffer_release: null name");
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    auto it = g_pool.find(name);
    if (it == g_pool.end()) return MIGEMM_OK;
    const PoolEntry e = it->second;
    g_pool.erase(it);
    return retire_locked(e);
}

int migemm_buffer_release_all(void) {
    clear_error();
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    int rc = MIGEMM_OK;
    for (auto &kv : g_pool) {
        const int r = retire_locked(kv.second);
        if (rc == MIGEMM_OK) rc = r;
    }
    g_pool.clear();
    return rc;
}

int migemm_buffer_count(size_t *count, size_t *total_bytes) {
    clear_error();
    std::shared_lock<std::shared_mutex> lock(g_rt_mutex);
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
    int device = -1;
    {
        std::shared_lock<std::shared_mutex> lock(g_rt_mutex);
        const Context *c = find_locked(ctx);
        if (c == nullptr)
            return set_error(MIGEMM_ERR_INVALID_ARG, "queue_register_current: unknown context");
        device = c->device;
    }
    int sdev = -1;
    MIGEMM_HIP(hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev));
    if (sdev != device)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "queue_register_current: the stream is on device %d, the context on "
                         "device %d", sdev, device);
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    if (find_locked(ctx) == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "queue_register_current: unknown context");
    unregister_locked(t_queue);
    t_queue.ctx = id_of(ctx);
    t_queue.stream = stream;
    t_queue.device = device;
    t_queue.set = true;
    ++g_registered[{device, stream}];
    return MIGEMM_OK;
}

int migemm_queue_get_current(void **ctx, void **stream) {
    clear_error();
    if (!t_queue.set)
        return set_error(MIGEMM_ERR_NO_QUEUE,
                         "no queue is registered on this thread: call "
                         "migemm_queue_register_current(ctx, stream) before computing");
    {
        std::shared_lock<std::shared_mutex> lock(g_rt_mutex);
        if (find_locked(handle_of(t_queue.ctx)) == nullptr)
            return set_error(MIGEMM_ERR_INVALID_ARG,
                             "queue_get_current: this thread's queue belongs to a destroyed "
                             "context");
    }
    if (ctx) *ctx = handle_of(t_queue.ctx);
    if (stream) *stream = t_queue.stream;
    return MIGEMM_OK;
}

int migemm_queue_clear_current(void) {
    clear_error();
    if (!t_queue.set) return MIGEMM_OK;
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    unregister_locked(t_queue);
    return MIGEMM_OK;
}

int migemm_tensor_buffer(const char *tensor_id, size_t bytes, void **ptr) {
    clear_error();
    if (ptr == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "tensor_buffer: null ptr");
    *ptr = nullptr;
    if (!t_queue.set)
        return set_error(MIGEMM_ERR_NO_QUEUE,
                         "tensor_buffer: no queue is registered on this thread");
    // a context destroyed by another thread is rejected here as an unknown context
    return migemm_buffer_get_or_create(handle_of(t_queue.ctx), tensor_id, bytes, ptr);
}

}  // extern "C"

namespace migemm {
// A stream the library is about to destroy stops being a registered queue (deferred frees
// must not record events on it afterwards).
void forget_stream(void *stream) {
    std::unique_lock<std::shared_mutex> lock(g_rt_mutex);
    for (auto it = g_registered.begin(); it != g_registered.end();)
        it = it->first.second == stream ? g_registered.erase(it) : std::next(it);
    if (t_queue.set && t_queue.stream == stream) t_queue = ThreadQueue{};
}
}  // namespace migemm
