// C ABI of libmigemm: argument validation, dispatch to the HIP kernels, and the device /
// memory / stream services the reference host obtains from OpenCL.
//
// Every compute entry point validates all of its arguments before the first HIP call, so
// argument errors behave the same with and without a GPU, mirroring the reference's
// checks that throw before any enqueue (cs/compiler/NnClGlob.cs:443-452, :1704-1714,
// cs/core/Tensor.cs:191-192; "cs/" = csharp/cstorchcl/cstorchcl/).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "migemm_internal.h"

namespace migemm {

namespace {
thread_local char g_last_error[512] = "";
constexpr int64_t kMaxElems = (int64_t)1 << 46;  // 256 TiB of fp32: beyond any device

// a*b + c with overflow detection for non-negative operands (bounded by kMaxElems).
bool mul_add_ok(int64_t a, int64_t b, int64_t c, int64_t *out) {
    if (a < 0 || b < 0 || c < 0) return false;
    if (a != 0 && b > kMaxElems / a) return false;
    const int64_t p = a * b;
    if (p > kMaxElems - c) return false;
    *out = p + c;
    return true;
}

bool ranges_overlap(const void *p0, int64_t n0, const void *p1, int64_t n1) {
    const uintptr_t a0 = reinterpret_cast<uintptr_t>(p0);
    const uintptr_t a1 = reinterpret_cast<uintptr_t>(p1);
    const uintptr_t e0 = a0 + (uintptr_t)n0 * sizeof(float);
    const uintptr_t e1 = a1 + (uintptr_t)n1 * sizeof(float);
    return a0 < e1 && a1 < e0;
}

// Element extent touched by a batched matrix operand: (batch-1)*stride + (rows-1)*ld + cols.
bool extent(int batch, int64_t stride, int rows, int64_t ld, int cols, int64_t *out) {
    int64_t inner;
    if (!mul_add_ok(rows - 1, ld, cols, &inner)) return false;
    return mul_add_ok(batch - 1, stride, inner, out);
}

struct DeviceWorkspace {
    void *ptr = nullptr;
    size_t bytes = 0;
    // Handed out to work captured into a HIP graph: the graph keeps the address, so the
    // buffer is never freed (a replay may run at any later time) and, once the capture has
    // ended, no longer lent to eager work (a replay on another stream could overlap it).
    bool captured = false;
};
std::mutex g_ws_mutex;
// keyed by (device, stream, slot)
std::map<std::tuple<int, uintptr_t, int>, DeviceWorkspace> g_ws;
// buffers that captured graphs refer to: kept until the process ends
std::vector<void *> g_graph_owned;
}  // namespace

int set_error(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error[0] = '\0'; }

int hip_check(hipError_t e, const char *what) {
    if (e == hipSuccess) return MIGEMM_OK;
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
        return set_error(MIGEMM_ERR_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
    return set_error(MIGEMM_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {
thread_local bool t_plan_only = false;
// An address that is never dereferenced: the partial-sum buffer of a plan-only dispatch.
float *const kPlanPlaceholder = reinterpret_cast<float *>(static_cast<uintptr_t>(1) << 12);
}  // namespace

bool plan_only() { return t_plan_only; }

int launch_status(const char *what) {
    if (t_plan_only) return MIGEMM_OK;
    return hip_check(hipGetLastError(), what);
}

int stream_device(hipStream_t stream, int *device) {
    if (stream == nullptr) {
        MIGEMM_HIP(hipGetDevice(device));
    } else {
        MIGEMM_HIP(hipStreamGetDevice(stream, device));
    }
    return MIGEMM_OK;
}

// One growing buffer per device, stream and slot: calls on one stream run in order, so
// they can share a buffer, and calls on different streams (the reference host keeps one
// queue per thread) never share one. Buffers come from the library's device memory pool
// (runtime.hip) in the stream's order, and an outgrown buffer is freed in the stream's
// order too (after the work already queued that uses it), so growing never waits on the
// host. A buffer a HIP graph captured is never freed and, once the capture has ended, is
// retired from eager use: the next eager call on the stream gets a buffer of its own.
// migemm_workspace_release / migemm_stream_destroy free a stream's live buffers.
// Nothing is allocated while the stream is being captured into a HIP graph (an allocation
// would invalidate the capture), and a capturing stream only uses its own buffer: work on
// another stream may run at the same time as a replay, so a borrowed buffer could race.
// A caller sizes the capturing stream's buffer beforehand with migemm_workspace_reserve or
// by running the same call once on that stream outside the capture.
void *workspace(hipStream_t stream, size_t bytes, int *status, int slot) {
    if (t_plan_only) {
        *status = MIGEMM_OK;
        return kPlanPlaceholder;
    }
    int dev = 0;
    *status = stream_device(stream, &dev);
    if (*status != MIGEMM_OK) return nullptr;
    if (slot < 0 || slot >= kWorkspaceSlots) {
        *status = set_error(MIGEMM_ERR_WORKSPACE, "workspace slot %d", slot);
        return nullptr;
    }
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(stream, &capture);
    if (e != hipSuccess) {
        *status = hip_check(e, "hipStreamIsCapturing");
        return nullptr;
    }
    const bool capturing = capture != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    const auto key = std::make_tuple(dev, reinterpret_cast<uintptr_t>(stream), slot);
    auto it = g_ws.find(key);
    if (it != g_ws.end() && it->second.bytes >= bytes && (capturing || !it->second.captured)) {
        if (capturing) it->second.captured = true;
        *status = MIGEMM_OK;
        return it->second.ptr;
    }
    if (capturing) {
        *status = set_error(MIGEMM_ERR_WORKSPACE,
                            "%zu bytes of workspace are needed during HIP graph capture but "
                            "the capturing stream holds %zu: call migemm_workspace_reserve on "
                            "that stream, or run the same call once on it, before capturing",
                            bytes, it != g_ws.end() ? it->second.bytes : (size_t)0);
        return nullptr;
    }
    DeviceWorkspace &w = g_ws[key];
    size_t want = bytes < ((size_t)8 << 20) ? ((size_t)8 << 20) : bytes;
    if (!w.captured && want < 2 * w.bytes) want = 2 * w.bytes;
    void *p = nullptr;
    *status = devmem_alloc_on(stream, dev, want, &p);
    if (*status != MIGEMM_OK) return nullptr;
    if (w.ptr != nullptr) {
        if (w.captured) {
            g_graph_owned.push_back(w.ptr);  // the graph keeps using it
        } else {
            *status = devmem_free_on(stream, w.ptr);  // after the queued work that uses it
            if (*status != MIGEMM_OK) {
                (void)devmem_free_on(stream, p);
                return nullptr;
            }
        }
    }
    w.ptr = p;
    w.bytes = want;
    w.captured = false;
    *status = MIGEMM_OK;
    return w.ptr;
}

float *partial_buffer(hipStream_t stream, const GemmDesc &d, size_t bytes, int *status) {
    if (d.scratch == nullptr) return static_cast<float *>(workspace(stream, bytes, status, 0));
    if (bytes > d.scratch_bytes) {
        *status = set_error(MIGEMM_ERR_WORKSPACE,
                            "this GEMM keeps %zu bytes of partial sums but the no-allocation "
                            "entry point's static scratch holds %zu "
                            "(MIGEMM_NOALLOC_SCRATCH_BYTES)", bytes, d.scratch_bytes);
        return nullptr;
    }
    *status = MIGEMM_OK;
    return d.scratch;
}

// Frees the live workspace buffers of `stream` (on the stream's device) in the stream's
// order. Buffers a graph captured are kept.
static int release_workspace(hipStream_t stream) {
    int dev = 0;
    int rc = stream_device(stream, &dev);
    if (rc != MIGEMM_OK) return rc;
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    for (int slot = 0; slot < kWorkspaceSlots; ++slot) {
        auto it = g_ws.find(std::make_tuple(dev, reinterpret_cast<uintptr_t>(stream), slot));
        if (it == g_ws.end()) continue;
        const DeviceWorkspace w = it->second;
        g_ws.erase(it);
        if (w.captured) {
            g_graph_owned.push_back(w.ptr);
        } else {
            rc = devmem_free_on(stream, w.ptr);
            if (rc != MIGEMM_OK) return rc;
        }
    }
    return MIGEMM_OK;
}

// ---------------------------------------------------------------------------------------
// Scratch of the no-allocation GEMM (migemm_gemm_strided_batched_noalloc): partial sums of
// split GEMMs in a static device array instead of the stream's workspace, so that entry
// point never allocates. Each GPU the library runs on holds its own copy until the process
// ends. In host code the array's name is only a stand-in symbol, never a device address:
// each device's address of it is looked up once, with that device current, and only that
// pointer is passed to kernels.
static __device__ __align__(256) float scratch[MIGEMM_NOALLOC_SCRATCH_BYTES / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::atomic<float *> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

// Device address of `scratch` on the device of `stream` (looked up on the first call there,
// with that device current).
static int scratch_address(hipStream_t stream, float **out) {
    int dev = 0;
    int rc = stream_device(stream, &dev);
    if (rc != MIGEMM_OK) return rc;
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(MIGEMM_ERR_UNSUPPORTED, "device %d: the no-allocation entry point "
                         "supports devices 0..%d", dev, kMaxDevices - 1);
    float *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mutex);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            int cur = 0;
            MIGEMM_HIP(hipGetDevice(&cur));
            if (cur != dev) MIGEMM_HIP(hipSetDevice(dev));
            void *addr = nullptr;
            const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
            if (cur != dev) MIGEMM_HIP(hipSetDevice(cur));
            MIGEMM_HIP(e);
            p = static_cast<float *>(addr);
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return MIGEMM_OK;
}

// Validates a general GEMM request and fills `d`. No HIP call is made.
static int validate_gemm(int transA, int transB, int M, int N, int K, const float *A,
                         int64_t lda, int64_t strideA, const float *B, int64_t ldb,
                         int64_t strideB, const float *bias, float *C, int64_t ldc,
                         int64_t strideC, int batch, GemmDesc *d) {
    if (M < 1 || N < 1 || K < 1 || batch < 1)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "gemm: sizes must be >= 1 (M=%d N=%d K=%d batch=%d)", M, N, K, batch);
    if (A == nullptr || B == nullptr || C == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: A, B and C must be non-null");
    if (transA != 0 && transA != 1)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: transA must be 0 or 1 (got %d)", transA);
    if (transB != 0 && transB != 1)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: transB must be 0 or 1 (got %d)", transB);
    const int a_rows = transA ? K : M, a_cols = transA ? M : K;
    const int b_rows = transB ? N : K, b_cols = transB ? K : N;
    if (lda < a_cols)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: lda=%lld < %d", (long long)lda, a_cols);
    if (ldb < b_cols)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: ldb=%lld < %d", (long long)ldb, b_cols);
    if (ldc < N)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: ldc=%lld < N=%d", (long long)ldc, N);
    if (strideA < 0 || strideB < 0 || strideC < 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: batch strides must be >= 0");
    int64_t ea, eb, ec;
    if (!extent(batch, strideA, a_rows, lda, a_cols, &ea) ||
        !extent(batch, strideB, b_rows, ldb, b_cols, &eb) ||
        !extent(batch, strideC, M, ldc, N, &ec))
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm: operand extent overflows");
    if (batch > 1 && strideC < (int64_t)(M - 1) * ldc + N)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "gemm: strideC=%lld makes batch entries of C overlap",
                         (long long)strideC);
    if (ranges_overlap(C, ec, A, ea) || ranges_overlap(C, ec, B, eb) ||
        (bias != nullptr && ranges_overlap(C, ec, bias, N)))
        return set_error(MIGEMM_ERR_ALIAS, "gemm: output overlaps an input");
    d->A = A;
    d->B = B;
    d->bias = bias;
    d->C = C;
    d->lda = lda;
    d->ldb = ldb;
    d->ldc = ldc;
    d->sA = batch > 1 ? strideA : 0;
    d->sB = batch > 1 ? strideB : 0;
    d->sC = batch > 1 ? strideC : 0;
    d->M = M;
    d->N = N;
    d->K = K;
    d->batch = batch;
    d->transA = transA != 0;
    d->transB = transB != 0;
    d->accumulate = false;
    return MIGEMM_OK;
}

// Kernel-family policy (migemm_set_gemm_policy) and tuning overrides (migemm_set_tuning),
// process-wide.
static std::atomic<int> g_policy{MIGEMM_POLICY_AUTO};
static std::atomic<int> g_tuning[MIGEMM_TUNE_SMALL_SPLITK + 1];

int tuning(int key) { return g_tuning[key].load(std::memory_order_relaxed); }

static thread_local PlanRecord g_plan = {"none", 0, 0, 0, 0, 0, 0, 0, 0, false, false};

void record_plan(const PlanRecord &p) { g_plan = p; }

void record_plan(const char *kernel, const GemmDesc &d, int bm, int bn, int splits,
                 int load_bytes) {
    g_plan = PlanRecord{kernel, bm, bn, splits, load_bytes, d.M, d.N, d.K, d.batch,
                        d.transA, d.transB};
}

static int run_gemm(hipStream_t stream, const GemmDesc &desc) {
    GemmDesc d = desc;
    const int policy = g_policy.load(std::memory_order_relaxed);
    // A batch of GEMMs that share B (batch stride 0), with A not transposed and the A and C
    // entries following each other without gaps, is one GEMM of batch * M rows: every output
    // element's sum is unchanged, and the larger M quantizes better onto the tiles. The
    // reference's LinearForward and BmmPermute calls with a shared weight are this case
    // (NnClGlob.cs:1502-1551, 1717-1751): Linear(500 -> 6565) on [8, 1500, 500] forward
    // 709.1 -> 648 us, dX 726.0 -> 659 us. Only under the AUTO policy, so the forced kernel
    // families keep running their own batch-stride code.
    if (policy == MIGEMM_POLICY_AUTO && d.batch > 1 && d.sB == 0 && !d.transA &&
        d.sA == (int64_t)d.M * d.lda && d.sC == (int64_t)d.M * d.ldc &&
        (int64_t)d.M * d.batch <= INT32_MAX) {
        d.M *= d.batch;
        d.batch = 1;
        d.sA = 0;
        d.sC = 0;
    }
    switch (policy) {
        case MIGEMM_POLICY_TILED: return launch_gemm_tiled(stream, d);
        case MIGEMM_POLICY_SMALL: return launch_gemm_small(stream, d);
        case MIGEMM_POLICY_SKINNY:
            if (skinny_supported(d)) return launch_gemm_skinny(stream, d);
            break;
        case MIGEMM_POLICY_PANEL:
            if (panel_supported(d)) return launch_gemm_panel(stream, d);
            break;
        case MIGEMM_POLICY_TINY:
            if (tiny_supported(d)) return launch_gemm_tiny(stream, d);
            break;
        default: break;
    }
    if (skinny_preferred(d)) return launch_gemm_skinny(stream, d);
    if (tiny_preferred(d)) return launch_gemm_tiny(stream, d);
    if (panel_preferred(d)) return launch_gemm_panel(stream, d);
    if (small_preferred(d)) return launch_gemm_small(stream, d);
    return launch_gemm_tiled(stream, d);
}

// C = opA(A) opB(B) + opA(A2) opB(B2) (+ bias) for a descriptor with a second operand pair:
// one panel launch over the k-groups of both pairs where the panel kernel applies and is
// the AUTO choice for the concatenated product (or is forced), otherwise the first product
// with the bias and then the second accumulated onto it, each dispatched as a GEMM of its
// own.
static int run_gemm_pair(hipStream_t stream, const GemmDesc &d) {
    const int policy = g_policy.load(std::memory_order_relaxed);
    if (panel_supported(d) && (policy == MIGEMM_POLICY_PANEL ||
                               (policy == MIGEMM_POLICY_AUTO && panel_preferred(d))))
        return launch_gemm_panel(stream, d);
    GemmDesc first = d;
    first.A2 = nullptr;
    first.B2 = nullptr;
    first.K2 = 0;
    int rc = run_gemm(stream, first);
    if (rc != MIGEMM_OK) return rc;
    GemmDesc second = first;
    second.A = d.A2;
    second.B = d.B2;
    second.lda = d.lda2;
    second.ldb = d.ldb2;
    second.K = d.K2;
    second.bias = nullptr;
    second.accumulate = true;
    return run_gemm(stream, second);
}

}  // namespace migemm

using namespace migemm;

extern "C" {

int migemm_gemm_strided_batched(void *stream, int transA, int transB, int M, int N, int K,
                                const float *A, int64_t lda, int64_t strideA, const float *B,
                                int64_t ldb, int64_t strideB, const float *bias, float *C,
                                int64_t ldc, int64_t strideC, int batch) {
    clear_error();
    GemmDesc d;
    int rc = validate_gemm(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, bias, C,
                           ldc, strideC, batch, &d);
    if (rc != MIGEMM_OK) return rc;
    return run_gemm(static_cast<hipStream_t>(stream), d);
}

int migemm_gemm_strided_batched_ex(void *stream, int transA, int transB, int M, int N, int K,
                                   const float *A, int64_t lda, int64_t strideA, const float *B,
                                   int64_t ldb, int64_t strideB, const float *bias, float *C,
                                   int64_t ldc, int64_t strideC, int batch, int flags) {
    clear_error();
    if ((flags & ~MIGEMM_GEMM_ACCUMULATE) != 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm_ex: unknown flags 0x%x", flags);
    GemmDesc d;
    int rc = validate_gemm(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, bias, C,
                           ldc, strideC, batch, &d);
    if (rc != MIGEMM_OK) return rc;
    d.accumulate = (flags & MIGEMM_GEMM_ACCUMULATE) != 0;
    return run_gemm(static_cast<hipStream_t>(stream), d);
}

int migemm_gemm_strided_batched_noalloc(void *stream, int transA, int transB, int M, int N,
                                        int K, const float *A, int64_t lda, int64_t strideA,
                                        const float *B, int64_t ldb, int64_t strideB,
                                        const float *bias, float *C, int64_t ldc,
                                        int64_t strideC, int batch, int flags) {
    clear_error();
    if ((flags & ~MIGEMM_GEMM_ACCUMULATE) != 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm_noalloc: unknown flags 0x%x", flags);
    GemmDesc d;
    int rc = validate_gemm(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, bias, C,
                           ldc, strideC, batch, &d);
    if (rc != MIGEMM_OK) return rc;
    d.accumulate = (flags & MIGEMM_GEMM_ACCUMULATE) != 0;
    rc = scratch_address(static_cast<hipStream_t>(stream), &d.scratch);
    if (rc != MIGEMM_OK) return rc;
    d.scratch_bytes = MIGEMM_NOALLOC_SCRATCH_BYTES;
    return run_gemm(static_cast<hipStream_t>(stream), d);
}

int migemm_gemm_plan(int transA, int transB, int M, int N, int K, const float *A, int64_t lda,
                     int64_t strideA, const float *B, int64_t ldb, int64_t strideB,
                     const float *bias, float *C, int64_t ldc, int64_t strideC, int batch,
                     int flags, char *plan, size_t plan_len) {
    clear_error();
    if (plan == nullptr || plan_len == 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm_plan: null or empty plan buffer");
    if ((flags & ~MIGEMM_GEMM_ACCUMULATE) != 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "gemm_plan: unknown flags 0x%x", flags);
    GemmDesc d;
    int rc = validate_gemm(transA, transB, M, N, K, A, lda, strideA, B, ldb, strideB, bias, C,
                           ldc, strideC, batch, &d);
    if (rc != MIGEMM_OK) return rc;
    d.accumulate = (flags & MIGEMM_GEMM_ACCUMULATE) != 0;
    t_plan_only = true;
    rc = run_gemm(nullptr, d);
    t_plan_only = false;
    if (rc != MIGEMM_OK) return rc;
    return migemm_last_plan(plan, plan_len);
}

int migemm_matmul_tiled(void *stream, const float *A, const float *B, float *C, int M, int K,
                        int N) {
    return migemm_gemm_strided_batched(stream, 0, 0, M, N, K, A, K, 0, B, N, 0, nullptr, C, N,
                                       0, 1);
}

static int check_ref_strides(const char *who, int sA, int sB, int sC) {
    if (sA < 0 || sB < 0 || sC < 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "%s: batch strides must be >= 0", who);
    return MIGEMM_OK;
}

int migemm_bmm_tiled(void *stream, const float *A, const float *B, float *C, int M, int K, int N,
                     int batch_stride_A, int batch_stride_B, int batch_stride_C, int batch) {
    clear_error();
    int rc = check_ref_strides("bmm_tiled", batch_stride_A, batch_stride_B, batch_stride_C);
    if (rc != MIGEMM_OK) return rc;
    return migemm_gemm_strided_batched(stream, 0, 0, M, N, K, A, K, batch_stride_A, B, N,
                                       batch_stride_B, nullptr, C, N, batch_stride_C, batch);
}

int migemm_bmm_permute_tiled(void *stream, const float *A, const float *B, float *C, int M,
                             int K, int N, int batch_stride_A, int batch_stride_B,
                             int batch_stride_C, int transA, int transB, int batch) {
    clear_error();
    int rc = check_ref_strides("bmm_permute_tiled", batch_stride_A, batch_stride_B,
                               batch_stride_C);
    if (rc != MIGEMM_OK) return rc;
    // The reference treats any non-zero flag as "transposed" (bmm_permute_tiled.cl:43-44).
    const int ta = transA != 0, tb = transB != 0;
    return migemm_gemm_strided_batched(stream, ta, tb, M, N, K, A, ta ? M : K, batch_stride_A,
                                       B, tb ? K : N, batch_stride_B, nullptr, C, N,
                                       batch_stride_C, batch);
}

int migemm_linear_forward(void *stream, const float *X, const float *W, const float *bias,
                          float *Y, int M, int K, int N, int batch_stride_X, int batch_stride_Y,
                          int batch) {
    clear_error();
    if (bias == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "linear_forward: bias must be non-null");
    int rc = check_ref_strides("linear_forward", batch_stride_X, 0, batch_stride_Y);
    if (rc != MIGEMM_OK) return rc;
    return migemm_gemm_strided_batched(stream, 0, 0, M, N, K, X, K, batch_stride_X, W, N, 0,
                                       bias, Y, N, batch_stride_Y, batch);
}

int migemm_lstm_gemm_xw(void *stream, const float *X, const float *W, const float *bias,
                        float *XW_out, int total_tokens, int in_features, int total_gates) {
    clear_error();
    if (bias == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_gemm_xw: bias must be non-null");
    return migemm_gemm_strided_batched(stream, 0, 0, total_tokens, total_gates, in_features, X,
                                       in_features, 0, W, total_gates, 0, bias, XW_out,
                                       total_gates, 0, 1);
}

int migemm_lstm_gemm_grad_x(void *stream, const float *all_grad_gates, const float *W,
                            float *grad_X, int total_tokens, int in_features, int total_gates) {
    clear_error();
    // grad_X[T, F] = G[T, 4H] * W^T, W stored [F, 4H] (B transposed: element (k, f) at
    // W[f * total_gates + k]).
    return migemm_gemm_strided_batched(stream, 0, 1, total_tokens, in_features, total_gates,
                                       all_grad_gates, total_gates, 0, W, total_gates, 0,
                                       nullptr, grad_X, in_features, 0, 1);
}

int migemm_lstm_gemm_grad_weights(void *stream, const float *X, const float *H_out,
                                  const float *all_grad_gates, float *grad_W, float *grad_U,
                                  float *grad_bias, int batch_size, int seq_len,
                                  int in_features, int hidden_size) {
    clear_error();
    if (X == nullptr || H_out == nullptr || all_grad_gates == nullptr || grad_W == nullptr ||
        grad_U == nullptr || grad_bias == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_gemm_grad_weights: null pointer argument");
    if (batch_size < 1 || seq_len < 1 || in_features < 1 || hidden_size < 1)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "lstm_gemm_grad_weights: sizes must be >= 1 (batch=%d seq=%d in=%d "
                         "hidden=%d)",
                         batch_size, seq_len, in_features, hidden_size);
    const int64_t tokens = (int64_t)batch_size * seq_len;
    const int64_t gates = (int64_t)4 * hidden_size;
    if (tokens > INT32_MAX || gates > INT32_MAX)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "lstm_gemm_grad_weights: batch*seq or 4*hidden exceeds 2^31-1");
    const int T = (int)tokens, G = (int)gates;
    // the three accumulated outputs must be disjoint from each other and from the inputs
    const struct {
        const void *p;
        int64_t n;
    } out[3] = {{grad_W, (int64_t)in_features * G},
                {grad_U, (int64_t)hidden_size * G},
                {grad_bias, G}},
      in[3] = {{X, tokens * in_features}, {H_out, tokens * hidden_size}, {all_grad_gates, tokens * G}};
    for (int i = 0; i < 3; ++i) {
        for (int j = 0; j < 3; ++j)
            if (ranges_overlap(out[i].p, out[i].n, in[j].p, in[j].n))
                return set_error(MIGEMM_ERR_ALIAS,
                                 "lstm_gemm_grad_weights: an output overlaps an input");
        for (int j = i + 1; j < 3; ++j)
            if (ranges_overlap(out[i].p, out[i].n, out[j].p, out[j].n))
                return set_error(MIGEMM_ERR_ALIAS, "lstm_gemm_grad_weights: outputs overlap");
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    // grad_W[F, 4H] += X^T * G (A transposed: X is stored [T, F])
    int rc = migemm_gemm_strided_batched_ex(stream, 1, 0, in_features, G, T, X, in_features, 0,
                                            all_grad_gates, G, 0, nullptr, grad_W, G, 0, 1,
                                            MIGEMM_GEMM_ACCUMULATE);
    if (rc != MIGEMM_OK) return rc;
    // grad_bias[4H] += column sums of G
    rc = launch_column_sum(st, all_grad_gates, grad_bias, 1, T, G, true);
    if (rc != MIGEMM_OK) return rc;
    // grad_U[H, 4H] += H_prev^T * G; H_prev is zero at every sequence's first step, so a
    // single-step sequence adds nothing
    if (seq_len == 1) return MIGEMM_OK;
    int st_ws = MIGEMM_OK;
    float *hprev = static_cast<float *>(
        workspace(st, (size_t)tokens * hidden_size * sizeof(float), &st_ws, 1));
    if (hprev == nullptr) return st_ws;
    rc = launch_shift_rows(st, H_out, hprev, T, seq_len, hidden_size);
    if (rc != MIGEMM_OK) return rc;
    return migemm_gemm_strided_batched_ex(stream, 1, 0, hidden_size, G, T, hprev, hidden_size, 0,
                                          all_grad_gates, G, 0, nullptr, grad_U, G, 0, 1,
                                          MIGEMM_GEMM_ACCUMULATE);
}

int migemm_lstm_recurrent_gates(void *stream, float *XW, const float *H_out, const float *U,
                                int batch_size, int seq_len, int hidden_size, int t) {
    clear_error();
    if (XW == nullptr || H_out == nullptr || U == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_recurrent_gates: null pointer argument");
    if (batch_size < 1 || seq_len < 1 || hidden_size < 1)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "lstm_recurrent_gates: sizes must be >= 1 (batch=%d seq=%d hidden=%d)",
                         batch_size, seq_len, hidden_size);
    if (t < 0 || t >= seq_len)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_recurrent_gates: step %d not in [0, %d)",
                         t, seq_len);
    const int64_t gates = (int64_t)4 * hidden_size;
    if (gates > INT32_MAX)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_recurrent_gates: 4*hidden exceeds 2^31-1");
    if (t == 0) return MIGEMM_OK;  // h_{-1} = 0: the gates are XW itself (lstm.cl:57-60)
    // XW[:, t, :] += H_out[:, t-1, :] * U: rows b of the two slices sit seq_len rows apart
    return migemm_gemm_strided_batched_ex(
        stream, 0, 0, batch_size, (int)gates, hidden_size, H_out + (int64_t)(t - 1) * hidden_size,
        (int64_t)seq_len * hidden_size, 0, U, gates, 0, nullptr, XW + (int64_t)t * gates,
        (int64_t)seq_len * gates, 0, 1, MIGEMM_GEMM_ACCUMULATE);
}

int migemm_lstm_hid_gates(void *stream, const float *X, const float *W, const float *U,
                          const float *bias, const float *H_prev, const float *H_out,
                          float *workspace, int batch_size, int seq_len, int in_features,
                          int hidden_size, int t) {
    clear_error();
    if (X == nullptr || W == nullptr || U == nullptr || bias == nullptr || workspace == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_hid_gates: null pointer argument");
    if (batch_size < 1 || seq_len < 1 || in_features < 1 || hidden_size < 1)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "lstm_hid_gates: sizes must be >= 1 (batch=%d seq=%d in=%d hidden=%d)",
                         batch_size, seq_len, in_features, hidden_size);
    if (t < 0 || t >= seq_len)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_hid_gates: step %d not in [0, %d)", t,
                         seq_len);
    // h_{t-1}: the chunk's incoming state at t = 0 (H_prev, lstm.cl:821), else the previous
    // step's output row of the same sequence (H_out, written at lstm.cl:861)
    const float *hsrc = t == 0 ? H_prev : H_out;
    if (hsrc == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_hid_gates: %s is null at step %d",
                         t == 0 ? "H_prev" : "H_out", t);
    const int64_t gates = (int64_t)4 * hidden_size;
    if (gates > INT32_MAX)
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_hid_gates: 4*hidden exceeds 2^31-1");
    const int G = (int)gates;
    int64_t n_x, n_w, n_u, n_h, n_ws, bs;
    if (!mul_add_ok(batch_size, seq_len, 0, &bs) || !mul_add_ok(bs, in_features, 0, &n_x) ||
        !mul_add_ok(in_features, gates, 0, &n_w) || !mul_add_ok(hidden_size, gates, 0, &n_u) ||
        !mul_add_ok(t == 0 ? batch_size : bs, hidden_size, 0, &n_h) ||
        !mul_add_ok(bs, gates, 0, &n_ws))
        return set_error(MIGEMM_ERR_INVALID_ARG, "lstm_hid_gates: size overflows");
    // the step's gates, workspace[t, 0..batch, 0..4H): one contiguous range
    float *out = workspace + (int64_t)t * batch_size * gates;
    const int64_t n_out = (int64_t)batch_size * gates;
    if (ranges_overlap(out, n_out, X, n_x) || ranges_overlap(out, n_out, W, n_w) ||
        ranges_overlap(out, n_out, U, n_u) || ranges_overlap(out, n_out, bias, gates) ||
        ranges_overlap(out, n_out, hsrc, n_h))
        return set_error(MIGEMM_ERR_ALIAS, "lstm_hid_gates: the step's gates overlap an input");
    GemmDesc d;
    d.A = X + (int64_t)t * in_features;  // x_t of sequence b: row b, seq_len*F apart
    d.lda = (int64_t)seq_len * in_features;
    d.B = W;
    d.ldb = gates;
    d.bias = bias;
    d.C = out;
    d.ldc = gates;
    d.sA = d.sB = d.sC = 0;
    d.M = batch_size;
    d.N = G;
    d.K = in_features;
    d.batch = 1;
    d.transA = d.transB = false;
    d.accumulate = false;
    d.A2 = t == 0 ? H_prev : H_out + (int64_t)(t - 1) * hidden_size;
    d.lda2 = t == 0 ? (int64_t)hidden_size : (int64_t)seq_len * hidden_size;
    d.B2 = U;
    d.ldb2 = gates;
    d.K2 = hidden_size;
    return run_gemm_pair(static_cast<hipStream_t>(stream), d);
}

int migemm_linear_weight_grad(void *stream, const float *X, const float *dY, float *dW, int M,
                              int K, int N, int batch) {
    clear_error();
    if (M < 1 || K < 1 || N < 1 || batch < 1)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "linear_weight_grad: sizes must be >= 1 (M=%d K=%d N=%d batch=%d)", M,
                         K, N, batch);
    const int64_t rows = (int64_t)batch * M;
    if (rows > INT32_MAX)
        return set_error(MIGEMM_ERR_INVALID_ARG, "linear_weight_grad: batch*M exceeds 2^31-1");
    // dW[K,N] = X'^T dY' with X' = X viewed [batch*M, K] and dY' = dY viewed [batch*M, N].
    return migemm_gemm_strided_batched(stream, 1, 0, K, N, (int)rows, X, K, 0, dY, N, 0,
                                       nullptr, dW, N, 0, 1);
}

int migemm_tensor_permute(void *stream, const float *src, float *dst, const int *src_dims,
                          const int *axes, int num_dims) {
    clear_error();
    if (src == nullptr || dst == nullptr || src_dims == nullptr || axes == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "tensor_permute: null pointer argument");
    if (num_dims < 1 || num_dims > 10)
        return set_error(MIGEMM_ERR_INVALID_ARG, "tensor_permute: num_dims=%d not in [1,10]",
                         num_dims);
    int64_t total = 1;
    bool seen[10] = {false};
    for (int i = 0; i < num_dims; ++i) {
        if (src_dims[i] < 1)
            return set_error(MIGEMM_ERR_INVALID_ARG, "tensor_permute: dim %d is %d (< 1)", i,
                             src_dims[i]);
        if (axes[i] < 0 || axes[i] >= num_dims || seen[axes[i]])
            return set_error(MIGEMM_ERR_INVALID_ARG,
                             "tensor_permute: axes is not a permutation of 0..%d", num_dims - 1);
        seen[axes[i]] = true;
        if (!mul_add_ok(total, src_dims[i], 0, &total))
            return set_error(MIGEMM_ERR_INVALID_ARG, "tensor_permute: size overflows");
    }
    if (ranges_overlap(src, total, dst, total))
        return set_error(MIGEMM_ERR_ALIAS, "tensor_permute: dst overlaps src");
    return launch_permute(static_cast<hipStream_t>(stream), src, dst, src_dims, axes, num_dims,
                          total);
}

int migemm_reduce_sum_axis(void *stream, const float *X, float *Y, int outer_size,
                           int axis_size, int inner_size) {
    clear_error();
    if (X == nullptr || Y == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "reduce_sum_axis: null pointer argument");
    if (outer_size < 1 || axis_size < 1 || inner_size < 1)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "reduce_sum_axis: sizes must be >= 1 (outer=%d axis=%d inner=%d)",
                         outer_size, axis_size, inner_size);
    int64_t nin, nout;
    if (!mul_add_ok((int64_t)outer_size * inner_size, axis_size, 0, &nin) ||
        !mul_add_ok(outer_size, inner_size, 0, &nout) || nout > INT32_MAX * (int64_t)256)
        return set_error(MIGEMM_ERR_INVALID_ARG, "reduce_sum_axis: size overflows");
    if (ranges_overlap(X, nin, Y, nout))
        return set_error(MIGEMM_ERR_ALIAS, "reduce_sum_axis: output overlaps input");
    return launch_column_sum(static_cast<hipStream_t>(stream), X, Y, outer_size, axis_size,
                             inner_size);
}

int migemm_stream_read(void *stream, const float *src, size_t n, float *sums, int blocks) {
    clear_error();
    if (src == nullptr || sums == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "stream_read: null pointer argument");
    if (n == 0 || n % 4 != 0 || (reinterpret_cast<uintptr_t>(src) & 15) != 0)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "stream_read: n must be a positive multiple of 4 and src 16-byte "
                         "aligned (n=%zu)", n);
    if (blocks < 1 || blocks > 65535 || (int64_t)(n / 4) < blocks)
        return set_error(MIGEMM_ERR_INVALID_ARG, "stream_read: blocks=%d not in [1, min(65535, "
                         "n/4)]", blocks);
    if (n > (size_t)kMaxElems)
        return set_error(MIGEMM_ERR_INVALID_ARG, "stream_read: n=%zu too large", n);
    if (ranges_overlap(sums, blocks, src, (int64_t)n))
        return set_error(MIGEMM_ERR_ALIAS, "stream_read: sums overlap src");
    return launch_stream_read(static_cast<hipStream_t>(stream), src, (int64_t)(n / 4), sums,
                              blocks);
}

int migemm_linear_bias_backward(void *stream, const float *grad_output, float *grad_bias,
                                int total_rows, int N) {
    clear_error();
    if (grad_output == nullptr || grad_bias == nullptr)
        return set_error(MIGEMM_ERR_INVALID_ARG, "linear_bias_backward: null pointer argument");
    if (total_rows < 1 || N < 1)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "linear_bias_backward: sizes must be >= 1 (rows=%d N=%d)", total_rows,
                         N);
    return migemm_reduce_sum_axis(stream, grad_output, grad_bias, 1, total_rows, N);
}

// ---------------------------------------------------------------------------------------
// Services.

int migemm_device_count(int *count) {
    clear_error();
    if (count == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "device_count: null pointer");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e == hipErrorNoDevice) {
        *count = 0;
        return MIGEMM_OK;
    }
    MIGEMM_HIP(e);
    *count = n;
    return MIGEMM_OK;
}

int migemm_set_device(int device) {
    clear_error();
    if (device < 0) return set_error(MIGEMM_ERR_INVALID_ARG, "set_device: device %d < 0", device);
    MIGEMM_HIP(hipSetDevice(device));
    return MIGEMM_OK;
}

int migemm_device_info(int device, char *arch_name, size_t arch_name_len, int *compute_units,
                       size_t *global_mem_bytes) {
    clear_error();
    if (device < 0) return set_error(MIGEMM_ERR_INVALID_ARG, "device_info: device %d < 0", device);
    hipDeviceProp_t prop;
    MIGEMM_HIP(hipGetDeviceProperties(&prop, device));
    if (arch_name != nullptr && arch_name_len > 0) {
        strncpy(arch_name, prop.gcnArchName, arch_name_len - 1);
        arch_name[arch_name_len - 1] = '\0';
    }
    if (compute_units != nullptr) *compute_units = prop.multiProcessorCount;
    if (global_mem_bytes != nullptr) *global_mem_bytes = prop.totalGlobalMem;
    return MIGEMM_OK;
}

int migemm_malloc(void **ptr, size_t bytes) {
    clear_error();
    if (ptr == nullptr || bytes == 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "malloc: null pointer or zero size");
    MIGEMM_HIP(hipMalloc(ptr, bytes));
    return MIGEMM_OK;
}

int migemm_free(void *ptr) {
    clear_error();
    if (ptr == nullptr) return MIGEMM_OK;
    MIGEMM_HIP(hipFree(ptr));
    return MIGEMM_OK;
}

int migemm_memcpy_h2d(void *stream, void *dst, const void *src, size_t bytes) {
    clear_error();
    if ((dst == nullptr || src == nullptr) && bytes != 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "memcpy_h2d: null pointer");
    if (bytes == 0) return MIGEMM_OK;
    MIGEMM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                              static_cast<hipStream_t>(stream)));
    return MIGEMM_OK;
}

int migemm_memcpy_d2h(void *stream, void *dst, const void *src, size_t bytes) {
    clear_error();
    if ((dst == nullptr || src == nullptr) && bytes != 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "memcpy_d2h: null pointer");
    if (bytes == 0) return MIGEMM_OK;
    MIGEMM_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                              static_cast<hipStream_t>(stream)));
    MIGEMM_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return MIGEMM_OK;
}

int migemm_memset(void *stream, void *dst, int value, size_t bytes) {
    clear_error();
    if (dst == nullptr && bytes != 0) return set_error(MIGEMM_ERR_INVALID_ARG, "memset: null pointer");
    if (bytes == 0) return MIGEMM_OK;
    MIGEMM_HIP(hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream)));
    return MIGEMM_OK;
}

int migemm_stream_create(void **stream) {
    clear_error();
    if (stream == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "stream_create: null pointer");
    hipStream_t s;
    MIGEMM_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return MIGEMM_OK;
}

int migemm_stream_destroy(void *stream) {
    clear_error();
    if (stream == nullptr) return MIGEMM_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // deferred frees must not record events on it any more
    forget_stream(stream);
    int rc = release_workspace(s);  // in the stream's order
    if (rc != MIGEMM_OK) return rc;
    MIGEMM_HIP(hipStreamSynchronize(s));
    MIGEMM_HIP(hipStreamDestroy(s));
    return MIGEMM_OK;
}

int migemm_workspace_reserve(void *stream, size_t bytes) {
    clear_error();
    if (bytes == 0) return MIGEMM_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    MIGEMM_HIP(hipStreamIsCapturing(s, &capture));
    if (capture != hipStreamCaptureStatusNone)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "workspace_reserve: the stream is being captured into a HIP graph");
    int st = MIGEMM_OK;
    for (int slot = 0; slot < kWorkspaceSlots; ++slot)
        if (workspace(s, bytes, &st, slot) == nullptr) return st;
    return MIGEMM_OK;
}

int migemm_workspace_release(void *stream) {
    clear_error();
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    MIGEMM_HIP(hipStreamIsCapturing(s, &capture));
    if (capture != hipStreamCaptureStatusNone)
        return set_error(MIGEMM_ERR_INVALID_ARG,
                         "workspace_release: the stream is being captured into a HIP graph");
    return release_workspace(s);
}

int migemm_workspace_size(void *stream, size_t *bytes) {
    clear_error();
    if (bytes == nullptr) return set_error(MIGEMM_ERR_INVALID_ARG, "workspace_size: null pointer");
    // no HIP call: the stream may already have been destroyed (then it holds nothing)
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    *bytes = 0;
    for (const auto &kv : g_ws)
        if (std::get<1>(kv.first) == reinterpret_cast<uintptr_t>(stream) &&
            std::get<2>(kv.first) == 0)
            *bytes = kv.second.bytes;
    return MIGEMM_OK;
}

int migemm_stream_synchronize(void *stream) {
    clear_error();
    MIGEMM_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return MIGEMM_OK;
}

const char *migemm_last_error(void) { return g_last_error; }

const char *migemm_version(void) { return "0.1.0"; }

int migemm_set_tuning(int key, int value, int *previous) {
    clear_error();
    bool ok;
    switch (key) {
        case MIGEMM_TUNE_TILE:
            ok = value == 0 || value == 32 || value == 64 || value == 128 || value == 256 ||
                 value == MIGEMM_TILE_128x256;
            break;
        case MIGEMM_TUNE_SPLITK:
        case MIGEMM_TUNE_SMALL_SPLITK: ok = value >= 0 && value <= 64; break;
        case MIGEMM_TUNE_DIRECT:
        case MIGEMM_TUNE_SMALL_TILES: ok = value >= 0 && value <= 2; break;
        default:
            return set_error(MIGEMM_ERR_INVALID_ARG, "set_tuning: unknown key %d", key);
    }
    if (!ok)
        return set_error(MIGEMM_ERR_INVALID_ARG, "set_tuning: value %d is not valid for key %d",
                         value, key);
    const int old = g_tuning[key].exchange(value);
    if (previous != nullptr) *previous = old;
    return MIGEMM_OK;
}

int migemm_last_plan(char *buf, size_t len) {
    clear_error();
    if (buf == nullptr || len == 0)
        return set_error(MIGEMM_ERR_INVALID_ARG, "last_plan: null or empty buffer");
    const PlanRecord &p = g_plan;
    snprintf(buf, len, "%s tile=%dx%d splits=%d load_bytes=%d M=%d N=%d K=%d batch=%d %c%c",
             p.kernel, p.bm, p.bn, p.splits, p.load_bytes, p.M, p.N, p.K, p.batch,
             p.transA ? 'T' : 'N', p.transB ? 'T' : 'N');
    return MIGEMM_OK;
}

int migemm_set_gemm_policy(int policy, int *previous) {
    clear_error();
    if (policy < MIGEMM_POLICY_AUTO || policy > MIGEMM_POLICY_TINY)
        return set_error(MIGEMM_ERR_INVALID_ARG, "set_gemm_policy: unknown policy %d", policy);
    const int old = g_policy.exchange(policy);
    if (previous != nullptr) *previous = old;
    return MIGEMM_OK;
}

}  // extern "C"
