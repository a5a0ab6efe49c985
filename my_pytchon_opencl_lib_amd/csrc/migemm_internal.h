// Internal declarations shared by the HIP translation units of libmigemm.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/migemm.h"

namespace migemm {

// Thread-local last-error message (returned by migemm_last_error()).
int set_error(int code, const char *fmt, ...);
void clear_error();

// Checks a HIP status; on failure records the message and returns MIGEMM_ERR_HIP.
int hip_check(hipError_t e, const char *what);

#define MIGEMM_HIP(call)                                   \
    do {                                                   \
        int _rc = ::migemm::hip_check((call), #call);      \
        if (_rc != MIGEMM_OK) return _rc;                  \
    } while (0)

// Division by an invariant divisor 1 <= d < 2^31 for numerators n < 2^31 (Granlund and
// Montgomery, "Division by Invariant Integers using Multiplication", PLDI 1994, the
// n + mulhi form): with l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1 (< 2^32),
//   n / d = (mulhi(n, m) + n) >> l,
// i.e. floor(n * M / 2^(32+l)) with M = 2^32 + m = floor(2^(32+l) / d) + 1, whose excess
// e = M d - 2^(32+l) <= d keeps n e / 2^(32+l) < 2^31 2^l / 2^(32+l) < 1 / d below the gap
// to the next multiple of d. The sum cannot overflow (mulhi(n, m) < n < 2^31), and d = 1
// (m = 1, l = 0) needs no special case, so the division is three instructions without a
// branch, against the long dependent sequence the GPU runs for a 32-bit division. Kernels
// take FastDiv values computed on the host for their launch-invariant divisors.
struct FastDiv {
    uint32_t d, mult, shift;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f{d, 1, 0};
    if (d == 0) return f;
    uint32_t l = 0;
    while (((uint64_t)1 << l) < d) ++l;
    f.mult = (uint32_t)((((uint64_t)1 << 32) * (((uint64_t)1 << l) - d)) / d + 1);
    f.shift = l;
    return f;
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv &f) {
    return (__umulhi(n, f.mult) + n) >> f.shift;
}

// Description of one (possibly batched, possibly transposed) fp32 GEMM after
// validation: C_b = opA(A_b) * opB(B_b) (+ bias).
struct GemmDesc {
    const float *A;
    const float *B;
    const float *bias;
    float *C;
    int64_t lda, ldb, ldc;
    int64_t sA, sB, sC;
    int M, N, K, batch;
    bool transA, transB;
    bool accumulate;  // C = C + (op(A) op(B) + bias) instead of C = op(A) op(B) + bias
    // Caller-provided scratch for partial sums (the no-allocation entry point's static
    // device array); nullptr = the library workspace of the stream.
    float *scratch = nullptr;
    size_t scratch_bytes = 0;
    // Optional second operand pair (batch 1): C = opA(A) opB(B) + opA(A2) opB(B2) (+ bias),
    // A2 [M, K2] and B2 [K2, N] in the orientations of A and B (the stateful LSTM gates
    // x_t W + h_{t-1} U). Only the panel kernel takes it; run_gemm_pair otherwise runs the
    // two products as two GEMMs.
    const float *A2 = nullptr;
    const float *B2 = nullptr;
    int64_t lda2 = 0, ldb2 = 0;
    int K2 = 0;
};

// Device memory for `bytes` of fp32 partial sums of the GEMM `d`: d.scratch when the call
// brought one (MIGEMM_ERR_WORKSPACE if it is too small), else the stream's workspace
// (slot 0). Returns nullptr and sets *status on failure.
float *partial_buffer(hipStream_t stream, const GemmDesc &d, size_t bytes, int *status);

// Tuning override `key` (MIGEMM_TUNE_*), set by migemm_set_tuning; 0 = the dispatcher's
// choice. A relaxed atomic load: production calls read no environment.
int tuning(int key);

// What the last dispatch on this host thread ran (migemm_last_plan formats it).
struct PlanRecord {
    const char *kernel;  // kernel family, e.g. "tiled-direct", "small", "skinny"
    int bm, bn;          // output tile (0 when the kernel has none)
    int splits;          // k ranges (1 = whole K)
    int load_bytes;      // bytes per lane of each operand load into LDS (16 or 4; 0 = n/a)
    int M, N, K, batch;
    bool transA, transB;
};
void record_plan(const PlanRecord &p);
void record_plan(const char *kernel, const GemmDesc &d, int bm, int bn, int splits,
                 int load_bytes);

// Plan-only dispatch (migemm_gemm_plan): on this host thread the launchers make every
// choice and record the plan exactly as for a real call, but enqueue nothing and make no HIP
// call: kernel launches go through MIGEMM_LAUNCH, their status through launch_status, and
// partial-sum / workspace requests return a placeholder address that nothing dereferences.
bool plan_only();
#define MIGEMM_LAUNCH(...)                                          \
    do {                                                            \
        if (!::migemm::plan_only()) hipLaunchKernelGGL(__VA_ARGS__); \
    } while (0)
// hip_check(hipGetLastError(), what) after a launch; MIGEMM_OK when planning only.
int launch_status(const char *what);

// Launchers. They assume a validated descriptor and only enqueue work.
int launch_gemm_tiled(hipStream_t stream, const GemmDesc &d);
int launch_gemm_skinny(hipStream_t stream, const GemmDesc &d);
// M <= 4 (gemm_skinny_kernel for B not transposed, gemv_rows_kernel for B transposed).
bool skinny_supported(const GemmDesc &d);
// Supported, and a shape where the streaming kernel beats the others (B not transposed:
// >= 64 MB of B; transposed: enough rows of B, gemm_skinny.hip).
bool skinny_preferred(const GemmDesc &d);
int launch_gemm_small(hipStream_t stream, const GemmDesc &d);
// Every operand layout with K % 32 == 0 (K2 % 32 == 0 for a second pair), N % 4 == 0,
// M % 4 == 0 when A is transposed, 16-byte aligned operand rows and lda, ldb <= 2^25
// (gemm_panel_kernel: 32x32 tiles, operands loaded straight into LDS).
bool panel_supported(const GemmDesc &d);
// Supported, and a shape where it beats the small and tiled families.
bool panel_preferred(const GemmDesc &d);

// Short-K kernel (gemm_tiny.hip): 16x16 tiles with all operands in registers, one
// wavefront per tile over K <= 80, two or four (each a share of K) for K = 96, 128, 160,
// 192, 256 or 320.
bool tiny_supported(const GemmDesc &d);
bool tiny_preferred(const GemmDesc &d);
int launch_gemm_tiny(hipStream_t stream, const GemmDesc &d);
int launch_gemm_panel(hipStream_t stream, const GemmDesc &d);
// True when C has too few 64x64 tiles to occupy the 256 CUs, or is 16 or fewer rows or
// columns wide (gemm_small_kernel).
bool small_preferred(const GemmDesc &d);
// 5-16 rows of C over a B (not transposed) of 256 MB or more: the tiled kernel's 32x32 tiles.
bool narrow_rows_streaming(const GemmDesc &d);

// Device memory owned by the library (runtime.hip): a memory pool per device whose frees
// are stream-ordered, so releasing memory never waits on the host (hipFree would
// synchronize the whole device).
// devmem_alloc: `bytes` usable on any stream of `device` when it returns.
int devmem_alloc(int device, size_t bytes, void **ptr);
// devmem_alloc_on: `bytes` usable by work queued on `stream` (of `device`) after the call.
int devmem_alloc_on(hipStream_t stream, int device, size_t bytes, void **ptr);
// devmem_free_on: frees pool memory once the work queued on `stream` so far has run.
int devmem_free_on(hipStream_t stream, void *ptr);
// devmem_free_after: frees pool memory of `device` once the work queued so far on each of
// the n streams has run (a null entry is the null stream).
int devmem_free_after(int device, void *ptr, void *const *streams, int n);
// devmem_trim: waits for pending frees of `device` and returns unused pool memory.
int devmem_trim(int device);
// A stream that is about to be destroyed stops being a registered queue.
void forget_stream(void *stream);
// The device a stream belongs to (the current device for the null stream).
int stream_device(hipStream_t stream, int *device);

// Device workspace owned by the library: one growing buffer per device, stream and slot.
// Slot 0 holds split-K partial sums (GEMM, column sums); slot 1 holds operands staged by
// an entry point for the GEMMs it then runs (which may use slot 0). Returns nullptr and
// records MIGEMM_ERR_WORKSPACE on failure.
constexpr int kWorkspaceSlots = 2;
void *workspace(hipStream_t stream, size_t bytes, int *status, int slot = 0);

// C_b[m, n] = sum over s = 0..S-1 (in order) of partial[s][b][m][n] (+ bias[n]); with
// `accumulate`, C_b[m, n] += that value.
int launch_reduce_slices(hipStream_t stream, const float *partial, int slices, int batch,
                         int M, int N, const float *bias, float *C, int64_t ldc,
                         int64_t strideC, bool accumulate = false);

int launch_permute(hipStream_t stream, const float *src, float *dst,
                   const int *src_dims, const int *axes, int num_dims, int64_t total);
// Y[o, i] (+)= sum over a of X[o][a][i] (accumulate: Y += sum).
int launch_column_sum(hipStream_t stream, const float *X, float *Y,
                      int outer, int axis, int inner, bool accumulate = false);

// sums[b] = sum of the b-th of `blocks` contiguous ranges of src[0 .. 4 n4), streamed once.
int launch_stream_read(hipStream_t stream, const float *src, int64_t n4, float *sums,
                       int blocks);

// Hp[t] = H[t - 1] when t % seq_len > 0, else 0 (rows of `hidden` floats).
int launch_shift_rows(hipStream_t stream, const float *H, float *Hp, int total_tokens,
                      int seq_len, int hidden);

}  // namespace migemm
