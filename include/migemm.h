/*
 * migemm.h -- C ABI of the MI355X (gfx950) fp32 matrix-multiplication library.
 *
 * This is the drop-in boundary for the matmul path of Dima3108/my_pytchon_opencl_lib.
 * Every entry point below replaces one OpenCL enqueue of the reference; the comment
 * above each declaration names the reference interface it replaces (file:line, paths
 * relative to the reference repository root; "cs/" abbreviates csharp/cstorchcl/cstorchcl/).
 *
 * Conventions (shared by every compute entry point):
 *   - All matrices are row-major fp32 in device memory (HIP device pointers).
 *   - Sizes are element counts; strides ("batch strides") are element offsets between
 *     consecutive matrices of a batch, exactly as the reference kernels take them.
 *     A batch stride of 0 broadcasts that operand over the batch
 *     (cs/compiler/NnClGlob.cs:467 and :1719-1720).
 *   - `stream` is a hipStream_t passed as void*; NULL means the null stream.
 *     Compute entry points are asynchronous on that stream (like BmmPermute /
 *     LinearForward in the reference); the host wrappers add the blocking
 *     synchronisation where the reference has one (cs/compiler/NnClGlob.cs:498).
 *   - The library never allocates or frees caller tensors. Outputs are written only
 *     inside [M x N] of each batch entry; memory around them (pooled buffers larger
 *     than M*N, cs/compiler/OpenCLBufferManager.cs:29-40) is left untouched.
 *   - An output range that overlaps an input range is rejected (MIGEMM_ERR_ALIAS):
 *     the reference kernels read inputs while other work-groups write C, so an
 *     aliased call has no defined result there either.
 *   - Every argument is validated before any HIP call is made, so argument errors are
 *     reported identically on machines with and without a GPU.
 *   - Arithmetic: each output element is an fp32 sum over k of fp32 products,
 *     accumulated by fp32 MFMA (v_mfma_f32_32x32x2_f32) or by fp32 FMA chains in the
 *     skinny kernels, plus an optional bias added after the k loop
 *     (cs/cl_kernels/linear.cl:119-122). Results match the reference kernels within a
 *     relative error of 1e-5*sqrt(K) against an fp64 evaluation.
 */
#ifndef MIGEMM_H
#define MIGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. 0 = success. The C# / Python wrappers map INVALID_ARG, ALIAS and
 * UNSUPPORTED to ArgumentException / ValueError (cs/compiler/NnClGlob.cs:443-452),
 * and HIP / NO_DEVICE / WORKSPACE to InvalidOperationException / RuntimeError
 * (cs/compiler/JITProgramCache.cs:40-43). */
enum {
    MIGEMM_OK = 0,
    MIGEMM_ERR_INVALID_ARG = 1, /* bad size, stride, pointer, flag or overflow        */
    MIGEMM_ERR_ALIAS = 2,       /* output range overlaps an input range              */
    MIGEMM_ERR_HIP = 3,         /* a HIP runtime call failed (message in last error) */
    MIGEMM_ERR_NO_DEVICE = 4,   /* no usable gfx950 device                           */
    MIGEMM_ERR_WORKSPACE = 5,   /* internal workspace could not be allocated         */
    MIGEMM_ERR_UNSUPPORTED = 6, /* valid request outside what this build implements  */
    MIGEMM_ERR_NO_QUEUE = 7     /* no queue registered on this thread (the reference's
                                   InvalidOperationException, DeviceQueueRegistry.cs:30-36) */
};

/* ------------------------------------------------------------------------------- */
/* (1) General strided-batched GEMM: the one entry point every form below reduces to.
 *
 *   C_b[m, n] = sum_k opA(A_b)[m, k] * opB(B_b)[k, n]  (+ bias[n] if bias != NULL)
 *   A_b = A + b*strideA, B_b = B + b*strideB, C_b = C + b*strideC, b in [0, batch)
 *   transA == 0: A_b element (m,k) at A_b[m*lda + k]   (A stored [M,K])
 *   transA != 0: A_b element (m,k) at A_b[k*lda + m]   (A stored [K,M])
 *   transB == 0: B_b element (k,n) at B_b[k*ldb + n]   (B stored [K,N])
 *   transB != 0: B_b element (k,n) at B_b[n*ldb + k]   (B stored [N,K])
 *   C_b element (m,n) at C_b[m*ldc + n].
 * Requirements: M,N,K,batch >= 1; lda/ldb/ldc at least the stored row length;
 * strideA, strideB >= 0 (0 = broadcast); when batch > 1, strideC >= (M-1)*ldc + N
 * so that no two batch entries write the same element.
 * Covers NN / NT / TN (TT too), stride-0 broadcast and the bias epilogue of
 * cs/cl_kernels/linear.cl:107-143 and cs/cl_kernels/lstm.cl:340-366.
 */
int migemm_gemm_strided_batched(void *stream, int transA, int transB,
                                int M, int N, int K,
                                const float *A, int64_t lda, int64_t strideA,
                                const float *B, int64_t ldb, int64_t strideB,
                                const float *bias,
                                float *C, int64_t ldc, int64_t strideC,
                                int batch);

/* The same with flags. MIGEMM_GEMM_ACCUMULATE: C_b = C_b + (opA(A_b) * opB(B_b) + bias),
 * the "+=" epilogue of the reference's gradient kernels (cs/cl_kernels/lstm.cl:546-560,
 * 621-632: grad_W / grad_U = old value + tile sum). Other bits are rejected. */
#define MIGEMM_GEMM_ACCUMULATE 1
int migemm_gemm_strided_batched_ex(void *stream, int transA, int transB,
                                   int M, int N, int K,
                                   const float *A, int64_t lda, int64_t strideA,
                                   const float *B, int64_t ldb, int64_t strideB,
                                   const float *bias,
                                   float *C, int64_t ldc, int64_t strideC,
                                   int batch, int flags);

/* The same as migemm_gemm_strided_batched_ex, allocating nothing: no hipMalloc, hipFree or
 * allocating library routine, on any call. It has no counterpart in the reference; it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation). The kernels and results are those of
 * migemm_gemm_strided_batched_ex; the partial sums that split-K GEMMs and sliced GEMVs keep
 * go to a static device array of MIGEMM_NOALLOC_SCRATCH_BYTES that each GPU the library
 * runs on holds until the process ends, instead of the stream's workspace. A call whose
 * partial sums exceed it fails with MIGEMM_ERR_WORKSPACE before any launch (e.g. 8 k ranges
 * of a 2048 x 2048 output; every BASELINE shape needs at most 0.7 MB). All calls on one GPU
 * share that array: calls that overlap in time on one GPU (two streams, two threads) race
 * on it, so callers order them (one stream, or events). */
#define MIGEMM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int migemm_gemm_strided_batched_noalloc(void *stream, int transA, int transB,
                                        int M, int N, int K,
                                        const float *A, int64_t lda, int64_t strideA,
                                        const float *B, int64_t ldb, int64_t strideB,
                                        const float *bias,
                                        float *C, int64_t ldc, int64_t strideC,
                                        int batch, int flags);

/* ------------------------------------------------------------------------------- */
/* (2) Reference-shaped entry points: same argument lists and meaning as the OpenCL
 *     kernels (plus the stream, and the batch count that the reference passes as the
 *     third global-size dimension), so every reference call site maps 1:1.          */

/* Replaces kernel matmul_tiled, cl_kernels/matmul.cl:8-14
 * (launched as in tests/test_matrix_ops.py:109-121): C[M,N] = A[M,K] * B[K,N]. */
int migemm_matmul_tiled(void *stream, const float *A, const float *B, float *C,
                        int M, int K, int N);

/* Replaces kernel bmm_tiled, cl_kernels/matmul.cl:78-87, enqueued by
 * NnClGlob.Bmm (cs/compiler/NnClGlob.cs:441-506) and nncl_glob.py:110-147.
 * batch_stride_B == 0 broadcasts B (NnClGlob.cs:467). */
int migemm_bmm_tiled(void *stream, const float *A, const float *B, float *C,
                     int M, int K, int N,
                     int batch_stride_A, int batch_stride_B, int batch_stride_C,
                     int batch);

/* Replaces kernel bmm_permute_tiled, cs/cl_kernels/bmm_permute_tiled.cl:7-19,
 * enqueued by NnClGlob.BmmPermute (cs/compiler/NnClGlob.cs:1702-1751).
 * transA: A stored [K,M] (element (r,k) = A[k*M + r], bmm_permute_tiled.cl:59);
 * transB: B stored [N,K] (element (k,c) = B[c*K + k], bmm_permute_tiled.cl:74). */
int migemm_bmm_permute_tiled(void *stream, const float *A, const float *B, float *C,
                             int M, int K, int N,
                             int batch_stride_A, int batch_stride_B, int batch_stride_C,
                             int transA, int transB, int batch);

/* Replaces kernel linear_forward_tiled, cs/cl_kernels/linear.cl:14-24, enqueued by
 * NnClGlob.LinearForward (cs/compiler/NnClGlob.cs:1493-1551):
 * Y_b = X_b * W + bias, W [K,N] shared by every batch entry, bias [N] (never NULL). */
int migemm_linear_forward(void *stream, const float *X, const float *W,
                          const float *bias, float *Y,
                          int M, int K, int N,
                          int batch_stride_X, int batch_stride_Y, int batch);

/* Replaces kernel lstm_gemm_xw, cs/cl_kernels/lstm.cl:273-279, enqueued by
 * NnClGlob.Lstm (cs/compiler/NnClGlob.cs:877-899):
 * XW_out[T,G] = X[T,F] * W[F,G] + bias[G]. */
int migemm_lstm_gemm_xw(void *stream, const float *X, const float *W,
                        const float *bias, float *XW_out,
                        int total_tokens, int in_features, int total_gates);

/* Replaces kernel lstm_gemm_grad_x, cs/cl_kernels/lstm.cl:372-376, enqueued by
 * NnClGlob.LstmBackward (cs/compiler/NnClGlob.cs:967-994):
 * grad_X[T,F] = all_grad_gates[T,G] * W^T with W stored [F,G] (G = 4 * hidden). */
int migemm_lstm_gemm_grad_x(void *stream, const float *all_grad_gates, const float *W,
                            float *grad_X, int total_tokens, int in_features, int total_gates);

/* Replaces kernel lstm_gemm_grad_weights, cs/cl_kernels/lstm.cl:459-468, enqueued by
 * NnClGlob.LstmBackward (cs/compiler/NnClGlob.cs:996-1024). Tokens are ordered
 * [batch_size][seq_len], T = batch_size * seq_len, G = 4 * hidden_size. Accumulates:
 *   grad_W[F,G]  += X[T,F]^T * all_grad_gates[T,G]
 *   grad_U[H,G]  += H_prev[T,H]^T * all_grad_gates, H_prev[t] = H_out[t-1] when
 *                   t % seq_len > 0, else 0 (each sequence's first step has no h_{t-1})
 *   grad_bias[G] += column sums of all_grad_gates
 * The three outputs must not overlap each other or the inputs. */
int migemm_lstm_gemm_grad_weights(void *stream, const float *X, const float *H_out,
                                  const float *all_grad_gates, float *grad_W, float *grad_U,
                                  float *grad_bias, int batch_size, int seq_len,
                                  int in_features, int hidden_size);

/* The recurrent product of one timestep inside kernel lstm_recurrent_forward,
 * cs/cl_kernels/lstm.cl:80-101 (enqueued by NnClGlob.Lstm, cs/compiler/NnClGlob.cs:912-928),
 * as a GEMM over the whole batch, in place on the step's slice of XW:
 *   XW[b, t, g] += sum_h H_out[b, t-1, h] * U[h, g]     for b < batch_size, g < 4*hidden
 * XW [batch_size, seq_len, 4*hidden] (X*W + bias from lstm_gemm_xw), H_out
 * [batch_size, seq_len, hidden], U [hidden, 4*hidden]. Afterwards XW[b, t, :] holds the
 * step's raw gates, which the reference kernel stores in its workspace
 * (workspace[(t*batch + b)*5H + g], lstm.cl:103-106) before applying the activations.
 * At t == 0 the previous hidden state is zero (lstm.cl:57-60) and XW is left unchanged. */
int migemm_lstm_recurrent_gates(void *stream, float *XW, const float *H_out, const float *U,
                                int batch_size, int seq_len, int hidden_size, int t);

/* The gate product of one timestep of kernel lstm_hid_forward, cs/cl_kernels/lstm.cl:788-870
 * (gate loop :832-844), enqueued by NnClGlob.LstmWithWithState
 * (cs/compiler/NnClGlob.cs:1067-1100) for layers/LSTMStateful.cs: with x, h, W and U as four
 * separate buffers, in one launch where the panel kernel applies (no x||h concatenation):
 *   workspace[t, b, g] = bias[g] + sum_i X[b, t, i] * W[i, g] + sum_h hp[b, h] * U[h, g]
 * for b < batch_size, g < 4*hidden_size, with hp = H_prev [batch_size, hidden_size] at t == 0
 * (the chunk's incoming state, lstm.cl:821) and hp[b] = H_out[b, t-1, :] after (the previous
 * step's output, lstm.cl:861). X [batch_size, seq_len, in_features], W [in_features, 4H],
 * U [hidden_size, 4H], bias [4H], H_out [batch_size, seq_len, hidden_size], workspace
 * [seq_len, batch_size, 4H] (the reference's gate buffer); only workspace[t] is written.
 * H_prev is read only at t == 0 and H_out only at t > 0: the other may be NULL. The
 * reference adds the bias first and the products in one fp32 chain (lstm.cl:833-843); this
 * sums the products by MFMA and adds the bias after them, within the tolerance above. The
 * activations and the cell update that follow in the reference kernel are not part of
 * this library (a caller applies them between steps). */
int migemm_lstm_hid_gates(void *stream, const float *X, const float *W, const float *U,
                          const float *bias, const float *H_prev, const float *H_out,
                          float *workspace, int batch_size, int seq_len, int in_features,
                          int hidden_size, int t);

/* Replaces kernel tensor_permute, cl_kernels/permute.cl:11-18, enqueued by
 * NnClGlob.Permute (cs/compiler/NnClGlob.cs:382-424) and nncl_glob.py:148-174.
 * dst = src.permute(axes); src_dims and axes are HOST int arrays of length num_dims
 * (1..10) -- the reference builds three device buffers from them on every call
 * (NnClGlob.cs:402-405); here they travel in the kernel arguments. */
int migemm_tensor_permute(void *stream, const float *src, float *dst,
                          const int *src_dims, const int *axes, int num_dims);

/* Replaces kernel linear_bias_backward, cs/cl_kernels/linear.cl:149-153, enqueued by
 * NnClGlob.LinearBiasBackward (cs/compiler/NnClGlob.cs:1557-1584):
 * grad_bias[n] = sum over r < total_rows of grad_output[r*N + n]. Summed r ascending
 * within chunks of 256 rows, the chunk sums added in chunk order: the reference's single
 * ascending chain (bit-identical) when total_rows <= 256, deterministic beyond. */
int migemm_linear_bias_backward(void *stream, const float *grad_output, float *grad_bias,
                                int total_rows, int N);

/* Replaces kernel reduce_sum_axis, cs/cl_kernels/reduce_sum_axis.cl:3-8, enqueued by
 * NnClGlob.Sum (cs/compiler/NnClGlob.cs:1595-1664):
 * Y[o, i] = sum over a < axis_size of X[(o*axis_size + a)*inner_size + i], in the order
 * of migemm_linear_bias_backward (the reference's ascending chain up to 256). */
int migemm_reduce_sum_axis(void *stream, const float *X, float *Y,
                           int outer_size, int axis_size, int inner_size);

/* Weight gradient of LinearOp.Backward (cs/core/LinearOp.cs:35-39):
 * dW[K,N] = sum_b X_b^T * dY_b for X [batch,M,K], dY [batch,M,N] contiguous.
 * The reference materialises BmmPermute(x, dY, transA) [batch,K,N] and then
 * Sum(axis 0); this runs one TN GEMM whose contraction runs over batch*M rows. */
int migemm_linear_weight_grad(void *stream, const float *X, const float *dY, float *dW,
                              int M, int K, int N, int batch);

/* ------------------------------------------------------------------------------- */
/* (3) Device, memory and stream services that replace the OpenCL context, queue
 *     registry, buffer manager and host read-back used by the reference host
 *     (cs/core/ComputeContext.cs:35-155, cs/core/DeviceQueueRegistry.cs:14-37,
 *     cs/compiler/OpenCLBufferManager.cs:22-88, cs/compiler/HostReturner.cs:17-74). */

/* Number of visible HIP devices (0 when there is none). */
int migemm_device_count(int *count);
/* Select the device used by later calls on this host thread. */
int migemm_set_device(int device);
/* Name (e.g. "gfx950"), compute-unit count and global memory of a device. */
int migemm_device_info(int device, char *arch_name, size_t arch_name_len,
                       int *compute_units, size_t *global_mem_bytes);
int migemm_malloc(void **ptr, size_t bytes);
int migemm_free(void *ptr);
int migemm_memcpy_h2d(void *stream, void *dst, const void *src, size_t bytes);
int migemm_memcpy_d2h(void *stream, void *dst, const void *src, size_t bytes);
int migemm_memset(void *stream, void *dst, int value, size_t bytes);
int migemm_stream_create(void **stream);
/* Frees the library workspace held for the stream (see migemm_workspace_release), stops
 * treating it as a registered queue (migemm_queue_register_current; a thread that still
 * names it as its current queue must not compute on it), waits for its queued work and
 * destroys it. */
int migemm_stream_destroy(void *stream);
int migemm_stream_synchronize(void *stream);

/* Library workspace. Split-K GEMMs, sliced GEMVs and long column sums keep fp32 partial
 * sums in device memory that the library owns: one growing buffer per (device, stream),
 * plus one for operands an entry point stages (lstm_gemm_grad_weights' H_prev), so calls
 * on different streams never share partial sums. The reference host has no counterpart
 * (its kernels never split K). The buffers come from a device memory pool of the library
 * in the stream's order, and an outgrown or released buffer is freed in the stream's order
 * (after the queued work that uses it): neither waits on the host.
 * Nothing is allocated while a stream is being captured into a HIP graph, and a capturing
 * stream uses only its own buffers: size them before the capture, with this call or by
 * running the same calls once on that stream. A call that needs more during a capture
 * fails with MIGEMM_ERR_WORKSPACE. A buffer that a graph captured lives until the process
 * ends and is no longer used by eager calls after the capture (the next eager call on the
 * stream gets a new one), so replaying the graph on another stream cannot race with them. */
/* Grows each of `stream`'s two workspace buffers (the stream's device) to >= bytes. */
int migemm_workspace_reserve(void *stream, size_t bytes);
/* Frees the stream's workspace buffers in the stream's order (the work queued so far still
 * uses them), except those a HIP graph captured. */
int migemm_workspace_release(void *stream);
/* Current size of `stream`'s partial-sum buffer (0 if none). */
int migemm_workspace_size(void *stream, size_t *bytes);
/* Message of the last failing call on this host thread ("" if none). */
const char *migemm_last_error(void);
/* Library version, e.g. "0.1.0". */
const char *migemm_version(void);

/* ------------------------------------------------------------------------------- */
/* (3b) The reference host's runtime objects on HIP, for a host that keeps its object model:
 *      a device context, the name-keyed buffer pool behind Tensor.DataBuffer and the
 *      per-thread current queue. Buffers are HIP device memory, the pointers the compute
 *      entry points take; queues are HIP streams (migemm_stream_create). */

/* Replaces new ComputeContext(preferAccelerator: true) (cs/core/ComputeContext.cs:35-159):
 * device -1 takes the first visible gfx950 device (the reference takes the first
 * accelerator / GPU of the first platform, :53-96; these kernels are built for gfx950
 * only), device >= 0 that device, which must be a gfx950. MIGEMM_ERR_NO_DEVICE when there
 * is none (the reference's InvalidOperationException, :92-93). */
int migemm_context_create(int device, void **ctx);
/* Replaces ComputeContext.Dispose (:161-170): frees every pooled buffer of the context and
 * clears this thread's current queue if it names the context. */
int migemm_context_destroy(void *ctx);
/* The device parameters ComputeContext exposes (:13-25, derived at :108-156): device index,
 * architecture name, compute units, wavefront size (warp_size), MAX_WORK_GROUP_SIZE and the
 * work-group shape MAX_WORK_GPOUP_SIZE_X / _Y the reference derives from them (Y = warp/8,
 * X = MAX/Y), global memory. Any output pointer may be NULL. */
int migemm_context_info(void *ctx, int *device, char *arch_name, size_t arch_name_len,
                        int *compute_units, int *wavefront_size, int *max_work_group_size,
                        int *work_group_x, int *work_group_y, size_t *global_mem_bytes);

/* Replaces OpenCLBufferManager.GetOrCreateBuffer (cs/compiler/OpenCLBufferManager.cs:22-61):
 * the device buffer called `name` if it belongs to `ctx` and holds >= bytes; otherwise a
 * buffer of exactly `bytes` is allocated on the context's device and the old one (if any)
 * is released. A released buffer is freed once the work queued before the release on every
 * registered queue of its device (and on the null stream) has run, as an OpenCL buffer
 * outlives its release until the kernels using it finish; the caller never waits for that.
 * Lookups that find their buffer run in parallel across threads. Errors as the reference's:
 * null context, empty name, zero size (:24-26); a handle of a destroyed context is rejected
 * on every thread. */
int migemm_buffer_get_or_create(void *ctx, const char *name, size_t bytes, void **ptr);
/* Replaces OpenCLBufferManager.ReleaseBuffer (:66-75); an unknown name is not an error. */
int migemm_buffer_release(const char *name);
/* Replaces OpenCLBufferManager.DisposeAll (:81-91). */
int migemm_buffer_release_all(void);
/* Number of pooled buffers and their total size (either pointer may be NULL). */
int migemm_buffer_count(size_t *count, size_t *total_bytes);

/* Replaces DeviceQueueRegistry.RegisterCurrent (cs/core/DeviceQueueRegistry.cs:19-22): the
 * calling thread's current queue is `stream` of `ctx`; a null stream is rejected (:21), and
 * so is a stream of another device than the context's. */
int migemm_queue_register_current(void *ctx, void *stream);
/* Replaces DeviceQueueRegistry.GetCurrent (:28-38): MIGEMM_ERR_NO_QUEUE when this thread has
 * registered none, MIGEMM_ERR_INVALID_ARG when its context has been destroyed (by any
 * thread). Either output may be NULL. */
int migemm_queue_get_current(void **ctx, void **stream);
/* Replaces DeviceQueueRegistry.Clear (:43-46). */
int migemm_queue_clear_current(void);
/* Replaces the Tensor.DataBuffer getter (cs/core/Tensor.cs:41): the pooled buffer named
 * tensor_id of the current queue's context (migemm_buffer_get_or_create), bytes =
 * 4 * Size. MIGEMM_ERR_NO_QUEUE when this thread has registered no queue. */
int migemm_tensor_buffer(const char *tensor_id, size_t bytes, void **ptr);

/* ------------------------------------------------------------------------------- */
/* (4) Kernel selection. The reference has one kernel per form (cl_kernels/matmul.cl:8,
 *     :78; cs/cl_kernels/bmm_permute_tiled.cl:7); this library chooses per shape among
 *     kernel families. The policy is process-wide and exists for tests and tuning:
 *     every policy computes the same product within the fp32 tolerance, only the kernel
 *     family (and so the association order of the sums) changes. */
#define MIGEMM_POLICY_AUTO 0   /* choice by shape (default) */
#define MIGEMM_POLICY_TILED 1  /* LDS-tiled 32x32x2 MFMA kernel (+ split-K) for every shape */
#define MIGEMM_POLICY_SMALL 2  /* k-split 16x16x4 MFMA small-output kernel for every shape */
#define MIGEMM_POLICY_SKINNY 3 /* fp32-FMA streaming kernels wherever they apply (M <= 4;
                                  B transposed: whole rows of B per wavefront), otherwise
                                  the AUTO choice */
#define MIGEMM_POLICY_PANEL 4  /* 32x32-tile panel kernel wherever it applies (any layout,
                                  K % 32 == 0, N % 4 == 0, M % 4 == 0 when A is
                                  transposed, 16-byte aligned rows, lda and ldb <= 2^25),
                                  otherwise the AUTO choice */
#define MIGEMM_POLICY_TINY 5   /* 16x16 tiles of 1, 2 or 4 wavefronts with all operands in
                                  registers wherever it applies (K <= 80, or K = 96, 128,
                                  160, 192, 256, 320), otherwise the AUTO choice */
/* Sets the policy; *previous (if not NULL) receives the one it replaces. Calls already
 * enqueued are unaffected. */
int migemm_set_gemm_policy(int policy, int *previous);

/* Tuning overrides of the dispatcher, process-wide, for tests and tuning sweeps; every
 * value computes the same product within the fp32 tolerance. 0 (the initial value of every
 * key) leaves the choice to the dispatcher. No other input (no environment variable)
 * changes which kernel runs. */
#define MIGEMM_TUNE_TILE 1         /* tiled kernel's output tile: 32, 64, 128, 256 (256x256)
                                      or MIGEMM_TILE_128x256 */
#define MIGEMM_TUNE_SPLITK 2       /* tiled kernel's k ranges: S in 1..64 */
#define MIGEMM_TUNE_DIRECT 3       /* operands loaded straight into LDS: 1 never,
                                      2 wherever the kernel applies (also split 128x256) */
#define MIGEMM_TUNE_SMALL_TILES 4  /* small-output kernel's 32x32 tiles: 1 never,
                                      2 always (M, N > 16) */
#define MIGEMM_TUNE_SMALL_SPLITK 5 /* small-output kernel's k ranges: S in 1..64 */
#define MIGEMM_TILE_128x256 128256
int migemm_set_tuning(int key, int value, int *previous);

/* Writes a one-line description of the kernel the last GEMM / permute / column-sum call of
 * this host thread ran (family, output tile, k ranges, load width, shape, layout) into
 * buf (NUL-terminated, truncated to len). For tests and tuning; the reference has none. */
int migemm_last_plan(char *buf, size_t len);

/* (5) Measurement. Streams src[0 .. n) once -- `blocks` work-groups, each a contiguous
 * range, 16-byte non-temporal loads -- and writes the sum of the b-th range to sums[b]. It
 * has no counterpart in the reference: it measures the read rate a kernel that only
 * streams reaches on the device, the ceiling the HBM-bound GEMV (M <= 4) is compared with.
 * n a positive multiple of 4, src 16-byte aligned, 1 <= blocks <= min(65535, n / 4). */
int migemm_stream_read(void *stream, const float *src, size_t n, float *sums, int blocks);

/* The plan migemm_gemm_strided_batched_ex would run for these arguments, written into
 * plan as by migemm_last_plan, without running it: the arguments are validated the same way
 * and the dispatcher makes every choice, but nothing is launched, no memory is touched or
 * allocated and no HIP call is made, so it works without a GPU. The pointers only take
 * part through their alignment and overlap checks. No counterpart in the reference: for
 * tests that pin the dispatcher's choices on the CPU. */
int migemm_gemm_plan(int transA, int transB, int M, int N, int K,
                     const float *A, int64_t lda, int64_t strideA,
                     const float *B, int64_t ldb, int64_t strideB,
                     const float *bias, float *C, int64_t ldc, int64_t strideC,
                     int batch, int flags, char *plan, size_t plan_len);

#ifdef __cplusplus
}
#endif

#endif /* MIGEMM_H */
