/*
 * oracle.c -- CPU restatement of the reference matmul path. TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker, never the product: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it. The shipped library (libmigemm.so) has no CPU
 * fallback and never calls into this code.
 *
 * Paths are relative to the reference repository; "cs/" = csharp/cstorchcl/cstorchcl/.
 *
 * What is restated, and how each function is pinned (tests/test_oracle.py):
 *  - oracle_matmul_tiled / oracle_bmm_tiled follow cl_kernels/matmul.cl:8-71 / :78-135:
 *    one fp32 accumulator per output starting at +0.0f, ceil(K/16) tiles of 16 k, out of
 *    range operands zero-filled (:37-52, :108-120), acc = fma(a, b, acc) in ascending k
 *    (OpenCL C contracts `acc += a*b` to an fma by default, :60 / :126), guarded store
 *    (:68-70, :132-134). Pinned by exact small-integer / identity / ones / rank-1 / probe
 *    known-answer tests, by brute force against an fp64 triple loop on every shape 1..33,
 *    and by the fp64 tolerance bound on the reference test shapes.
 *  - oracle_bmm_permute_tiled follows cs/cl_kernels/bmm_permute_tiled.cl:7-122: the same
 *    per-output fma chain over 16-wide k tiles with the transposed index formulas
 *    (A[k*M + r] :59, B[c*K + k] :74). Pinned by NT(A,B) == NN(A, B^T) and TN(A,B) ==
 *    NN(A^T, B) bit-for-bit and by the known-answer tests.
 *  - oracle_linear_forward_tiled / oracle_lstm_gemm_xw follow cs/cl_kernels/linear.cl:14-144
 *    and cs/cl_kernels/lstm.cl:273-367: the fma chain, then ONE fp32 add of bias[n] after
 *    the k loop (linear.cl:119-122, lstm.cl:356). Pinned by == bmm + row-broadcast add.
 *  - oracle_lstm_gemm_grad_x / oracle_lstm_gemm_grad_weights follow cs/cl_kernels/lstm.cl:
 *    372-457 / 459-636: fma chains over 16-wide zero-padded tiles, the weight gradients
 *    accumulated onto the old value (old + chain), grad_U's left operand the previous
 *    step's hidden state of the same sequence (zero at each sequence's first step). Pinned
 *    by the reference kernels themselves on the GPU (tests/test_reference_gpu.py), by exact
 *    small-integer products against independent numpy constructions, and by
 *    grad_x == bmm_permute_tiled(G, W, transB) bit for bit.
 *  - oracle_lstm_recurrent_gates follows the recurrent product of
 *    cs/cl_kernels/lstm.cl:80-101: the step's XW value as the accumulator's start, then an
 *    fma chain over h ascending of h_{t-1}[h] * U[h][g]. Pinned by the reference kernel's
 *    own stored gates (lstm_recurrent_forward's workspace, tests/test_reference_gpu.py and
 *    the committed fixture tests/golden/reference_outputs.npz), by exact small-integer
 *    products against an independent numpy construction, and by a planted mistake (the
 *    hidden state of step t instead of t-1) that the known answers reject.
 *  - oracle_lstm_hid_gates follows the gate loop of lstm_hid_forward,
 *    cs/cl_kernels/lstm.cl:826-844: the accumulator starts at bias[g], then one fma chain
 *    over the step's input row against W (i ascending) continued over h_{t-1} against U (h
 *    ascending); h_{t-1} is H_prev at t == 0, else the kernel's own previous output. Pinned
 *    by the reference kernel's stored gates (its workspace, tests/test_reference_gpu.py and
 *    the committed fixture tests/golden/reference_outputs.npz), by exact small-integer
 *    answers against an independent numpy construction, and by planted mistakes (bias
 *    added last, h_t instead of h_{t-1}, the U chain before the W chain) that the fixture
 *    rejects.
 *  - oracle_tensor_permute follows cl_kernels/permute.cl:11-50. Pinned by numpy.transpose.
 *  - oracle_reduce_sum_axis / oracle_linear_bias_backward follow
 *    cs/cl_kernels/reduce_sum_axis.cl:3-24 and cs/cl_kernels/linear.cl:149-168: sequential
 *    fp32 sum from +0.0f in ascending order. Pinned by exact integer sums and by
 *    numpy's float32 cumulative sum (same order).
 *  - oracle_gemm_f64 evaluates the same contraction in double precision (the accuracy
 *    reference); oracle_gemm_absprod its |A|*|B| (componentwise error denominator).
 *    Pinned against numpy float64 matmul.
 *  - oracle_fill_uniform / oracle_fill_normal: the synthetic input generator shared with
 *    numpy (oracle/__init__.py). Pinned by golden values in tests/golden/ and by the
 *    numpy mirror.
 *
 * Build (gcc only, no GPU): see oracle/Makefile. Compiled with -ffp-contract=off so that
 * the only fused operations are the explicit fmaf() calls.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define REF_TILE 16 /* TILE_SIZE of matmul.cl:1 and TILE_K of bmm_permute_tiled.cl:5 */

/* ------------------------------------------------------------------------------------ */
/* Generator: counter-based SplitMix64 of (seed, tensor_id, index).                      */

static uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t tensor_id) {
    return splitmix64(splitmix64(seed) ^ (tensor_id * 0xD1B54A32D192ED03ULL));
}

/* Uniform in [lo, hi): top 24 bits -> u in [0,1) (exact in fp32), then lo + (hi-lo)*u
 * evaluated in double and rounded once to float. */
void oracle_fill_uniform(float *out, int64_t n, uint64_t seed, uint64_t tensor_id, double lo,
                         double hi) {
    const uint64_t key = stream_key(seed, tensor_id);
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t r = splitmix64(key + (uint64_t)i);
        const double u = (double)(r >> 40) * (1.0 / 16777216.0);
        out[i] = (float)(lo + (hi - lo) * u);
    }
}

/* Normal(mean, std) by Box-Muller in double: element i uses the 64-bit draw at counter i
 * (two 26-bit fractions), and only the cosine branch, so every element is independent of
 * n. */
void oracle_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t tensor_id, double mean,
                        double std) {
    const uint64_t key = stream_key(seed, tensor_id);
    const double two_pi = 6.283185307179586476925286766559;
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t r = splitmix64(key + (uint64_t)i);
        const double u1 = ((double)(r >> 38) + 0.5) * (1.0 / 67108864.0); /* (0,1) */
        const double u2 = (double)((r >> 12) & 0x3FFFFFFULL) * (1.0 / 67108864.0);
        const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)(mean + std * z);
    }
}

/* ------------------------------------------------------------------------------------ */
/* Reference kernels, restated per output element.                                      */

/* matmul.cl:78-135 (bmm_tiled) for batch entry z; matmul_tiled is batch 1, strides 0. */
static void bmm_tiled_one(const float *A, const float *B, float *C, int M, int K, int N,
                          int row, int col) {
    float acc = 0.0f;
    const int num_tiles = (K + REF_TILE - 1) / REF_TILE;
    for (int t = 0; t < num_tiles; ++t) {
        for (int k = 0; k < REF_TILE; ++k) {
            const int kk = t * REF_TILE + k;
            /* Asub[row][k]: zero when out of range (matmul.cl:109-113) */
            const float a = (row < M && kk < K) ? A[(int64_t)row * K + kk] : 0.0f;
            /* Bsub[k][col]: zero when out of range (matmul.cl:116-120) */
            const float b = (kk < K && col < N) ? B[(int64_t)kk * N + col] : 0.0f;
            acc = fmaf(a, b, acc);
        }
    }
    C[(int64_t)row * N + col] = acc;
}

void oracle_bmm_tiled(const float *A, const float *B, float *C, int M, int K, int N, int sA,
                      int sB, int sC, int batch) {
    for (int z = 0; z < batch; ++z) {
        const float *a = A + (int64_t)z * sA;
        const float *b = B + (int64_t)z * sB;
        float *c = C + (int64_t)z * sC;
        for (int row = 0; row < M; ++row)
            for (int col = 0; col < N; ++col) bmm_tiled_one(a, b, c, M, K, N, row, col);
    }
}

void oracle_matmul_tiled(const float *A, const float *B, float *C, int M, int K, int N) {
    oracle_bmm_tiled(A, B, C, M, K, N, 0, 0, 0, 1);
}

/* bmm_permute_tiled.cl:46-99 for one output element: the 64x64 tile / 4x4 register block
 * only distributes outputs; each accumulator is its own fma chain over ascending k. */
static float permute_chain(const float *A, const float *B, int M, int K, int N, int r, int c,
                           int transA, int transB) {
    float acc = 0.0f;
    const int num_tiles = (K + REF_TILE - 1) / REF_TILE;
    for (int t = 0; t < num_tiles; ++t) {
        for (int k = 0; k < REF_TILE; ++k) {
            const int kk = t * REF_TILE + k;
            float a = 0.0f, b = 0.0f;
            if (r < M && kk < K) a = transA ? A[(int64_t)kk * M + r] : A[(int64_t)r * K + kk];
            if (kk < K && c < N) b = transB ? B[(int64_t)c * K + kk] : B[(int64_t)kk * N + c];
            acc = fmaf(a, b, acc);
        }
    }
    return acc;
}

void oracle_bmm_permute_tiled(const float *A, const float *B, float *C, int M, int K, int N,
                              int sA, int sB, int sC, int transA, int transB, int batch) {
    for (int z = 0; z < batch; ++z) {
        const float *a = A + (int64_t)z * sA;
        const float *b = B + (int64_t)z * sB;
        float *cz = C + (int64_t)z * sC;
        for (int r = 0; r < M; ++r)
            for (int c = 0; c < N; ++c)
                cz[(int64_t)r * N + c] = permute_chain(a, b, M, K, N, r, c, transA != 0, transB != 0);
    }
}

/* linear.cl:14-144: fma chain (W shared by every batch entry), then acc + bias[c]. */
void oracle_linear_forward_tiled(const float *X, const float *W, const float *bias, float *Y,
                                 int M, int K, int N, int sX, int sY, int batch) {
    for (int z = 0; z < batch; ++z) {
        const float *x = X + (int64_t)z * sX;
        float *y = Y + (int64_t)z * sY;
        for (int r = 0; r < M; ++r)
            for (int c = 0; c < N; ++c) {
                const float acc = permute_chain(x, W, M, K, N, r, c, 0, 0);
                y[(int64_t)r * N + c] = acc + bias[c];
            }
    }
}

/* lstm.cl:273-367: identical arithmetic to linear_forward_tiled with batch 1. */
void oracle_lstm_gemm_xw(const float *X, const float *W, const float *bias, float *XW,
                         int total_tokens, int in_features, int total_gates) {
    oracle_linear_forward_tiled(X, W, bias, XW, total_tokens, in_features, total_gates, 0, 0, 1);
}

/* lstm.cl:372-457 (lstm_gemm_grad_x): grad_X[t][f] = fma chain over the gates k in
 * ascending, zero-padded 16-wide tiles of G[t][k] * W[f][k] (the tile WTsub[k][f] is read
 * from W[f*G + k], :413-419): the bmm_permute_tiled arithmetic with B transposed. */
void oracle_lstm_gemm_grad_x(const float *Gr, const float *W, float *gX, int total_tokens,
                             int in_features, int total_gates) {
    for (int t = 0; t < total_tokens; ++t)
        for (int f = 0; f < in_features; ++f)
            gX[(int64_t)t * in_features + f] =
                permute_chain(Gr, W, total_tokens, total_gates, in_features, t, f, 0, 1);
}

/* lstm.cl:459-636 (lstm_gemm_grad_weights), tokens t = b*seq_len + s in ascending,
 * zero-padded 16-wide tiles (:484, :497-517), each output its own fp32 chain from +0.0f:
 *   grad_W[f][c] = grad_W[f][c] + (fma chain of X[t][f] * G[t][c])              :518-560
 *   grad_bias[c] = grad_bias[c] + (plain sum of G[t][c], padded zeros included)  :524-575
 *   grad_U[h][c] = grad_U[h][c] + (fma chain of Hprev[t][h] * G[t][c]),
 *                  Hprev[t][h] = H_out[(t-1)*H + h] if t % seq_len > 0 else 0    :579-632 */
void oracle_lstm_gemm_grad_weights(const float *X, const float *Hout, const float *Gr,
                                   float *gW, float *gU, float *gB, int batch_size,
                                   int seq_len, int in_features, int hidden) {
    const int T = batch_size * seq_len, Gt = 4 * hidden;
    const int Tp = (T + REF_TILE - 1) / REF_TILE * REF_TILE;
    for (int f = 0; f < in_features; ++f)
        for (int c = 0; c < Gt; ++c) {
            float acc = 0.0f;
            for (int t = 0; t < Tp; ++t) {
                const float x = t < T ? X[(int64_t)t * in_features + f] : 0.0f;
                const float g = t < T ? Gr[(int64_t)t * Gt + c] : 0.0f;
                acc = fmaf(x, g, acc);
            }
            gW[(int64_t)f * Gt + c] = gW[(int64_t)f * Gt + c] + acc;
        }
    for (int c = 0; c < Gt; ++c) {
        float acc = 0.0f;
        for (int t = 0; t < Tp; ++t) acc = acc + (t < T ? Gr[(int64_t)t * Gt + c] : 0.0f);
        gB[c] = gB[c] + acc;
    }
    for (int h = 0; h < hidden; ++h)
        for (int c = 0; c < Gt; ++c) {
            float acc = 0.0f;
            for (int t = 0; t < Tp; ++t) {
                const float hv =
                    (t < T && t % seq_len > 0) ? Hout[(int64_t)(t - 1) * hidden + h] : 0.0f;
                const float g = t < T ? Gr[(int64_t)t * Gt + c] : 0.0f;
                acc = fmaf(hv, g, acc);
            }
            gU[(int64_t)h * Gt + c] = gU[(int64_t)h * Gt + c] + acc;
        }
}

/* lstm.cl:80-101 (inside lstm_recurrent_forward): the raw gates of step t of sequence b,
 *   acc = XW[(b*seq_len + t)*4H + g]                                            :82-87
 *   acc = fma(h_prev[h], U[h*4H + g], acc) for h = 0..H-1 ascending             :90-101
 * with h_prev = H_out[(b*seq_len + t-1)*H + h] (the previous step's hidden state, which the
 * kernel keeps in h_local, :122-123) and 0 at t == 0 (:57-60). The kernel stores acc in
 * workspace[(t*batch + b)*5H + g] (:103-106); gates[b*4H + g] receives it here. */
void oracle_lstm_recurrent_gates(const float *XW, const float *Hout, const float *U,
                                 float *gates, int batch_size, int seq_len, int hidden, int t) {
    const int Gt = 4 * hidden;
    for (int b = 0; b < batch_size; ++b)
        for (int g = 0; g < Gt; ++g) {
            float acc = XW[((int64_t)b * seq_len + t) * Gt + g];
            for (int h = 0; h < hidden; ++h) {
                const float hv = t > 0 ? Hout[((int64_t)b * seq_len + t - 1) * hidden + h] : 0.0f;
                acc = fmaf(hv, U[(int64_t)h * Gt + g], acc);
            }
            gates[(int64_t)b * Gt + g] = acc;
        }
}

/* The gate loop of lstm_hid_forward, cs/cl_kernels/lstm.cl:826-844, for one step t:
 *   x_offset  = b*(seq_len*in_features) + t*in_features                          :827
 *   ws_offset = t*(batch*4H) + b*4H                                               :828
 *   val = bias[g]                                                                 :833
 *   val = fma(X[x_offset + i], W[i*4H + g], val) for i = 0..in_features-1          :835-837
 *   val = fma(h_curr[h], U[h*4H + g], val)        for h = 0..hidden-1              :839-841
 *   workspace[ws_offset + g] = val                                                :843
 * (OpenCL C contracts `val += a*b` to an fma by default). h_curr is H_prev[b*H + h] at t == 0
 * (:819-822) and afterwards the previous step's hidden state, which the kernel also stores
 * as H_out[b*(seq_len*H) + (t-1)*H + h] (:861). gates[b*4H + g] receives val. */
void oracle_lstm_hid_gates(const float *X, const float *W, const float *U, const float *bias,
                           const float *Hprev, const float *Hout, float *gates, int batch_size,
                           int seq_len, int in_features, int hidden, int t) {
    const int Gt = 4 * hidden;
    /* Each gate's chain is the kernel's, in its order; the loops run g innermost so W and U
     * are read by rows (the chains of different g are independent). */
#pragma omp parallel for schedule(static)
    for (int b = 0; b < batch_size; ++b) {
        const float *x = X + (int64_t)b * seq_len * in_features + (int64_t)t * in_features;
        const float *hp = t == 0 ? Hprev + (int64_t)b * hidden
                                 : Hout + (int64_t)b * seq_len * hidden + (int64_t)(t - 1) * hidden;
        float *val = gates + (int64_t)b * Gt;
        for (int g = 0; g < Gt; ++g) val[g] = bias[g];
        for (int i = 0; i < in_features; ++i) {
            const float *w = W + (int64_t)i * Gt;
            for (int g = 0; g < Gt; ++g) val[g] = fmaf(x[i], w[g], val[g]);
        }
        for (int h = 0; h < hidden; ++h) {
            const float *u = U + (int64_t)h * Gt;
            for (int g = 0; g < Gt; ++g) val[g] = fmaf(hp[h], u[g], val[g]);
        }
    }
}

/* permute.cl:11-50: dst[tid] = src[src_index(permuted coords)], up to 10 dimensions. */
void oracle_tensor_permute(const float *src, float *dst, const int *src_dims, const int *axes,
                           int num_dims) {
    int64_t total = 1;
    int dst_dims[10];
    for (int i = 0; i < num_dims; ++i) {
        total *= src_dims[i];
        dst_dims[i] = src_dims[axes[i]];
    }
    for (int64_t tid = 0; tid < total; ++tid) {
        int64_t dst_coords[10], src_coords[10];
        int64_t rem = tid;
        for (int i = num_dims - 1; i >= 0; --i) {
            dst_coords[i] = rem % dst_dims[i];
            rem /= dst_dims[i];
        }
        for (int i = 0; i < num_dims; ++i) src_coords[axes[i]] = dst_coords[i];
        int64_t idx = 0, stride = 1;
        for (int i = num_dims - 1; i >= 0; --i) {
            idx += src_coords[i] * stride;
            stride *= src_dims[i];
        }
        dst[tid] = src[idx];
    }
}

/* reduce_sum_axis.cl:3-24: Y[o, i] = sum over a (ascending, from +0.0f). */
void oracle_reduce_sum_axis(const float *X, float *Y, int outer, int axis, int inner) {
    for (int o = 0; o < outer; ++o)
        for (int i = 0; i < inner; ++i) {
            float sum = 0.0f;
            const int64_t base = (int64_t)o * axis * inner + i;
            for (int a = 0; a < axis; ++a) sum += X[base + (int64_t)a * inner];
            Y[(int64_t)o * inner + i] = sum;
        }
}

/* linear.cl:149-168: grad_bias[col] = sum over rows (ascending, from +0.0f). */
void oracle_linear_bias_backward(const float *grad_output, float *grad_bias, int total_rows,
                                 int N) {
    oracle_reduce_sum_axis(grad_output, grad_bias, 1, total_rows, N);
}

/* ------------------------------------------------------------------------------------ */
/* fp64 accuracy reference (any layout), with the same operand conventions as the C ABI's
 * migemm_gemm_strided_batched. Row range [row0, row1) lets callers evaluate a sample. */
void oracle_gemm_f64(int transA, int transB, int M, int N, int K, const float *A, int64_t lda,
                     int64_t sA, const float *B, int64_t ldb, int64_t sB, const float *bias,
                     double *C, int batch, int row0, int row1) {
    (void)M; /* rows come from [row0, row1) */
    for (int z = 0; z < batch; ++z) {
        const float *a = A + (int64_t)z * sA;
        const float *b = B + (int64_t)z * sB;
        double *c = C + (int64_t)z * (int64_t)(row1 - row0) * N;
        for (int r = row0; r < row1; ++r) {
            double *crow = c + (int64_t)(r - row0) * N;
            for (int n = 0; n < N; ++n) crow[n] = 0.0;
            for (int k = 0; k < K; ++k) {
                const double av = transA ? a[(int64_t)k * lda + r] : a[(int64_t)r * lda + k];
                if (transB) {
                    for (int n = 0; n < N; ++n) crow[n] += av * (double)b[(int64_t)n * ldb + k];
                } else {
                    const float *brow = b + (int64_t)k * ldb;
                    for (int n = 0; n < N; ++n) crow[n] += av * (double)brow[n];
                }
            }
            if (bias != NULL)
                for (int n = 0; n < N; ++n) crow[n] += (double)bias[n];
        }
    }
}

/* |opA(A)| * |opB(B)| (+ |bias|) in fp64: the componentwise error denominator. */
void oracle_gemm_absprod(int transA, int transB, int M, int N, int K, const float *A,
                         int64_t lda, int64_t sA, const float *B, int64_t ldb, int64_t sB,
                         const float *bias, double *C, int batch, int row0, int row1) {
    (void)M; /* rows come from [row0, row1) */
    for (int z = 0; z < batch; ++z) {
        const float *a = A + (int64_t)z * sA;
        const float *b = B + (int64_t)z * sB;
        double *c = C + (int64_t)z * (int64_t)(row1 - row0) * N;
        for (int r = row0; r < row1; ++r) {
            double *crow = c + (int64_t)(r - row0) * N;
            for (int n = 0; n < N; ++n) crow[n] = 0.0;
            for (int k = 0; k < K; ++k) {
                const double av =
                    fabs((double)(transA ? a[(int64_t)k * lda + r] : a[(int64_t)r * lda + k]));
                for (int n = 0; n < N; ++n) {
                    const float bv = transB ? b[(int64_t)n * ldb + k] : b[(int64_t)k * ldb + n];
                    crow[n] += av * fabs((double)bv);
                }
            }
            if (bias != NULL)
                for (int n = 0; n < N; ++n) crow[n] += fabs((double)bias[n]);
        }
    }
}

/* ------------------------------------------------------------------------------------ */
/* CPU baseline: the matmul_tiled arithmetic (per output: fp32 fma chain over ascending k
 * from +0.0f; the zero-padded tail adds fma(0,0,acc) == acc) for rows [row0, row1),
 * evaluated i-k-j so the compiler vectorises across independent outputs. Results are
 * bit-identical to oracle_matmul_tiled. Threads split the rows (OpenMP when built with
 * it). */
void oracle_matmul_rows(const float *A, const float *B, float *C, int M, int K, int N, int row0,
                        int row1, int threads) {
    (void)M;
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1)
#else
    (void)threads;
#endif
    for (int r = row0; r < row1; ++r) {
        float *crow = C + (int64_t)(r - row0) * N;
        for (int n = 0; n < N; ++n) crow[n] = 0.0f;
        const float *arow = A + (int64_t)r * K;
        for (int k = 0; k < K; ++k) {
            const float av = arow[k];
            const float *brow = B + (int64_t)k * N;
            for (int n = 0; n < N; ++n) crow[n] = fmaf(av, brow[n], crow[n]);
        }
        /* the zero-padded k of the last 16-wide tile: fma(0, 0, acc) == acc + 0 (turns an
         * underflowed -0 into +0 exactly as the padded chain does) */
        if (K % REF_TILE != 0)
            for (int n = 0; n < N; ++n) crow[n] = crow[n] + 0.0f;
    }
}

int oracle_openmp_enabled(void) {
#if defined(_OPENMP)
    return 1;
#else
    return 0;
#endif
}
