/* Runs every function of the CPU oracle (oracle/oracle.c) over edge-case shapes with each
 * buffer allocated to exactly the extent the function may touch, for the sanitizer build of
 * tests/test_sanitizers.py (AddressSanitizer + UndefinedBehaviorSanitizer): an access one
 * element past an operand, a signed overflow in an index or a misaligned access aborts the
 * run. The results themselves are checked elsewhere (tests/test_oracle.py); here only a few
 * cheap identities guard against the driver silently doing nothing. TEST INFRASTRUCTURE. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void oracle_fill_uniform(float *out, int64_t n, uint64_t seed, uint64_t tensor_id, double lo,
                         double hi);
void oracle_fill_normal(float *out, int64_t n, uint64_t seed, uint64_t tensor_id, double mean,
                        double std);
void oracle_bmm_tiled(const float *A, const float *B, float *C, int M, int K, int N, int sA,
                      int sB, int sC, int batch);
void oracle_matmul_tiled(const float *A, const float *B, float *C, int M, int K, int N);
void oracle_bmm_permute_tiled(const float *A, const float *B, float *C, int M, int K, int N,
                              int sA, int sB, int sC, int transA, int transB, int batch);
void oracle_linear_forward_tiled(const float *X, const float *W, const float *bias, float *Y,
                                 int M, int K, int N, int sX, int sY, int batch);
void oracle_lstm_gemm_xw(const float *X, const float *W, const float *bias, float *XW,
                         int total_tokens, int in_features, int total_gates);
void oracle_lstm_gemm_grad_x(const float *Gr, const float *W, float *gX, int total_tokens,
                             int in_features, int total_gates);
void oracle_lstm_gemm_grad_weights(const float *X, const float *Hout, const float *Gr,
                                   float *gW, float *gU, float *gB, int batch_size,
                                   int seq_len, int in_features, int hidden);
void oracle_lstm_recurrent_gates(const float *XW, const float *Hout, const float *U,
                                 float *gates, int batch_size, int seq_len, int hidden, int t);
void oracle_lstm_hid_gates(const float *X, const float *W, const float *U, const float *bias,
                           const float *Hprev, const float *Hout, float *gates, int batch_size,
                           int seq_len, int in_features, int hidden, int t);
void oracle_tensor_permute(const float *src, float *dst, const int *src_dims, const int *axes,
                           int num_dims);
void oracle_reduce_sum_axis(const float *X, float *Y, int outer, int axis, int inner);
void oracle_linear_bias_backward(const float *grad_output, float *grad_bias, int total_rows,
                                 int N);
void oracle_gemm_f64(int transA, int transB, int M, int N, int K, const float *A, int64_t lda,
                     int64_t sA, const float *B, int64_t ldb, int64_t sB, const float *bias,
                     double *C, int batch, int row0, int row1);
void oracle_gemm_absprod(int transA, int transB, int M, int N, int K, const float *A,
                         int64_t lda, int64_t sA, const float *B, int64_t ldb, int64_t sB,
                         const float *bias, double *C, int batch, int row0, int row1);
void oracle_matmul_rows(const float *A, const float *B, float *C, int M, int K, int N, int row0,
                        int row1, int threads);
int oracle_openmp_enabled(void);

static int failures = 0;
static uint64_t next_id = 0;

/* exactly n floats, seeded (n >= 1) */
static float *fv(int64_t n) {
    float *p = malloc((size_t)n * sizeof(float));
    if (!p) abort();
    oracle_fill_uniform(p, n, 7, next_id++, -1.0, 1.0);
    return p;
}

static double *dv(int64_t n) {
    double *p = malloc((size_t)n * sizeof(double));
    if (!p) abort();
    return p;
}

#define EXPECT(cond, ...)                                      \
    do {                                                       \
        if (!(cond)) {                                         \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                      \
            fprintf(stderr, "\n");                             \
            ++failures;                                        \
        }                                                      \
    } while (0)

static void gemms(int M, int K, int N, int batch) {
    /* bmm_tiled / matmul_tiled: A [batch, M, K], B [batch, K, N] (and a broadcast B) */
    float *A = fv((int64_t)batch * M * K), *B = fv((int64_t)batch * K * N),
          *B1 = fv((int64_t)K * N), *C = fv((int64_t)batch * M * N),
          *bias = fv(N);
    oracle_bmm_tiled(A, B, C, M, K, N, M * K, K * N, M * N, batch);
    oracle_bmm_tiled(A, B1, C, M, K, N, M * K, 0, M * N, batch);
    oracle_matmul_tiled(A, B1, C, M, K, N);
    for (int ta = 0; ta < 2; ++ta)
        for (int tb = 0; tb < 2; ++tb)
            oracle_bmm_permute_tiled(A, B, C, M, K, N, M * K, K * N, M * N, ta, tb, batch);
    oracle_linear_forward_tiled(A, B1, bias, C, M, K, N, M * K, M * N, batch);
    /* fp64 evaluation and |A||B| over all rows, then over the last row only */
    double *C64 = dv((int64_t)batch * M * N);
    for (int ta = 0; ta < 2; ++ta)
        for (int tb = 0; tb < 2; ++tb) {
            const int64_t lda = ta ? M : K, ldb = tb ? K : N;
            oracle_gemm_f64(ta, tb, M, N, K, A, lda, (int64_t)M * K, B, ldb, (int64_t)K * N,
                            bias, C64, batch, 0, M);
            oracle_gemm_absprod(ta, tb, M, N, K, A, lda, (int64_t)M * K, B, ldb,
                                (int64_t)K * N, bias, C64, batch, M - 1, M);
            EXPECT(C64[0] >= 0.0, "absprod is negative");
        }
    oracle_matmul_rows(A, B1, C, M, K, N, 0, M, 1);
    oracle_matmul_rows(A, B1, C, M, K, N, M / 2, M, 4);
    free(A), free(B), free(B1), free(C), free(bias), free(C64);
}

static void lstm(int batch, int seq, int F, int H) {
    const int T = batch * seq, G = 4 * H;
    float *X = fv((int64_t)T * F), *W = fv((int64_t)F * G), *U = fv((int64_t)H * G),
          *bias = fv(G), *XW = fv((int64_t)T * G), *Hout = fv((int64_t)T * H),
          *Gr = fv((int64_t)T * G), *gX = fv((int64_t)T * F), *gW = fv((int64_t)F * G),
          *gU = fv((int64_t)H * G), *gB = fv(G), *gates = fv((int64_t)batch * G),
          *Hprev = fv((int64_t)batch * H);
    oracle_lstm_gemm_xw(X, W, bias, XW, T, F, G);
    oracle_lstm_gemm_grad_x(Gr, W, gX, T, F, G);
    oracle_lstm_gemm_grad_weights(X, Hout, Gr, gW, gU, gB, batch, seq, F, H);
    for (int t = 0; t < seq; ++t) {
        oracle_lstm_recurrent_gates(XW, Hout, U, gates, batch, seq, H, t);
        oracle_lstm_hid_gates(X, W, U, bias, Hprev, Hout, gates, batch, seq, F, H, t);
    }
    free(X), free(W), free(U), free(bias), free(XW), free(Hout), free(Gr), free(gX), free(gW),
        free(gU), free(gB), free(gates), free(Hprev);
}

static void permute(int nd, const int *dims, const int *axes) {
    int64_t n = 1;
    for (int i = 0; i < nd; ++i) n *= dims[i];
    float *src = fv(n), *dst = fv(n);
    oracle_tensor_permute(src, dst, dims, axes, nd);
    /* a permutation moves values without changing them: the sums agree */
    double s0 = 0, s1 = 0;
    for (int64_t i = 0; i < n; ++i) s0 += src[i], s1 += dst[i];
    EXPECT(fabs(s0 - s1) < 1e-3, "permute changed the values (%g vs %g)", s0, s1);
    free(src), free(dst);
}

static void reductions(int outer, int axis, int inner) {
    float *X = fv((int64_t)outer * axis * inner), *Y = fv((int64_t)outer * inner);
    oracle_reduce_sum_axis(X, Y, outer, axis, inner);
    float *gb = fv(inner);
    oracle_linear_bias_backward(X, gb, outer * axis, inner);
    free(X), free(Y), free(gb);
}

int main(void) {
    const int shapes[][4] = {{1, 1, 1, 1}, {17, 33, 5, 1}, {16, 16, 16, 2}, {65, 31, 129, 1},
                             {3, 47, 29, 3}, {64, 64, 64, 1}, {1, 100, 1, 4}, {33, 1, 17, 2}};
    for (size_t i = 0; i < sizeof(shapes) / sizeof(shapes[0]); ++i)
        gemms(shapes[i][0], shapes[i][1], shapes[i][2], shapes[i][3]);
    const int lstms[][4] = {{1, 1, 1, 1}, {3, 4, 10, 12}, {2, 5, 33, 20}, {4, 2, 16, 16}};
    for (size_t i = 0; i < sizeof(lstms) / sizeof(lstms[0]); ++i)
        lstm(lstms[i][0], lstms[i][1], lstms[i][2], lstms[i][3]);
    const int d1[] = {7}, a1[] = {0};
    const int d2[] = {5, 9}, a2[] = {1, 0};
    const int d3[] = {3, 17, 29}, a3[] = {0, 2, 1};
    const int d4[] = {2, 3, 5, 7}, a4[] = {3, 1, 0, 2};
    const int d5[] = {2, 1, 4, 3, 5}, a5[] = {4, 0, 3, 1, 2};
    permute(1, d1, a1);
    permute(2, d2, a2);
    permute(3, d3, a3);
    permute(4, d4, a4);
    permute(5, d5, a5);
    reductions(1, 1, 1);
    reductions(3, 300, 7);
    reductions(2, 257, 33);
    float *u = fv(1001), *nrm = malloc(1001 * sizeof(float));
    oracle_fill_normal(nrm, 1001, 3, 1, 0.0, 1.0);
    double mean = 0;
    for (int i = 0; i < 1001; ++i) mean += u[i];
    EXPECT(fabs(mean / 1001) < 0.2, "uniform fill mean %g", mean / 1001);
    free(u), free(nrm);
    printf("oracle_san: %s (openmp %d)\n", failures ? "FAILED" : "ok", oracle_openmp_enabled());
    return failures ? 1 : 0;
}
