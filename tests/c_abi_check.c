/* A plain C99 caller of libmigemm, with no torch and no Python: the way a non-Python host
 * (the reference's C# host through P/Invoke, cs/compiler/NnClGlob.cs) uses the library.
 *
 *   c_abi_check validate   argument checks only; needs no GPU
 *   c_abi_check gpu        device memory, copies and the GEMM entry points on GPU 0,
 *                          checked exactly against a CPU loop on small-integer operands
 *   c_abi_check runtime    the reference host's runtime objects on GPU 0: a context, the
 *                          name-keyed buffer pool, one registered queue per POSIX thread,
 *                          and Bmm -> BmmOp.Backward on pooled buffers with fresh names
 *
 * Exit status 0 on success; every failure prints what failed. */
#define _POSIX_C_SOURCE 200809L
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "migemm.h"

static int failures = 0;
static pthread_mutex_t failures_lock = PTHREAD_MUTEX_INITIALIZER;

#define CHECK(cond, ...)                              \
    do {                                              \
        if (!(cond)) {                                \
            pthread_mutex_lock(&failures_lock);       \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);             \
            fprintf(stderr, "\n");                    \
            ++failures;                               \
            pthread_mutex_unlock(&failures_lock);     \
        }                                             \
    } while (0)

/* Argument checks of every entry point; all of them fail before any HIP call, so no GPU is
 * needed. Run from several threads at once (each thread has its own last-error message). */
static void *validate_thread(void *arg) {
    float *fake = (float *)(uintptr_t)0x100000;
    (void)arg;
    CHECK(strlen(migemm_version()) > 0, "empty version");
    int rc = migemm_gemm_strided_batched(NULL, 0, 0, 0, 4, 4, fake, 4, 0, fake + 64, 4, 0, NULL,
                                         fake + 128, 4, 0, 1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "M = 0 gave %d", rc);
    CHECK(strstr(migemm_last_error(), "sizes must be >= 1") != NULL, "message for M = 0: %s",
          migemm_last_error());
    rc = migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, fake, 4, 0, fake, 4, 0, NULL, fake, 4,
                                     0, 1);
    CHECK(rc == MIGEMM_ERR_ALIAS, "aliased output gave %d", rc);
    rc = migemm_gemm_strided_batched(NULL, 2, 0, 4, 4, 4, fake, 4, 0, fake + 64, 4, 0, NULL,
                                     fake + 128, 4, 0, 1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "transA = 2 gave %d", rc);
    rc = migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, fake, 3, 0, fake + 64, 4, 0, NULL,
                                     fake + 128, 4, 0, 1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "lda < K gave %d", rc);
    rc = migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, fake, 4, 16, fake + 64, 4, 16, NULL,
                                     fake + 256, 4, 4, 2);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "overlapping batch entries of C gave %d", rc);
    rc = migemm_gemm_strided_batched(NULL, 0, 0, 1 << 30, 1 << 30, 4, fake, 4, 0, fake, 1 << 30,
                                     0, NULL, fake, (int64_t)1 << 40, 0, 1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "overflowing extent gave %d", rc);
    rc = migemm_gemm_strided_batched_ex(NULL, 0, 0, 4, 4, 4, fake, 4, 0, fake + 64, 4, 0, NULL,
                                        fake + 128, 4, 0, 1, 4);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "unknown flag gave %d", rc);
    rc = migemm_gemm_strided_batched_noalloc(NULL, 0, 0, 4, 4, 0, fake, 4, 0, fake + 64, 4, 0,
                                             NULL, fake + 128, 4, 0, 1, 0);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "noalloc K = 0 gave %d", rc);
    rc = migemm_bmm_tiled(NULL, fake, fake + 64, fake + 128, 4, 4, 4, -1, 0, 16, 2);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "negative stride gave %d", rc);
    rc = migemm_bmm_permute_tiled(NULL, fake, fake + 64, fake + 128, 4, 4, 4, 16, 16, -16, 1, 0, 2);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "negative C stride gave %d", rc);
    rc = migemm_linear_forward(NULL, fake, fake + 64, NULL, fake + 128, 4, 4, 4, 16, 16, 1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "linear_forward without bias gave %d", rc);
    rc = migemm_lstm_gemm_xw(NULL, fake, fake + 64, NULL, fake + 128, 4, 4, 4);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "lstm_gemm_xw without bias gave %d", rc);
    rc = migemm_lstm_gemm_grad_weights(NULL, fake, fake + 64, fake + 128, fake + 256, fake + 256,
                                       fake + 512, 2, 3, 4, 5);
    CHECK(rc == MIGEMM_ERR_ALIAS, "grad_weights with overlapping outputs gave %d", rc);
    rc = migemm_lstm_recurrent_gates(NULL, fake, fake + 4096, fake + 8192, 2, 3, 4, 3);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "recurrent step 3 of 3 gave %d", rc);
    rc = migemm_lstm_hid_gates(NULL, fake, fake + 4096, fake + 8192, fake + 12288, NULL,
                               fake + 16384, fake + 20480, 2, 3, 4, 5, 0);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "hid gates with no H_prev at step 0 gave %d", rc);
    /* step 1's gates (batch 2 x 20 gates, from workspace + 40) start where H_out starts */
    rc = migemm_lstm_hid_gates(NULL, fake, fake + 4096, fake + 8192, fake + 12288, fake + 16384,
                               fake + 20480, fake + 20440, 2, 3, 4, 5, 1);
    CHECK(rc == MIGEMM_ERR_ALIAS, "hid gates over H_out gave %d", rc);
    rc = migemm_lstm_hid_gates(NULL, fake, fake + 4096, fake + 8192, fake + 12288, fake + 16384,
                               fake + 20480, fake + 40960, 2, 3, 4, 5, -1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "hid gates step -1 gave %d", rc);
    {
        int dims[3] = {2, 3, 4}, axes[3] = {0, 2, 2};
        rc = migemm_tensor_permute(NULL, fake, fake + 64, dims, axes, 3);
        CHECK(rc == MIGEMM_ERR_INVALID_ARG, "axes with a repeat gave %d", rc);
        axes[2] = 1;
        rc = migemm_tensor_permute(NULL, fake, fake + 8, dims, axes, 3);
        CHECK(rc == MIGEMM_ERR_ALIAS, "permute into its source gave %d", rc);
        rc = migemm_tensor_permute(NULL, fake, fake + 64, dims, axes, 11);
        CHECK(rc == MIGEMM_ERR_INVALID_ARG, "11 dimensions gave %d", rc);
    }
    rc = migemm_reduce_sum_axis(NULL, fake, fake + 2, 1, 4, 4);
    CHECK(rc == MIGEMM_ERR_ALIAS, "reduce into its input gave %d", rc);
    rc = migemm_linear_bias_backward(NULL, fake, fake + 1024, 0, 4);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "no rows gave %d", rc);
    rc = migemm_linear_weight_grad(NULL, fake, fake + 64, fake + 128, 4, 0, 4, 1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "K = 0 gave %d", rc);
    /* runtime services */
    void *p = NULL, *ctx = NULL, *st = NULL;
    CHECK(migemm_buffer_get_or_create(NULL, "x", 16, &p) == MIGEMM_ERR_INVALID_ARG, "null ctx");
    CHECK(migemm_buffer_get_or_create((void *)(uintptr_t)12345, "x", 16, &p) ==
              MIGEMM_ERR_INVALID_ARG && strstr(migemm_last_error(), "unknown context"),
          "unknown context accepted");
    CHECK(migemm_buffer_get_or_create((void *)(uintptr_t)12345, "", 16, &p) ==
              MIGEMM_ERR_INVALID_ARG, "empty name accepted");
    CHECK(migemm_queue_register_current((void *)(uintptr_t)12345, NULL) ==
              MIGEMM_ERR_INVALID_ARG, "null queue accepted");
    CHECK(migemm_queue_get_current(&ctx, &st) == MIGEMM_ERR_NO_QUEUE, "a queue without register");
    CHECK(migemm_tensor_buffer("t", 16, &p) == MIGEMM_ERR_NO_QUEUE, "tensor_buffer without queue");
    CHECK(migemm_queue_clear_current() == MIGEMM_OK, "clear");
    CHECK(migemm_buffer_release("never-created") == MIGEMM_OK, "release of an unknown name");
    CHECK(migemm_context_destroy((void *)(uintptr_t)12345) == MIGEMM_ERR_INVALID_ARG,
          "destroy of an unknown context");
    CHECK(migemm_context_create(-2, &ctx) == MIGEMM_ERR_INVALID_ARG, "device -2 accepted");
    {
        size_t n = 1, b = 1;
        CHECK(migemm_buffer_count(&n, &b) == MIGEMM_OK && n == 0 && b == 0, "empty pool");
        CHECK(migemm_workspace_size(NULL, &b) == MIGEMM_OK && b == 0, "workspace of no stream");
        CHECK(migemm_workspace_size(NULL, NULL) == MIGEMM_ERR_INVALID_ARG, "null size pointer");
    }
    /* policy, tuning and the plan record */
    int prev = -1;
    CHECK(migemm_set_gemm_policy(9, NULL) == MIGEMM_ERR_INVALID_ARG, "policy 9 accepted");
    CHECK(migemm_set_tuning(MIGEMM_TUNE_TILE, 48, &prev) == MIGEMM_ERR_INVALID_ARG, "tile 48");
    CHECK(migemm_set_tuning(99, 0, &prev) == MIGEMM_ERR_INVALID_ARG, "tuning key 99");
    {
        char plan[8];
        CHECK(migemm_last_plan(plan, sizeof(plan)) == MIGEMM_OK && strlen(plan) < sizeof(plan),
              "plan truncation");
        CHECK(migemm_last_plan(NULL, 4) == MIGEMM_ERR_INVALID_ARG, "null plan buffer");
    }
    return NULL;
}

static int validate(void) {
    enum { T = 4 };
    pthread_t th[T];
    for (int i = 0; i < T; ++i) pthread_create(&th[i], NULL, validate_thread, NULL);
    for (int i = 0; i < T; ++i) pthread_join(th[i], NULL);
    validate_thread(NULL);
    return failures;
}

/* C[b] = op(A[b]) op(B[b]) (+ bias) in double; small integers keep it exact. */
static void ref_gemm(int ta, int tb, int M, int N, int K, const float *A, const float *B,
                     const float *bias, float *C, int batch, int bcastB) {
    for (int b = 0; b < batch; ++b)
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j) {
                double s = 0;
                for (int k = 0; k < K; ++k) {
                    const float a = ta ? A[(size_t)b * M * K + (size_t)k * M + i]
                                       : A[(size_t)b * M * K + (size_t)i * K + k];
                    const size_t bo = bcastB ? 0 : (size_t)b * K * N;
                    const float v = tb ? B[bo + (size_t)j * K + k] : B[bo + (size_t)k * N + j];
                    s += (double)a * v;
                }
                if (bias) s += bias[j];
                C[((size_t)b * M + i) * N + j] = (float)s;
            }
}

static float *dev_copy(void *stream, const float *h, size_t n) {
    void *d = NULL;
    if (migemm_malloc(&d, n * sizeof(float)) != MIGEMM_OK) return NULL;
    if (migemm_memcpy_h2d(stream, d, h, n * sizeof(float)) != MIGEMM_OK) return NULL;
    return (float *)d;
}

static int gpu(void) {
    int count = 0;
    CHECK(migemm_device_count(&count) == MIGEMM_OK && count >= 1, "no device (%s)",
          migemm_last_error());
    if (failures) return failures;
    CHECK(migemm_set_device(0) == MIGEMM_OK, "set_device: %s", migemm_last_error());
    void *stream = NULL;
    CHECK(migemm_stream_create(&stream) == MIGEMM_OK, "stream_create: %s", migemm_last_error());

    enum { BATCH = 3, M = 70, N = 45, K = 131 };
    const size_t na = (size_t)BATCH * M * K, nb = (size_t)BATCH * K * N, nc = (size_t)BATCH * M * N;
    float *hA = malloc(na * sizeof(float)), *hB = malloc(nb * sizeof(float));
    float *hC = malloc(nc * sizeof(float)), *hR = malloc(nc * sizeof(float));
    float hbias[N];
    unsigned s = 12345u;
    for (size_t i = 0; i < na; ++i) { s = s * 1103515245u + 12345u; hA[i] = (float)((int)(s >> 16) % 7 - 3); }
    for (size_t i = 0; i < nb; ++i) { s = s * 1103515245u + 12345u; hB[i] = (float)((int)(s >> 16) % 7 - 3); }
    for (int j = 0; j < N; ++j) hbias[j] = (float)(j % 5 - 2);
    float *dA = dev_copy(stream, hA, na), *dB = dev_copy(stream, hB, nb);
    float *dbias = dev_copy(stream, hbias, N);
    void *dCv = NULL;
    CHECK(dA && dB && dbias && migemm_malloc(&dCv, nc * sizeof(float)) == MIGEMM_OK,
          "device buffers: %s", migemm_last_error());
    if (failures) return failures;
    float *dC = (float *)dCv;

    /* every layout of the general entry point, batched, with bias */
    for (int form = 0; form < 4; ++form) {
        const int ta = form >> 1, tb = form & 1;
        int rc = migemm_gemm_strided_batched(stream, ta, tb, M, N, K, dA, ta ? M : K,
                                             (int64_t)M * K, dB, tb ? K : N, (int64_t)K * N,
                                             dbias, dC, N, (int64_t)M * N, BATCH);
        CHECK(rc == MIGEMM_OK, "gemm form %d: %s", form, migemm_last_error());
        CHECK(migemm_memcpy_d2h(stream, hC, dC, nc * sizeof(float)) == MIGEMM_OK, "d2h: %s",
              migemm_last_error());
        ref_gemm(ta, tb, M, N, K, hA, hB, hbias, hR, BATCH, 0);
        CHECK(memcmp(hC, hR, nc * sizeof(float)) == 0, "gemm form %d differs", form);
    }
    /* reference-shaped entry points: bmm_tiled with a broadcast B, linear_forward */
    CHECK(migemm_bmm_tiled(stream, dA, dB, dC, M, K, N, M * K, 0, M * N, BATCH) == MIGEMM_OK,
          "bmm_tiled: %s", migemm_last_error());
    CHECK(migemm_memcpy_d2h(stream, hC, dC, nc * sizeof(float)) == MIGEMM_OK, "d2h");
    ref_gemm(0, 0, M, N, K, hA, hB, NULL, hR, BATCH, 1);
    CHECK(memcmp(hC, hR, nc * sizeof(float)) == 0, "bmm_tiled (broadcast B) differs");
    CHECK(migemm_linear_forward(stream, dA, dB, dbias, dC, M, K, N, M * K, M * N, BATCH) ==
              MIGEMM_OK, "linear_forward: %s", migemm_last_error());
    CHECK(migemm_memcpy_d2h(stream, hC, dC, nc * sizeof(float)) == MIGEMM_OK, "d2h");
    ref_gemm(0, 0, M, N, K, hA, hB, hbias, hR, BATCH, 1);
    CHECK(memcmp(hC, hR, nc * sizeof(float)) == 0, "linear_forward differs");

    CHECK(migemm_stream_synchronize(stream) == MIGEMM_OK, "sync: %s", migemm_last_error());
    migemm_free(dA);
    migemm_free(dB);
    migemm_free(dbias);
    migemm_free(dC);
    CHECK(migemm_stream_destroy(stream) == MIGEMM_OK, "stream_destroy");
    free(hA);
    free(hB);
    free(hC);
    free(hR);
    return failures;
}

/* ---- runtime objects: context, pool, per-thread queues (cs/core/ComputeContext.cs,
 *      cs/compiler/OpenCLBufferManager.cs, cs/core/DeviceQueueRegistry.cs) ---- */
struct worker {
    void *ctx;
    void *stream;
    int index;
    int ok;
    void *seen_stream;
    float *buf;
};

/* Registers its own queue, reads it back, and fills its own pooled tensor with its index. */
static void *worker_main(void *arg) {
    struct worker *w = (struct worker *)arg;
    void *c = NULL, *s = NULL, *p = NULL;
    char name[32];
    w->ok = migemm_queue_get_current(NULL, NULL) == MIGEMM_ERR_NO_QUEUE &&
            migemm_queue_register_current(w->ctx, w->stream) == MIGEMM_OK &&
            migemm_queue_get_current(&c, &s) == MIGEMM_OK && c == w->ctx;
    w->seen_stream = s;
    snprintf(name, sizeof(name), "worker%d", w->index);
    if (w->ok && migemm_tensor_buffer(name, 256 * sizeof(float), &p) == MIGEMM_OK) {
        float h[256];
        for (int i = 0; i < 256; ++i) h[i] = (float)w->index;
        w->ok = migemm_memcpy_h2d(s, p, h, sizeof(h)) == MIGEMM_OK &&
                migemm_stream_synchronize(s) == MIGEMM_OK;
        w->buf = (float *)p;
    } else {
        w->ok = 0;
    }
    migemm_queue_clear_current();
    return NULL;
}

static int runtime(void) {
    void *ctx = NULL, *other = NULL, *p0 = NULL, *p1 = NULL;
    int dev = -1, wave = 0, wx = 0, wy = 0;
    char arch[64];
    CHECK(migemm_context_create(-1, &ctx) == MIGEMM_OK, "context_create: %s", migemm_last_error());
    if (failures) return failures;
    CHECK(migemm_context_info(ctx, &dev, arch, sizeof(arch), NULL, &wave, NULL, &wx, &wy, NULL) ==
              MIGEMM_OK && dev >= 0 && wave == 64 && wy == 8 && strncmp(arch, "gfx950", 6) == 0,
          "context_info: dev %d wave %d wx %d wy %d arch %s", dev, wave, wx, wy, arch);
    /* pool: reuse while large enough, replace when larger or from another context */
    CHECK(migemm_buffer_get_or_create(ctx, "x", 1024, &p0) == MIGEMM_OK, "pool: %s",
          migemm_last_error());
    CHECK(migemm_buffer_get_or_create(ctx, "x", 512, &p1) == MIGEMM_OK && p1 == p0, "pool reuse");
    CHECK(migemm_buffer_get_or_create(ctx, "x", 4096, &p1) == MIGEMM_OK && p1 != NULL,
          "pool growth: %s", migemm_last_error());
    CHECK(migemm_context_create(-1, &other) == MIGEMM_OK, "second context");
    CHECK(migemm_buffer_get_or_create(other, "x", 16, &p0) == MIGEMM_OK, "other context");
    size_t n = 0, total = 0;
    CHECK(migemm_buffer_count(&n, &total) == MIGEMM_OK && n == 1 && total == 16,
          "count %zu %zu", n, total);
    CHECK(migemm_context_destroy(other) == MIGEMM_OK, "context_destroy: %s", migemm_last_error());
    CHECK(migemm_buffer_count(&n, &total) == MIGEMM_OK && n == 0, "destroy kept %zu", n);

    /* one queue per thread */
    enum { T = 4 };
    pthread_t th[T];
    struct worker w[T];
    for (int i = 0; i < T; ++i) {
        w[i].ctx = ctx;
        w[i].index = i;
        w[i].ok = 0;
        w[i].buf = NULL;
        CHECK(migemm_stream_create(&w[i].stream) == MIGEMM_OK, "stream_create");
    }
    for (int i = 0; i < T; ++i) pthread_create(&th[i], NULL, worker_main, &w[i]);
    for (int i = 0; i < T; ++i) pthread_join(th[i], NULL);
    CHECK(migemm_queue_get_current(NULL, NULL) == MIGEMM_ERR_NO_QUEUE, "main thread has a queue");
    for (int i = 0; i < T; ++i) {
        float h[256];
        void *p = NULL;
        char name[32];
        snprintf(name, sizeof(name), "worker%d", i);
        CHECK(w[i].ok && w[i].seen_stream == w[i].stream, "worker %d: %s", i, migemm_last_error());
        CHECK(migemm_buffer_get_or_create(ctx, name, 1024, &p) == MIGEMM_OK && p == w[i].buf,
              "worker %d buffer", i);
        CHECK(migemm_memcpy_d2h(w[i].stream, h, p, sizeof(h)) == MIGEMM_OK && h[0] == (float)i &&
                  h[255] == (float)i, "worker %d data", i);
        CHECK(migemm_stream_destroy(w[i].stream) == MIGEMM_OK, "stream_destroy");
    }

    /* Bmm -> BmmOp.Backward on pooled buffers, a fresh name per output */
    enum { B = 2, M = 24, K = 40, N = 16 };
    void *q = NULL, *da, *db, *dg, *dc, *dga, *dgb;
    CHECK(migemm_stream_create(&q) == MIGEMM_OK && migemm_queue_register_current(ctx, q) == MIGEMM_OK,
          "register: %s", migemm_last_error());
    static float hA[B * M * K], hB[B * K * N], hG[B * M * N], hC[B * M * N], hR[B * M * N];
    static float hGA[B * M * K], hGB[B * K * N], rGA[B * M * K], rGB[B * K * N];
    unsigned s = 7u;
    for (int i = 0; i < B * M * K; ++i) { s = s * 1103515245u + 12345u; hA[i] = (float)((int)(s >> 16) % 7 - 3); }
    for (int i = 0; i < B * K * N; ++i) { s = s * 1103515245u + 12345u; hB[i] = (float)((int)(s >> 16) % 7 - 3); }
    for (int i = 0; i < B * M * N; ++i) { s = s * 1103515245u + 12345u; hG[i] = (float)((int)(s >> 16) % 7 - 3); }
    CHECK(migemm_tensor_buffer("a", sizeof(hA), &da) == MIGEMM_OK &&
              migemm_tensor_buffer("b", sizeof(hB), &db) == MIGEMM_OK &&
              migemm_tensor_buffer("grad_c", sizeof(hG), &dg) == MIGEMM_OK, "tensor buffers");
    migemm_memcpy_h2d(q, da, hA, sizeof(hA));
    migemm_memcpy_h2d(q, db, hB, sizeof(hB));
    migemm_memcpy_h2d(q, dg, hG, sizeof(hG));
    CHECK(migemm_tensor_buffer("bmm_c#1", sizeof(hC), &dc) == MIGEMM_OK &&
              migemm_bmm_tiled(q, da, db, dc, M, K, N, M * K, K * N, M * N, B) == MIGEMM_OK &&
              migemm_stream_synchronize(q) == MIGEMM_OK, "Bmm: %s", migemm_last_error());
    CHECK(migemm_tensor_buffer("bmm_c#2", sizeof(hGA), &dga) == MIGEMM_OK &&
              migemm_bmm_permute_tiled(q, dg, db, dga, M, N, K, M * N, K * N, M * K, 0, 1, B) ==
                  MIGEMM_OK, "gradA: %s", migemm_last_error());
    CHECK(migemm_tensor_buffer("bmm_c#3", sizeof(hGB), &dgb) == MIGEMM_OK &&
              migemm_bmm_permute_tiled(q, da, dg, dgb, K, M, N, M * K, M * N, K * N, 1, 0, B) ==
                  MIGEMM_OK, "gradB: %s", migemm_last_error());
    migemm_memcpy_d2h(q, hC, dc, sizeof(hC));
    migemm_memcpy_d2h(q, hGA, dga, sizeof(hGA));
    migemm_memcpy_d2h(q, hGB, dgb, sizeof(hGB));
    ref_gemm(0, 0, M, N, K, hA, hB, NULL, hR, B, 0);
    CHECK(memcmp(hC, hR, sizeof(hC)) == 0, "Bmm output differs");
    for (int b = 0; b < B; ++b)
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < K; ++j) {
                double a = 0;
                for (int k = 0; k < N; ++k)
                    a += (double)hG[(b * M + i) * N + k] * hB[(b * K + j) * N + k];
                rGA[(b * M + i) * K + j] = (float)a;
            }
    for (int b = 0; b < B; ++b)
        for (int i = 0; i < K; ++i)
            for (int j = 0; j < N; ++j) {
                double a = 0;
                for (int k = 0; k < M; ++k)
                    a += (double)hA[(b * M + k) * K + i] * hG[(b * M + k) * N + j];
                rGB[(b * K + i) * N + j] = (float)a;
            }
    CHECK(memcmp(hGA, rGA, sizeof(hGA)) == 0, "gradA did not survive gradB");
    CHECK(memcmp(hGB, rGB, sizeof(hGB)) == 0, "gradB differs");
    migemm_queue_clear_current();
    CHECK(migemm_stream_destroy(q) == MIGEMM_OK, "stream_destroy");
    CHECK(migemm_context_destroy(ctx) == MIGEMM_OK, "context_destroy: %s", migemm_last_error());
    CHECK(migemm_buffer_count(&n, NULL) == MIGEMM_OK && n == 0, "buffers left: %zu", n);
    return failures;
}

int main(int argc, char **argv) {
    if (argc != 2 || (strcmp(argv[1], "validate") != 0 && strcmp(argv[1], "gpu") != 0 &&
                      strcmp(argv[1], "runtime") != 0)) {
        fprintf(stderr, "usage: %s validate|gpu|runtime\n", argv[0]);
        return 2;
    }
    const int bad = strcmp(argv[1], "gpu") == 0       ? gpu()
                    : strcmp(argv[1], "runtime") == 0 ? runtime()
                                                      : validate();
    printf("c_abi_check %s: %s\n", argv[1], bad ? "FAILED" : "ok");
    return bad ? 1 : 0;
}
