/* A plain C99 caller of libmigemm, with no torch and no Python: the way a non-Python host
 * (the reference's C# host through P/Invoke, cs/compiler/NnClGlob.cs) uses the library.
 *
 *   c_abi_check validate   argument checks only; needs no GPU
 *   c_abi_check gpu        device memory, copies and the GEMM entry points on GPU 0,
 *                          checked exactly against a CPU loop on small-integer operands
 *
 * Exit status 0 on success; every failure prints what failed. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "migemm.h"

static int failures = 0;

#define CHECK(cond, ...)                              \
    do {                                              \
        if (!(cond)) {                                \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);             \
            fprintf(stderr, "\n");                    \
            ++failures;                               \
        }                                             \
    } while (0)

static int validate(void) {
    float *fake = (float *)(uintptr_t)0x100000;
    CHECK(strlen(migemm_version()) > 0, "empty version");
    int rc = migemm_gemm_strided_batched(NULL, 0, 0, 0, 4, 4, fake, 4, 0, fake + 64, 4, 0, NULL,
                                         fake + 128, 4, 0, 1);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "M = 0 gave %d", rc);
    CHECK(strlen(migemm_last_error()) > 0, "no message for M = 0");
    rc = migemm_gemm_strided_batched(NULL, 0, 0, 4, 4, 4, fake, 4, 0, fake, 4, 0, NULL, fake, 4,
                                     0, 1);
    CHECK(rc == MIGEMM_ERR_ALIAS, "aliased output gave %d", rc);
    rc = migemm_bmm_tiled(NULL, fake, fake + 64, fake + 128, 4, 4, 4, -1, 0, 16, 2);
    CHECK(rc == MIGEMM_ERR_INVALID_ARG, "negative stride gave %d", rc);
    CHECK(migemm_set_gemm_policy(9, NULL) == MIGEMM_ERR_INVALID_ARG, "policy 9 accepted");
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

int main(int argc, char **argv) {
    if (argc != 2 || (strcmp(argv[1], "validate") != 0 && strcmp(argv[1], "gpu") != 0)) {
        fprintf(stderr, "usage: %s validate|gpu\n", argv[0]);
        return 2;
    }
    const int bad = strcmp(argv[1], "gpu") == 0 ? gpu() : validate();
    printf("c_abi_check %s: %s\n", argv[1], bad ? "FAILED" : "ok");
    return bad ? 1 : 0;
}
