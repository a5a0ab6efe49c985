// Skinny fp32 GEMM (M <= 4 rows of C, B not transposed): the decode-like GEMV of the
// matmul path, C[M,N] = A[M,K] * B[K,N] (+ bias), which reads each element of B once and
// is therefore bound by HBM bandwidth (0.5 FLOP/byte at M = 1), not by the matrix cores.
//
// Work split: a work-group of 4 wavefronts owns 256 consecutive columns (one float4 of
// B per lane) and a slice of KC rows of K; wavefront w accumulates rows w, w+4, ... of
// its slice with fp32 FMA chains and the 4 wavefronts are combined through LDS. With
// S = ceil(K / KC) > 1 slices, each slice writes its partial sums to the library
// workspace and a second kernel (reduce_slices_kernel, gemm_mfma.hip) adds the S partials
// of every output in slice order, then the bias. The result is deterministic: the
// association order depends only on (K, KC), never on timing. (A single-kernel
// "last work-group combines" variant needs an agent-scope release fence per work-group,
// which writes back the XCD's whole L2 on MI355X and cost more than the GEMV itself.)
#include "migemm_internal.h"

namespace migemm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int SK_THREADS = 256;
constexpr int SK_COLS = 256;  // columns per work-group (64 lanes x float4)
constexpr int SK_MAXM = 4;

struct SkinnyArgs {
    const float *A;
    const float *B;
    const float *bias;
    float *C;
    int64_t a_rs, a_ks;  // A(m, k) = A[m*a_rs + k*a_ks]
    int64_t ldb, ldc;
    int64_t sA, sB, sC;
    int M, N, K;
    int kc;        // rows of K per slice (multiple of 4)
    int slices;    // ceil(K / kc)
    int cblocks;   // ceil(N / 256)
    float *partial;  // [slices][batch][M][N] when slices > 1
    int batch;
};

template <int MR, bool VEC>
__global__ void __launch_bounds__(SK_THREADS) gemm_skinny_kernel(SkinnyArgs p) {
    __shared__ f4 red[4][MR][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int cb = blockIdx.x;
    const int s = blockIdx.y;
    const int b = blockIdx.z;
    const int n = cb * SK_COLS + lane * 4;

    const float *Ab = p.A + (int64_t)b * p.sA;
    const float *Bb = p.B + (int64_t)b * p.sB;
    const int kb = s * p.kc;
    const int ke = min(p.K, kb + p.kc);

    f4 acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = f4{0.f, 0.f, 0.f, 0.f};

    // Columns beyond N read a clamped, in-bounds column; their sums are never stored.
    int nc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) nc[e] = min(n + e, p.N - 1);

    auto row_of_b = [&](int k) -> f4 {
        const float *rowp = Bb + (int64_t)k * p.ldb;
        if constexpr (VEC) {
            return *reinterpret_cast<const f4 *>(rowp + (n < p.N ? n : p.N - 4));
        } else {
            return f4{rowp[nc[0]], rowp[nc[1]], rowp[nc[2]], rowp[nc[3]]};
        }
    };

    int k = kb + w;
    // 4 rows in flight per wavefront per iteration.
    for (; k + 12 < ke; k += 16) {
        f4 v0 = row_of_b(k), v1 = row_of_b(k + 4), v2 = row_of_b(k + 8), v3 = row_of_b(k + 12);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float *ap = Ab + m * p.a_rs;
            const float a0 = ap[(int64_t)k * p.a_ks], a1 = ap[(int64_t)(k + 4) * p.a_ks];
            const float a2 = ap[(int64_t)(k + 8) * p.a_ks], a3 = ap[(int64_t)(k + 12) * p.a_ks];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                acc[m][e] = __builtin_fmaf(a0, v0[e], acc[m][e]);
                acc[m][e] = __builtin_fmaf(a1, v1[e], acc[m][e]);
                acc[m][e] = __builtin_fmaf(a2, v2[e], acc[m][e]);
                acc[m][e] = __builtin_fmaf(a3, v3[e], acc[m][e]);
            }
        }
    }
    for (; k < ke; k += 4) {
        f4 v = row_of_b(k);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float a = Ab[m * p.a_rs + (int64_t)k * p.a_ks];
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[m][e] = __builtin_fmaf(a, v[e], acc[m][e]);
        }
    }

#pragma unroll
    for (int m = 0; m < MR; ++m) red[w][m][lane] = acc[m];
    __syncthreads();

    // Wavefront 0 combines the 4 wavefronts in order (w = 0, 1, 2, 3).
    if (w == 0) {
        f4 tot[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            tot[m] = red[0][m][lane];
            tot[m] += red[1][m][lane];
            tot[m] += red[2][m][lane];
            tot[m] += red[3][m][lane];
        }
        if (p.slices == 1) {
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float *crow = p.C + (int64_t)b * p.sC + (int64_t)m * p.ldc;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    if (n + e < p.N) {
                        float v = tot[m][e];
                        if (p.bias != nullptr) v = v + p.bias[n + e];
                        crow[n + e] = v;
                    }
                }
            }
        } else {
            float *part = p.partial + (((int64_t)s * p.batch + b) * p.M) * p.N;
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n + e < p.N) part[(int64_t)m * p.N + n + e] = tot[m][e];
        }
    }
}

template <int MR>
int launch_mr(hipStream_t st, const SkinnyArgs &a, bool vec, int batch) {
    dim3 grid(a.cblocks, a.slices, batch);
    if (vec)
        hipLaunchKernelGGL((gemm_skinny_kernel<MR, true>), grid, dim3(SK_THREADS), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_skinny_kernel<MR, false>), grid, dim3(SK_THREADS), 0, st, a);
    return hip_check(hipGetLastError(), "gemm_skinny_kernel launch");
}

}  // namespace

bool skinny_applicable(const GemmDesc &d) {
    return d.M <= SK_MAXM && !d.transB && d.N >= 4 && d.batch <= 65535;
}

int launch_gemm_skinny(hipStream_t stream, const GemmDesc &d) {
    SkinnyArgs a;
    a.A = d.A;
    a.B = d.B;
    a.bias = d.bias;
    a.C = d.C;
    a.a_rs = d.transA ? 1 : d.lda;
    a.a_ks = d.transA ? d.lda : 1;
    a.ldb = d.ldb;
    a.ldc = d.ldc;
    a.sA = d.sA;
    a.sB = d.sB;
    a.sC = d.sC;
    a.M = d.M;
    a.N = d.N;
    a.K = d.K;
    a.cblocks = (d.N + SK_COLS - 1) / SK_COLS;

    // Aim for >= ~2048 work-groups so every CU holds several and HBM sees enough
    // requests in flight; slices are at least 64 rows so the final combine stays small.
    const int64_t want = 2048;
    int64_t slices = (want + (int64_t)a.cblocks * d.batch - 1) / ((int64_t)a.cblocks * d.batch);
    int kc = (int)((d.K + slices - 1) / slices);
    kc = (kc + 15) / 16 * 16;
    if (kc < 64) kc = 64;
    if (kc > d.K) kc = (d.K + 3) / 4 * 4;
    a.kc = kc;
    a.slices = (d.K + kc - 1) / kc;
    if (a.slices > 65535) {
        a.kc = (d.K + 65534) / 65535;
        a.kc = (a.kc + 3) / 4 * 4;
        a.slices = (d.K + a.kc - 1) / a.kc;
    }
    a.partial = nullptr;
    a.batch = d.batch;
    if (a.slices > 1) {
        const size_t part_bytes = (size_t)a.slices * d.batch * d.M * d.N * sizeof(float);
        int st = MIGEMM_OK;
        a.partial = static_cast<float *>(workspace(part_bytes, &st));
        if (a.partial == nullptr) return st;
    }
    const bool vec = (reinterpret_cast<uintptr_t>(d.B) & 15u) == 0 && d.ldb % 4 == 0 &&
                     d.N % 4 == 0 && (d.batch == 1 || d.sB % 4 == 0);
    int rc;
    switch (d.M) {
        case 1: rc = launch_mr<1>(stream, a, vec, d.batch); break;
        case 2: rc = launch_mr<2>(stream, a, vec, d.batch); break;
        case 3: rc = launch_mr<3>(stream, a, vec, d.batch); break;
        default: rc = launch_mr<4>(stream, a, vec, d.batch); break;
    }
    if (rc != MIGEMM_OK || a.slices == 1) return rc;
    return launch_reduce_slices(stream, a.partial, a.slices, d.batch, d.M, d.N, d.bias, d.C,
                                d.ldc, d.sC);
}

}  // namespace migemm
