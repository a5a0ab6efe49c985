// Skinny fp32 GEMM (M <= 4 rows of C, B not transposed): the decode-like GEMV of the
// matmul path, C[M,N] = A[M,K] * B[K,N] (+ bias), which reads each element of B once and
// is therefore bound by HBM bandwidth (0.5 FLOP/byte at M = 1), not by the matrix cores.
//
// Work split: a work-group of 4 wavefronts owns 256 consecutive columns (one float4 of
// B per lane) and a slice of KC rows of K; the slice of A is staged in LDS, wavefront w
// accumulates the w-th quarter of the slice with fp32 FMA chains, 16 rows of loads in
// flight at a time (8 for 3-4 rows of C), and the 4 wavefronts are combined through LDS.
// With S = ceil(K / KC) > 1 slices, each slice writes its partial sums to the library
// workspace and a second kernel (reduce_slices_kernel, gemm_mfma.hip) adds the S partials
// of every output in slice order, then the bias. The result is deterministic: the
// association order depends only on (K, KC), never on timing. (A single-kernel
// "last work-group combines" variant needs an agent-scope release fence per work-group,
// which writes back the XCD's whole L2 on MI355X and cost more than the GEMV itself.)
#include <stdlib.h>

#include "migemm_internal.h"

namespace migemm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
// The same vector with 4-byte alignment: B's base may sit at any float offset (a strided
// view), and 16-byte loads need only 4-byte alignment on gfx950.
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

constexpr int SK_THREADS = 256;
constexpr int SK_COLS = 256;  // columns per work-group (64 lanes x float4)
constexpr int SK_MAXM = 4;
// rows of B in flight per wavefront: 16, or 8 for 3-4 rows of C, whose A values and
// accumulators would otherwise hold 256 VGPRs (one wavefront per SIMD)
template <int MR>
struct SkUnroll {
    static constexpr int value = MR <= 2 ? 16 : 8;
};
constexpr int SK_KC_MAX = 512;  // rows of K per slice at most (A's slice is staged in LDS)

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
    int accumulate;  // C += result instead of C = result
};

template <int MR, bool VEC, bool NTL>
__global__ void __launch_bounds__(SK_THREADS) gemm_skinny_kernel(SkinnyArgs p) {
    __shared__ f4 red[4][MR][64];
    __shared__ float a_s[MR][SK_KC_MAX];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int cb = blockIdx.x;
    const int s = blockIdx.y;
    const int b = blockIdx.z;
    const int n = cb * SK_COLS + lane * 4;

    const float *Ab = p.A + (int64_t)b * p.sA;
    const float *Bb = p.B + (int64_t)b * p.sB;
    // Wavefront w owns the contiguous rows [k_lo, k_hi) of this work-group's slice.
    const int kb = s * p.kc;
    const int ke = min(p.K, kb + p.kc);
    const int per_wave = p.kc / 4;
    const int k_lo = min(ke, kb + w * per_wave);
    const int k_hi = min(ke, k_lo + per_wave);

    // The slice of A (MR x (ke - kb) values) goes to LDS once: every lane reads all of it,
    // and as per-element global loads it took 4 vector-memory instructions per row of B at
    // M = 4, more than the B stream itself.
    const int span = ke - kb;
    for (int i = tid; i < MR * span; i += SK_THREADS) {
        const int m = i / span;
        const int kk = i - m * span;
        a_s[m][kk] = Ab[m * p.a_rs + (int64_t)(kb + kk) * p.a_ks];
    }
    __syncthreads();

    // Columns beyond N read a clamped, in-bounds column; their sums are never stored.
    const float *colp = Bb + (VEC ? (n < p.N ? n : p.N - 4) : 0);
    int nc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) nc[e] = min(n + e, p.N - 1);

    f4 acc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m] = f4{0.f, 0.f, 0.f, 0.f};

    // Batches of SK_UNROLL rows: every load of a batch is issued before its FMAs, so each
    // wavefront keeps SK_UNROLL x 1 KiB of B in flight. Full batches carry no bounds
    // checks; the last, partial batch re-reads its final row and multiplies it by zero.
    constexpr int SK_UNROLL = SkUnroll<MR>::value;
    auto load_row = [&](int k) {
        const float *rowp = colp + (int64_t)k * p.ldb;
        f4 v;
        if constexpr (VEC && NTL)
            v = __builtin_nontemporal_load(reinterpret_cast<const f4u *>(rowp));
        else if constexpr (VEC)
            __builtin_memcpy(&v, rowp, sizeof(f4));
        else
            v = f4{rowp[nc[0]], rowp[nc[1]], rowp[nc[2]], rowp[nc[3]]};
        return v;
    };
    int k0 = k_lo;
    for (; k0 + SK_UNROLL <= k_hi; k0 += SK_UNROLL) {
        f4 v[SK_UNROLL];
#pragma unroll
        for (int u = 0; u < SK_UNROLL; ++u) v[u] = load_row(k0 + u);
#pragma unroll
        for (int u = 0; u < SK_UNROLL; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float a = a_s[m][k0 + u - kb];
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[m][e] = __builtin_fmaf(a, v[u][e], acc[m][e]);
            }
    }
    if (k0 < k_hi) {
        f4 v[SK_UNROLL];
#pragma unroll
        for (int u = 0; u < SK_UNROLL; ++u) v[u] = load_row(min(k0 + u, k_hi - 1));
#pragma unroll
        for (int u = 0; u < SK_UNROLL; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const bool ok = k0 + u < k_hi;
                const float a = ok ? a_s[m][k0 + u - kb] : 0.f;
                const f4 vv = ok ? v[u] : f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[m][e] = __builtin_fmaf(a, vv[e], acc[m][e]);
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
                        crow[n + e] = p.accumulate ? crow[n + e] + v : v;
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
    // B is streamed once: non-temporal loads (measured 1x11008x4096: 32.0 us against 36.6 us
    // with ordinary loads, 3 rotating copies of B).
    if (vec)
        hipLaunchKernelGGL((gemm_skinny_kernel<MR, true, true>), grid, dim3(SK_THREADS), 0, st, a);
    else
        hipLaunchKernelGGL((gemm_skinny_kernel<MR, false, false>), grid, dim3(SK_THREADS), 0, st, a);
    return hip_check(hipGetLastError(), "gemm_skinny_kernel launch");
}

}  // namespace

bool skinny_supported(const GemmDesc &d) {
    return d.M <= SK_MAXM && !d.transB && d.N >= 4 && d.batch <= 65535 &&
           (int64_t)d.K <= (int64_t)65535 * 256;
}

// Streaming B pays once B is too large to sit in the caches: from 64 MB of B the kernel
// beats the small kernel at every M <= 4 (graph replay, rotating copies of B, us, skinny /
// small: 1 x 11008 x 4096 32.2 / 60.6; 4 x 11008 x 4096 38.9 / 61.4; 2 x 8192 x 2048
// 19.1 / 27.0; 3 x 4096 x 4096 16.7 / 23.9). At 32 MB they tie (1 x 4096 x 2048 12.0 /
// 12.1; 4 x 4096 x 2048 14.9 / 12.3) and below that the small kernel wins (3 x 6565 x 500
// 20.1 / 7.7).
bool skinny_preferred(const GemmDesc &d) {
    return skinny_supported(d) && (int64_t)d.K * d.N * d.batch >= ((int64_t)16 << 20);
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

    // Slices of KC = 4 wavefronts x 64 rows (four batches of 16 per wavefront) give the
    // 5b shape (11008 x 4096) 43 x 16 = 688 work-groups, all resident at once, each
    // wavefront streaming 64 KiB of B; small K gets one slice.
    int kc = 256;
    const int64_t blocks = (int64_t)a.cblocks * d.batch;
    if (blocks >= 1024) kc = 512;  // enough column blocks already: fewer partials
    if (kc >= d.K) kc = (d.K + 3) / 4 * 4;
    a.kc = kc;
    a.slices = (d.K + kc - 1) / kc;
    if (a.slices > 65535)  // K <= 65535 * SK_KC_MAX is part of skinny_supported
        return set_error(MIGEMM_ERR_UNSUPPORTED, "gemm_skinny: K=%d needs %d slices", d.K,
                         a.slices);
    a.partial = nullptr;
    a.batch = d.batch;
    a.accumulate = d.accumulate;
    if (a.slices > 1) {
        const size_t part_bytes = (size_t)a.slices * d.batch * d.M * d.N * sizeof(float);
        int st = MIGEMM_OK;
        a.partial = partial_buffer(stream, d, part_bytes, &st);
        if (a.partial == nullptr) return st;
    }
    // 4-column groups never straddle N when N % 4 == 0 (16-byte loads need only 4-byte
    // alignment on gfx950).
    const bool vec = d.N % 4 == 0;
    int rc;
    switch (d.M) {
        case 1: rc = launch_mr<1>(stream, a, vec, d.batch); break;
        case 2: rc = launch_mr<2>(stream, a, vec, d.batch); break;
        case 3: rc = launch_mr<3>(stream, a, vec, d.batch); break;
        default: rc = launch_mr<4>(stream, a, vec, d.batch); break;
    }
    record_plan("skinny", d, 0, SK_COLS, a.slices, 0);
    if (rc != MIGEMM_OK || a.slices == 1) return rc;
    return launch_reduce_slices(stream, a.partial, a.slices, d.batch, d.M, d.N, d.bias, d.C,
                                d.ldc, d.sC, d.accumulate);
}

}  // namespace migemm
