// Skinny fp32 GEMM (M <= 4 rows of C): the decode-like GEMV of the matmul path,
// C[M,N] = A[M,K] * op(B) (+ bias), which reads each element of B once and is therefore
// bound by HBM bandwidth (0.5 FLOP/byte at M = 1), not by the matrix cores. B stored [N, K]
// (transposed, the weight layout of the Python reference's Linear, core/layers.py:21-33)
// runs gemv_rows_kernel below: a wavefront streams whole rows of B. B stored [K, N]:
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

    // Column of accumulator e: four adjacent columns per lane with 16-byte loads; otherwise
    // (N % 4 != 0) lane + 64 e, so each 4-byte load instruction reads 256 contiguous bytes
    // of the row instead of touching 1 KB at a 16-byte stride.
    auto col = [&](int e) { return VEC ? n + e : cb * SK_COLS + e * 64 + lane; };
    // Columns beyond N read a clamped, in-bounds column; their sums are never stored.
    const float *colp = Bb + (VEC ? (n < p.N ? n : p.N - 4) : 0);
    int nc[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) nc[e] = min(col(e), p.N - 1);

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
        else if constexpr (NTL)
            v = f4{__builtin_nontemporal_load(rowp + nc[0]), __builtin_nontemporal_load(rowp + nc[1]),
                   __builtin_nontemporal_load(rowp + nc[2]), __builtin_nontemporal_load(rowp + nc[3])};
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
                    const int c = col(e);
                    if (c < p.N) {
                        float v = tot[m][e];
                        if (p.bias != nullptr) v = v + p.bias[c];
                        crow[c] = p.accumulate ? crow[c] + v : v;
                    }
                }
            }
        } else {
            float *part = p.partial + (((int64_t)s * p.batch + b) * p.M) * p.N;
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (col(e) < p.N) part[(int64_t)m * p.N + col(e)] = tot[m][e];
        }
    }
}

// B transposed (stored [N, K]): output column n is the dot product of A's rows with row n
// of the stored B, whose K floats are contiguous. A wavefront owns RW consecutive rows of B
// and streams each over the whole K, 16 bytes per lane, U 1 KB loads per row in flight;
// lane L covers k = 256 i + 4 L .. +3. The lanes' partial sums are added by a butterfly
// over the wavefront (a fixed order), so nothing leaves the wavefront but the result and
// the call is one launch. A's rows (MR <= 4) are read through the caches with each chunk of
// B; every wavefront shares them, and RW rows per wavefront reuse each chunk of A RW times.
// Measured (graph replay, rotating copies of B, us; RW x U = 1 x 4 / 1 x 8 / 2 x 4 / 4 x 4):
// 1 x 11008 x 4096 29.2 / 28.9 / 30.6 / 35.7; 2 x 11008 x 4096 37.5 / 36.4 / 34.6 / 37.7;
// 4 x 11008 x 4096 50.8 / 50.6 / 42.8 / 38.0; 1 x 8192 x 8192 43.9 / 43.8 / 48.2 / 55.5.
template <int MR>
struct RowsPlan {
    static constexpr int RW = MR == 1 ? 1 : (MR == 2 ? 2 : 4);  // rows of B per wavefront
    static constexpr int U = MR <= 2 ? 8 : 4;                    // 1 KB chunks per row in flight
};
constexpr int RW_WAVES = 4;  // wavefronts per work-group

// AM: how A is read. 0 = A's rows are contiguous; 1 = strided, one element at a time;
// 2 = A stored transposed and dense ([K, MR], lda = MR): the MR values of 4 consecutive k
// are 4 MR contiguous floats, fetched as MR 16-byte loads.
template <int MR, int AM>
__global__ void __launch_bounds__(RW_WAVES * 64) gemv_rows_kernel(SkinnyArgs p) {
    constexpr int RW = RowsPlan<MR>::RW;
    constexpr int U = RowsPlan<MR>::U;
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * RW_WAVES + w) * RW;
    const int b = blockIdx.y;
    if (n0 >= p.N) return;  // no barrier below: whole wavefronts may leave
    const float *Ab = p.A + (int64_t)b * p.sA;
    const float *Bb = p.B + (int64_t)b * p.sB;
    const float *brow[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) brow[r] = Bb + (int64_t)min(n0 + r, p.N - 1) * p.ldb;

    f4 acc[MR][RW];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[m][r] = f4{0.f, 0.f, 0.f, 0.f};

    auto load_a = [&](int m, int k) {
        const float *q = Ab + (int64_t)m * p.a_rs;
        f4 v;
        if constexpr (AM == 0)
            v = *reinterpret_cast<const f4u *>(q + k);
        else
            v = f4{q[(int64_t)k * p.a_ks], q[(int64_t)(k + 1) * p.a_ks],
                   q[(int64_t)(k + 2) * p.a_ks], q[(int64_t)(k + 3) * p.a_ks]};
        return v;
    };
    // A's values at k .. k+3 for every row m (k + 4 <= K)
    auto load_a_all = [&](f4 (&av)[MR], int k) {
        if constexpr (AM == 2) {
            f4 t[MR];
#pragma unroll
            for (int j = 0; j < MR; ++j)
                t[j] = *reinterpret_cast<const f4u *>(Ab + (int64_t)k * MR + 4 * j);
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) av[m][e] = t[(e * MR + m) / 4][(e * MR + m) % 4];
        } else {
#pragma unroll
            for (int m = 0; m < MR; ++m) av[m] = load_a(m, k);
        }
    };
    auto fma4 = [&](f4 &c, const f4 &x, const f4 &y) {
#pragma unroll
        for (int e = 0; e < 4; ++e) c[e] = __builtin_fmaf(x[e], y[e], c[e]);
    };
    // whole batches of U chunks of 256 k: no bounds checks
    constexpr int STEP = 256 * U;
    const int kfull = p.K / STEP * STEP;
    for (int kb = 0; kb < kfull; kb += STEP) {
        f4 bv[U][RW], av[U][MR];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int r = 0; r < RW; ++r)
                bv[u][r] = __builtin_nontemporal_load(
                    reinterpret_cast<const f4u *>(brow[r] + kb + 256 * u + 4 * lane));
#pragma unroll
        for (int u = 0; u < U; ++u) load_a_all(av[u], kb + 256 * u + 4 * lane);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int r = 0; r < RW; ++r) fma4(acc[m][r], av[u][m], bv[u][r]);
    }
    // the rest of K, one chunk of 256 at a time; k >= K contributes nothing
    for (int kb = kfull; kb < p.K; kb += 256) {
        const int k = kb + 4 * lane;
        if (k + 4 <= p.K) {
            f4 av[MR];
            load_a_all(av, k);
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const f4 bv = *reinterpret_cast<const f4u *>(brow[r] + k);
#pragma unroll
                for (int m = 0; m < MR; ++m) fma4(acc[m][r], av[m], bv);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (k + e < p.K) {
#pragma unroll
                    for (int r = 0; r < RW; ++r) {
                        const float bv = brow[r][k + e];
#pragma unroll
                        for (int m = 0; m < MR; ++m)
                            acc[m][r][e] = __builtin_fmaf(
                                Ab[(int64_t)m * p.a_rs + (int64_t)(k + e) * p.a_ks], bv,
                                acc[m][r][e]);
                    }
                }
            }
        }
    }
    // lane sums, then the wavefront butterfly: every lane ends with the same total
#pragma unroll
    for (int m = 0; m < MR; ++m) {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            float v = (acc[m][r][0] + acc[m][r][1]) + (acc[m][r][2] + acc[m][r][3]);
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
            const int n = n0 + r;
            if (lane == 0 && n < p.N) {
                if (p.bias != nullptr) v = v + p.bias[n];
                float *c = p.C + (int64_t)b * p.sC + (int64_t)m * p.ldc + n;
                *c = p.accumulate ? *c + v : v;
            }
        }
    }
}

template <int MR>
int launch_rows(hipStream_t st, const SkinnyArgs &a, int am, int batch) {
    constexpr int per_wg = RW_WAVES * RowsPlan<MR>::RW;
    dim3 grid((a.N + per_wg - 1) / per_wg, batch);
    if (am == 0)
        MIGEMM_LAUNCH((gemv_rows_kernel<MR, 0>), grid, dim3(RW_WAVES * 64), 0, st, a);
    else if (am == 2)
        MIGEMM_LAUNCH((gemv_rows_kernel<MR, 2>), grid, dim3(RW_WAVES * 64), 0, st, a);
    else
        MIGEMM_LAUNCH((gemv_rows_kernel<MR, 1>), grid, dim3(RW_WAVES * 64), 0, st, a);
    return launch_status("gemv_rows_kernel launch");
}

template <int MR>
int launch_mr(hipStream_t st, const SkinnyArgs &a, bool vec, int batch) {
    dim3 grid(a.cblocks, a.slices, batch);
    // B is streamed once: non-temporal loads (measured 1x11008x4096: 32.0 us against 36.6 us
    // with ordinary loads, 3 rotating copies of B).
    if (vec)
        MIGEMM_LAUNCH((gemm_skinny_kernel<MR, true, true>), grid, dim3(SK_THREADS), 0, st, a);
    else
        MIGEMM_LAUNCH((gemm_skinny_kernel<MR, false, true>), grid, dim3(SK_THREADS), 0, st, a);
    return launch_status("gemm_skinny_kernel launch");
}

}  // namespace

bool skinny_supported(const GemmDesc &d) {
    if (d.M > SK_MAXM || d.batch > 65535) return false;
    // gemv_rows_kernel: its k loops step in int, 256 x 8 floats at a time
    if (d.transB) return d.K <= (1 << 30);
    return d.N >= 4 && (int64_t)d.K <= (int64_t)65535 * 256;
}

// B transposed: where the rows kernel beats the other families (graph replay, rotating
// copies of B, M 1-4 x N 1024-11008 x K 512-8192, us, rows / small kernel). At M = 1 (a
// wavefront per row) at every shape: 1 x 1024 x 512 2.58 / 4.87, 1 x 4096 x 1024 5.04 /
// 5.49, 1 x 11008 x 4096 30.0 / 39.5. With 2-4 rows per wavefront it needs many rows: at
// N = 11008 from K = 1024 (M = 2: 12.46 / 13.62) or K = 2048 (M = 3-4: 21.3 / 24.5), but at
// N = 4096 the small kernel wins (4 x 4096 x 4096 22.4 / 15.3, 2 x 4096 x 4096 15.2 / 14.8).
static bool rows_preferred(const GemmDesc &d) {
    const int64_t rows = (int64_t)d.N * d.batch;
    // M = 1: every row count, except many short rows, whose per-row reduction outweighs
    // the stream (graph replay, us, rows kernel / small kernel: 1 x 1301 x 440 3.58 / 5.55,
    // batch-8 1 x 1755 x 40 3.89 / 5.51, 1 x 173 x 17 2.72 / 3.06; batch-32 1 x 302 x 5262
    // 56.1 / 45.2, 1 x 134 x 29895 9.33 / 6.45). A wavefront streams a whole row at ~8 GB/s,
    // so rows longer than 10000 take this kernel only if there are >= 768 of them; fewer,
    // longer rows go to the small kernel's k ranges (batch-8 1 x 137946 x 25 78.9 / 24.6,
    // 1 x 32279 x 52 16.9 / 9.2; a dot product, 1 x 10^7 x 1, 91 there; 1 x 31706 x 877 27.2 /
    // 34.1)
    if (d.M == 1) return !(d.K < 320 && rows >= 16384) && (d.K <= 10000 || rows >= 768);
    if (d.M == 2) return rows >= 8192 && d.K >= 1024;
    return rows >= 8192 && d.K >= 2048;
}

// Streaming B pays once B is too large to sit in the caches: from 64 MB of B the kernel
// beats the small kernel at every M <= 4 (graph replay, rotating copies of B, us, skinny /
// small: 1 x 11008 x 4096 32.2 / 60.6; 4 x 11008 x 4096 38.9 / 61.4; 2 x 8192 x 2048
// 19.1 / 27.0; 3 x 4096 x 4096 16.7 / 23.9). At 32 MB they tie (1 x 4096 x 2048 12.0 /
// 12.1; 4 x 4096 x 2048 14.9 / 12.3) and below that the small kernel wins (3 x 6565 x 500
// 20.1 / 7.7).
bool skinny_preferred(const GemmDesc &d) {
    if (!skinny_supported(d)) return false;
    if (d.transB) return rows_preferred(d);
    // 3-4 rows of C over a batch: each entry's B must reach the bound itself (graph replay,
    // us, this kernel / small kernel: batch-4 4 x 824 x 5425 36.2 / 18.9, batch-8 4 x 1028 x
    // 2151 36.3 / 19.9; batch-2 4 x 7959 x 4144, 132 MB per entry, 57.2 / 87.3). With
    // N % 4 != 0, 96 MB of B over the whole batch is enough (rotating copies of B: batch-16
    // 3 x 9907 x 526 76.4 / 120.1, batch-8 4 x 11128 x 1349 106.6 / 148.2, batch-4 4 x 11887
    // x 529 34.8 / 44.7; 48 of 48 such shapes of two seeds 0.57-0.99x; below it batch-8 3 x
    // 3350 x 866, 93 MB, 26.5 / 22.6, batch-4 3 x 995 x 4479 23.6 / 17.9).
    if (d.M >= 3)
        return (int64_t)d.K * d.N >= ((int64_t)16 << 20) ||
               (d.N % 4 != 0 && (int64_t)d.K * d.N * d.batch >= ((int64_t)23 << 20));
    return (int64_t)d.K * d.N * d.batch >= ((int64_t)16 << 20);
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
    a.batch = d.batch;
    a.accumulate = d.accumulate;
    a.partial = nullptr;

    if (d.transB) {  // rows of the stored B streamed whole: one launch, no partial sums
        a.kc = d.K;
        a.slices = 1;
        // A's row is contiguous also when A is stored transposed with one row and lda = 1
        // (a [K, 1] column); the 4-byte loads would otherwise touch 1 KB per instruction at
        // a 16-byte stride for every 1 KB of B.
        const int am = !d.transA || (d.M == 1 && d.lda == 1) ? 0 : d.lda == d.M ? 2 : 1;
        int rc;
        switch (d.M) {
            case 1: rc = launch_rows<1>(stream, a, am, d.batch); break;
            case 2: rc = launch_rows<2>(stream, a, am, d.batch); break;
            case 3: rc = launch_rows<3>(stream, a, am, d.batch); break;
            default: rc = launch_rows<4>(stream, a, am, d.batch); break;
        }
        record_plan("skinny-rows", d, 0, 0, 1, 16);
        return rc;
    }

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
