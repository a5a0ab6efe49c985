// Short-K fp32 GEMM for gfx950 (v_mfma_f32_16x16x4_f32): C = op(A) * op(B) (+ bias) with
// K <= 80, such as the batch-32 attention score product Q * K^T of matmul.cl:78-135 at
// BASELINE config 2a (K = 64) or a narrow Linear layer.
//
// With so short a K the small-output kernel's division of K over the wavefronts of a work-
// group buys a chain of a few MFMAs per wavefront at the price of an LDS reduction and a
// barrier, and its wavefronts spend most of their lifetime waiting (wave-level counters).
// Here one wavefront owns one 16x16 tile of C over the whole K:
//  * every operand value goes from global memory (L2) straight to registers, all loads of
//    the wavefront issued before its first MFMA (K <= 80: at most five 16-wide k-groups,
//    8 to 40 registers);
//  * fragments in the MFMA's own order: in step j of k-group g, lane l supplies row / column
//    l % 16 at k = 16 g + 4 (l / 16) + j. A K-contiguous operand is one 16-byte load per
//    k-group (4 rows x 64 contiguous bytes per 16 lanes); an M- or N-contiguous one is four
//    4-byte loads, 16 lanes covering 64 contiguous bytes of one k-row;
//  * one accumulator, MFMAs in ascending k: a fixed association order (one fp32 chain per
//    output over k-steps of 4), no cross-wavefront reduction, no LDS, no barrier;
//  * four independent tiles per work-group (consecutive tiles along N, so the four
//    wavefronts read the same rows of A), work-groups dealt to the XCDs in contiguous
//    chunks;
//  * edges: rows beyond M and columns beyond N are clamped on load and not stored; the last,
//    partial k-group (K % 16 != 0) is loaded element by element with k >= K zero in both
//    operands; bias after the k sum (linear.cl:119-122), then C is written or added to.
#include <type_traits>

#include "migemm_internal.h"

namespace migemm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

struct TinyArgs {
    const float *A;
    const float *B;
    const float *bias;
    float *C;
    int64_t lda, ldb, ldc;
    int64_t sA, sB, sC;
    int M, N, K;
    int total;          // 16x16 tiles over all batch entries
    int accumulate;     // C += result instead of C = result
    FastDiv per_batch;  // tiles per batch entry
    FastDiv tiles_n;    // tiles along N
};

constexpr int TT = 16;   // tile edge
constexpr int TWG = 4;   // wavefronts (tiles) per work-group
constexpr int TG_MAX = 5;  // full 16-wide k-groups at most (K <= 80)

// G: number of full k-groups (K / 16), a template parameter so every load and MFMA of the
// wavefront is straight-line code.
template <bool AKC, bool BKC, int G>
__global__ void __launch_bounds__(TWG * 64) gemm_tiny_kernel(TinyArgs p) {
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int nwg = gridDim.x;
    int wg = blockIdx.x;
    wg = (nwg & 7) == 0 ? (wg & 7) * (nwg >> 3) + (wg >> 3) : wg;
    const int tile = wg * TWG + w;
    if (tile >= p.total) return;  // the whole wavefront (the last work-group's spare tiles)
    const int b = (int)fast_div((uint32_t)tile, p.per_batch);
    const int t = tile - b * (int)p.per_batch.d;
    const int tm = (int)fast_div((uint32_t)t, p.tiles_n);
    const int tn = t - tm * (int)p.tiles_n.d;
    const int m0 = tm * TT;
    const int n0 = tn * TT;
    const int li = lane & 15;
    const int lq = lane >> 4;
    const int row = min(m0 + li, p.M - 1);
    const int col = min(n0 + li, p.N - 1);
    const float bias_v = p.bias != nullptr ? p.bias[col] : 0.f;

    const float *Ab = p.A + (int64_t)b * p.sA;
    const float *Bb = p.B + (int64_t)b * p.sB;
    // A(i, k) = Ab[i*lda + k] (AKC) or Ab[k*lda + i]; B(k, n) = Bb[n*ldb + k] (BKC) or
    // Bb[k*ldb + n]. pa / pb: this lane's row / column at k = 4 * lq.
    const float *pa = AKC ? Ab + (int64_t)row * p.lda + 4 * lq : Ab + (int64_t)(4 * lq) * p.lda + row;
    const float *pb = BKC ? Bb + (int64_t)col * p.ldb + 4 * lq : Bb + (int64_t)(4 * lq) * p.ldb + col;
    const int64_t a_g = AKC ? TT : (int64_t)TT * p.lda;  // per k-group
    const int64_t b_g = BKC ? TT : (int64_t)TT * p.ldb;

    f4 fa[G > 0 ? G : 1], fb[G > 0 ? G : 1];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float *qa = pa + g * a_g;
        const float *qb = pb + g * b_g;
        if constexpr (AKC)
            __builtin_memcpy(&fa[g], qa, sizeof(f4));
        else
            fa[g] = f4{qa[0], qa[p.lda], qa[2 * p.lda], qa[3 * p.lda]};
        if constexpr (BKC)
            __builtin_memcpy(&fb[g], qb, sizeof(f4));
        else
            fb[g] = f4{qb[0], qb[p.ldb], qb[2 * p.ldb], qb[3 * p.ldb]};
    }
    // the partial k-group, issued with the others
    const bool part = G * TT < p.K;
    f4 xa = {0.f, 0.f, 0.f, 0.f}, xb = {0.f, 0.f, 0.f, 0.f};
    if (part) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = G * TT + 4 * lq + j;
            if (k < p.K) {
                xa[j] = Ab[AKC ? (int64_t)row * p.lda + k : (int64_t)k * p.lda + row];
                xb[j] = Bb[BKC ? (int64_t)col * p.ldb + k : (int64_t)k * p.ldb + col];
            }
        }
    }
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[g][j], fb[g][j], acc, 0, 0, 0);
    if (part) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[j], xb[j], acc, 0, 0, 0);
    }

    // lane l, register r: row 4 (l / 16) + r, column l % 16 of the tile
    const int n = n0 + li;
    if (n < p.N) {
        float *Cb = p.C + (int64_t)b * p.sC + n;
        auto store = [&](auto accumulate) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 4 * lq + r;
                if (m < p.M) {
                    float v = acc[r];
                    if (p.bias != nullptr) v = v + bias_v;
                    float *c = Cb + (int64_t)m * p.ldc;
                    if constexpr (decltype(accumulate)::value)
                        *c = *c + v;
                    else
                        *c = v;
                }
            }
        };
        if (p.accumulate)
            store(std::true_type{});
        else
            store(std::false_type{});
    }
}

template <int G>
int launch_g(hipStream_t st, const TinyArgs &a, bool akc, bool bkc) {
    const dim3 grid((unsigned)((a.total + TWG - 1) / TWG)), block(TWG * 64);
    if (akc && bkc)
        hipLaunchKernelGGL((gemm_tiny_kernel<true, true, G>), grid, block, 0, st, a);
    else if (akc)
        hipLaunchKernelGGL((gemm_tiny_kernel<true, false, G>), grid, block, 0, st, a);
    else if (bkc)
        hipLaunchKernelGGL((gemm_tiny_kernel<false, true, G>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((gemm_tiny_kernel<false, false, G>), grid, block, 0, st, a);
    return hip_check(hipGetLastError(), "gemm_tiny_kernel launch");
}

int64_t tiles16(const GemmDesc &d) {
    return (int64_t)((d.M + TT - 1) / TT) * ((d.N + TT - 1) / TT) * d.batch;
}

}  // namespace

bool tiny_supported(const GemmDesc &d) {
    return d.K <= TG_MAX * TT && tiles16(d) <= (int64_t)0x7fffffff - TWG;
}

// Where the tiny kernel beats the previous choice (graph replay, 50 calls, us, previous /
// tiny; K in 16..80, M x N from 64 x 64 x 64 batches to 4096 x 4096, NN, NT, TN):
// 32 x 128 x 64 @ 64 x 128 (config 2a) 4.37 / 3.83; 1024 x 32 x 1024 5.44 / 4.32 (tiled);
// 32 x 128 x 80 @ 80 x 128 6.63 / 4.06 (the register-staged tiled kernel); 32 x 64 x 128
// TN 4.65 / 3.62. It loses with few tiles, where the small kernel's k division shortens
// each wavefront's MFMA chain (64 x 64 x 64 2.18 / 2.78; 256 x 64 x 512 2.86 / 3.03), and on
// large outputs, where the tiled kernels reuse operands from LDS (2048 x 32 x 2048 9.83 /
// 10.59; 1024 x 64 x 2048 8.02 / 9.11) -- except at K = 16 (4096 x 16 x 4096 24.5 / 20.5).
bool tiny_preferred(const GemmDesc &d) {
    if (!tiny_supported(d) || d.M < 16 || d.N < 16) return false;
    const int64_t t = tiles16(d);
    if (t < (d.K <= 48 ? 512 : 1024)) return false;
    if (d.K <= 16) return true;
    return t <= (d.K <= 48 ? 8192 : 4096);
}

int launch_gemm_tiny(hipStream_t stream, const GemmDesc &d) {
    if (!tiny_supported(d))
        return set_error(MIGEMM_ERR_UNSUPPORTED, "gemm_tiny: K=%d > %d", d.K, TG_MAX * TT);
    TinyArgs a;
    a.A = d.A;
    a.B = d.B;
    a.bias = d.bias;
    a.C = d.C;
    a.lda = d.lda;
    a.ldb = d.ldb;
    a.ldc = d.ldc;
    a.sA = d.sA;
    a.sB = d.sB;
    a.sC = d.sC;
    a.M = d.M;
    a.N = d.N;
    a.K = d.K;
    const int tm = (d.M + TT - 1) / TT;
    const int tn = (d.N + TT - 1) / TT;
    a.total = (int)tiles16(d);
    a.accumulate = d.accumulate;
    a.per_batch = make_fastdiv((uint32_t)((int64_t)tm * tn));
    a.tiles_n = make_fastdiv((uint32_t)tn);
    const bool akc = !d.transA;
    const bool bkc = d.transB;
    int rc;
    switch (d.K / TT) {
        case 0: rc = launch_g<0>(stream, a, akc, bkc); break;
        case 1: rc = launch_g<1>(stream, a, akc, bkc); break;
        case 2: rc = launch_g<2>(stream, a, akc, bkc); break;
        case 3: rc = launch_g<3>(stream, a, akc, bkc); break;
        case 4: rc = launch_g<4>(stream, a, akc, bkc); break;
        default: rc = launch_g<5>(stream, a, akc, bkc); break;
    }
    record_plan("tiny", d, TT, TT, 1, 0);
    return rc;
}

}  // namespace migemm
