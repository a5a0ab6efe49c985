// Short-K fp32 GEMM for gfx950 (v_mfma_f32_16x16x4_f32): C = op(A) * op(B) (+ bias) with
// K <= 320, such as the batch-32 attention products of matmul.cl:78-135 at BASELINE config 2
// (Q * K^T with K = 64, P * V with K = 128) or a narrow Linear layer.
//
// With so short a K the small-output kernel's division of K over eight wavefronts buys a
// chain of a few MFMAs per wavefront at the price of lane permutations, an LDS reduction and
// a barrier, and its wavefronts spend most of their lifetime waiting (wave-level counters).
// Here a 16x16 tile of C is computed by KS = 1, 2 or 4 wavefronts of one work-group, each over
// a contiguous 1/KS of K (at most five 16-wide k-groups, K <= 80 per wavefront; K = 128 on
// four wavefronts of 32):
//  * every operand value of a wavefront goes from global memory (L2) straight to registers,
//    all its loads issued before its first MFMA (8 to 40 registers);
//  * fragments in the MFMA's own order: in step j of k-group g, lane l supplies row / column
//    l % 16 at k = 16 g + 4 (l / 16) + j. A K-contiguous operand is one 16-byte load per
//    k-group, 16 lanes reading 4 rows x 64 contiguous bytes, put in fragment order by a lane
//    permutation; an M- or N-contiguous one is four 4-byte loads, 16 lanes covering 64
//    contiguous bytes of one k-row;
//  * one accumulator per wavefront, MFMAs in ascending k; with KS > 1 the wavefronts' partial
//    tiles are added through LDS in k order after one barrier: a fixed association order;
//  * 4 / KS tiles per work-group (consecutive along N, so the wavefronts read the same rows of
//    A), work-groups dealt to the XCDs in contiguous chunks;
//  * edges: rows beyond M and columns beyond N are clamped on load and not stored; with KS = 1
//    the last, partial k-group (K % 16 != 0) is loaded element by element with k >= K zero in
//    both operands (KS > 1 takes only K a multiple of 16 KS); bias after the k sum
//    (linear.cl:119-122), then C is written or added to.
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

constexpr int TT = 16;     // tile edge
constexpr int TWG = 4;     // wavefronts per work-group
constexpr int TG_MAX = 5;  // full 16-wide k-groups per wavefront at most (80 values of K)

// G: full k-groups per wavefront (K / (16 KS), or K / 16 plus a partial group with KS = 1),
// a template parameter so every load and MFMA of the wavefront is straight-line code. KS:
// wavefronts per tile, each over k in [kp 16 G, (kp + 1) 16 G).
template <bool AKC, bool BKC, int G, int KS>
__global__ void __launch_bounds__(TWG * 64) gemm_tiny_kernel(TinyArgs p) {
    __shared__ f4 red[KS > 1 ? TWG : 1][64];
    const int lane = threadIdx.x & 63;
    const int w = threadIdx.x >> 6;
    const int kp = w % KS;  // this wavefront's part of K
    const int nwg = gridDim.x;
    int wg = blockIdx.x;
    wg = (nwg & 7) == 0 ? (wg & 7) * (nwg >> 3) + (wg >> 3) : wg;
    const int tile = wg * (TWG / KS) + w / KS;
    const bool live = tile < p.total;  // false only for the last work-group's spare tiles
    if (KS == 1 && !live) return;      // (with KS > 1 every wavefront reaches the barrier)
    const int tile_c = live ? tile : p.total - 1;
    const int b = (int)fast_div((uint32_t)tile_c, p.per_batch);
    const int t = tile_c - b * (int)p.per_batch.d;
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
    // Bb[k*ldb + n]. pa / pb: this lane's row / column at k = k0 + 4 * lq.
    const int k0 = kp * G * TT;
    // A K-contiguous operand read in fragment order would give each 16-lane group 16
    // different rows; it is read coalesced instead: lane (lq, li = 4a + c) loads the 16
    // bytes of row 4 lq + a at k = 4c .. 4c+3 (a 16-lane group reads 4 rows x 64 contiguous
    // bytes), and a lane permutation (ds_bpermute, no LDS storage) gives lane (lq, li) row
    // li at k = 4 lq + j, the same values as the fragment-order load.
    const int crow = 4 * lq + (li >> 2);
    const int ck = 4 * (li & 3);
    const int perm_src = (16 * (li >> 2) + 4 * (li & 3) + lq) * 4;  // byte index of the source
    const float *pa = AKC ? Ab + (int64_t)min(m0 + crow, p.M - 1) * p.lda + k0 + ck
                          : Ab + (int64_t)(k0 + 4 * lq) * p.lda + row;
    const float *pb = BKC ? Bb + (int64_t)min(n0 + crow, p.N - 1) * p.ldb + k0 + ck
                          : Bb + (int64_t)(k0 + 4 * lq) * p.ldb + col;
    auto permute = [&](f4 v) {
        f4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            r[j] = __int_as_float(__builtin_amdgcn_ds_bpermute(perm_src, __float_as_int(v[j])));
        return r;
    };
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
    // the partial k-group (KS = 1 only), issued with the others
    const bool part = KS == 1 && G * TT < p.K;
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
    auto permute_group = [&](int g) {
        if constexpr (AKC) fa[g] = permute(fa[g]);
        if constexpr (BKC) fb[g] = permute(fb[g]);
    };
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (G >= 3 && KS > 1) {
        // The permutations of k-group g + 1 are issued right after the MFMAs of k-group g,
        // so their latency runs under those MFMAs, while the MFMAs of k-group g still start
        // as soon as its own operands have landed; left to itself the compiler paired each
        // permute with the MFMA that consumes it and waited for it in between (graph replay,
        // 100 calls, us, paired / pipelined: 256^3 NN 2.45 / 2.40, NT 2.58 / 2.48). Where a
        // wavefront has the whole tile or two k-groups the pairing stays ahead: config 2a
        // 3.107 / 3.126, config 2b 3.04 / 3.07.
        permute_group(0);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[g][j], fb[g][j], acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (g + 1 < G) permute_group(g + 1);
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) permute_group(g);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa[g][j], fb[g][j], acc, 0, 0, 0);
    }
    if (part) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[j], xb[j], acc, 0, 0, 0);
    }

    if constexpr (KS > 1) {  // add the other parts' tiles in k order
        red[w][lane] = acc;
        __syncthreads();
        if (kp != 0 || !live) return;
#pragma unroll
        for (int q = 1; q < KS; ++q) acc += red[w + q][lane];
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

template <int G, int KS>
int launch_g(hipStream_t st, const TinyArgs &a, bool akc, bool bkc) {
    constexpr int TPW = TWG / KS;  // tiles per work-group
    const dim3 grid((unsigned)((a.total + TPW - 1) / TPW)), block(TWG * 64);
    if (akc && bkc)
        MIGEMM_LAUNCH((gemm_tiny_kernel<true, true, G, KS>), grid, block, 0, st, a);
    else if (akc)
        MIGEMM_LAUNCH((gemm_tiny_kernel<true, false, G, KS>), grid, block, 0, st, a);
    else if (bkc)
        MIGEMM_LAUNCH((gemm_tiny_kernel<false, true, G, KS>), grid, block, 0, st, a);
    else
        MIGEMM_LAUNCH((gemm_tiny_kernel<false, false, G, KS>), grid, block, 0, st, a);
    return launch_status("gemm_tiny_kernel launch");
}

int64_t tiles16(const GemmDesc &d) {
    return (int64_t)((d.M + TT - 1) / TT) * ((d.N + TT - 1) / TT) * d.batch;
}

// Wavefronts per tile: 1 for K <= 80 (any K), 2 for K = 96 and 160, 4 for K = 128, 192, 256,
// 320 (whole 16-wide k-groups, at most five per wavefront); 0: not supported. K = 128 takes
// four wavefronts of two k-groups rather than two of four: the shorter MFMA chains and the
// extra wavefronts in flight outweigh the larger reduction (graph replay, 100 calls, us, two
// / four: config 2b 32 x 128 x 128 @ 128 x 64 3.54 / 3.35, 16 x 128 x 128 @ 128 x 64 2.91 /
// 2.68, 32 x 128 x 128 @ 128 x 128 4.83 / 4.68, 512 x 128 x 512 3.53 / 3.27, 4 x 256 x 128 @
// 128 x 256 TN 3.37 / 3.30, NT 32 x 128 x 128 @ 128 x 64 3.82 / 3.84).
int tiny_parts(const GemmDesc &d) {
    if (d.K <= TG_MAX * TT) return 1;
    if (d.K % (4 * TT) == 0 && d.K <= 4 * TG_MAX * TT) return 4;
    if (d.K % (2 * TT) == 0 && d.K <= 2 * TG_MAX * TT) return 2;
    return 0;
}

}  // namespace

bool tiny_supported(const GemmDesc &d) {
    return tiny_parts(d) > 0 && tiles16(d) <= (int64_t)0x7fffffff - TWG;
}

// Where the tiny kernel beats the other families (graph replay, 50 calls, us, previous
// choice / tiny):
//  * K <= 80, one wavefront per tile (K in 16..80, M x N from 64 x 64 x 64 batches to
//    4096 x 4096, NN, NT, TN): 32 x 128 x 64 @ 64 x 128 (config 2a) 4.37 / 3.83; 1024 x 32 x
//    1024 5.44 / 4.32 (tiled); 32 x 128 x 80 @ 80 x 128 6.63 / 4.06 (the register-staged
//    tiled kernel); 32 x 64 x 128 TN 4.65 / 3.62. It loses with few tiles, where the small
//    kernel's k division shortens each wavefront's MFMA chain (64 x 64 x 64 2.18 / 2.78;
//    256 x 64 x 512 2.86 / 3.03), and on large outputs, where the tiled kernels reuse operands
//    from LDS (2048 x 32 x 2048 9.83 / 10.59; 1024 x 64 x 2048 8.02 / 9.11) -- except at
//    K = 16 (4096 x 16 x 4096 24.5 / 20.5).
//  * K = 96..320, two or four wavefronts per tile (96 shapes, 60 won): 512-2048 tiles, e.g.
//    32 x 128 x 128 @ 128 x 64 (config 2b) 3.79 / 3.59 (two wavefronts per tile; four: 3.35),
//    32 x 128 x 96 @ 96 x 128 6.31 / 4.19
//    and 32 x 128 x 192 TN 8.25 / 6.30 (the register-staged tiled kernel), 4 x 64 x 320 @
//    320 x 512 5.30 / 3.98. It loses with 256 tiles (256 x 128 x 256 2.63 / 2.90), at 4096
//    tiles (1024 x 128 x 1024 7.21 / 8.03) and where the panel kernel applies (64 x 256 x
//    4096 4.19 / 4.85; batch-32 128 x 256 x 128 NT 5.40 / 5.94), which is therefore asked
//    first.
bool tiny_preferred(const GemmDesc &d) {
    // Outputs under 16 rows or columns only with one wavefront per tile (batch-32 15 x 77 x 1550
    // 6.1 us against 6.8 on the small kernel, batch-8 5 x 62 x 4700 TT 5.0 / 5.7; but 8 x 256
    // x 4096 on four wavefronts per tile 5.0 / 4.2).
    if (!tiny_supported(d)) return false;
    if ((d.M < 16 || d.N < 16) && tiny_parts(d) != 1) return false;
    const int64_t t = tiles16(d);
    if (tiny_parts(d) == 1) {
        // (B transposed took the small kernel above K = 48 while the K-contiguous loads
        // read 16 rows per 16 lanes; read coalesced it runs as NN does: batch-32 128 x 64 x
        // 128 NT 3.11 us against 4.01 on the small kernel, 512 x 64 x 512 2.63 / 3.31)
        if (t < (d.K <= 48 ? 512 : 1024)) return false;
        // Outputs of 64 MB or more over K <= 16 are bound by writing C: where C's rows start
        // on 128-byte lines the tiled kernel's 128x128 tiles store whole lines, these 16x16
        // tiles half lines (graph replay, us, this kernel / 128x128: 65536 x 3 x 4096 395.3
        // / 220.3, 16384 x 8 x 16384 429.2 / 268.6, 9868 x 8 x 6208 NT 136.9 / 61.0, batch-16
        // 1024 x 8 x 1024 31.7 / 21.5; a torch fill of the same C: 157.3 for the first).
        // Rows off the lines make each of the larger tiles' row stores straddle two lines,
        // and this kernel stays (7008 x 6 x 6220 54.0 / 128.7, 4556 x 1 x 14292 65.5 /
        // 204.5).
        if (d.K <= 16 && t >= 65536 && d.ldc % 32 == 0 && (d.batch == 1 || d.sC % 32 == 0) &&
            ((uintptr_t)d.C & 127) == 0)
            return false;
        if (d.K <= 16) return true;
        // Above these tile counts larger outputs go to the tiled kernel (graph replay, us, this
        // kernel / 64x64 tiles: 1 x 4296 x 33 x 618 10.0 / 11.3, batch-8 615 x 17 x 711 10.5 /
        // 11.7, 269 x 68 x 5623 8.8 / 10.3; batch-8 512 x 79 x 681 TN 17.2 / 12.1, 2195 x 26 x
        // 6327 NT 30.2 / 25.8); outputs under 16 rows or columns stay here (small kernel /
        // this one: batch-32 11 x 33 x 18406 38.0 / 20.8, batch-32 2 x 35 x 7626 TN 18.9 /
        // 12.0, 8 x 40 x 200000 16.0 / 11.0; 29 of 30 such shapes faster here).
        return t <= (d.K <= 48 ? 16384 : 8192) || d.M < 16 || d.N < 16;
    }
    // From 64 tiles when A is K-contiguous (coalesced loads; graph replay, us, small kernel
    // / this one: 256 x 256 x 256 NN 2.94 / 2.50, NT 2.83 / 2.63, 128 x 256 x 128 NN 2.81 /
    // 2.32, 256 x 320 x 256 NN 3.41 / 2.81); a transposed A (four 4-byte loads per
    // fragment) keeps the small kernel below 512 tiles (256 x 256 x 256 TN 2.83 / 2.95).
    if (t < (d.transA ? 512 : 64) || t > 2048) return false;
    return !panel_preferred(d);
}

int launch_gemm_tiny(hipStream_t stream, const GemmDesc &d) {
    if (!tiny_supported(d))
        return set_error(MIGEMM_ERR_UNSUPPORTED,
                         "gemm_tiny: K=%d (needs K <= 80, or K = 96, 128, 160, 192, 256, 320)",
                         d.K);
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
    const int ks = tiny_parts(d);
    if (ks == 1) {
        switch (d.K / TT) {
            case 0: rc = launch_g<0, 1>(stream, a, akc, bkc); break;
            case 1: rc = launch_g<1, 1>(stream, a, akc, bkc); break;
            case 2: rc = launch_g<2, 1>(stream, a, akc, bkc); break;
            case 3: rc = launch_g<3, 1>(stream, a, akc, bkc); break;
            case 4: rc = launch_g<4, 1>(stream, a, akc, bkc); break;
            default: rc = launch_g<5, 1>(stream, a, akc, bkc); break;
        }
    } else if (ks == 2) {  // K = 96, 160
        switch (d.K / (2 * TT)) {
            case 3: rc = launch_g<3, 2>(stream, a, akc, bkc); break;
            default: rc = launch_g<5, 2>(stream, a, akc, bkc); break;
        }
    } else {  // K = 128, 192, 256, 320
        switch (d.K / (4 * TT)) {
            case 2: rc = launch_g<2, 4>(stream, a, akc, bkc); break;
            case 3: rc = launch_g<3, 4>(stream, a, akc, bkc); break;
            case 4: rc = launch_g<4, 4>(stream, a, akc, bkc); break;
            default: rc = launch_g<5, 4>(stream, a, akc, bkc); break;
        }
    }
    record_plan("tiny", d, TT, TT, ks, 0);
    return rc;
}

}  // namespace migemm
