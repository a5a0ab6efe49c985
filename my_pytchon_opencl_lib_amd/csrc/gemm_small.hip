// Small-output fp32 GEMM for gfx950 (v_mfma_f32_16x16x4_f32): shapes whose C has too few
// 64x64 tiles to occupy the 256 CUs. These are the latency-bound calls of the matmul path:
// the 256^3 matmul_tiled test GEMM, the batch-32 attention BMMs, and the 64-row gate GEMM
// of lstm_gemm_xw (cs/cl_kernels/lstm.cl:273) and linear_forward_tiled
// (cs/cl_kernels/linear.cl:14) at small batch ("cs/" = csharp/cstorchcl/cstorchcl/).
//
// In the tiled kernel one wavefront walks the whole K range of its 32x32 sub-tile, so with
// few tiles the MFMA chain of a single wavefront is the run time. Here the K range is
// divided among the wavefronts instead:
//  * A work-group owns a (16*MB) x (16*NB) tile of C and has NW wavefronts; wavefront w
//    multiplies the w-th contiguous share of the work-group's 16-wide k-groups, and the NW
//    partial tiles are added in LDS in the order w = 0..NW-1 (deterministic).
//  * Work-groups are dealt to the 8 XCDs in contiguous chunks of tiles, and consecutive
//    tiles step along the shorter side of C, so each XCD's L2 holds a contiguous share of
//    the larger operand.
//  * No LDS staging of operands: wavefronts of one work-group share no operand data (each
//    has its own k range), so fragments go from global memory (L2) straight to registers,
//    three k-groups in flight per wavefront.
//  * Fragments: in step j (0..3) of a k-group, lane l supplies row/column l%16 at
//    k = 4*(l/16) + j. An operand contiguous in M or N fetches four 32-bit values, 16
//    lanes covering 64 contiguous bytes. A K-contiguous operand is fetched with one
//    coalesced 128-bit load per lane (4 rows x 64 bytes per 16 lanes) and moved into
//    fragment order by a lane permutation. Both operands use the same k order, so the
//    sum is the full dot product; only the fp32 association order differs from the
//    reference's ascending chain.
//  * Edges: rows beyond M and columns beyond N are clamped on load and never stored; the
//    last, partial k-group (K % 16 != 0) is loaded element by element with k >= K set to
//    zero in both operands.
//  * If the output tiles times the wavefronts still cannot fill the chip, the k-groups
//    are further divided into S ranges over work-groups; range s writes its partial tile
//    to the library workspace and reduce_slices_kernel adds the ranges in order (then the
//    bias), as the tiled kernel's split-K does.
#include <stdlib.h>

#include <algorithm>

#include "migemm_internal.h"

namespace migemm {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

struct SmallArgs {
    const float *A;
    const float *B;
    const float *bias;
    float *C;
    int64_t lda, ldb, ldc;
    int64_t sA, sB, sC;
    int M, N, K;
    int tiles_m, tiles_n;  // tiles per batch entry
    int batch;
    int total;             // tiles_m * tiles_n * batch * splits
    int splits;            // k ranges over work-groups (1 = none)
    int groups_per_split;  // 16-wide k-groups per range
    float *partial;        // [splits][batch][M][N] when splits > 1
    int accumulate;        // C += result instead of C = result
    int m_fast;            // consecutive tiles step along M (else along N)
    // launch-invariant divisors of the work-group decomposition (multiply-high divisions:
    // with hardware-less 32-bit divisions the prologue before the first load took ~0.6 us
    // of the 256^3 GEMM's 2.4 us)
    FastDiv per_split;     // tiles_m * tiles_n * batch
    FastDiv per_batch;     // tiles_m * tiles_n
    FastDiv fast;          // tiles_m if m_fast, else tiles_n
};

constexpr int KG = 16;       // k values per k-group (4 MFMA steps of 4)
constexpr int INFLIGHT = 3;  // k-groups of loads in flight per wavefront

__device__ __forceinline__ f4 load16(const float *p) {
    f4 v;
    __builtin_memcpy(&v, p, sizeof(v));
    return v;
}

// One k-group (16 values of k, four MFMA steps j of 4) of a wavefront's operands: a[blk]
// for 16-row block blk of A, b[nb] for 16-column block nb of B. M/N-contiguous operand: the
// fragment values of steps j = 0..3. K-contiguous operand: the 128-bit load, before the
// lane permutation.
template <int MB, int NB>
struct Frag {
    f4 a[MB];
    f4 b[NB];
};

template <int MB, int NB, int NW, bool AKC, bool BKC>
__global__ void __launch_bounds__(NW * 64) gemm_small_kernel(SmallArgs p) {
    __shared__ float red[NW][MB * NB * 4][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int li = lane & 15;  // fragment row (A) / column (B) of this lane in a 16-block
    const int lq = lane >> 4;  // fragment k quarter of this lane in a k-group

    // ---- work-group -> (split, batch, tile); consecutive tiles share an XCD ----
    int pid = blockIdx.x;
    const int total = p.total;
    // (a select, not a branch: a branch here splits the kernel-argument loads in two rounds)
    pid = (total & 7) == 0 ? (pid & 7) * (total >> 3) + (pid >> 3) : pid;
    const int split = (int)fast_div((uint32_t)pid, p.per_split);
    pid -= split * (int)p.per_split.d;
    const int b = (int)fast_div((uint32_t)pid, p.per_batch);
    const int t = pid - b * (int)p.per_batch.d;
    const int slow = (int)fast_div((uint32_t)t, p.fast);
    const int quick = t - slow * (int)p.fast.d;
    const int tm = p.m_fast ? quick : slow;
    const int tn = p.m_fast ? slow : quick;
    const int m0 = tm * 16 * MB;
    const int n0 = tn * 16 * NB;

    const float *Ab = p.A + (int64_t)b * p.sA;
    const float *Bb = p.B + (int64_t)b * p.sB;

    // The bias of this thread's output column (every element it stores in the epilogue is
    // in column n0 + tid % (16 NB)), loaded now so its latency overlaps the k loop.
    const int ncol = n0 + tid % (16 * NB);
    const float bias_v =
        p.bias != nullptr && p.splits == 1 && ncol < p.N ? p.bias[ncol] : 0.f;

    // Per-lane operand pointers at k-group 0 (rows / columns clamped).
    // AKC: A(i, k) = Ab[i*lda + k]; else A(i, k) = Ab[k*lda + i]. BKC: B(k, n) = Bb[n*ldb + k];
    // else B(k, n) = Bb[k*ldb + n].
    // An operand contiguous in M or N is read in fragment order: lane (lq, li) loads
    // row/column li at k = 4*lq + j, and each 16-lane group covers 64 contiguous bytes.
    // A K-contiguous operand read in fragment order would give every 16-lane group 16
    // different rows (16 bytes each, 4x the L1 accesses of the data), so it is read
    // coalesced instead: lane (lq, li = 4a + c) loads the 16 bytes of row 4*lq + a at
    // k = 4c .. 4c+3 (a 16-lane group reads 4 rows x 64 contiguous bytes), and a lane
    // permutation (ds_bpermute, no LDS storage) gives lane (lq, li) row li at k = 4*lq + j.
    const int crow = 4 * lq + (li >> 2);
    const int ck = 4 * (li & 3);
    const int perm_src = (16 * (li >> 2) + 4 * (li & 3) + lq) * 4;  // byte index of source lane
    const float *pa[MB];
#pragma unroll
    for (int blk = 0; blk < MB; ++blk) {
        if constexpr (AKC)
            pa[blk] = Ab + (int64_t)min(m0 + blk * 16 + crow, p.M - 1) * p.lda + ck;
        else
            pa[blk] = Ab + (int64_t)(4 * lq) * p.lda + min(m0 + blk * 16 + li, p.M - 1);
    }
    const float *pb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        if constexpr (BKC)
            pb[nb] = Bb + (int64_t)min(n0 + nb * 16 + crow, p.N - 1) * p.ldb + ck;
        else
            pb[nb] = Bb + (int64_t)(4 * lq) * p.ldb + min(n0 + nb * 16 + li, p.N - 1);
    }
    // distance between consecutive k-groups
    const int64_t a_gstep = AKC ? KG : (int64_t)KG * p.lda;
    const int64_t b_gstep = BKC ? KG : (int64_t)KG * p.ldb;

    auto load = [&](Frag<MB, NB> &f, int g) {
#pragma unroll
        for (int blk = 0; blk < MB; ++blk) {
            const float *q = pa[blk] + g * a_gstep;
            if constexpr (AKC)
                f.a[blk] = load16(q);
            else
                f.a[blk] = f4{q[0], q[p.lda], q[2 * p.lda], q[3 * p.lda]};
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const float *q = pb[nb] + g * b_gstep;
            if constexpr (BKC)
                f.b[nb] = load16(q);
            else
                f.b[nb] = f4{q[0], q[p.ldb], q[2 * p.ldb], q[3 * p.ldb]};
        }
    };

    auto permute = [&](f4 v) {
        f4 r;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            r[j] = __int_as_float(__builtin_amdgcn_ds_bpermute(perm_src, __float_as_int(v[j])));
        return r;
    };

    f4 acc[MB][NB];
#pragma unroll
    for (int blk = 0; blk < MB; ++blk)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[blk][nb] = f4{0.f, 0.f, 0.f, 0.f};

    // `direct`: the operands were loaded in fragment order (the partial k-group).
    auto mma = [&](const Frag<MB, NB> &f, bool direct) {
        f4 fa[MB], fb[NB];
#pragma unroll
        for (int blk = 0; blk < MB; ++blk)
            fa[blk] = AKC && !direct ? permute(f.a[blk]) : f.a[blk];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
            fb[nb] = BKC && !direct ? permute(f.b[nb]) : f.b[nb];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int blk = 0; blk < MB; ++blk)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
                    acc[blk][nb] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                        fa[blk][j], fb[nb][j], acc[blk][nb], 0, 0, 0);
    };

    // ---- k-groups of this wavefront ----
    const int K = p.K;
    const int G = (K + KG - 1) / KG;
    const int gfull = K / KG;  // k-groups entirely inside K
    const int gs0 = split * p.groups_per_split;
    const int gs1 = min(G, gs0 + p.groups_per_split);
    const int per_wave = (gs1 - gs0 + NW - 1) / NW;
    const int glo = min(gs1, gs0 + w * per_wave);
    const int ghi = min(gs1, glo + per_wave);
    const int gend = min(ghi, gfull);

    if (glo < gend) {
        // Each work-group starts its wavefronts' ranges at its own rotation, so the work-
        // groups of an XCD, which read the same A (or B) panel, do not all request the
        // same lines from the same L2 channels at the same time.
        const int nfg = gend - glo;
        // rotation in [0, nfg): the top 10 bits of a multiplicative hash of the work-group
        // id, scaled (a remainder would be another division in the prologue)
        const unsigned hash = (blockIdx.x * 2654435761u) >> 22;
        const int rot = (int)((hash * (unsigned)nfg) >> 10);
        auto kgroup = [&](int i) {  // i-th k-group of the range, i < nfg
            const int x = i + rot;
            return glo + (x >= nfg ? x - nfg : x);
        };
        // INFLIGHT register sets rotate; every load in the loop is unconditional (past the
        // end it re-reads the last k-group, which is never multiplied). The scheduling
        // barriers keep each set's loads together and in order: left free, the scheduler
        // sinks all refills to the end of the iteration and interleaves the sets, so the
        // first MFMA of an iteration has to wait for almost every load in flight.
        Frag<MB, NB> f[INFLIGHT];
#pragma unroll
        for (int i = 0; i < INFLIGHT; ++i) {
            load(f[i], kgroup(min(i, nfg - 1)));
            __builtin_amdgcn_sched_barrier(0);
        }
        int i0 = 0;
        for (; i0 + INFLIGHT <= nfg; i0 += INFLIGHT) {
#pragma unroll
            for (int i = 0; i < INFLIGHT; ++i) {
                mma(f[i], false);
                __builtin_amdgcn_sched_barrier(0);
                load(f[i], kgroup(min(i0 + INFLIGHT + i, nfg - 1)));
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll
        for (int i = 0; i < INFLIGHT; ++i)
            if (i < nfg - i0) mma(f[i], false);
    }
    if (ghi > gfull && glo <= gfull) {
        // the partial k-group: element-wise loads in fragment order, k >= K zero in both
        // operands
        Frag<MB, NB> f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = gfull * KG + 4 * lq + j;
            const bool ok = k < K;
#pragma unroll
            for (int blk = 0; blk < MB; ++blk) {
                const int i = min(m0 + blk * 16 + li, p.M - 1);
                const int64_t off = AKC ? (int64_t)i * p.lda + k : (int64_t)k * p.lda + i;
                f.a[blk][j] = ok ? Ab[off] : 0.f;
            }
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int nc = min(n0 + nb * 16 + li, p.N - 1);
                const int64_t off = BKC ? (int64_t)nc * p.ldb + k : (int64_t)k * p.ldb + nc;
                f.b[nb][j] = ok ? Bb[off] : 0.f;
            }
        }
        mma(f, true);
    }

    // ---- combine the NW wavefronts in order, then store (or write the partial) ----
    // Output layout of v_mfma_f32_16x16x4_f32: lane l, register r holds row 4*(l/16) + r,
    // column l%16 of its 16x16 block.
#pragma unroll
    for (int blk = 0; blk < MB; ++blk)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[w][(blk * NB + nb) * 4 + r][lane] = acc[blk][nb][r];
    __syncthreads();

    for (int e = tid; e < MB * NB * 256; e += NW * 64) {
        const int row = e / (16 * NB);  // 0 .. 16*MB-1
        const int col = e % (16 * NB);  // 0 .. 16*NB-1
        const int slot = ((row >> 4) * NB + (col >> 4)) * 4 + (row & 3);
        const int src = ((row & 15) >> 2) * 16 + (col & 15);
        float v = red[0][slot][src];
#pragma unroll
        for (int q = 1; q < NW; ++q) v += red[q][slot][src];
        const int m = m0 + row;
        const int n = n0 + col;
        if (m < p.M && n < p.N) {
            if (p.splits == 1) {
                if (p.bias != nullptr) v = v + bias_v;  // n = ncol: NW * 64 % (16 NB) == 0
                float *c = p.C + (int64_t)b * p.sC + (int64_t)m * p.ldc + n;
                *c = p.accumulate ? *c + v : v;
            } else {
                p.partial[(((int64_t)split * p.batch + b) * p.M + m) * p.N + n] = v;
            }
        }
    }
}

template <int MB, int NB, int NW>
int launch_layout(hipStream_t st, const SmallArgs &a, bool akc, bool bkc) {
    const dim3 grid(a.total), block(NW * 64);
    if (akc && bkc)
        MIGEMM_LAUNCH((gemm_small_kernel<MB, NB, NW, true, true>), grid, block, 0, st, a);
    else if (akc)
        MIGEMM_LAUNCH((gemm_small_kernel<MB, NB, NW, true, false>), grid, block, 0, st, a);
    else if (bkc)
        MIGEMM_LAUNCH((gemm_small_kernel<MB, NB, NW, false, true>), grid, block, 0, st, a);
    else
        MIGEMM_LAUNCH((gemm_small_kernel<MB, NB, NW, false, false>), grid, block, 0, st, a);
    return launch_status("gemm_small_kernel launch");
}

template <int MB, int NB = 1>
int launch_nw(hipStream_t st, const SmallArgs &a, int nw, bool akc, bool bkc) {
    return nw == 8 ? launch_layout<MB, NB, 8>(st, a, akc, bkc)
                   : launch_layout<MB, NB, 4>(st, a, akc, bkc);
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct SmallPlan {
    int mb, nb, nw, splits;
    int64_t wgs;  // work-groups without the k split
};

// Largest row block MB (<= 4, no larger than M needs) whose tiles, after dividing K over
// at most 16 ranges of >= 2 k-groups per wavefront, give the 256 CUs a work-group each;
// failing that MB = 1. A larger MB reads B fewer times (B is re-read once per 16*MB rows).
SmallPlan plan_small(const GemmDesc &d) {
    const int G = (int)cdiv(d.K, KG);
    const int nw = G >= 16 ? 8 : 4;
    const int mb_max = (int)(d.M > 48 ? 4 : cdiv(d.M, 16));
    SmallPlan pl{1, 1, nw, 1, 0};
    // k ranges that give `wgs` work-groups a CU each: at most 16, of >= 2 k-groups per
    // wavefront. Fewer than 16 tiles of one row block (`wide`, the plan the row-block search
    // below ends on for tiny outputs) may take more: as many as keep one work-group per CU,
    // of >= 8 k-groups per wavefront, and a multiple of 8 over several tiles so that each
    // XCD's contiguous chunk holds whole k ranges and the tiles of a range share its L2.
    // A dot product over K = 10^7 (1 x 10^7 x 1) streamed 40 MB through 16 work-groups in
    // 1151 us (70 GB/s), 95 us in 256 ranges; 40 tiny outputs over K = 4000-400000, graph
    // replay: 0.62x the total time, none more than 3 % slower.
    auto split_for = [&](int64_t wgs, bool wide = false) {
        const int64_t need = cdiv(256, wgs);
        int64_t cap = G / (2 * nw);
        if (cap > 16) cap = 16;
        if (cap < 1) cap = 1;
        int64_t s = need < cap ? need : cap;
        if (wide && wgs < 16) {
            int64_t w = std::min<int64_t>(256 / wgs, G / (8 * nw));
            if (wgs > 1) w -= w % 8;
            if (w > s) s = w;
        }
        return (int)s;
    };
    for (int mb = mb_max; mb >= 1; --mb) {
        const int64_t wgs = cdiv(d.M, 16 * mb) * cdiv(d.N, 16) * d.batch;
        const int s = split_for(wgs, mb == 1);
        pl = SmallPlan{mb, 1, nw, s, wgs};
        if (wgs * s >= 256) break;
    }
    // 32x32 tiles (2 row blocks x 2 column blocks) instead of 64x16 or 48x16 when A is
    // K-contiguous, with the same k split: a work-group then reads 4 fragments per k-group
    // instead of 5 (4), and a 32-row share of A. Measured (graph replay, us, 32x32 /
    // 64x16): 64 x 1536 x 4096 + bias 12.35 / 14.17; 64 x 1024 x 4096 9.55 / 11.18;
    // 128 x 2048 x 2048 14.82 / 19.07; 777 x 300 x 300 6.20 / 8.69; 200 x 1024 x 1536
    // 15.31 / 17.19; 80 x 1024 x 4096 15.04 / 16.37; 200 x 777 x 300 (48x16) 8.82 / 10.10;
    // batch-32 128 x 128 x 64 4.24 / 4.71, 128 x 64 x 128 NT 4.60 / 4.76; 256^3 (16x16
    // plan, kept) 3.52 / 3.51; 100 x 777 x 300 (16x16 plan, kept) 9.00 / 8.11. With A
    // transposed they ran slower (64 x 1536 x 4096 TN 18.84 / 16.84).
    // MIGEMM_TUNE_SMALL_TILES (tests and tuning): 1 never, 2 always (M, N > 16).
    // The k split is recomputed for the 32x32 grid, so the split and small_preferred's
    // whole-K test judge the grid that is launched.
    const int force_nb = tuning(MIGEMM_TUNE_SMALL_TILES);
    if (force_nb == 2 ? d.M > 16 && d.N > 16
                      : force_nb != 1 && pl.mb >= 3 && d.N > 16 && !d.transA) {
        const int64_t wgs22 = cdiv(d.M, 32) * cdiv(d.N, 32) * d.batch;
        pl = SmallPlan{2, 2, nw, split_for(wgs22), wgs22};
    }
    // 16 MB or more of operands already split into 2-15 k ranges over fewer than 384
    // work-groups: 1.5x the ranges, rounded to an even count (graph replay, us, before /
    // after: 1846 x 4713 x 17 19.98 / 16.15, batch-8 29 x 19424 x 142 44.56 / 33.30, 13 x
    // 5919 x 1365 24.14 / 15.83; 19 of 19 such shapes 0.66-0.96x; on 70 others 21 of 23
    // changed plans faster, 0.973x the total, batch-8 249 x 5255 x 8 TN 14.56 / 17.85 the
    // worst). Not from 16 ranges (237 x 15478 x 15 8.34 / 9.76) nor from 384 work-groups (12
    // x 2713 x 4013 NT 15.24 / 16.16).
    const double bytes = 4.0 * d.batch * ((double)d.M * d.K + (double)d.K * d.N);
    if (bytes >= 16e6 && pl.splits >= 2 && pl.splits < 16 && pl.wgs * pl.splits < 384) {
        int s = 3 * pl.splits / 2;
        if ((3 * pl.splits) % 2 != 0 && s % 2 != 0) ++s;
        if (2 * s <= G) pl.splits = s;
    }
    return pl;
}

}  // namespace

// Where the small kernel beats the tiled one (graph replay over a grid of M, N in 1..6000
// and K in 16..8192, NN and TN, then a sweep of M in {64, 128, 200}, N in {512, 1536, 4096},
// K in {1024 .. 8192}; shapes are M x K x N, us, small / tiled):
//  * M or N <= 4 (unless B is large enough for the skinny kernel): the tiled kernel's
//    64-wide tiles would be almost empty (6000 x 8192 x 1 48 / 63; 3 x 300 x 300 4.5 / 10.0).
//  * fewer 64x64 tiles than CUs, and then
//    - a thin output (M or N <= 32) or K <= 64 (17 x 8192 x 1024 14.4 / 18.5);
//    - K <= 1024: fewer than 24 tiles, or a plan without a k split (no reduce launch) and
//      then, with 32x32 tiles, fewer than 128 tiles or K >= 768 (128 x 1024 x 4096 16.1 /
//      20.7; 512 x 1024 x 1024 16.1 / 20.8; 2048 x 300 x 300 15.8 / 11.1); with 64x16 tiles
//      fewer than 128 (777 x 300 x 300 9.1 / 10.6; 200 x 1024 x 1536 17.7 / 18.4), or 80
//      with A transposed (TN: 64 x 1024 x 4096 12.1 / 14.0, 200 x 1024 x 1536 22.8 / 18.6,
//      512 x 1024 x 1024 22.7 / 21.1); with a k split the tiled kernel wins: 64 x 1024 x
//      1536 12.7 / 11.6, 200 x 1024 x 512 13.1 / 11.8;
//    - K <= 2048: fewer than 12 tiles, or a plan without a k split and then, with 32x32
//      tiles, fewer than 80 tiles or M <= 128 (64 x 1536 x 4096 14.1 / 19.0; 128 x 2048 x
//      4096 28.3 / 30.3; 200 x 2048 x 1536 33.1 / 27.1; 6000 x 2048 x 64 28.5 / 26.4); with 64x16
//      tiles fewer than 80, with A transposed and K > 1536 fewer than 48 (TN: 64 x 1536 x
//      4096 17.4 / 19.8, 64 x 2048 x 4096 21.8 / 19.3, 128 x 2048 x 4096 43.7 / 30.7);
//      200 x 2048 x 300 14.7 / 11.6 and 6000 x 2048 x 64 28.7 / 26.8 split;
//    - longer K with at most 8 tiles (64 x 4096 x 512 10.5 / 11.8; 128 x 8192 x 128 11.7 /
//      13.4; 256 x 4096 x 256 takes the tiled split, 14.2 / 13.6).
bool narrow_rows_streaming(const GemmDesc &d) {
    return d.M > 4 && d.M <= 16 && !d.transB &&
           (int64_t)d.K * d.N * d.batch * 4 >= ((int64_t)256 << 20);
}

bool small_preferred(const GemmDesc &d) {
    // Outputs 16 or fewer rows (or columns) wide: the tiled kernels' 64-256 wide tiles would
    // be mostly empty (graph replay, us, small / tiled: batch-32 8 x 195 x 3480 20.9 / 53.9,
    // batch-32 3000 x 200 x 12 21.0 / 33.0, batch-16 2048 x 512 x 16 TN 16.8 / 22.6,
    // batch-16 16 x 1024 x 4096 58.9 / 68.0).
    // Except few rows over a B of 256 MB or more (B not transposed): the tiled kernel's 32x32
    // tiles stream B in longer row segments (batch-16 16 x 2048 x 4096 100.8 / 157.4 us on
    // this kernel, batch-16 8 x 6000 x 1024 89.0 / 115.8, batch-16 16 x 1024 x 4096 46.1 /
    // 57.6; batch-16 8 x 2048 x 1024, 134 MB, 32.8 / 28.9).
    if (narrow_rows_streaming(d)) return false;
    if (d.M <= 16 || d.N <= 16) return true;
    const int64_t tiles64 = cdiv(d.M, 64) * cdiv(d.N, 64) * d.batch;
    if (tiles64 >= 256) return false;
    // Short K below one round of 64x64 tiles: the tiled kernel's 32x32 tiles lose to these
    // (1000 x 100 x 700 6.95 / 9.15, 3567 x 164 x 199 TN 11.1 / 15.5, batch-2 187 x 129 x
    // 1259 TN 7.8 / 12.3, batch-8 300 x 84 x 200 6.4 / 7.9).
    if (d.K < 256) return true;
    const int mn = d.M < d.N ? d.M : d.N;
    if (mn <= 32 || d.K <= 64) return true;
    if (d.K <= 2048) {
        const SmallPlan pl = plan_small(d);
        const bool whole = pl.splits == 1;
        if (pl.nb == 2) {  // 32x32 tiles
            if (d.K <= 1024) return tiles64 < 24 || (whole && (tiles64 < 128 || d.K >= 768));
            // up to 16 tiles also with a k split (256 x 2048 x 256 9.2 against 10.2 us tiled)
            return tiles64 <= 16 || (whole && (tiles64 < 80 || d.M <= 128));
        }
        if (!d.transA) {  // 64x16 tiles, A K-contiguous
            if (d.K <= 1024) return tiles64 < 24 || (whole && tiles64 < 128);
            return tiles64 < 12 || (whole && tiles64 < 80);
        }
        // (A transposed) up to K = 512 also with a k split at <= 32 tiles: 256 x 512 x 512 TN
        // 8.0 against 10.3 us tiled, batch-8 128 x 512 x 128 TN 8.1 / 10.3
        if (d.K <= 512 && tiles64 <= 32) return true;
        if (d.K <= 1024) return tiles64 < 24 || (whole && tiles64 < 80);
        return tiles64 < 12 || (whole && tiles64 < (d.K <= 1536 ? 80 : 48));
    }
    // longer K: up to 8 tiles, or 16 with A K-contiguous (256 x 8192 x 256 17.7 against
    // 18.8 us tiled, 512 x 8192 x 128 17.6 / 18.9)
    return tiles64 <= (d.transA ? 8 : 16);
}

int launch_gemm_small(hipStream_t stream, const GemmDesc &d) {
    SmallPlan pl = plan_small(d);
    const int force_split = tuning(MIGEMM_TUNE_SMALL_SPLITK);
    if (force_split >= 1) pl.splits = force_split;

    SmallArgs a;
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
    a.accumulate = d.accumulate;
    a.tiles_m = (int)cdiv(d.M, 16 * pl.mb);
    a.tiles_n = (int)cdiv(d.N, 16 * pl.nb);
    // Consecutive tiles (which share an XCD's L2) step along the shorter side, so each XCD
    // reads a contiguous share of the larger operand. Against stepping along N (us):
    // 64 x 1536 x 4096 (32x32 tiles) 12.35 / 13.73; 80 x 1024 x 4096 16.55 / 19.21;
    // 80 x 2048 x 2048 15.31 / 18.56; 128 x 1024 x 4096 TN 22.32 / 22.94.
    a.m_fast = d.N >= d.M;
    a.batch = d.batch;
    const int G = (int)cdiv(d.K, KG);
    a.groups_per_split = (int)cdiv(G, pl.splits);
    a.splits = (int)cdiv(G, a.groups_per_split);  // no empty range
    // More than 16 ranges over several tiles: whole k ranges per XCD chunk (a range count
    // that is a multiple of 8) also after the rounding above; the next such count down.
    // With a range split over two XCDs its tiles' operand lines are fetched into both L2s
    // (33 x 100000 x 33 TN in 9 tiles: 29 ranges 44.2 us, 16 ranges 23.6).
    if (a.splits > 16 && pl.wgs > 1 && a.splits % 8 != 0) {
        for (int s = a.splits - 1; s >= 16; --s) {
            const int gps = (int)cdiv(G, s);
            const int s2 = (int)cdiv(G, gps);
            if (s2 % 8 == 0) {
                a.groups_per_split = gps;
                a.splits = s2;
                break;
            }
        }
    }
    const int64_t total = pl.wgs * a.splits;
    if (total > 0x7fffffff)
        return set_error(MIGEMM_ERR_UNSUPPORTED, "gemm_small: %lld work-groups", (long long)total);
    a.total = (int)total;
    a.per_split = make_fastdiv((uint32_t)(pl.wgs));
    a.per_batch = make_fastdiv((uint32_t)(a.tiles_m * a.tiles_n));
    a.fast = make_fastdiv((uint32_t)(a.m_fast ? a.tiles_m : a.tiles_n));
    a.partial = nullptr;
    if (a.splits > 1) {
        int st = MIGEMM_OK;
        a.partial = partial_buffer(stream, d,
                                   (size_t)a.splits * d.batch * d.M * d.N * sizeof(float), &st);
        if (a.partial == nullptr) return st;
    }
    const bool akc = !d.transA;
    const bool bkc = d.transB;
    int rc;
    switch (pl.mb) {
        case 4: rc = launch_nw<4>(stream, a, pl.nw, akc, bkc); break;
        case 3: rc = launch_nw<3>(stream, a, pl.nw, akc, bkc); break;
        case 2:
            rc = pl.nb == 2 ? launch_nw<2, 2>(stream, a, pl.nw, akc, bkc)
                            : launch_nw<2>(stream, a, pl.nw, akc, bkc);
            break;
        default: rc = launch_nw<1>(stream, a, pl.nw, akc, bkc); break;
    }
    record_plan("small", d, 16 * pl.mb, 16 * pl.nb, a.splits, 0);
    if (rc != MIGEMM_OK || a.splits == 1) return rc;
    return launch_reduce_slices(stream, a.partial, a.splits, d.batch, d.M, d.N, d.bias, d.C,
                                d.ldc, d.sC, d.accumulate);
}

}  // namespace migemm
