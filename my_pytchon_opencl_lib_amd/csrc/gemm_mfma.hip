// Tiled fp32 GEMM for gfx950 on the matrix cores (v_mfma_f32_32x32x2_f32).
//
// One kernel template covers every form of the reference matmul path:
//   matmul_tiled / bmm_tiled        (cl_kernels/matmul.cl:8-135)         -> NN
//   bmm_permute_tiled transA/transB (cs/cl_kernels/bmm_permute_tiled.cl) -> TN / NT
//   linear_forward_tiled, lstm_gemm_xw bias epilogue (cs/cl_kernels/linear.cl:107-143,
//   cs/cl_kernels/lstm.cl:340-366)
// ("cs/" = csharp/cstorchcl/cstorchcl/ in the reference repository.)
//
// Design (what differs from the reference's one-output-per-work-item 16x16 tiles):
//  * A work-group of WM x WN wavefronts computes a BM x BN tile of C; each wavefront owns
//    a (BM/WM) x (BN/WN) sub-tile made of 32x32 MFMA blocks whose fp32 accumulators stay
//    in registers for the whole K loop.
//  * Operands move global -> registers -> LDS with 128-bit loads and stores, double
//    buffered: tile k+1 is fetched from HBM/L2 while tile k is multiplied out of LDS, with
//    one barrier per BK step.
//  * Each operand keeps its global orientation in LDS. A K-contiguous operand (A not
//    transposed, B transposed) is stored [i][BK+4]; the +4 float pad puts the 8 (or 16)
//    rows touched by one 128-bit LDS read phase on disjoint banks, and one ds_read_b128
//    feeds four MFMA steps. An I-contiguous operand (A transposed, B not transposed) is
//    stored [k][T+8] and read with conflict-free 32-bit reads of 32 consecutive floats.
//  * The K order inside an MFMA step is permuted consistently for both operands: in step
//    s of k-group g, lanes 0-31 supply k = 8g+s and lanes 32-63 supply k = 8g+4+s. The
//    sum over k is unchanged; only the fp32 association order differs from the
//    reference's ascending chain (covered by the 1e-5*sqrt(K) tolerance).
//  * Edges: rows beyond M / columns beyond N are clamped on load (they only feed outputs
//    that are never stored); k >= K is zero-filled in both operands, as the reference's
//    zero padding does (matmul.cl:39-52). Stores are guarded to [M x N].
//  * Split-K: when the output has too few tiles to occupy the 256 CUs (skinny M, e.g. the
//    64-row LSTM gate GEMM), the k-tiles are divided into S contiguous ranges; range s
//    writes its fp32 partial tile to the library workspace and reduce_slices_kernel adds
//    the S partials of each output in order s = 0..S-1, then the bias (deterministic).
//  * Work-group ids are remapped so that consecutive output tiles land on the same XCD
//    (the dispatcher deals work-groups round-robin over the 8 XCDs, each with its own
//    L2), then rastered in groups of 8 tile-rows so concurrently running tiles share
//    A and B panels in that L2.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <type_traits>

#include "tiled_common.h"

namespace migemm {
namespace {

constexpr int PAD_K = 4;  // pad of a K-contiguous LDS tile row [i][BK + 4]
constexpr int PAD_I = 8;  // pad of an I-contiguous LDS tile row [k][T + 8]

// LDS layout of a K-contiguous tile: rows of BK floats padded to BK + 4 (row strides of 20
// and 36 floats). Measured on gfx950 with SQ_LDS_BANK_CONFLICT for 64-lane 128-bit
// accesses: the MFMA fragment reads (32 consecutive rows x 2 chunks) are conflict-free at
// both strides, and so are writes whose lanes cover 8 rows x 8 chunks (BK = 32) or 16
// rows x 4 chunks (BK = 16). Writes covering 16 rows as 4 consecutive lanes per row
// conflict (8 extra cycles per instruction at stride 20), which is why Operand lays its
// BK = 16 lanes out row-fastest.
template <int BK>
__device__ __forceinline__ int kc_off(int row, int chunk) {
    return row * (BK + PAD_K) + 4 * chunk;
}

template <int T, int BK, bool KC>
struct TileFloats {
    static constexpr int value = KC ? T * (BK + PAD_K) : BK * (T + PAD_I);
};

// 16 contiguous bytes from a 4-byte aligned address: gfx950 global loads do not need
// natural alignment (the target has unaligned-buffer-access), so this is one
// global_load_dwordx4 whatever the row stride of the operand.
__device__ __forceinline__ f4 load16(const float *p) {
    f4 v;
    __builtin_memcpy(&v, p, sizeof(v));
    return v;
}

// One operand tile (T rows of the M or N dimension by BK of the K dimension).
//  KC  : element (i, k) lives at base[i*ld + k] (K contiguous) else at base[k*ld + i].
//  VEC : the contiguous extent (K for KC, else the M or N extent) is a multiple of 4, so
//        every group of 4 contiguous elements is entirely inside or entirely outside the
//        matrix and is fetched with one 128-bit load. Otherwise a KC operand still uses
//        128-bit loads for full k-tiles and 32-bit loads only in the tail tile, and an
//        I-contiguous operand fetches its 4 columns (clamped at the edge) one by one.
// Per-thread source pointers are formed once per tile (rows beyond `rows` clamped), so a
// k-step only adds a uniform offset. load<false> is the unpredicated main-loop fetch;
// load<true> zero-fills k >= K for the single tail tile. The fetched registers are
// written to LDS one k-tile later (see the main loop), so loads stay in flight across a
// whole k-tile of MFMA work.
template <int T, int BK, int NT, bool KC, bool VEC>
struct Operand {
    static_assert((T * BK) % (4 * NT) == 0, "operand tile does not split over the threads");
    static constexpr int NLOAD = T * BK / (4 * NT);
    static constexpr int TPR = KC ? BK / 4 : T / 4;  // threads per LDS tile row
    static constexpr int RPP = NT / TPR;             // LDS tile rows per pass
    typedef f4 Regs[NLOAD];                          // one k-tile in flight
    const float *ptr[NLOAD];  // KC: start of global row i; else element (k = kr + p*RPP, i)
    int coff[4];              // !KC && !VEC: clamped column offsets of the 4 elements
    int c, rr;                // this thread's column (x4) and first tile row

    __device__ __forceinline__ void init(const float *__restrict__ base, int64_t ld, int i0,
                                         int rows, int tid) {
        if constexpr (KC && BK == 16) {
            // lanes row-fastest: a wavefront's 64 lanes cover 16 rows x 4 chunks
            const int lane = tid & 63;
            rr = (tid >> 6) * 16 + (lane & 15);
            c = (lane >> 4) * 4;
        } else {
            c = (tid % TPR) * 4;
            rr = tid / TPR;
        }
        if constexpr (KC) {
#pragma unroll
            for (int p = 0; p < NLOAD; ++p) {
                int gi = i0 + rr + p * RPP;
                gi = gi < rows ? gi : rows - 1;
                ptr[p] = base + (int64_t)gi * ld;
            }
        } else {
            int gi = i0 + c;
            if constexpr (VEC) {
                gi = gi < rows ? gi : rows - 4;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int g = i0 + c + e;
                    coff[e] = (g < rows ? g : rows - 1) - i0 - c;
                }
            }
#pragma unroll
            for (int p = 0; p < NLOAD; ++p) ptr[p] = base + (int64_t)(rr + p * RPP) * ld + gi;
        }
    }

    // Fetch k-tile k0.. into registers. TAIL (the tile holding K's end) only clamps the
    // addresses of k >= K to column / row 0 so every access stays inside the operand; the
    // fetched values there are discarded by store<true>. Both forms issue the same loads,
    // which keeps the compiler's load counters exact across the main loop.
    template <bool TAIL>
    __device__ __forceinline__ void load(Regs &r, int64_t ld, int k0, int K) const {
        if constexpr (KC) {
            const int gk = k0 + c;
#pragma unroll
            for (int p = 0; p < NLOAD; ++p) {
                if constexpr (VEC) {
                    r[p] = load16(ptr[p] + ((!TAIL || gk < K) ? gk : 0));
                } else if constexpr (!TAIL) {
                    r[p] = load16(ptr[p] + gk);  // a full k-tile: gk + 3 < K
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[p][e] = ptr[p][gk + e < K ? gk + e : 0];
                }
            }
        } else {
            const int64_t koff = (int64_t)k0 * ld;
#pragma unroll
            for (int p = 0; p < NLOAD; ++p) {
                const float *src = ptr[p] + koff;
                if constexpr (TAIL) {
                    // a k row past K is replaced by row 0 of the tile's source
                    if (k0 + rr + p * RPP >= K) src = ptr[p] - (int64_t)(rr + p * RPP) * ld;
                }
                if constexpr (VEC) {
                    r[p] = load16(src);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[p][e] = src[coff[e]];
                }
            }
        }
    }

    // Write a fetched k-tile to LDS; TAIL zero-fills k >= K (matmul.cl:39-52 pads both
    // operands with zeros) before the write.
    template <bool TAIL>
    __device__ __forceinline__ void store(const Regs &r, float *lds, int k0, int K) const {
#pragma unroll
        for (int p = 0; p < NLOAD; ++p) {
            f4 v = r[p];
            if constexpr (TAIL) {
                if constexpr (KC) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = (k0 + c + e < K) ? v[e] : 0.f;
                } else {
                    if (k0 + rr + p * RPP >= K) v = f4{0.f, 0.f, 0.f, 0.f};
                }
            }
            if constexpr (KC)
                *reinterpret_cast<f4 *>(lds + kc_off<BK>(rr + p * RPP, c >> 2)) = v;
            else
                *reinterpret_cast<f4 *>(lds + (rr + p * RPP) * (T + PAD_I) + c) = v;
        }
    }
};

// MFMA operand fragments of k-group g (8 consecutive k of the LDS tile) for F blocks of
// 32 rows starting at `off`: fr[f][s] is this lane's value for MFMA step s.
template <int T, int BK, bool KC, int F>
__device__ __forceinline__ void read_frags(const float *lds, int off, int g, int lane,
                                           f4 (&fr)[F]) {
    const int lo = lane & 31;
    const int hi = lane >> 5;
    if constexpr (KC) {
#pragma unroll
        for (int f = 0; f < F; ++f)
            fr[f] = *reinterpret_cast<const f4 *>(lds + kc_off<BK>(off + f * 32 + lo, 2 * g + hi));
    } else {
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                fr[f][s] = lds[(8 * g + 4 * hi + s) * (T + PAD_I) + off + f * 32 + lo];
    }
}

template <int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, bool AV, bool BV>
__global__ void __launch_bounds__(WM *WN * 64) __attribute__((amdgpu_waves_per_eu(2)))
gemm_mfma_kernel(TiledArgs p) {
    constexpr int NT = WM * WN * 64;
    constexpr int WTM = BM / WM;
    constexpr int WTN = BN / WN;
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "bad wave tile");
    static_assert(BK % 8 == 0, "BK must be a multiple of 8");
    constexpr int A_FL = TileFloats<BM, BK, AKC>::value;
    constexpr int B_FL = TileFloats<BN, BK, BKC>::value;
    constexpr int STAGE = A_FL + B_FL;
    __shared__ __attribute__((aligned(16))) float smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN;
    const int wn = wave % WN;

    const TileCoord tc = tile_coord<BM, BN>(p, blockIdx.x);
    const int split = tc.split;
    const int b = tc.b;
    const int m0 = tc.m0;
    const int n0 = tc.n0;

    const float *Ab = p.A + (int64_t)b * p.sA;
    const float *Bb = p.B + (int64_t)b * p.sB;

    typedef Operand<BM, BK, NT, AKC, AV> OpA;
    typedef Operand<BN, BK, NT, BKC, BV> OpB;
    OpA opa;
    OpB opb;

    f16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int K = p.K;
    const int nfull = K / BK;  // k-tiles entirely inside K; a later one is the zero-filled tail
    const int kt0 = split * p.kt_per_split;
    const int kt1 = min((K + BK - 1) / BK, kt0 + p.kt_per_split);

    opa.init(Ab, p.lda, m0, p.M, tid);
    opb.init(Bb, p.ldb, n0, p.N, tid);

    // Pipeline: global loads run two k-tiles ahead of the MFMAs in two register sets, the
    // LDS holds two stages. While tile kt is multiplied out of stage kt%2, the registers
    // of tile kt+1 (fetched one iteration earlier) are written to the other stage halfway
    // through, and tile kt+2 is being fetched. The barrier closing tile kt then only
    // orders LDS traffic; it never waits on global memory.
    // Full k-tiles [kt0, kf) run through the pipelined main loop, which contains no tail
    // code; the zero-filled tail tile (K % BK != 0, index nfull) follows it.
    auto fetch = [&](typename OpA::Regs &ra, typename OpB::Regs &rb, int kt) {
        opa.template load<false>(ra, p.lda, kt * BK, K);
        opb.template load<false>(rb, p.ldb, kt * BK, K);
    };
    auto put = [&](const typename OpA::Regs &ra, const typename OpB::Regs &rb, float *stage,
                   int kt) {
        opa.template store<false>(ra, stage, kt * BK, K);
        opb.template store<false>(rb, stage + A_FL, kt * BK, K);
    };
    auto group = [&](const float *cur, int g) {
        f4 fa[FM];
        f4 fb[FN];
        read_frags<BM, BK, AKC, FM>(cur, wm * WTM, g, lane, fa);
        read_frags<BN, BK, BKC, FN>(cur + A_FL, wn * WTN, g, lane, fb);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s],
                                                                     acc[i][j], 0, 0, 0);
    };
    const int kf = min(kt1, nfull);  // end of the full k-tiles of this range
    // One k-tile: `held` carries tile kt+1 in, `spare` receives tile kt+2. Every fetch and
    // LDS write in the main loop is unconditional (past the last full tile the fetch
    // re-reads it and the write lands in the stage nobody reads again), and the loop runs
    // whole pairs of steps, so the compiler's load counters see one straight-line pattern
    // and each LDS write waits only on the previous step's loads.
    auto step = [&](int kt, typename OpA::Regs &helda, typename OpB::Regs &heldb,
                    typename OpA::Regs &sparea, typename OpB::Regs &spareb) {
        const float *cur = smem + ((kt - kt0) & 1) * STAGE;
        float *nxt = smem + ((kt - kt0 + 1) & 1) * STAGE;
        fetch(sparea, spareb, min(kt + 2, kf - 1));
        constexpr int G = BK / 8;
#pragma unroll
        for (int g = 0; g < (G + 1) / 2; ++g) group(cur, g);
        put(helda, heldb, nxt, kt + 1);
#pragma unroll
        for (int g = (G + 1) / 2; g < G; ++g) group(cur, g);
        __syncthreads();
    };

    typename OpA::Regs ra0, ra1;
    typename OpB::Regs rb0, rb1;
    int kt = kt0;
    if (kt0 < kf) {
        fetch(ra0, rb0, kt0);
        put(ra0, rb0, smem, kt0);
        fetch(ra0, rb0, min(kt0 + 1, kf - 1));
        __syncthreads();
        for (; kt + 1 < kf; kt += 2) {
            step(kt, ra0, rb0, ra1, rb1);
            step(kt + 1, ra1, rb1, ra0, rb0);
        }
        if (kt < kf) {  // an odd last full tile, already in its LDS stage
            const float *cur = smem + ((kt - kt0) & 1) * STAGE;
#pragma unroll
            for (int g = 0; g < BK / 8; ++g) group(cur, g);
            ++kt;
        }
    }
    if (kt < kt1) {  // the tail tile: k >= K zero-filled in both operands
        opa.template load<true>(ra1, p.lda, kt * BK, K);
        opb.template load<true>(rb1, p.ldb, kt * BK, K);
        __syncthreads();  // every wavefront is done reading the stages
        opa.template store<true>(ra1, smem, kt * BK, K);
        opb.template store<true>(rb1, smem + A_FL, kt * BK, K);
        __syncthreads();
#pragma unroll
        for (int g = 0; g < BK / 8; ++g) group(smem, g);
    }

    store_tile<FM, FN>(p, tc, m0 + wm * WTM, n0 + wn * WTN, lane, acc);
}

// C_b[m, n] = partial[0][b][m][n] + ... + partial[S-1][b][m][n] (+ bias[n]), added in
// slice order. Each thread owns VW consecutive outputs of the flattened [batch][M][N]
// partial array (VW = 4, one 128-bit load per slice, only when the array's size is a
// multiple of 4; VW = 1 also spreads a small output, such as a GEMV's, over more CUs) and
// reads RS_GROUP slices at a time with every load of a group issued before the group is
// summed (a serial load-add chain would pay one full memory latency per slice).
// The kernel runs right after the kernel that wrote the partials, usually with its
// instructions out of every cache, so it is kept short: no tail path, slice addresses
// stepped in vector registers, 32-bit index arithmetic where the output allows. A general
// version (tail path, 64-bit division, 16 scalar slice offsets: 1300 instructions and ~95
// spilled scalar registers) added ~1.1 us to the 11008-column GEMV's 2 us reduction.
constexpr int RS_GROUP = 16;

// PLAIN: no bias, no accumulation and C contiguous ([batch][M][N] with ldc = N), so output
// t is C[t] and the epilogue needs no index arithmetic (the GEMV's and most split-K cases).
template <int VW, bool PLAIN>
__global__ void __launch_bounds__(256)
reduce_slices_kernel(const float *__restrict__ partial, int slices, int64_t total, int M, int N,
                     const float *__restrict__ bias, float *__restrict__ C, int64_t ldc,
                     int64_t strideC, int accumulate) {
    typedef float vec __attribute__((ext_vector_type(VW)));
    const int64_t nvec = total / VW;
    const int64_t step = (int64_t)gridDim.x * blockDim.x;
    for (int64_t vi = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; vi < nvec; vi += step) {
        const int64_t t = vi * VW;
        const float *src = partial + t;
        vec v;
        __builtin_memcpy(&v, src, sizeof(vec));
        for (int s0 = 1; s0 < slices; s0 += RS_GROUP) {
            vec x[RS_GROUP];
            const float *q = src + (int64_t)s0 * total;
#pragma unroll
            for (int g = 0; g < RS_GROUP; ++g) {
                if (s0 + g < slices) __builtin_memcpy(&x[g], q, sizeof(vec));
                q += total;
            }
#pragma unroll
            for (int g = 0; g < RS_GROUP; ++g)
                if (s0 + g < slices) v += x[g];
        }
        if constexpr (PLAIN) {
            __builtin_memcpy(C + t, &v, sizeof(vec));
            continue;
        }
        // (b, m, n) of element t
        int64_t b;
        int m, n;
        if (total <= INT32_MAX) {
            const uint32_t tt = (uint32_t)t;
            const uint32_t row = tt / (uint32_t)N;
            n = (int)(tt - row * (uint32_t)N);
            const uint32_t bb = row / (uint32_t)M;
            m = (int)(row - bb * (uint32_t)M);
            b = bb;
        } else {
            const int64_t row = t / N;
            n = (int)(t - row * N);
            b = row / M;
            m = (int)(row - b * M);
        }
#pragma unroll
        for (int e = 0; e < VW; ++e) {
            float o = v[e];
            if (bias != nullptr) o = o + bias[n];
            float *c = C + b * strideC + (int64_t)m * ldc + n;
            *c = accumulate ? *c + o : o;
            if (VW > 1 && ++n == N) {
                n = 0;
                if (++m == M) {
                    m = 0;
                    ++b;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------
// Host-side selection.

struct TileCfg {
    int bm, bn;
};

template <int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC, bool AV, bool BV>
int launch_one(hipStream_t s, const TiledArgs &a) {
    MIGEMM_LAUNCH((gemm_mfma_kernel<BM, BN, BK, WM, WN, AKC, BKC, AV, BV>),
                       dim3(a.total), dim3(WM * WN * 64), 0, s, a);
    return launch_status("gemm_mfma_kernel launch");
}

template <int BM, int BN, int BK, int WM, int WN, bool AKC, bool BKC>
int launch_vec(hipStream_t s, const TiledArgs &a, bool av, bool bv) {
    if (av) {
        if (bv) return launch_one<BM, BN, BK, WM, WN, AKC, BKC, true, true>(s, a);
        return launch_one<BM, BN, BK, WM, WN, AKC, BKC, true, false>(s, a);
    }
    if (bv) return launch_one<BM, BN, BK, WM, WN, AKC, BKC, false, true>(s, a);
    return launch_one<BM, BN, BK, WM, WN, AKC, BKC, false, false>(s, a);
}

template <int BM, int BN, int BK, int WM, int WN>
int launch_layout(hipStream_t s, const TiledArgs &a, bool akc, bool bkc, bool av, bool bv) {
    if (akc) {
        if (bkc) return launch_vec<BM, BN, BK, WM, WN, true, true>(s, a, av, bv);
        return launch_vec<BM, BN, BK, WM, WN, true, false>(s, a, av, bv);
    }
    if (bkc) return launch_vec<BM, BN, BK, WM, WN, false, true>(s, a, av, bv);
    return launch_vec<BM, BN, BK, WM, WN, false, false>(s, a, av, bv);
}

// Sets the tile grid for a BM x BN tile and the split-K ranges (a.splits requested on
// entry; on return the number of non-empty ranges, each of kt_per_split BK-wide k-tiles),
// then launches.
// ONLY: -1 instantiates every operand layout; 0..3 only the layout (akc = ONLY >> 1,
// bkc = ONLY & 1), for tile shapes that one form alone uses.
template <int BM, int BN, int BK, int WM, int WN, int ONLY = -1>
int launch_tiles(hipStream_t s, TiledArgs &a, bool akc, bool bkc, bool av, bool bv) {
    a.tiles_m = (a.M + BM - 1) / BM;
    a.tiles_n = (a.N + BN - 1) / BN;
    const int nk = (a.K + BK - 1) / BK;
    const int want = a.splits < nk ? a.splits : nk;
    a.kt_per_split = (nk + want - 1) / want;
    a.splits = (nk + a.kt_per_split - 1) / a.kt_per_split;
    const int64_t total = (int64_t)a.tiles_m * a.tiles_n * a.batch * a.splits;
    if (total > INT32_MAX)
        return set_error(MIGEMM_ERR_UNSUPPORTED, "gemm: %lld tiles exceed one launch",
                         (long long)total);
    a.total = (int)total;
    set_tile_divisors(a);
    if constexpr (ONLY >= 0)
        return launch_vec<BM, BN, BK, WM, WN, (ONLY >> 1) != 0, (ONLY & 1) != 0>(s, a, av, bv);
    else
        return launch_layout<BM, BN, BK, WM, WN>(s, a, akc, bkc, av, bv);
}

}  // namespace

int launch_reduce_slices(hipStream_t stream, const float *partial, int slices, int batch,
                         int M, int N, const float *bias, float *C, int64_t ldc,
                         int64_t strideC, bool accumulate) {
    const int64_t total = (int64_t)batch * M * N;
    // 4 outputs per thread once that still gives every CU a work-group (and the size is a
    // multiple of 4, so no thread has a partial vector)
    const bool wide = total >= 4 * 256 * 256 && total % 4 == 0;
    int64_t blocks = ((wide ? total / 4 : total) + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    const bool plain = bias == nullptr && !accumulate && ldc == N &&
                       (batch == 1 || strideC == (int64_t)M * N) &&
                       (!wide || ((uintptr_t)C & 15) == 0);
#define MIGEMM_REDUCE(VW, PLAIN)                                                              \
    MIGEMM_LAUNCH((reduce_slices_kernel<VW, PLAIN>), dim3((unsigned)blocks), dim3(256), 0, \
                       stream, partial, slices, total, M, N, bias, C, ldc, strideC,            \
                       (int)accumulate)
    if (wide) {
        if (plain) MIGEMM_REDUCE(4, true);
        else MIGEMM_REDUCE(4, false);
    } else {
        if (plain) MIGEMM_REDUCE(1, true);
        else MIGEMM_REDUCE(1, false);
    }
#undef MIGEMM_REDUCE
    return launch_status("reduce_slices_kernel launch");
}

namespace {

// An operand's rows and batch entries all start on 16-byte boundaries, as
// global_load_lds_dwordx4 needs.
bool rows16(const float *p, int64_t ld, int64_t stride) {
    return ((uintptr_t)p & 15) == 0 && ld % 4 == 0 && stride % 4 == 0;
}

// The tile cost model. A macro-tile shape runs at a fitted rate with a fixed per-tile
// overhead of `over` k-steps: time = rounds of 256 work-groups (one round as long as one
// tile) x 2 x tile area x (K + over) / rate. Fitted to NN at 4096 x K x 4096, K = 256 ..
// 4096, in one process on one box; every dispatcher rule below that weighs tile shapes
// takes its constants from these tables.
struct TileFit {
    double rate;  // TFLOP/s (kElementFit: relative to 256x256)
    double over;  // k-steps per tile
};
enum TileShape { T64 = 0, T128 = 1, T128x256 = 2, T256 = 3 };
// operands loaded straight into LDS (gemm_direct_kernel, 16-byte aligned rows)
constexpr TileFit kDirectFit[4] = {{135.2, 95}, {147.6, 90}, {152.1, 98}, {152.6, 75}};
// register-staged kernels (other 128-bit operands)
constexpr TileFit kStagedFit[4] = {{134.2, 75}, {138.9, 78}, {140.6, 99}, {147.2, 73}};
// element-wise loads (M, N or K not a multiple of 4): the earlier three-shape model, rates
// relative to 256x256; 256x256 work-groups fill a CU alone, their prologue and C store not
// overlapped (about 32 k-steps per tile, 16 for 128x256). 64x64 at 0.91: fitted first to
// five shapes (graph replay, us, 64x64 / 128x128: 1231 x 4246 x 7348 NT 598 / 745, batch-8
// 701 x 1107 x 1602 TT 166 / 209, 12000 x 500 x 6565 702 / 633, 6000 x 1000 x 6001 595 /
// 542, 4096 x 4095 x 4095 980 / 951 with 256x256 at 941), then raised from 0.88 on 49
// audited outputs of 256-16384 per side (picks' time above the per-shape best 1.13 -> 0.84
// %) and checked on 40 others: 5 picks changed, each 2-12 % faster (8948 x 1088 x 3283
// 558.0 -> 489.6), 0.5 % less in total.
constexpr TileFit kElementFit[4] = {{0.91, 0}, {0.966, 0}, {0.981, 16}, {1.0, 32}};
// Operands loaded 4 bytes per lane (not 16-byte aligned rows) lower the rates of split
// 64x64 and 128x128 tiles to these fractions (long-K regime below).
constexpr double kUnalignedRate64 = 0.85, kUnalignedRate128 = 0.95;
// Split-K partial sums cost (2S + 1) M N 4 bytes of HBM traffic at this rate (bytes / us).
constexpr double kPartialBytesPerUs = 6e6;
}  // namespace

int launch_gemm_tiled(hipStream_t stream, const GemmDesc &d) {
    // Operand orientation: A is K-contiguous unless transposed; B is K-contiguous only
    // when transposed.
    const bool akc = !d.transA;
    const bool bkc = d.transB;
    // Groups of 4 contiguous elements never straddle the matrix edge when the
    // contiguous extent is a multiple of 4 (alignment does not matter, see load16).
    const bool av = akc ? d.K % 4 == 0 : d.M % 4 == 0;
    const bool bv = bkc ? d.K % 4 == 0 : d.N % 4 == 0;

    TiledArgs a;
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
    a.batch = d.batch;
    a.accumulate = d.accumulate;

    auto tiles = [&](int bm, int bn) {
        return (int64_t)((d.M + bm - 1) / bm) * ((d.N + bn - 1) / bn) * d.batch;
    };
    const int nk32 = (d.K + 31) / 32;
    // Largest tile that still gives the 256 CUs two work-groups each. Below that, a long K
    // (>= 4096) with M, N >= 128 and at least 128 tiles of 128x128 keeps 128x128 tiles and
    // splits K until there are >= 1024 work-groups (an even number of ranges, at most 8).
    // Otherwise 64x64 tiles, mostly whole when there are >= 256 of them (a split then mostly
    // adds the reduce: 1024^3 in 2 ranges 62.7 TFLOP/s, whole 75.7). A long K over 48-128 is
    // split into 8 ranges: the XCD remap in the kernel then gives each XCD one k-range of
    // every tile, so the A and B panels of that range are shared in its L2. Other splits aim
    // at 640 work-groups, at most 32 ranges of >= 8 k-tiles of 32. Measured (graph replay,
    // us): the Linear(500 -> 6565) gradients dX 12000x500x6565 (NT) 128x128 / 4 ranges 664,
    // 64x64 767; dW 500x6565x12000 (TN) 128x128 / 6 ranges 691, 64x64 916. With few 128x128
    // tiles, 8 ranges leave most CUs idle: 256x4096x256 41.5 against 64x64 / 16 ranges 14.1;
    // 128x4096x4096 64x64 with 4 / 5 / 8 / 16 ranges: 49.2 / 55.0 / 47.9 / 51.5;
    // 512x16384x512 TN with 5 / 8 / 10: 119.9 / 78.4 / 91.0.
    // gemm_direct_kernel applies when a lane's offset within a 256-row panel fits its loads'
    // 32-bit offsets: an operand with 16-byte aligned rows and a contiguous extent that is a
    // multiple of 4 is loaded 16 bytes per lane (wa / wb = 4), any other 4 bytes per lane.
    const int wa = av && rows16(d.A, d.lda, d.sA) ? 4 : 1;
    const int wb = bv && rows16(d.B, d.ldb, d.sB) ? 4 : 1;
    // MIGEMM_TUNE_DIRECT: 1 = never load straight into LDS, 2 = wherever the kernel applies
    const int direct_mode = tuning(MIGEMM_TUNE_DIRECT);
    const bool fits = direct_mode != 1 && d.lda <= (1 << 21) && d.ldb <= (1 << 21);
    const bool direct = fits && wa == 4 && wb == 4;
    // Estimated time (us) of `t` tiles of `area` outputs over k at a fitted rate (TFLOP/s,
    // scaled by `scale`) with its per-tile overhead: the work-groups are dealt over the 256
    // CUs in rounds, each round as long as one tile.
    auto est = [](int64_t t, double area, double k, TileFit f, double scale = 1.0) {
        return (double)((t + 255) / 256) * 256.0 * 2.0 * area * (k + f.over) /
               (f.rate * scale * 1e6);
    };
    // Whole 128x256 or 256x256 tiles (loaded straight into LDS) instead of 64x64 ones for
    // outputs with few 128x128 tiles, when the estimate says so: 8000 x 4096 x 1000 runs
    // 476.1 us in 128x256 tiles against 538.9 in 64x64, 1000 x 4096 x 8000 TN 485.6 / 519.0,
    // 8000 x 1024 x 1000 131.6 / 147.0.
    auto wider = [&](double c64, int &cfg_out, int &big_out) {
        const double c1 = est(tiles(128, 256), 32768, d.K, kDirectFit[T128x256]);
        const double c2 = est(tiles(256, 256), 65536, d.K, kDirectFit[T256]);
        if (c1 < c64 && c1 <= c2) {
            cfg_out = 128;
            big_out = 1;
        } else if (c2 < c64) {
            cfg_out = 128;
            big_out = 2;
        }
    };
    int cfg, splits = 1;
    int big = 0;  // 128x128 tiles; 1: 128x256, 2: 256x256 (see below)
    if (narrow_rows_streaming(d)) {
        // few rows over a large B (gemm_small.hip, small_preferred): 32x32 tiles, the k loop
        // split until there are ~1536 work-groups (ranges of >= 8 k-tiles of 32): batch-16
        // 8 x 6000 x 1024 (512 tiles) 89.0 us in 3 ranges, 178.5 whole
        cfg = 32;
        const int64_t t32 = tiles(32, 32);
        const int64_t want = (1536 + t32 - 1) / t32;
        int64_t cap = nk32 / 8 < 8 ? nk32 / 8 : 8;
        if (cap < 1) cap = 1;
        splits = (int)(want < cap ? want : cap);
    } else if (tiles(128, 128) >= 512) {
        cfg = 128;
    } else if (d.K >= 4096 && d.M >= 128 && d.N >= 128 && tiles(128, 128) >= 128) {
        // Long K over few tiles. Weighed by time ~ rounds of 256 work-groups x 2 area
        // (k + o) / rate (the fitted rates of the tile cost model below), plus for split
        // ranges the partial sums' HBM traffic, (2S + 1) M N 4 bytes at ~6 TB/s:
        //   128x128 tiles (register-staged) in S ranges, an even S <= 8 giving ~1024
        //     work-groups;
        //   256x256 tiles split so that every CU holds one work-group (32 or 64 tiles);
        //   whole 64x64 tiles (loaded straight into LDS).
        // Measured against the estimate's choice (us): 2048 x 4096 x 1024 256-split 144.6,
        // 64x64 130.7 (chosen); 1024 x 6400 x 4096 TN 256-split 386.5 (chosen), 64x64 396.1;
        // 512 x 6400 x 4096 TN 256-split 207.9, 64x64 203.2 (chosen); 1000 x 4096 x 3000
        // 128-split 249.7, 64x64 198.4 (chosen); 500 x 12000 x 6565 TN 128-split 685.0
        // (chosen), 64x64 722.4; 12000 x 6565 x 500 NT 128-split 669.8, 64x64 633.1 (chosen).
        // 64x64 tiles are also weighed in 2-4 ranges, and operands loaded 4 bytes per lane
        // (not `direct`) lower the rates of 64x64 and 128x128 tiles (kUnalignedRate*): on 30
        // shapes of this regime (K 4096-16384, every tile and range count timed) the picks'
        // time above the per-shape best fell from 7.1 % to 2.7 % (800 x 5000 x 2500 NT 213.4
        // -> 184.0 us in four 64x64 ranges, 160 x 10116 x 11952 490.6 -> 418.7, the LSTM
        // gate gradient 6400 x 4096 x 512 NT 230.9 -> 220.3 in three).
        const double e64 = direct ? 1.0 : kUnalignedRate64;
        const double e128 = direct ? 1.0 : kUnalignedRate128;
        auto traffic = [&](int s) {
            return (2.0 * s + 1) * d.M * d.N * 4.0 * d.batch / kPartialBytesPerUs;
        };
        const int64_t t128 = tiles(128, 128), t256 = tiles(256, 256), t64 = tiles(64, 64);
        int64_t want = (1024 + t128 - 1) / t128;
        want += want & 1;
        const int s128 = (int)(want < 8 ? want : 8);
        double best =
            est(t128 * s128, 16384, (double)d.K / s128, kStagedFit[T128], e128) + traffic(s128);
        cfg = 128;
        splits = s128;
        if (av && bv && (t256 == 32 || t256 == 64)) {
            const int s256 = (int)(256 / t256);
            const double c = est(256, 65536, (double)d.K / s256,
                                 direct ? kDirectFit[T256] : kStagedFit[T256]) + traffic(s256);
            if (c < best) {
                best = c;
                big = 2;
                splits = s256;
            }
        }
        for (int s = 1; s <= 4 && fits; ++s) {
            const double c = est(t64 * s, 4096, (double)d.K / s, kDirectFit[T64], e64) +
                             (s > 1 ? traffic(s) : 0.0);
            if (c < best) {
                best = c;
                cfg = 64;
                big = 0;
                splits = s;
            }
        }
        if (direct) {
            int c = cfg, b = big;
            wider(best, c, b);
            if (c != cfg || b != big) {
                cfg = c;
                big = b;
                splits = 1;
            }
        }
    } else if (tiles(64, 64) >= 256 || nk32 < 8) {
        cfg = tiles(64, 64) >= 256 ? 64 : 32;
        // About one tile per CU (one wavefront per SIMD) with a long k loop, or a few tiles
        // left over for a second round: 3 ranges fill the CUs (1024x2048x1024 NT 77.3 ->
        // 89.6 TFLOP/s, 1100x1100x900 49.6 -> 57.2; 1024^3, balanced and short, stays whole)
        const int64_t t64 = tiles(64, 64);
        if (t64 >= 256 && t64 < 320 && nk32 >= 24 &&
            (d.K >= 2048 || (t64 % 256 != 0 && d.K >= 768)))
            splits = 3;
        if (direct && splits == 1 && cfg == 64)
            wider(est(t64, 4096, d.K, kDirectFit[T64]), cfg, big);
    } else {
        cfg = 64;
        const int64_t t64 = tiles(64, 64);
        if (d.K >= 4096 && t64 >= 48 && t64 <= 128) {
            splits = 8;
        } else {
            const int64_t want = (640 + t64 - 1) / t64;
            const int64_t cap = nk32 / 8 < 32 ? nk32 / 8 : 32;
            splits = (int)(want < cap ? want : cap);
            if (splits < 1) splits = 1;
        }
    }
    // Large outputs: pick the macro-tile by the busiest CU's share of the work. The work-
    // groups are dealt over the 256 CUs, so a CU carries ceil(tiles / 256) tiles of area x
    // (K + a per-tile overhead), at each tile's own rate (kDirectFit, kStagedFit,
    // kElementFit). The tile count's quantization then decides: 3072 x 1024 x 3072 runs 168.7 us in 64x64
    // tiles (9 per CU) against 190.1 in 128x128 (2.25 per CU); 4096 x 256 x 4096 74.4 in
    // 256x256 against 82.1 in 128x128. (Outputs of 256-511 tiles of 128x128 stay on 64x64
    // tiles: one 4-wavefront work-group per CU hides latency poorly, 2048 x 1024 x 2048 TN
    // 81.0 us in direct 64x64 tiles against 86.3 in 128x128.)
    // Element-wise loads (M, N or K not a multiple of 4) keep the earlier three-shape model
    // (kElementFit), whose 256x256 overhead decides short K: 12000 x 6565 x 500 runs 729 us
    // at 128x128, 747 at 256x256.
    // C's rows start on 64-byte boundaries (every batch entry's too)
    const bool rows64 = d.ldc % 16 == 0 && ((uintptr_t)d.C & 63) == 0 &&
                        (d.batch == 1 || d.sC % 16 == 0);
    if (cfg == 128 && splits == 1 && tiles(128, 128) >= 512 && d.K <= 16) {
        // K <= 16: writing C is the work; 128x128 tiles, whole 128-byte lines per row and
        // four work-groups per CU (us, 64x64 / 128x128 / 256x256: 65536 x 3 x 4096 297.4 /
        // 217.5 / 241.0; 16384 x 8 x 16384 271.8 / 275.0 / 284.8; 20000 x 16 x 20000 446.0 /
        // 336.1 / 376.6)
        big = 0;
    } else if (cfg == 128 && splits == 1 && tiles(128, 128) >= 512) {
        const double k = d.K;
        auto cost = [&](int bm, int bn, TileFit f, double over) {
            return (double)((tiles(bm, bn) + 255) / 256) * bm * bn * (k + over) / f.rate;
        };
        const TileFit *fit = direct ? kDirectFit : av && bv ? kStagedFit : kElementFit;
        if (av && bv) {
            double c64, c0, c1, c2;
            if (direct) {
                // At K <= 512 the per-tile prologue and C store of the larger tiles weigh
                // 1.5x their fitted overhead: on a grid of 200 shapes (M, N in 1000..8000, K
                // in 256..4096, NN and TN, every tile timed) the picks' total time above the
                // per-shape best falls from 0.32 % to 0.18 %, and 3000 x 256 x 8000 takes
                // 64x64 tiles (115.1 us) instead of 128x256 (136.7 us). Outputs of 4096 or
                // more 128x128 tiles (8 or more rounds of 128x256) are exempt: over that many
                // rounds the work-groups drift apart and overlap one another's prologue and
                // store. On 84 outputs of 2000-16000 x 2048-8192 at K = 256-768 the picks'
                // total time above the per-shape best falls from 1.1 % to 0.25 %; the
                // Python Linear(500 -> 6565) forward, 12000 x 500 x 6565 NT, takes 128x256
                // tiles (670 us) instead of 64x64 (740-754).
                const double s = d.K <= 512 && tiles(128, 128) < 4096 ? 1.5 : 1.0;
                // C rows that do not start on 128-byte lines are stored as partial lines, and
                // a 256x256 work-group (one per CU) cannot hide that store burst behind other
                // work-groups' k loops; up to K = 1024 its overhead counts twice then (graph
                // replay, us, 64x64 / 128x128 / 128x256 / 256x256): 12000 x 500 x 6565 NT
                // (the Python Linear(500 -> 6565) forward) 683-755 / 645 / 656 / 742, TT
                // 674-710 / 634 / 641 / 734, 8192 x 512 x 8191 NT 527 / 517 / 535 / 608,
                // 4096 x 300 x 4095 NT 101 / 115 / 116 / 126, 8192 x 1024 x 8190 TT 980 / 1011
                // / 954 / 1033; with N = 6560 all four 616-690 and 256x256 among the best. On
                // the dispatcher grid (M, N 1000-8000, K 256-4096, NN / NT / TN) the 256x256
                // picks with such C rows ran 0.76-0.96x as long at K <= 1024 (5000 x 256 x
                // 3000 NT 93.9 -> 71.7 us in 64x64 tiles), but 1.01x at K = 4096.
                const bool cmis = (d.ldc % 32 != 0 || ((uintptr_t)d.C & 127) != 0) && d.K <= 1024;
                // Rows off 64-byte boundaries as well cost every tile wider than 64 about 110
                // k-steps more per tile at K <= 256 (the C store; 8192 x 64 x 8180 against
                // 8192 x 64 x 8192, us: 128x128 215.8 / 114.8, 256x256 220.4 / 120.8, 64x64
                // 124.0 / 121.1), which then replaces the 256x256 term above. By K = 500 the
                // other work-groups' k loops hide it (12000 x 500 x 6565 NT 728 in 128x256
                // tiles, 787 in 64x64).
                const double om = !rows64 && d.K <= 256 ? 110.0 : 0.0;
                c64 = cost(64, 64, fit[T64], fit[T64].over);
                c0 = cost(128, 128, fit[T128], fit[T128].over * s + om);
                c1 = cost(128, 256, fit[T128x256], fit[T128x256].over * s + om);
                const double o256 = fit[T256].over * s;
                c2 = cost(256, 256, fit[T256], o256 + (om > 0 ? om : cmis ? o256 : 0.0));
            } else {
                c64 = cost(64, 64, fit[T64], fit[T64].over);
                c0 = cost(128, 128, fit[T128], fit[T128].over);
                c1 = cost(128, 256, fit[T128x256], fit[T128x256].over);
                c2 = cost(256, 256, fit[T256], fit[T256].over);
            }
            const double best = std::min(std::min(c64, c0), std::min(c1, c2));
            cfg = best == c64 ? 64 : 128;
            big = best == c2 ? 2 : (best == c1 ? 1 : 0);
        } else if (d.K <= 320 && fits) {
            // Element-wise loads and a short k loop, where the C store weighs: 64x64 tiles
            // when C's rows are off 64-byte boundaries (graph replay, us, 64x64 / 128x128:
            // 4001 x 101 x 4003 48.1 / 72.0, 3001 x 203 x 5001 67.6 / 85.1, 6000 x 250 x 6001
            // NT 183.2 / 214.0, 2047 x 61 x 8191 TT 36.8 / 62.8, 3001 x 301 x 3001 TN 55.8 /
            // 70.0; from K = 400 the larger tiles win: 8000 x 400 x 4001 238.5 / 222.7),
            // 128x128 when they are on them and there are >= 6 rounds of tiles (11079 x 94 x
            // 11104 TN 314.5 / 265.2, 15658 x 73 x 10496 TN 363.7 / 306.8, 12110 x 41 x 11152
            // TT 232.4 / 196.0; with fewer 64x64 still wins: 2501 x 96 x 5008 TT 36.3 / 42.0,
            // 3343 x 85 x 6128 NT 53.1 / 60.8).
            cfg = rows64 && tiles(128, 128) >= 1536 ? 128 : 64;
            big = 0;
        } else {
            // element-wise loads: kElementFit (64x64 only where gemm_direct_kernel applies)
            const double c64 = fits ? cost(64, 64, fit[T64], fit[T64].over) : 1e300;
            const double c0 = cost(128, 128, fit[T128], fit[T128].over);
            const double c1 = cost(128, 256, fit[T128x256], fit[T128x256].over);
            const double c2 = cost(256, 256, fit[T256], fit[T256].over);
            const double best = std::min(std::min(c64, c0), std::min(c1, c2));
            cfg = best == c64 ? 64 : 128;
            big = best == c2 ? 2 : (best == c1 ? 1 : 0);
        }
    }
    // tuning overrides (migemm_set_tuning), validated when they were set
    const int force_tile = tuning(MIGEMM_TUNE_TILE);
    const int force_split = tuning(MIGEMM_TUNE_SPLITK);
    if (force_tile == MIGEMM_TILE_128x256) {
        cfg = 128;
        big = 1;
    } else if (force_tile == 32 || force_tile == 64 || force_tile == 128) {
        cfg = force_tile;
        big = 0;
    } else if (force_tile == 256) {
        cfg = 128;
        big = 2;
    }
    if (force_split >= 1) splits = force_split;
    // gemm_direct_kernel runs every 64x64, 128x128, 128x256 and 256x256 tile except split
    // 128x256 ranges (which the dispatcher does not pick; MIGEMM_DIRECT=2 forces them too).
    // Measured against the register-staged kernel (us): unsplit 64x64 1024^3 24.7 / 21.5,
    // 2048 x 1024 x 2048 TN 77.8 / 68.9; split 64x64 ranges 512 x 16384 x 512 TN 78.6 / 72.3,
    // 256 x 8192 x 1024 43.9 / 40.0, 1024 x 2048 x 1024 NT 46.2 / 42.6; split 128x128 ranges
    // in the uncapped variant (gemm_direct_128.hip) 6400 x 4096 x 512 NT 244.4 / 230.6;
    // split 256x256 tiles 1024 x 6400 x 4096 TN 396.6 / 386.1. An unaligned operand is loaded
    // 4 bytes per lane (Linear(500 -> 6565) forward 12000 x 500 x 6565 735.3 -> 648.8 us,
    // 4096 x 4096 x 4095 TN 1015.6 -> 924.1).
    const bool use_direct =
        fits && cfg != 32 && (splits == 1 || big != 1 || direct_mode == 2);

    a.splits = splits;
    // C stored through L2 by tiles 128 or more wide whose rows are off 64-byte boundaries
    // (tiled_common.h, store_tile)
    a.write_back = cfg == 128 && !rows64;
    a.partial = nullptr;
    if (splits > 1) {
        int st = MIGEMM_OK;
        a.partial =
            partial_buffer(stream, d, (size_t)splits * d.batch * d.M * d.N * sizeof(float), &st);
        if (a.partial == nullptr) return st;
    }
    int rc;
    switch (cfg) {
        case 128:
            // Wavefronts of 32x128 (124-128 VGPRs, 4 per SIMD). Measured at 4096^3
            // (graph replay, 5 rounds), NN / NT / TN TFLOP/s: 256x256 with 16 wavefronts
            // 141.4 / 145.4 / 144.6; 128x256 with 8: 141.2 / 140.5 / 141.5; 128x128 with
            // 4: 140.2 / 136.1 / 140.3; 128x128 with 2x2 wavefronts of 64x64: 140.1 /
            // 125.9 / 140.2.
            // NT (both operands K-contiguous) runs BK = 32: half the barriers, 144 KB of
            // LDS; measured NT 146.3 against 144.1 TFLOP/s at 4096^3, 148.6 against 145.5
            // at 8192^3. With an I-contiguous operand BK = 32 spills and is slower (NN
            // 133.0 against 143.5), so NN / TN keep BK = 16. TN (both operands
            // I-contiguous) runs 8 wavefronts of 64x128 (2 per SIMD, ~220 VGPRs): 143.2
            // against 142.5 at 4096^3, 145.9 against 144.3 at 8192^3; NN and NT are
            // slower that way (142.7 / 143.0).
            if (use_direct)
                rc = launch_gemm_direct(stream, a, big == 2 ? 256 : 128, big >= 1 ? 256 : 128,
                                        akc, bkc, wa, wb);
            else if (big == 2 && akc && bkc)
                rc = launch_tiles<256, 256, 32, 8, 2, 3>(stream, a, akc, bkc, av, bv);
            else if (big == 2 && !akc && !bkc)
                rc = launch_tiles<256, 256, 16, 4, 2, 0>(stream, a, akc, bkc, av, bv);
            else if (big == 2)
                rc = launch_tiles<256, 256, 16, 8, 2>(stream, a, akc, bkc, av, bv);
            else if (big == 1)
                rc = launch_tiles<128, 256, 16, 4, 2>(stream, a, akc, bkc, av, bv);
            else
                rc = launch_tiles<128, 128, 16, 4, 1>(stream, a, akc, bkc, av, bv);
            break;
        case 64:
            if (use_direct)
                rc = launch_gemm_direct(stream, a, 64, 64, akc, bkc, wa, wb);
            else
                rc = launch_tiles<64, 64, 32, 2, 2>(stream, a, akc, bkc, av, bv);
            break;
        default: rc = launch_tiles<32, 32, 32, 1, 1>(stream, a, akc, bkc, av, bv); break;
    }
    splits = a.splits;  // the launch drops empty k ranges
    record_plan(use_direct ? "tiled-direct" : "tiled-staged", d,
                cfg == 128 && big == 2 ? 256 : cfg, cfg == 128 && big >= 1 ? 256 : cfg, splits,
                use_direct ? (wa == 4 && wb == 4 ? 16 : 4) : 0);
    if (rc != MIGEMM_OK || splits == 1) return rc;
    return launch_reduce_slices(stream, a.partial, splits, d.batch, d.M, d.N, d.bias, d.C,
                                d.ldc, d.sC, d.accumulate);
}

}  // namespace migemm
