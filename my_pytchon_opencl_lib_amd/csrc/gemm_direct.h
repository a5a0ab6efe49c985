// Kernel template and launch helpers of gemm_direct_kernel, shared by the translation
// units that instantiate it per tile shape (gemm_direct_<tile>.hip; the dispatcher is in
// gemm_direct.hip, which also describes the kernel).
#pragma once

#include <stdlib.h>

#include "tiled_common.h"

namespace migemm {

// Per tile shape: launches gemm_direct_kernel for the operand layouts (akc, bkc) and load
// widths (wa, wb: 4 or 1 floats per lane).
int launch_direct_256(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa, int wb);
int launch_direct_128x256(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa,
                          int wb);
int launch_direct_128(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa, int wb);
int launch_direct_64(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa, int wb);

namespace {

// s_waitcnt vmcnt(N) with expcnt and lgkmcnt left at their maxima. The 6-bit vmcnt field
// is split over bits 3:0 and 15:14 of the immediate.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

typedef __attribute__((address_space(3))) float *lds_ptr_t;

// global_load_lds_dwordx4 in its scalar-base form: each lane's 16 bytes at sbase + voff go
// to LDS at `dst` + 16 * lane (dst wave-uniform, through M0). Written as inline assembly
// rather than __builtin_amdgcn_global_load_lds: with the builtin the compiler made every
// later LDS read wait for all outstanding LDS loads (s_waitcnt vmcnt(0)), which serializes
// the pipeline. The kernel orders these loads itself: each wavefront waits for its own with
// s_waitcnt vmcnt before the barrier that publishes them. Nothing else in the kernels of
// this file uses M0 (checked in the generated code).
__device__ __forceinline__ void dma16(const char *sbase, uint32_t voff, float *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_ptr_t)dst;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
}

// global_load_lds_dword, the 4-byte form for operands whose rows are not 16-byte aligned:
// each lane's float at sbase + voff goes to LDS at `dst` + 4 * lane.
__device__ __forceinline__ void dma4(const char *sbase, uint32_t voff, float *dst) {
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_ptr_t)dst;
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1"
                 :
                 : "v"(voff), "s"(sbase), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ f4 dl_load16(const float *p) {
    f4 v;
    __builtin_memcpy(&v, p, sizeof(v));
    return v;
}

// K-contiguous LDS tile: rows of BK floats (CPR = BK / 4 chunks of 16 bytes), unpadded.
// Chunk c of row r is stored in slot c ^ kc_swz(r). A fragment read phase covers 16
// consecutive rows at one chunk; kc_swz spreads them over the 16 bank groups of 16 bytes:
// BK = 16: (r / 4) % 4, BK = 32: (r / 2) % 8.
template <int BK>
__device__ __forceinline__ int kc_swz(int r) {
    constexpr int CPR = BK / 4;
    return (r / (16 / CPR)) % CPR;
}

// I-contiguous LDS tile: BK k-rows of T floats, unpadded. Column c of k-row k is stored at
// c ^ ic_swz(k): the two half-wavefronts of a fragment read take k-rows 4 apart (whose
// starts fall on the same banks) at 32 consecutive columns each; flipping bit 5 of the
// column on alternate groups of 4 k-rows puts them on complementary halves of the 64 banks.
__device__ __forceinline__ int ic_swz(int k) { return ((k >> 2) & 1) << 5; }

// One operand of a T x BK tile (T = 64, 128 or 256 rows of the M or N dimension), loaded W
// floats per lane (W = 4: global_load_lds_dwordx4, rows 16-byte aligned and the contiguous
// extent a multiple of 4; W = 1: global_load_lds_dword, any operand). A load instruction
// fills the next 64 W floats of the tile in LDS order: lane L the W floats at LDS position
// 64 W q + W L, which hold tile row / k-row f / BK (KC) or f / T (I-contiguous), de-swizzled
// to the element they must contain. NS = instructions per wavefront per tile. The loads
// address memory as a wave-uniform base (the tile's first row / column at k-tile 0,
// advanced per k-tile in scalar registers) plus a 32-bit per-lane byte offset, which keeps
// the per-lane state to one register per instruction; the launcher checks that the offsets
// fit.
template <int NT, bool KC, int BK, int T, int W>
struct DlOperand {
    static_assert(T == 64 || T == 128 || T == 256, "tile edge");
    static_assert(W == 1 || W == 4, "floats per lane");
    static constexpr int NW = NT / 64;
    static constexpr int FPI = 64 * W;       // floats per load instruction
    static constexpr int NI = T * BK / FPI;  // load instructions per tile
    static constexpr int NS = NI / NW;
    static_assert(NS >= 1 && NS * NW == NI, "the tile's loads split evenly over the wavefronts");
    static constexpr int FLOATS = T * BK;
    const char *base;      // wave-uniform: element (i0, 0) of the operand
    uint32_t voff[NS];     // this lane's byte offset from `base` at k-tile 0
    int kk[NS];            // the k (within a tile) of this lane's first float
    int q0;                // first instruction of this wavefront (wave-uniform)

    __device__ __forceinline__ void init(const float *op, int64_t ld, int i0, int rows,
                                         int wave, int lane) {
        q0 = wave * NS;
        base = reinterpret_cast<const char *>(op + (KC ? (int64_t)i0 * ld : (int64_t)i0));
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const int f = FPI * (q0 + j) + W * lane;  // LDS position within the tile
            if constexpr (KC) {
                const int r = f / BK;                 // tile row
                const int pos = f % BK;
                const int k = 4 * ((pos / 4) ^ kc_swz<BK>(r)) + pos % 4;
                int gi = i0 + r;
                gi = gi < rows ? gi : rows - 1;
                kk[j] = k;
                voff[j] = (uint32_t)(((gi - i0) * (uint32_t)ld + k) * 4);
            } else {
                const int k = f / T;                  // k-row of the tile
                int gi = i0 + ((f % T) ^ ic_swz(k));
                gi = gi < rows ? gi : rows - W;
                kk[j] = k;
                voff[j] = (uint32_t)((k * (uint32_t)ld + (gi - i0)) * 4);
            }
        }
    }

    __device__ __forceinline__ int lds_off(int j) const { return (q0 + j) * FPI; }

    __device__ __forceinline__ const char *tile_base(int kt, int64_t ld) const {
        return base + (KC ? (int64_t)kt * BK * 4 : (int64_t)kt * BK * ld * 4);
    }

    // Full k-tile kt straight into `stage`.
    __device__ __forceinline__ void issue(float *stage, int kt, int64_t ld) const {
        const char *tb = tile_base(kt, ld);
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            if constexpr (W == 4)
                dma16(tb, voff[j], stage + lds_off(j));
            else
                dma4(tb, voff[j], stage + lds_off(j));
        }
    }

    // This lane's floats of the tail tile kt (k0 = BK kt, k0 + BK > K), k >= K zero-filled.
    typedef typename std::conditional<W == 4, f4, float>::type TailElem;
    struct Tail {
        TailElem v[NS];
    };
    __device__ __forceinline__ void tail_fetch(Tail &t, int kt, int K, int64_t ld) const {
        const int k0 = kt * BK;
        const char *tb = tile_base(kt, ld);
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            const float *src = reinterpret_cast<const float *>(tb + voff[j]);
            if constexpr (W == 4) {
                f4 v = {0.f, 0.f, 0.f, 0.f};
                if constexpr (KC) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (k0 + kk[j] + e < K) v[e] = src[e];
                } else {
                    if (k0 + kk[j] < K) v = dl_load16(src);
                }
                t.v[j] = v;
            } else {
                t.v[j] = k0 + kk[j] < K ? *src : 0.f;
            }
        }
    }

    // Writes a fetched tail tile where the direct loads would have put it.
    __device__ __forceinline__ void tail_put(const Tail &t, float *stage, int lane) const {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            if constexpr (W == 4)
                *reinterpret_cast<f4 *>(stage + lds_off(j) + 4 * lane) = t.v[j];
            else
                stage[lds_off(j) + lane] = t.v[j];
        }
    }
};

// Fragments of k-group g (8 consecutive k of the tile) for F blocks of 32 rows from `off`:
// fr[f][s] is this lane's operand for MFMA step s (lanes 0-31: k = 8g + s, lanes 32-63:
// k = 8g + 4 + s).
template <bool KC, int BK, int T, int F>
__device__ __forceinline__ void dl_frags(const float *lds, int off, int g, int lane,
                                         f4 (&fr)[F]) {
    const int lo = lane & 31;
    const int hi = lane >> 5;
    if constexpr (KC) {
        const int slot = (2 * g + hi) ^ kc_swz<BK>(lo);  // off + 32 f keeps kc_swz(r)
#pragma unroll
        for (int f = 0; f < F; ++f)
            fr[f] = *reinterpret_cast<const f4 *>(lds + (off + f * 32 + lo) * BK + 4 * slot);
    } else {
        // k-row 8g + 4hi + s has ic_swz = 32 hi
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                fr[f][s] = lds[(8 * g + 4 * hi + s) * T + ((off + f * 32 + lo) ^ (hi << 5))];
    }
}

// BM x BN tiles, WM x WN wavefronts; S LDS stages; tile kt lives in stage (kt - kt0) % S
// and is loaded D (<= S) tiles ahead. OCC: wavefronts per SIMD the register allocation must
// allow (4 for four 4-wavefront work-groups per CU).
template <int BM, int BN, int WM, int WN, bool AKC, bool BKC, int BK, int S, int D, int OCC,
          int WA, int WB>
__global__ void __launch_bounds__(WM *WN * 64) __attribute__((amdgpu_waves_per_eu(OCC)))
gemm_direct_kernel(TiledArgs p) {
    static_assert(D >= 2 && D <= S, "loads run 2..S tiles ahead");
    constexpr int NT = WM * WN * 64;
    constexpr int WTM = BM / WM;
    constexpr int WTN = BN / WN;
    constexpr int FM = WTM / 32;
    constexpr int FN = WTN / 32;
    constexpr int G = BK / 8;  // k-groups per tile
    static_assert(FM >= 1 && FN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "bad wave tile");
    typedef DlOperand<NT, AKC, BK, BM, WA> OpA;
    typedef DlOperand<NT, BKC, BK, BN, WB> OpB;
    constexpr int A_FL = OpA::FLOATS;
    constexpr int B_FL = OpB::FLOATS;
    // One array per operand, so each wavefront reads every stage of an operand from one
    // base register with immediate offsets (the stages of one operand span < 64 KB).
    __shared__ __attribute__((aligned(16))) float lds_a[S * A_FL];
    __shared__ __attribute__((aligned(16))) float lds_b[S * B_FL];
    constexpr int LPT = OpA::NS + OpB::NS;  // load instructions per tile per wavefront

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN;
    const int wn = wave % WN;

    // The tile mapping divides in VALU registers; the results are wave-uniform, and keeping
    // them (and everything derived from them: k-tile indices, load bases) in scalar
    // registers leaves the vector registers to the accumulators and fragments.
    TileCoord tc = tile_coord<BM, BN>(p, blockIdx.x);
    tc.split = __builtin_amdgcn_readfirstlane(tc.split);
    tc.b = __builtin_amdgcn_readfirstlane(tc.b);
    tc.m0 = __builtin_amdgcn_readfirstlane(tc.m0);
    tc.n0 = __builtin_amdgcn_readfirstlane(tc.n0);
    const float *Ab = p.A + (int64_t)tc.b * p.sA;
    const float *Bb = p.B + (int64_t)tc.b * p.sB;

    OpA opa;
    OpB opb;
    opa.init(Ab, p.lda, tc.m0, p.M, wave, lane);
    opb.init(Bb, p.ldb, tc.n0, p.N, wave, lane);

    f16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int K = p.K;
    const int kt0 = tc.split * p.kt_per_split;
    const int kt1 = min((K + BK - 1) / BK, kt0 + p.kt_per_split);
    const int kf = min(kt1, K / BK);  // end of the full k-tiles of this range

    auto issue = [&](int kt, int st) {
        opa.issue(lds_a + st * A_FL, kt, p.lda);
        opb.issue(lds_b + st * B_FL, kt, p.ldb);
    };
    auto frags = [&](int st, int g, f4(&fa)[FM], f4(&fb)[FN]) {
        dl_frags<AKC, BK, BM, FM>(lds_a + st * A_FL, wm * WTM, g, lane, fa);
        dl_frags<BKC, BK, BN, FN>(lds_b + st * B_FL, wn * WTN, g, lane, fb);
    };
    auto mfmas = [&](const f4(&fa)[FM], const f4(&fb)[FN]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][s], fb[j][s],
                                                                     acc[i][j], 0, 0, 0);
    };
    // Tile kt out of stage ST: every fragment read of the stage is issued before the
    // barrier, which (1) publishes tile kt+1 (each wavefront first waits for its own loads
    // of it; the D-2 tiles issued after it may stay in flight) and (2) retires the stage of
    // tile kt+D-S, so the loads of tile kt+D can go there. The last k-group's MFMAs follow
    // the barrier, and the first of tile kt+1 follow them with no barrier in between.
    auto step = [&](int kt, auto st) {
        constexpr int ST = decltype(st)::value;
        f4 fa[2][FM], fb[2][FN];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            frags(ST, g, fa[g & 1], fb[g & 1]);
            if (g > 0) mfmas(fa[(g - 1) & 1], fb[(g - 1) & 1]);
        }
        if constexpr (D > 2) {
            if (kt + D - 1 < kf)
                wait_vmcnt<(D - 2) * LPT>();
            else
                wait_vmcnt<0>();
        } else {
            wait_vmcnt<0>();
        }
        __syncthreads();
        if (kt + D < kf) issue(kt + D, (ST + D) % S);
        mfmas(fa[(G - 1) & 1], fb[(G - 1) & 1]);
    };

    // 64x64 tiles fetch the tail tile into registers before the first direct loads (16
    // registers per lane, which these tiles have to spare), so its memory latency overlaps
    // the k loop; a work-group runs the whole k loop with others of the same launch wave,
    // and latency left at the end is not hidden by other work-groups. Issued first, these
    // loads are the oldest in the vmcnt order and every wait below also covers them.
    constexpr bool TAIL_EARLY = BM == 64 && BN == 64;
    typename OpA::Tail ta;
    typename OpB::Tail tb;
    if constexpr (TAIL_EARLY) {
        if (kf < kt1) {
            opa.tail_fetch(ta, kf, K, p.lda);
            opb.tail_fetch(tb, kf, K, p.ldb);
        }
    }

    int kt = kt0;
    if (kt0 < kf) {
#pragma unroll
        for (int t = 0; t < D; ++t)
            if (kt0 + t < kf) issue(kt0 + t, t);
        if (kt0 + D - 1 < kf)
            wait_vmcnt<(D - 1) * LPT>();
        else
            wait_vmcnt<0>();
        __syncthreads();
        // S steps per pass, so every stage index is a compile-time constant
        for (; kt + S - 1 < kf; kt += S) {
            step(kt, std::integral_constant<int, 0>{});
            step(kt + 1, std::integral_constant<int, 1 % S>{});
            if constexpr (S > 2) step(kt + 2, std::integral_constant<int, 2 % S>{});
            if constexpr (S > 3) step(kt + 3, std::integral_constant<int, 3 % S>{});
        }
        if (kt < kf) step(kt++, std::integral_constant<int, 0>{});
        if constexpr (S > 2)
            if (kt < kf) step(kt++, std::integral_constant<int, 1 % S>{});
        if constexpr (S > 3)
            if (kt < kf) step(kt++, std::integral_constant<int, 2 % S>{});
    }
    wait_vmcnt<0>();  // no load into LDS outlives the loop
    if (kt < kt1) {  // the tail tile: k >= K zero-filled in both operands
        if constexpr (!TAIL_EARLY) {
            opa.tail_fetch(ta, kt, K, p.lda);
            opb.tail_fetch(tb, kt, K, p.ldb);
        }
        __syncthreads();  // every wavefront is done reading the stages
        opa.tail_put(ta, lds_a, lane);
        opb.tail_put(tb, lds_b, lane);
        __syncthreads();
        // k-groups wholly at k >= K hold zeros in both operands; their MFMAs would add
        // exact zeros (an accumulator that starts at +0 is never -0), so they are skipped.
        const int groups = (K - kt * BK + 7) / 8;
        f4 fa[FM], fb[FN];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            if (g < groups) {
                frags(0, g, fa, fb);
                mfmas(fa, fb);
            }
        }
    }
    store_tile<FM, FN>(p, tc, tc.m0 + wm * WTM, tc.n0 + wn * WTN, lane, acc);
}

template <int BM, int BN, int WM, int WN, bool AKC, bool BKC, int BK, int S, int D, int OCC,
          int WA = 4, int WB = 4>
int launch_direct(hipStream_t s, TiledArgs &a) {
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
    MIGEMM_LAUNCH((gemm_direct_kernel<BM, BN, WM, WN, AKC, BKC, BK, S, D, OCC, WA, WB>),
                       dim3(a.total),
                       dim3(WM * WN * 64), 0, s, a);
    return launch_status("gemm_direct_kernel launch");
}

// Every operand layout (NN, NT, TN, TT) with wavefronts of 32x128 (64x64 tiles: 2 x 2
// wavefronts of 32x32).
template <int BM, int BN, int BK, int S, int D, int OCC = 1, int WA = 4, int WB = 4>
int launch_layouts(hipStream_t s, TiledArgs &a, bool akc, bool bkc) {
    constexpr int WM = BN >= 128 ? BM / 32 : 2;
    constexpr int WN = BN >= 128 ? BN / 128 : 2;
    if (akc && bkc) return launch_direct<BM, BN, WM, WN, true, true, BK, S, D, OCC, WA, WB>(s, a);
    if (akc) return launch_direct<BM, BN, WM, WN, true, false, BK, S, D, OCC, WA, WB>(s, a);
    if (!bkc) return launch_direct<BM, BN, WM, WN, false, false, BK, S, D, OCC, WA, WB>(s, a);
    return launch_direct<BM, BN, WM, WN, false, true, BK, S, D, OCC, WA, WB>(s, a);
}

}  // namespace

}  // namespace migemm
