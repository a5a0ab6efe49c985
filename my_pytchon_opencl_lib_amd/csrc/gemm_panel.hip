// Panel fp32 GEMM for gfx950: C = op(A) * op(B) (+ bias) for outputs with few rows, in every
// operand layout: an activation panel such as the 64 x 1536 input of the LSTM gate GEMM
// (lstm_gemm_xw, cs/cl_kernels/lstm.cl:273) or the h_{t-1} rows of its recurrent product
// (lstm.cl:80-101) times a weight matrix stored [K, N], or [N, K] as the Python reference's
// Linear keeps it (core/layers.py:21-33), and the transposed forms of bmm_permute_tiled
// (cs/cl_kernels/bmm_permute_tiled.cl:7-122); "cs/" = csharp/cstorchcl/cstorchcl/.
//
// Such a GEMM has too few output tiles for the tiled kernel, and every 32x32 tile of C needs
// its 32-row slice of A and 32-column slice of B over the whole K (393 KB at K = 1536).
//  * A work-group owns a 32x32 tile of C and has NW wavefronts (8, two per SIMD, when K has
//    8 or more k-groups of 32); wavefront w multiplies the w-th contiguous share of the
//    k-groups and the NW partial tiles are added in LDS in the order w = 0..NW-1
//    (deterministic), each partial written into its own wavefront's ring, so the epilogue
//    has one barrier.
//  * The product is computed as C^T = B^T A^T with v_mfma_f32_32x32x2_f32: the MFMA's first
//    operand is B (lane l supplies column n0 + l%32), its second A (lane l supplies row
//    m0 + l%32). In step s of each 8-wide sub-group, lanes 0-31 supply k = s and lanes 32-63
//    k = 4 + s, for both operands. A K-contiguous operand (A not transposed, B transposed)
//    is staged as 32 rows of 32 k, and a lane's four values of a sub-group are one 16-byte
//    read; a k-row operand (B not transposed, A transposed) as 32 k-rows of 32 columns, and
//    they are four 4-byte reads of consecutive k-rows. Every layout sums each output over k
//    in the same order.
//  * Every operand byte moves with global_load_lds_dwordx4 (16 bytes per lane, straight
//    into LDS). A k-group of 32 is 4 KB of each operand, 8 load instructions per wavefront,
//    each covering 8 whole 128-byte lines: with 8-wide k-groups every line of A was fetched
//    by 4 instructions and the loads ran at ~23 bytes per clock per CU.
//  * Each wavefront keeps its own LDS ring of D k-groups (shipped D = 1: one k-group in
//    flight while the previous one is multiplied) and waits for its own loads
//    (s_waitcnt vmcnt), so the k loop has no barrier. k-group i's fragments are in
//    registers before its first MFMA (k-group 0's first sub-group starts as soon as both
//    operands' first 8 k have landed); its slot is refilled after the first 4 of its 16
//    MFMAs, and k-group i+1's fragments are read into a second register set before the
//    last 4. Past the end the loads re-read the last k-group (never multiplied), so the
//    wait count is constant.
//  * K-contiguous rows are stored with chunk c of row r in slot c ^ ((r / 2) % 8), which
//    makes the 128-bit fragment reads conflict-free.
//  * Work-groups are dealt to the 8 XCDs in contiguous chunks, both row tiles of a column
//    block on one XCD, so each XCD's L2 holds a contiguous 1/8 of B (3.1 MB for the gate
//    GEMM) and B is fetched into L2 once.
//  * Edges: rows beyond M and columns beyond N are clamped on load and not stored. The
//    kernel needs K % 32 == 0, N % 4 == 0, M % 4 == 0 when A is transposed, and 16-byte
//    aligned rows (the dispatcher checks).
//  * Epilogue as the other kernels: bias after the k sum (linear.cl:119-122), then C is
//    written or added to.
#include "gemm_direct.h"

namespace migemm {
namespace {

// A 16-byte vector at 4-byte alignment (bias and C rows may start at any float).
typedef float f4u __attribute__((ext_vector_type(4), aligned(4)));

struct PanelArgs {
    const float *A;
    const float *B;
    const float *bias;
    float *C;
    int64_t lda, ldb, ldc;
    int64_t sA, sB, sC;
    int M, N, K;
    int tiles_m, tiles_n, batch, total;
    int accumulate;
    FastDiv per_batch;  // tiles_m * tiles_n (multiply-high division in the prologue)
    FastDiv tm_div;     // tiles_m
    // Second operand pair (kernels with TWO, batch 1): C = op(A) op(B) + op(A2) op(B2)
    // (+ bias), A2 / B2 in the orientations of A / B with K2 = K - 32 G1 k; k-groups G1..
    // of the sum are theirs. The stateful LSTM gates x_t W + h_{t-1} U.
    const float *A2;
    const float *B2;
    int64_t lda2, ldb2;
    int G1;  // k-groups of the first pair
};

constexpr int PT = 32;         // output tile edge
constexpr int PKG = 32;        // k per k-group: 4 KB of each operand, whole 128-byte lines
constexpr int PSTAGE = 2048;   // floats per ring stage: B 32 k-rows x 32, then A 32 rows x 32
constexpr int PRS = 36;        // floats between the rows of a partial tile in the reduction

// A rows in LDS: 32 floats (8 chunks of 16 bytes) per row; chunk c of row r is stored in
// slot c ^ ((r / 2) % 8), so the 16 rows a 128-bit fragment read phase covers fall on 16
// distinct bank groups.
__device__ __forceinline__ int pa_swz(int r) { return (r >> 1) & 7; }

template <int NW, int D, bool AKC, bool BKC, bool TWO>
__global__ void __launch_bounds__(NW * 64) gemm_panel_kernel(PanelArgs p) {
    static_assert(D * PSTAGE >= PT * PRS, "a partial tile fits in its wavefront's ring");
    static_assert(8 * (D - 1) < 64, "vmcnt range");
    __shared__ float ring[NW * D * PSTAGE];

    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

    // ---- work-group -> (batch, tile); both row tiles of a column block on one XCD ----
    int pid = blockIdx.x;
    // (a select, not a branch: a branch here splits the kernel-argument loads in two rounds)
    pid = (p.total & 7) == 0 ? (pid & 7) * (p.total >> 3) + (pid >> 3) : pid;
    const int b = (int)fast_div((uint32_t)pid, p.per_batch);
    const int t = pid - b * (int)p.per_batch.d;
    const int tn = (int)fast_div((uint32_t)t, p.tm_div);
    const int tm = t - tn * p.tiles_m;
    const int m0 = __builtin_amdgcn_readfirstlane(tm * PT);
    const int n0 = __builtin_amdgcn_readfirstlane(tn * PT);
    const int bb = __builtin_amdgcn_readfirstlane(b);

    // ---- this wavefront's k-groups ----
    const int G = p.K / PKG;
    const int per = (G + NW - 1) / NW;
    const int g0 = min(G, w * per);
    const int ng = min(G, g0 + per) - g0;

    // The bias of this thread's 4 output columns (every group a thread stores below starts
    // at column n0 + 4 (tid % 8)), loaded now: in the epilogue its memory latency was ~0.5 us
    // of the 64 x 1536 x 4096 gate GEMM's ~8.7 us.
    f4 bias4 = f4{0.f, 0.f, 0.f, 0.f};
    {
        const int nb = n0 + (threadIdx.x & 7) * 4;
        if (p.bias != nullptr && nb < p.N) bias4 = *reinterpret_cast<const f4u *>(p.bias + nb);
    }
    // Likewise the C group a thread adds onto (accumulate) when each thread stores one group
    // (NW >= 4): in the epilogue its latency was ~0.15 us of the 64 x 1024 x 4096 recurrent
    // step. C overlaps no operand (the entry points reject aliasing) and only this thread
    // writes it, after the k loop.
    constexpr bool CPRE = NW * 64 >= PT * PT / 4;
    f4 c4 = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (CPRE) {
        const int mi = threadIdx.x >> 3;
        const int nq = (threadIdx.x & 7) * 4;
        if (p.accumulate && mi < PT && m0 + mi < p.M && n0 + nq < p.N)
            c4 = *reinterpret_cast<const f4u *>(p.C + (int64_t)bb * p.sC +
                                                (int64_t)(m0 + mi) * p.ldc + n0 + nq);
    }

    float *my = ring + w * D * PSTAGE;
    f16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;

    if (ng > 0) {
        // Each operand's 32 x 32 slice of a k-group is 4 load instructions of 1 KB per
        // wavefront (lane L: 16 bytes at LDS float 256 q + 4 L of the operand's half of the
        // stage), in one of two layouts:
        //  * K-contiguous (A not transposed, B transposed): rows of 32 k. Lane L of
        //    instruction q loads row 8q + L/8 (clamped) into slot L % 8, the row's k chunk
        //    (L % 8) ^ pa_swz(row); a fragment of 4 consecutive k is one 16-byte read.
        //  * k-rows (A transposed, B not): 32 k-rows of 32 columns. Lane L of instruction q
        //    loads k-row 8q + L/8, columns i0 + 4 (L % 8) .. +3 (clamped to the last whole
        //    chunk); a fragment is 4 reads of one column in consecutive k-rows.
        // Offsets are bytes from the operand's element (i0, k-group 0) of this wavefront.
        auto offsets = [&](auto kc, int i0, int extent, int64_t ld, uint32_t(&off)[4]) {
            if constexpr (decltype(kc)::value) {
                const int rl = lane >> 3;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = 8 * q + rl;
                    int row = i0 + r;
                    row = row < extent - 1 ? row : extent - 1;
                    const int chunk = (lane & 7) ^ pa_swz(r);
                    off[q] = (uint32_t)((((uint32_t)(row - i0)) * (uint32_t)ld + 4u * chunk) * 4u);
                }
            } else {
                int col = i0 + 4 * (lane & 7);
                col = col < extent - 4 ? col : extent - 4;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    off[q] = (uint32_t)((((uint32_t)(8 * q + (lane >> 3))) * (uint32_t)ld +
                                         (uint32_t)(col - i0)) * 4u);
            }
        };
        uint32_t aoffs[4], boffs[4];
        offsets(std::integral_constant<bool, AKC>{}, m0, p.M, p.lda, aoffs);
        offsets(std::integral_constant<bool, BKC>{}, n0, p.N, p.ldb, boffs);
        // (TWO: the bases are the pairs' k-group 0 and issue() adds the absolute k-group)
        const int gb = TWO ? 0 : g0;
        const char *abase = reinterpret_cast<const char *>(
            p.A + (int64_t)bb * p.sA +
            (AKC ? (int64_t)m0 * p.lda + (int64_t)gb * PKG : (int64_t)gb * PKG * p.lda + m0));
        const char *bbase = reinterpret_cast<const char *>(
            p.B + (int64_t)bb * p.sB +
            (BKC ? (int64_t)n0 * p.ldb + (int64_t)gb * PKG : (int64_t)gb * PKG * p.ldb + n0));
        // bytes per k-group
        const int64_t astep = AKC ? (int64_t)PKG * 4 : (int64_t)PKG * p.lda * 4;
        const int64_t bstep = BKC ? (int64_t)PKG * 4 : (int64_t)PKG * p.ldb * 4;
        uint32_t aoffs2[4] = {0, 0, 0, 0}, boffs2[4] = {0, 0, 0, 0};
        const char *abase2 = nullptr, *bbase2 = nullptr;
        int64_t astep2 = 0, bstep2 = 0;
        if constexpr (TWO) {
            offsets(std::integral_constant<bool, AKC>{}, m0, p.M, p.lda2, aoffs2);
            offsets(std::integral_constant<bool, BKC>{}, n0, p.N, p.ldb2, boffs2);
            abase2 = reinterpret_cast<const char *>(p.A2 + (AKC ? (int64_t)m0 * p.lda2 : m0));
            bbase2 = reinterpret_cast<const char *>(p.B2 + (BKC ? (int64_t)n0 * p.ldb2 : n0));
            astep2 = AKC ? (int64_t)PKG * 4 : (int64_t)PKG * p.lda2 * 4;
            bstep2 = BKC ? (int64_t)PKG * 4 : (int64_t)PKG * p.ldb2 * 4;
        }

        // The first MFMA sub-group of a k-group needs k 0..7 of both operands: all four
        // instructions of a K-contiguous operand, the first of a k-row one. K-contiguous
        // operands are issued first and k-row operands interleaved by instruction, so those
        // loads are the oldest PEEL of the 8.
        constexpr int PEEL = 4 * ((int)AKC + (int)BKC) + ((int)!AKC + (int)!BKC);
        // the 8 loads of one k-group from operand bases ag / bg with lane offsets ao / bo
        auto issue_from = [&](const char *ag, const char *bg, const uint32_t(&ao)[4],
                              const uint32_t(&bo)[4], float *st) {
            if constexpr (AKC) {
#pragma unroll
                for (int q = 0; q < 4; ++q) dma16(ag, ao[q], st + 1024 + 256 * q);
            }
            if constexpr (BKC) {
#pragma unroll
                for (int q = 0; q < 4; ++q) dma16(bg, bo[q], st + 256 * q);
            }
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if constexpr (!AKC) dma16(ag, ao[q], st + 1024 + 256 * q);
                if constexpr (!BKC) dma16(bg, bo[q], st + 256 * q);
            }
        };
        auto issue = [&](int j, int slot) {
            const int g = j < ng ? j : ng - 1;
            float *st = my + slot * PSTAGE;
            if constexpr (TWO) {
                // absolute k-group g0 + g: a wave-uniform branch to the pair that holds it
                // (per-lane selects of the 8 offsets cost ~35 instructions per k-group)
                const int ga = g0 + g;
                if (ga >= p.G1)
                    issue_from(abase2 + (int64_t)(ga - p.G1) * astep2,
                               bbase2 + (int64_t)(ga - p.G1) * bstep2, aoffs2, boffs2, st);
                else
                    issue_from(abase + (int64_t)ga * astep, bbase + (int64_t)ga * bstep, aoffs,
                               boffs, st);
            } else {
                issue_from(abase + (int64_t)g * astep, bbase + (int64_t)g * bstep, aoffs, boffs,
                           st);
            }
        };
        // Fragments of sub-group j (k = 8j .. 8j+7 of the k-group), step s: B lane l holds
        // column l%32 at k-row 8j + 4(l/32) + s; A lane l holds row l%32 at the same k.
        const int lo = lane & 31;
        const int hi = lane >> 5;
        auto frag = [&](auto kc, const float *half, int j) {
            f4 v;
            if constexpr (decltype(kc)::value) {
                v = dl_load16(half + lo * PT + 4 * ((2 * j + hi) ^ pa_swz(lo)));
            } else {
#pragma unroll
                for (int s = 0; s < 4; ++s) v[s] = half[(8 * j + 4 * hi + s) * PT + lo];
            }
            return v;
        };
        auto frag_a = [&](int slot, int j) {
            return frag(std::integral_constant<bool, AKC>{}, my + slot * PSTAGE + 1024, j);
        };
        auto frag_b = [&](int slot, int j) {
            return frag(std::integral_constant<bool, BKC>{}, my + slot * PSTAGE, j);
        };

        struct Frags {
            f4 b[4];
            f4 a[4];
        };
        auto read = [&](int slot, Frags &f) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f.b[j] = frag_b(slot, j);
                f.a[j] = frag_a(slot, j);
            }
        };
        auto mma = [&](const Frags &f, int j) {
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(f.b[j][s], f.a[j][s], acc, 0, 0, 0);
        };
        // D k-groups in flight; k-group i+1's fragments are read into a second register set
        // while k-group i's last MFMAs run, so LDS latency is not exposed.
#pragma unroll
        for (int j = 0; j < D; ++j) issue(j, j);
        Frags cur, nxt;
        int i0 = 0;
        if constexpr (D == 1) {
            // k-group 0 peeled: its first sub-group starts once the loads it needs have
            // landed (PEEL of the 8), while the rest of the k-group is still arriving
            wait_vmcnt<8 - PEEL>();
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (AKC || j == 0) cur.a[j] = frag_a(0, j);
                if (BKC || j == 0) cur.b[j] = frag_b(0, j);
            }
            __builtin_amdgcn_sched_barrier(0);
            mma(cur, 0);
            // MFMA intrinsics do not touch memory, so without a use here the compiler moves
            // them past the wait below
            asm volatile("" ::"v"(acc[0]));
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<0>();
#pragma unroll
            for (int j = 1; j < 4; ++j) {
                if constexpr (!AKC) cur.a[j] = frag_a(0, j);
                if constexpr (!BKC) cur.b[j] = frag_b(0, j);
            }
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the slot is read
            issue(1, 0);
            __builtin_amdgcn_sched_barrier(0);
            mma(cur, 1);
            mma(cur, 2);
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<0>();  // k-group 1 has landed
            read(0, nxt);
            __builtin_amdgcn_sched_barrier(0);
            mma(cur, 3);
            cur = nxt;
            i0 = 1;
        } else {
            wait_vmcnt<8 * (D - 1)>();  // k-group 0 has landed
            read(0, cur);
        }
        for (int i = i0; i < ng; ++i) {
            mma(cur, 0);
            __builtin_amdgcn_sched_barrier(0);
            // cur's fragments are all in registers: refill slot i%D after the first 4 MFMAs,
            // so k-group i+D's loads have 8 MFMAs (and the other wavefront's work) to land
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            issue(i + D, i % D);
            __builtin_amdgcn_sched_barrier(0);
            mma(cur, 1);
            mma(cur, 2);
            __builtin_amdgcn_sched_barrier(0);
            wait_vmcnt<8 * (D - 1)>();  // k-group i+1 has landed
            read((i + 1) % D, nxt);
            __builtin_amdgcn_sched_barrier(0);
            mma(cur, 3);
            cur = nxt;
        }
        wait_vmcnt<0>();
    }

    // ---- combine the NW wavefronts in order, add the bias, store ----
    // Each wavefront writes its partial tile into its own ring (all of its loads have landed
    // and its own reads are done), so a single barrier precedes the sum. acc register 4g + j
    // of lane l is C(row l % 32, column 8g + 4(l / 32) + j); partial rows are 36 floats apart
    // (16-byte aligned), so a thread adds 4 columns per LDS read.
    {
        float *red = ring + w * D * PSTAGE;
        const int lo = lane & 31;
        const int hi = lane >> 5;
#pragma unroll
        for (int g = 0; g < 4; ++g)
            *reinterpret_cast<f4 *>(red + lo * PRS + 8 * g + 4 * hi) =
                f4{acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
    }
    __syncthreads();
    float *Cb = p.C + (int64_t)bb * p.sC;
    for (int e = threadIdx.x; e < PT * PT / 4; e += NW * 64) {
        const int mi = e >> 3;
        const int nq = (e & 7) * 4;  // = the bias group loaded above: NW * 64 % 8 == 0
        f4 v = *reinterpret_cast<const f4 *>(ring + mi * PRS + nq);
#pragma unroll
        for (int q = 1; q < NW; ++q)
            v += *reinterpret_cast<const f4 *>(ring + q * D * PSTAGE + mi * PRS + nq);
        const int m = m0 + mi;
        const int n = n0 + nq;
        if (m < p.M && n < p.N) {  // N % 4 == 0: the whole group is inside
            if (p.bias != nullptr) v = v + bias4;
            f4u *c = reinterpret_cast<f4u *>(Cb + (int64_t)m * p.ldc + n);
            if (p.accumulate) v = (CPRE ? c4 : f4(*c)) + v;
            *c = v;
        }
    }
}

// One k-group ring slot per wavefront (D = 1), NW wavefronts along K; operand layouts AKC
// (A K-contiguous, i.e. not transposed) and BKC (B K-contiguous, i.e. transposed); TWO: a
// second operand pair.
template <bool AKC, bool BKC, bool TWO>
int launch_nw(hipStream_t stream, const PanelArgs &a, int nw) {
    switch (nw) {
        case 8: MIGEMM_LAUNCH((gemm_panel_kernel<8, 1, AKC, BKC, TWO>), dim3(a.total), dim3(8 * 64), 0, stream, a); break;
        case 4: MIGEMM_LAUNCH((gemm_panel_kernel<4, 1, AKC, BKC, TWO>), dim3(a.total), dim3(4 * 64), 0, stream, a); break;
        case 2: MIGEMM_LAUNCH((gemm_panel_kernel<2, 1, AKC, BKC, TWO>), dim3(a.total), dim3(2 * 64), 0, stream, a); break;
        default: MIGEMM_LAUNCH((gemm_panel_kernel<1, 1, AKC, BKC, TWO>), dim3(a.total), dim3(64), 0, stream, a); break;
    }
    return launch_status("gemm_panel_kernel launch");
}

template <bool TWO>
int launch_layout(hipStream_t stream, const PanelArgs &a, const GemmDesc &d, int nw) {
    if (!d.transA && !d.transB) return launch_nw<true, false, TWO>(stream, a, nw);
    if (!d.transA) return launch_nw<true, true, TWO>(stream, a, nw);
    if (!d.transB) return launch_nw<false, false, TWO>(stream, a, nw);
    return launch_nw<false, true, TWO>(stream, a, nw);
}

bool aligned16(const float *p, int64_t ld, int64_t stride) {
    return ((uintptr_t)p & 15) == 0 && ld % 4 == 0 && stride % 4 == 0;
}

}  // namespace

bool panel_supported(const GemmDesc &d) {
    // Whole 32-wide k-groups; 16-byte chunks of C's rows (the epilogue) and of a k-row
    // operand's rows (B not transposed: N % 4 == 0; A transposed: M % 4 == 0); every
    // operand row 16-byte aligned; each lane's load offset within a k-group fits 32 bits:
    // below 32 ld * 4 bytes for a K-contiguous operand, (31 ld + extent) * 4 <= 128 ld bytes
    // for a k-row one. A second operand pair (batch 1) meets the same conditions.
    const bool pair1 = d.K % PKG == 0 && d.N % 4 == 0 && d.N >= 4 &&
                       (!d.transA || d.M % 4 == 0) && aligned16(d.A, d.lda, d.sA) &&
                       aligned16(d.B, d.ldb, d.sB) && d.lda <= ((int64_t)1 << 25) &&
                       d.ldb <= ((int64_t)1 << 25);
    if (d.A2 == nullptr) return pair1;
    return pair1 && d.batch == 1 && d.K2 % PKG == 0 && aligned16(d.A2, d.lda2, 0) &&
           aligned16(d.B2, d.ldb2, 0) && d.lda2 <= ((int64_t)1 << 25) &&
           d.ldb2 <= ((int64_t)1 << 25);
}

// Where the panel kernel beats the other families (graph replay, NN, M in 16..256, N in
// 512..8192, K in 256..4096, 246 shapes; us, panel / the previous choice): one to three
// rounds of 32x32 tiles, 128-768 tiles (64 x 1536 x 4096 10.3 / 13.3, 96 x 1536 x 2048 9.8 /
// 18.1 split 64x64 tiles, 256 x 512 x 2048 8.7 / 13.9, 96 x 4096 x 8192 59.5 / 76.4); fewer
// tiles while K is short enough that one CU per tile is not the bottleneck (64 x 1024 x 1024
// 7.2 / 8.5, 128 x 512 x 512 5.3 / 7.0; but 32 x 1024 x 512 7.0 / 6.4 and 64 x 4096 x 1024
// 19.0 / 12.7 with K split over work-groups). It loses at K = 256 below 192 tiles (4.1-4.4
// against 3.4-4.0: its fixed cost is higher), above 768 tiles (256 x 512 x 4096 16.1 / 13.7
// in 64x64 tiles) and at M <= 16, where half of each 32-row tile is empty. A later audit
// (288 shapes, batch 1 / 8 / 32, M and N 64-512, K 384-1024) moved two bounds: K = 384 pays
// from 128 tiles (batch-8 64 x 384 x 256 5.1 against 5.9 us on the small kernel) and with
// 32-63 tiles K stops at 768 (256 x 1024 x 128 7.0 against 6.3 us).
bool panel_preferred(const GemmDesc &d) {
    // (N <= 16 too: three quarters of each 32-column tile would be empty; batch-16 1024 x 1024
    // x 8 TN 16.7 us here, 14.6 on the small kernel)
    if (d.M <= 16 || d.N <= 16 || !panel_supported(d)) return false;
    const int64_t tiles = (int64_t)((d.M + PT - 1) / PT) * ((d.N + PT - 1) / PT) * d.batch;
    // a second operand pair runs as one GEMM over the concatenated k: K + K2
    if (d.A2 != nullptr) {
        GemmDesc one = d;
        one.A2 = nullptr;
        one.K = d.K + d.K2;
        return panel_preferred(one);
    }
    if (tiles < 16 || tiles > 768) return false;
    // Long K with many tiles: every XCD streams the A panels of all its tiles' rows, and the
    // tiled kernel's 64x64 tiles (split over k) re-read half as much (768 x 4096 x 768: 54.6
    // against 45.8 us; 1024 x 4096 x 768 63.7 / 54.9; batch-8 256 x 8192 x 256 77.1 / 71.1),
    // while up to 512 tiles the panel kernel stays ahead with 512 rows (512 x 2048 x 512 11.8
    // against 15.5; batch-8 512 x 1536 x 128 17.1 / 23.7) and with few rows at 768 tiles
    // (96 x 4096 x 8192 59.5 / 76.4).
    if ((d.M > 256 && tiles > 512 && d.K > 1024) || (d.K >= 8192 && tiles >= 512)) return false;
    if (d.K < (tiles < 128 ? 512 : tiles < 192 ? 384 : 256)) return false;
    const int kmax = tiles < 32 ? 512 : tiles < 64 ? 768 : tiles < 128 ? 1536
                     : tiles < 192 ? 2048 : 1 << 30;
    return d.K <= kmax;
}

int launch_gemm_panel(hipStream_t stream, const GemmDesc &d) {
    PanelArgs a;
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
    a.tiles_m = (d.M + PT - 1) / PT;
    a.tiles_n = (d.N + PT - 1) / PT;
    a.batch = d.batch;
    const int64_t total = (int64_t)a.tiles_m * a.tiles_n * d.batch;
    if (total > 0x7fffffff)
        return set_error(MIGEMM_ERR_UNSUPPORTED, "gemm_panel: %lld work-groups", (long long)total);
    a.total = (int)total;
    a.accumulate = d.accumulate;
    a.per_batch = make_fastdiv((uint32_t)(a.tiles_m * a.tiles_n));
    a.tm_div = make_fastdiv((uint32_t)a.tiles_m);
    const bool two = d.A2 != nullptr;
    a.A2 = d.A2;
    a.B2 = d.B2;
    a.lda2 = d.lda2;
    a.ldb2 = d.ldb2;
    a.G1 = d.K / PKG;
    if (two) a.K = d.K + d.K2;  // the kernel walks the k-groups of both pairs
    // NW wavefronts split the k-groups (8, two per SIMD, unless K has fewer k-groups), each
    // with one k-group (8 KB) in flight while it multiplies the previous one: 64 KB of LDS.
    // Measured at 64 x 1536 x 4096 (100 rotating inputs, graph replay, us): 8 wavefronts
    // with 1 / 2 k-groups in flight 9.65 / 10.24, 4 with 2 / 3 / 4 10.86 / 11.01 / 11.86, 16
    // with 1 10.8. Deeper queues do not pay: the k loop alone (no loads) runs at ~91 % of
    // the MFMA rate, and more loads in flight only slowed the loads. Where the refill is
    // issued (min of 7 graph replays of 100 calls, two processes each, us, after 12 MFMAs
    // / at the k-group's start / after 4): 64 x 1536 x 4096 9.41 / 9.42 / 9.06, 256 x 512 x
    // 2048 9.11 / 8.86 / 8.54, 96 x 4096 x 8192 58.6 / 56.8 / 55.3; after 2 or 14 MFMAs
    // within 1 % of after 4. With the one-barrier epilogue (same harness, another box):
    // 9.20 -> 9.03, 9.01 -> 8.17 and 57.6 -> 55.1. Starting k-group 0 after 5 of its 8
    // loads: 8.95 -> 8.90, 8.15 -> 7.91, 64 x 1024 x 4096 7.03 -> 6.75.
    const int G = a.K / PKG;
    int nw = G >= 8 ? 8 : (G >= 4 ? 4 : (G >= 2 ? 2 : 1));
    const int rc = two ? launch_layout<true>(stream, a, d, nw)
                       : launch_layout<false>(stream, a, d, nw);
    GemmDesc shown = d;
    shown.K = a.K;
    record_plan(two ? "panel-pair" : "panel", shown, PT, PT, 1, 16);
    return rc;
}

}  // namespace migemm
