// Pieces shared by the tiled MFMA GEMM kernels (gemm_mfma.hip: operands staged through
// registers; gemm_direct.hip: operands loaded straight into LDS): the argument block, the
// work-group -> tile mapping and the epilogue that writes a wavefront's 32x32 accumulator
// blocks to C (or to the split-K partial buffer).
#pragma once

#include <type_traits>

#include "migemm_internal.h"

namespace migemm {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16 __attribute__((ext_vector_type(16)));

struct TiledArgs {
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
    int splits;            // split-K ranges (1 = no split)
    int kt_per_split;      // k-tiles per range
    float *partial;        // [splits][batch][M][N] partial sums when splits > 1
    int accumulate;        // C += result instead of C = result
    int write_back;        // C stored through L2 (write-back) instead of non-temporally
    // launch-invariant divisors of tile_coord (multiply-high divisions), set by
    // set_tile_divisors once tiles_m, tiles_n, batch are final
    FastDiv per_split;     // tiles_m * tiles_n * batch
    FastDiv per_batch;     // tiles_m * tiles_n
    FastDiv in_group;      // GROUP * tiles_n
    FastDiv last_group;    // rows of tiles in the last group of 8 (tiles_m % 8, or 8)
};

constexpr int TILE_GROUP = 8;  // tile-rows rastered together

inline void set_tile_divisors(TiledArgs &a) {
    a.per_batch = make_fastdiv((uint32_t)(a.tiles_m * a.tiles_n));
    a.per_split = make_fastdiv((uint32_t)(a.tiles_m * a.tiles_n * a.batch));
    a.in_group = make_fastdiv((uint32_t)(TILE_GROUP * a.tiles_n));
    const int rem = a.tiles_m % TILE_GROUP;
    a.last_group = make_fastdiv((uint32_t)(rem == 0 ? TILE_GROUP : rem));
}

struct TileCoord {
    int split, b, m0, n0;
};

// Work-group id -> (split range, batch entry, tile origin). The dispatcher deals work-groups
// round-robin over the 8 XCDs (each with its own L2), so ids are first remapped to give each
// XCD a contiguous chunk of tiles, then rastered in groups of 8 tile-rows so concurrently
// running tiles share A and B panels in that L2.
template <int BM, int BN>
__device__ __forceinline__ TileCoord tile_coord(const TiledArgs &p, int pid) {
    const int total = p.total;
    // (a select, not a branch: a branch here splits the kernel-argument loads in two rounds)
    pid = (total & 7) == 0 ? (pid & 7) * (total >> 3) + (pid >> 3) : pid;
    TileCoord tc;
    tc.split = (int)fast_div((uint32_t)pid, p.per_split);
    pid -= tc.split * (int)p.per_split.d;
    tc.b = (int)fast_div((uint32_t)pid, p.per_batch);
    const int t = pid - tc.b * (int)p.per_batch.d;
    const int grp = (int)fast_div((uint32_t)t, p.in_group);
    const int first_m = grp * TILE_GROUP;
    const int tg = t - grp * (int)p.in_group.d;  // index within the group
    int tm, tn;
    if (p.tiles_m - first_m >= TILE_GROUP) {  // a whole group of 8 tile-rows
        tm = first_m + (tg & (TILE_GROUP - 1));
        tn = tg / TILE_GROUP;
    } else {  // the last, shorter group
        tn = (int)fast_div((uint32_t)tg, p.last_group);
        tm = first_m + tg - tn * (int)p.last_group.d;
    }
    tc.m0 = tm * BM;
    tc.n0 = tn * BN;
    return tc;
}

// Writes FM x FN accumulator blocks of 32x32 whose top-left output is (r0, c0). Register r
// of block (i, j) holds row r0 + 32i + 8(r/4) + 4(lane/32) + r%4, column c0 + 32j + lane%32.
// Split ranges write raw partial sums to p.partial (reduce_slices_kernel adds them in range
// order and applies bias / accumulate); otherwise the bias is added after the k loop
// (linear.cl:119-122) and C is written, or added to with p.accumulate.
template <int FM, int FN>
__device__ __forceinline__ void store_tile(const TiledArgs &p, const TileCoord &tc, int r0,
                                           int c0, int lane, const f16 (&acc)[FM][FN]) {
    const int lo = lane & 31;
    const int hi = lane >> 5;
    if (p.splits > 1) {
        float *Pb = p.partial + ((int64_t)tc.split * p.batch + tc.b) * p.M * p.N;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = c0 + j * 32 + lo;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = r0 + i * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
                    if (col < p.N && row < p.M) Pb[(int64_t)row * p.N + col] = acc[i][j][r];
                }
        }
        return;
    }
    float *Cb = p.C + (int64_t)tc.b * p.sC;
    // Copies of the store loop behind a uniform branch, so a plain store never carries a
    // (speculated) load of C. The plain store is non-temporal: every work-group of a large
    // GEMM writes its tile at about the same time, at the end, and dirty C lines held in L2
    // are written back when the kernel ends, before the next kernel on the stream can start
    // (4096^3 forms back to back: 2.758-2.768 -> 2.750-2.756 ms per step of three).
    // p.write_back (tiles 128 or more wide whose C rows do not start on 64-byte boundaries)
    // stores through L2 instead: each row of such a tile begins and ends in a line it shares
    // with a neighbouring tile, and L2 merges the two parts before the line goes to HBM
    // (graph replay, us, non-temporal / write-back: 8192 x 64 x 8180 in 128x128 tiles
    // 213.3 / 129.4, 12000 x 500 x 6565 NT in 128x256 686.7 / 647.8, 4096 x 4096 x 4095 TN
    // in 256x256 942.9 / 924.2; 64x64 tiles lose with it, 12000 x 80 x 6565 NT 172.7 /
    // 189.0). Split-K partials keep ordinary stores: the reduction reads them right away.
    auto store = [&](auto mode) {  // 0: non-temporal, 1: write-back, 2: C += result
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = c0 + j * 32 + lo;
            const bool cok = col < p.N;
            float bv = 0.f;
            if (p.bias != nullptr && cok) bv = p.bias[col];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = r0 + i * 32 + 8 * (r >> 2) + 4 * hi + (r & 3);
                    if (cok && row < p.M) {
                        float v = acc[i][j][r];
                        if (p.bias != nullptr) v = v + bv;
                        float *c = Cb + (int64_t)row * p.ldc + col;
                        if constexpr (decltype(mode)::value == 2)
                            *c = *c + v;
                        else if constexpr (decltype(mode)::value == 1)
                            *c = v;
                        else
                            __builtin_nontemporal_store(v, c);
                    }
                }
            }
        }
    };
    if (p.accumulate)
        store(std::integral_constant<int, 2>{});
    else if (p.write_back)
        store(std::integral_constant<int, 1>{});
    else
        store(std::integral_constant<int, 0>{});
}

// Tiles of bm x bn (256x256, 128x256, 128x128 or 64x64) with operands loaded straight into
// LDS (gemm_direct.hip). wa / wb: floats per lane of each operand's loads, 4 (every row and
// batch entry 16-byte aligned and the contiguous extent a multiple of 4: K for a
// K-contiguous operand, M or N otherwise) or 1 (any operand).
// On entry a.splits is the requested number of split-K ranges; on return `a` holds the grid
// (tiles_m, tiles_n, kt_per_split in the kernel's k-tiles, total) and the non-empty range
// count.
int launch_gemm_direct(hipStream_t stream, TiledArgs &a, int bm, int bn, bool akc, bool bkc,
                       int wa = 4, int wb = 4);

}  // namespace migemm
