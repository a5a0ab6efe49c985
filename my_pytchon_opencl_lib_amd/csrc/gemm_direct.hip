// Tiled fp32 GEMM for gfx950 with operands loaded straight from global memory into LDS.
//
// The same product as gemm_mfma_kernel (matmul.cl:8-135 NN, bmm_permute_tiled.cl NT / TN,
// the bias epilogue of linear.cl:119-122) for 256x256 output tiles whose operands allow
// 128-bit loads everywhere (every contiguous extent a multiple of 4). It differs in how the
// operands reach LDS:
//  * global_load_lds_dwordx4 (gfx950) moves each lane's 16 bytes from global memory to LDS
//    without passing through registers. One wavefront instruction fills 1 KB of LDS: lane L's
//    bytes land at M0 + 16 L. The kernel holds no staging registers, which leaves room for
//    BK = 32 k-tiles (the register-staged kernel spills at BK = 32 with an I-contiguous
//    operand) and for the next k-group's fragments.
//  * S LDS stages, loads D tiles ahead (shipped: BK = 32, S = D = 2; 2 x 130 KB). Every
//    fragment read of a tile's stage is issued before the tile's one barrier, so the
//    barrier (1) publishes tile kt+1, for which each wavefront first waits with
//    s_waitcnt vmcnt (the compiler does not track these loads), and (2) retires the stage
//    just read, which the loads of tile kt+D then reuse. The last k-group's MFMAs follow the
//    barrier, and the first MFMAs of tile kt+1 follow them without a barrier in between.
//  * LDS layouts (per stage, unpadded where a wavefront's 1 KB write must be contiguous):
//      K-contiguous operand (A not transposed, B transposed): 256 rows x BK k, row r at
//        BK r floats. Chunk c (4 floats) of row r is stored in slot c ^ kc_swz(r), so a
//        16-lane phase of an MFMA fragment read (16 consecutive rows, one chunk each) hits
//        16 distinct 16-byte bank groups. A load instruction covers 64 / (BK / 4) whole rows
//        and each lane fetches the chunk that belongs in its slot.
//      I-contiguous operand (A transposed, B not transposed): BK k-rows of 256 floats, row k
//        at k * 264 floats (one load instruction per k-row; the 8-float pad keeps the two
//        half-wavefronts of a fragment read, k-rows 4 apart, on different banks).
//  * Edges: rows / columns beyond M / N are clamped on load (they feed outputs that are not
//    stored); the k tail (K % BK != 0) is fetched through registers with k >= K zero-filled
//    (matmul.cl:39-52) and written into the same layout after the pipelined loop (64x64
//    tiles fetch it before the loop, so its latency is hidden); k-groups wholly past K
//    are skipped.
//  * K order within an MFMA step, split-K ranges, the XCD-aware raster and the epilogue are
//    those of gemm_mfma_kernel (tiled_common.h); each output's k sum runs in the same order
//    as in gemm_mfma_kernel, so both give identical bits for one split.
#include "gemm_direct.h"

namespace migemm {

int launch_gemm_direct(hipStream_t stream, TiledArgs &a, int bm, int bn, bool akc, bool bkc,
                       int wa, int wb) {
    // An operand with wa / wb = 1 (rows not 16-byte aligned, or a contiguous extent that is
    // not a multiple of 4) is loaded 4 bytes per lane in the same pipeline.
    if (bm == 256) return launch_direct_256(stream, a, akc, bkc, wa, wb);
    if (bm == 64) return launch_direct_64(stream, a, akc, bkc, wa, wb);
    if (bn == 256) return launch_direct_128x256(stream, a, akc, bkc, wa, wb);
    return launch_direct_128(stream, a, akc, bkc, wa, wb);
}

}  // namespace migemm
