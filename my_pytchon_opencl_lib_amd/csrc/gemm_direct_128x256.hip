// gemm_direct_kernel instantiations for 128x256 tiles (kernel: gemm_direct.hip, gemm_direct.h).
#include "gemm_direct.h"

namespace migemm {

int launch_direct_128x256(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa,
                          int wb) {
    if (wa != 4 || wb != 4) {
        if (wa == 1 && wb == 1) return launch_layouts<128, 256, 16, 3, 2, 1, 1, 1>(stream, a, akc, bkc);
        if (wa == 1) return launch_layouts<128, 256, 16, 3, 2, 1, 1, 4>(stream, a, akc, bkc);
        return launch_layouts<128, 256, 16, 3, 2, 1, 4, 1>(stream, a, akc, bkc);
    }
    // BK = 16 with three stages (2 x 72 KB: two work-groups per CU). At 4096 x K x 4096
    // (K = 256 .. 4096) and 4096 x 2048 x 2048 NT within 1 % of two stages
    // and 7-11 % faster than the register-staged 128x256 kernel.
    return launch_layouts<128, 256, 16, 3, 2>(stream, a, akc, bkc);
}

}  // namespace migemm
