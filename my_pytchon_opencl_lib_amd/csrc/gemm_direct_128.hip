// gemm_direct_kernel instantiations for 128x128 tiles (kernel: gemm_direct.hip, gemm_direct.h).
#include "gemm_direct.h"

namespace migemm {

int launch_direct_128(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa, int wb) {
    // Split-K ranges take the variant without the 128-VGPR cap (three work-groups per CU):
    // the ranges are sized for ~1024 work-groups, which at four per CU leave a nearly empty
    // second round. Measured (us, capped / uncapped / register-staged): 6400 x 4096 x 512 NT
    // in 6 ranges 263.1 / 230.6 / 244.4; 500 x 12000 x 6564 TN in 6 ranges 700.7 / 603.6 /
    // 651.2.
    const bool split = a.splits > 1;
    if (wa != 4 || wb != 4) {
        if (split) {
            if (wa == 1 && wb == 1) return launch_layouts<128, 128, 16, 2, 2, 1, 1, 1>(stream, a, akc, bkc);
            if (wa == 1) return launch_layouts<128, 128, 16, 2, 2, 1, 1, 4>(stream, a, akc, bkc);
            return launch_layouts<128, 128, 16, 2, 2, 1, 4, 1>(stream, a, akc, bkc);
        }
        if (wa == 1 && wb == 1) return launch_layouts<128, 128, 16, 2, 2, 4, 1, 1>(stream, a, akc, bkc);
        if (wa == 1) return launch_layouts<128, 128, 16, 2, 2, 4, 1, 4>(stream, a, akc, bkc);
        return launch_layouts<128, 128, 16, 2, 2, 4, 4, 1>(stream, a, akc, bkc);
    }
    // BK = 16, two stages (32 KB) and at most 128 VGPRs: four work-groups (16 wavefronts) per
    // CU. Measured (us; direct with this occupancy / with up to 168 VGPRs, three work-groups
    // / three stages / BK = 32 / register-staged): 4096 x 1024 x 4096 NN 249.6 / 293.9 /
    // 307.0 / 258.5 / 271.0; 4096^3 949.7 / 1141.4 / 943.5 / 957.2 / 1033.0; 2048^3 TN 142.2 / 145.6 / 147.0 / 154.3 / 164.3;
    // 6400 x 512 x 4096 226.9 / 230.6 / 230.5 / 243.3 / 243.0. With three work-groups per CU
    // the 1024 tiles of a 4096-wide output leave a ragged last round.
    if (split) return launch_layouts<128, 128, 16, 2, 2>(stream, a, akc, bkc);
    return launch_layouts<128, 128, 16, 2, 2, 4>(stream, a, akc, bkc);
}

}  // namespace migemm
