// gemm_direct_kernel instantiations for 64x64 tiles (kernel: gemm_direct.hip, gemm_direct.h).
#include "gemm_direct.h"

namespace migemm {

int launch_direct_64(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa, int wb) {
    if (wa != 4 || wb != 4) {
        if (wa == 1 && wb == 1) return launch_layouts<64, 64, 32, 2, 2, 1, 1, 1>(stream, a, akc, bkc);
        if (wa == 1) return launch_layouts<64, 64, 32, 2, 2, 1, 1, 4>(stream, a, akc, bkc);
        return launch_layouts<64, 64, 32, 2, 2, 1, 4, 1>(stream, a, akc, bkc);
    }
    // 2 x 2 wavefronts of 32x32, BK = 32, two stages (32 KB). Against BK = 16
    // and three stages, us: 1024^3 22.4 / 22.6 / 22.5,
    // 2048 x 512 x 2048 38.8 / 40.1 / 43.6, 3072 x 1024 x 3072 157.1 / 156.0 / 151.9.
    // Loading further ahead did not pay either (us, shipped / BK = 32 with three stages
    // loaded three tiles ahead / BK = 16 with four stages four ahead): 1000 x 777 x 3000
    // 45.9 / 46.2 / 45.6, 2048 x 512 x 2048 38.4 / 40.5 / 38.3, 4096 x 1024 x 4096 263.2 /
    // 258.8 / 261.4, 12000 x 6565 x 500 NT 638.8 / 637.0 / 687.0. Nor did 5 or 8 stages
    // loaded as many tiles ahead on few-tile long-K shapes (us, shipped / BK = 32 with 8
    // stages / BK = 32 with 5 / BK = 16 with 8): 512 x 16384 x 512 TN 71.8 / 79.9 / 73.5 /
    // 72.7, 384 x 6000 x 384 27.8 / 33.1 / 29.5 / 28.4, 128 x 4096 x 4096 43.2 / 52.0 /
    // 45.9 / 45.1; the config-3 gate GEMM in 4 ranges 16.0 / 16.8 / 16.1 / 16.2 (the
    // small-output kernel: 14.7).
    return launch_layouts<64, 64, 32, 2, 2>(stream, a, akc, bkc);
}

}  // namespace migemm
