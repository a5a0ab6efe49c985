// gemm_direct_kernel instantiations for 256x256 tiles (kernel: gemm_direct.hip, gemm_direct.h).
#include "gemm_direct.h"

namespace migemm {

int launch_direct_256(hipStream_t stream, TiledArgs &a, bool akc, bool bkc, int wa, int wb) {
    if (wa != 4 || wb != 4) {
        if (wa == 1 && wb == 1) return launch_layouts<256, 256, 32, 2, 2, 1, 1, 1>(stream, a, akc, bkc);
        if (wa == 1) return launch_layouts<256, 256, 32, 2, 2, 1, 1, 4>(stream, a, akc, bkc);
        return launch_layouts<256, 256, 32, 2, 2, 1, 4, 1>(stream, a, akc, bkc);
    }
    // BK = 32 with two stages, loads two tiles ahead (2 x 128 KB of LDS, one barrier per
    // 32 k). Measured at 4096^3 against BK = 16 with three stages,
    // interleaved in one process, TFLOP/s NN / NT / TN: 148.2 / 150.9 / 147.4 against
    // 148.0 / 150.3 / 147.8; with loads three tiles ahead (three stages) 146.7 / 150.0 /
    // 143.4; four stages 145.9 / 149.9 / 142.9; TN with 8 wavefronts of 64x128
    // 144.3-145.5. The register-staged kernel: 144.6 / 147.7 / 143.0. Raising the wavefront
    // priority (s_setprio 1 or 3) around each k-group's MFMAs: 126.3 / 129.5 / 133.5 against
    // 149.6 / 150.1 / 149.3. Eight wavefronts of 64x128 with this pipeline (176-184 VGPRs):
    // 146.7 / 147.4 / 146.6 against 150.4 / 150.5 / 150.3.
    return launch_layouts<256, 256, 32, 2, 2>(stream, a, akc, bkc);
}

}  // namespace migemm
