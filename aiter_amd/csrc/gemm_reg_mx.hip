// Kernel instances, part 1: A4W4 and A8W4 tiles and skinny kernels.
#include "gemm_registry.h"

namespace aiter_amd {

void RegBuilder::part_mx() {
    // ---- a4w4 (B preshuffled): 32x32x64 tile kernels; the 256-column
    // tiles read B straight into registers (gemm_flat.h), the others stage
    // A and B through LDS (gemm_t32.h) ----
    const Variant pre = kPre, plain = kPlain;
    tile(kA4W4, 256, 256, pre, launch_flat<kFp4, 256>, "a4w4");
    tile(kA4W4, 256, 128, pre, launch_t32<kFp4, true, 256, 128, 2>, "a4w4");
    tile(kA4W4, 128, 256, pre, launch_flat<kFp4, 128>, "a4w4");
    tile(kA4W4, 128, 128, pre, launch_t32<kFp4, true, 128, 128, 2>, "a4w4");
    tile(kA4W4, 64, 256, pre, launch_t32<kFp4, true, 64, 256, 1>, "a4w4");
    tile(kA4W4, 64, 128, pre, launch_t32<kFp4, true, 64, 128, 1>, "a4w4");
    skinny(kA4W4, 1, false, pre, launch_skinny<kFp4, 1, true, false, false>, "a4w4");
    skinny(kA4W4, 2, false, pre, launch_skinny<kFp4, 2, true, false, false>, "a4w4");
    skinny(kA4W4, 4, false, pre, launch_skinny<kFp4, 4, true, false, false>, "a4w4");
    skinny(kA4W4, 1, true, pre, launch_skinny<kFp4, 1, true, true, false>, "a4w4");
    skinny(kA4W4, 2, true, pre, launch_skinny<kFp4, 2, true, true, false>, "a4w4");
    skinny(kA4W4, 4, true, pre, launch_skinny<kFp4, 4, true, true, false>, "a4w4");
    // a4w4 with row-major B (bpreshuffle = 0)
    tile(kA4W4, 128, 128, plain, launch_t32<kFp4, false, 128, 128, 2>, "a4w4");
    tile(kA4W4, 64, 128, plain, launch_t32<kFp4, false, 64, 128, 1>, "a4w4");
    skinny(kA4W4, 1, false, plain, launch_skinny<kFp4, 1, false, false, false>, "a4w4");
    skinny(kA4W4, 2, false, plain, launch_skinny<kFp4, 2, false, false, false>, "a4w4");
    skinny(kA4W4, 4, false, plain, launch_skinny<kFp4, 4, false, false, false>, "a4w4");
    // ---- a8w4 ----
    const Variant a8 = kPre, a8p = kA8Pre;
    tile(kA8W4, 128, 256, a8, launch_flat<kFp8, 128>, "a8w4");
    tile(kA8W4, 128, 128, a8, launch_t32<kFp8, true, 128, 128, 2>, "a8w4");
    tile(kA8W4, 64, 256, a8, launch_t32<kFp8, true, 64, 256, 1>, "a8w4");
    tile(kA8W4, 64, 128, a8, launch_t32<kFp8, true, 64, 128, 1>, "a8w4");
    tile(kA8W4, 128, 256, a8p, launch_tile<kFp8, kFp4, 128, 256, true, true, false>, "a8w4");
    tile(kA8W4, 128, 128, a8p, launch_tile<kFp8, kFp4, 128, 128, true, true, false>, "a8w4");
    tile(kA8W4, 64, 128, a8p, launch_tile<kFp8, kFp4, 64, 128, true, true, false>, "a8w4");
    skinny(kA8W4, 1, false, a8, launch_skinny<kFp8, 1, true, false, false>, "a8w4");
    skinny(kA8W4, 2, false, a8, launch_skinny<kFp8, 2, true, false, false>, "a8w4");
    skinny(kA8W4, 4, false, a8, launch_skinny<kFp8, 4, true, false, false>, "a8w4");
    skinny(kA8W4, 1, true, a8, launch_skinny<kFp8, 1, true, true, false>, "a8w4");
    skinny(kA8W4, 2, true, a8, launch_skinny<kFp8, 2, true, true, false>, "a8w4");
    skinny(kA8W4, 4, true, a8, launch_skinny<kFp8, 4, true, true, false>, "a8w4");
}

}  // namespace aiter_amd
