// Kernel instances, part 5: the short-K direct skinny kernels (decode).
#include "gemm_registry.h"

namespace aiter_amd {

void RegBuilder::part_direct() {
    // rank 0: the heuristic keeps its split / LDS-staged forms; the tuned
    // tables name these where they win
    const Variant pre = kPre, a8 = kPre;
    staged(kA4W4, 1, pre, launch_skinny_direct<kFp4, 1, 1, 8>, "a4w4", 16, "_direct_k8", 0);
    staged(kA4W4, 1, pre, launch_skinny_direct<kFp4, 1, 1, 16>, "a4w4", 16, "_direct_k16", 0);
    staged(kA4W4, 1, pre, launch_skinny_direct<kFp4, 1, 2, 8>, "a4w4", 32, "_direct_k8", 0);
    staged(kA4W4, 2, pre, launch_skinny_direct<kFp4, 2, 1, 8>, "a4w4", 16, "_direct_k8", 0);
    staged(kA4W4, 2, pre, launch_skinny_direct<kFp4, 2, 2, 8>, "a4w4", 32, "_direct_k8", 0);
    staged(kA4W4, 4, pre, launch_skinny_direct<kFp4, 4, 1, 8>, "a4w4", 16, "_direct_k8", 0);
    staged(kA8W4, 1, a8, launch_skinny_direct<kFp8, 1, 1, 8>, "a8w4", 16, "_direct_k8", 0);
    staged(kA8W4, 2, a8, launch_skinny_direct<kFp8, 2, 1, 8>, "a8w4", 16, "_direct_k8", 0);
}

}  // namespace aiter_amd
