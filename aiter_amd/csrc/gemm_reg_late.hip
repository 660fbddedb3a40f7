// Kernel instances, part 7: instances added after the earlier parts, so
// that the ids those parts assign stay put.
#include "gemm_registry.h"

namespace aiter_amd {

void RegBuilder::part_late() {
    // bf16 row-major B, f32 output, on the flat tile with whole-line B
    // copies into wave-private LDS regions (gemm_flat.h, BLDS)
    tile(kA16W16, 256, 256, Variant{false, false, true}, launch_flat<kBf16, 256, true, false>, "a16w16");
    reg.back().name += "_flat";
}

}  // namespace aiter_amd
