// Kernel instances, part 7: instances added after the earlier parts, so
// that the ids those parts assign stay put.
#include "gemm_registry.h"

namespace aiter_amd {

void RegBuilder::part_late() {
    // bf16 row-major B, f32 output, on the flat tile with whole-line B
    // copies into wave-private LDS regions (gemm_flat.h, BLDS)
    tile(kA16W16, 256, 256, Variant{false, false, true}, launch_flat<kBf16, 256, true, false>, "a16w16");
    reg.back().name += "_flat";
    // stream-K skinny kernels, row-major bf16 B through LDS (gemm_skinny_lds.h):
    // tuned tables only (rank -1: never the heuristic's choice)
    const Variant b16r{false, false, false};
    auto sk = [&](int mf, LaunchFn fn) {
        skinny(kA16W16, mf, false, b16r, fn, "a16w16", 32);
        reg.back().name += "_lds_sk";
        reg.back().rank = -1;
        reg.back().stream_k = true;
    };
    sk(1, launch_skinny_sk<1, 2, 8>);
    sk(2, launch_skinny_sk<2, 2, 8>);
    sk(4, launch_skinny_sk<4, 2, 4>);
}

}  // namespace aiter_amd
