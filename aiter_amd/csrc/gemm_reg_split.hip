// Kernel instances, part 3: persistent tiles and split-K tiles.
#include "gemm_registry.h"

namespace aiter_amd {

void RegBuilder::part_persist_split() {
    const Variant pre = kPre, plain = kPlain, a8 = kPre;
    // ---- persistent forms of the flat tiles (gemm_flat_persist.h);
    // appended so that the ids above stay stable ----
    persist(kA4W4, 256, kPre, launch_flat_persist<kFp4, 256>, "a4w4");
    persist(kA4W4, 128, kPre, launch_flat_persist<kFp4, 128>, "a4w4");
    persist(kA8W4, 128, kPre, launch_flat_persist<kFp8, 128>, "a8w4");
    persist(kA16W16, 256, Variant{false, true, false}, launch_flat_persist<kBf16, 256>, "a16w16");
    persist(kA16W16, 128, Variant{false, true, false}, launch_flat_persist<kBf16, 128>, "a16w16");
    // ---- split-K forms of the smaller t32 tiles (K split over gridDim.y,
    // f32 partial slices summed by splitk_reduce_kernel), for shapes
    // whose tiles cannot fill the CUs ----
    tsplit(kA4W4, 64, 128, pre, launch_t32<kFp4, true, 64, 128, 1, false, true>, "a4w4");
    tsplit(kA4W4, 64, 256, pre, launch_t32<kFp4, true, 64, 256, 1, false, true>, "a4w4");
    tsplit(kA4W4, 128, 128, pre, launch_t32<kFp4, true, 128, 128, 2, false, true>, "a4w4");
    tsplit(kA4W4, 64, 128, plain, launch_t32<kFp4, false, 64, 128, 1, false, true>, "a4w4");
    tsplit(kA8W4, 64, 128, a8, launch_t32<kFp8, true, 64, 128, 1, false, true>, "a8w4");
    tsplit(kA8W4, 64, 256, a8, launch_t32<kFp8, true, 64, 256, 1, false, true>, "a8w4");
    for (int of = 0; of < 2; ++of) {
        for (int bp = 0; bp < 2; ++bp) {
            const Variant v{false, bp != 0, of != 0};
#define AA_T16S(BM, BN, WMW)                                                                      \
    tsplit(kA16W16, BM, BN, v,                                                                    \
           of ? (bp ? launch_t32<kBf16, true, BM, BN, WMW, true, true>                            \
                    : launch_t32<kBf16, false, BM, BN, WMW, true, true>)                          \
              : (bp ? launch_t32<kBf16, true, BM, BN, WMW, false, true>                           \
                    : launch_t32<kBf16, false, BM, BN, WMW, false, true>),                        \
           "a16w16");
            AA_T16S(64, 64, 2) AA_T16S(64, 128, 1) AA_T16S(128, 128, 2)
#undef AA_T16S
        }
    }
}

}  // namespace aiter_amd
