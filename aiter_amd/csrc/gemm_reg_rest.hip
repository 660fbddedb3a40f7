// Kernel instances, part 4: row-major-B flat tiles, f32-output A4W4, 32-column
// skinny kernels, LDS-staged persistent and skinny kernels, long-K split tiles.
#include "gemm_registry.h"

namespace aiter_amd {

void RegBuilder::part_rest() {
    const Variant pre = kPre, plain = kPlain;
    // ---- a4w4 with row-major B on the flat kernels (B straight to VGPRs:
    // 16 contiguous bytes of one row per lane) ----
    tile(kA4W4, 256, 256, plain, launch_flat<kFp4, 256, false, false>, "a4w4");
    persist(kA4W4, 256, plain, launch_flat_persist<kFp4, 256, false, false>, "a4w4");
    // ---- a4w4 with f32 output (the tile that mxfp4_gemm_asm quantises to
    // e2m1 / MXFP8) ----
    // (no 256x256 flat f32 tile: its epilogue spills; the persistent form does not)
    const Variant pre32{false, true, true};
    tile(kA4W4, 128, 256, pre32, launch_flat<kFp4, 128, true>, "a4w4");
    tile(kA4W4, 128, 128, pre32, launch_t32<kFp4, true, 128, 128, 2, true>, "a4w4");
    tile(kA4W4, 64, 128, pre32, launch_t32<kFp4, true, 64, 128, 1, true>, "a4w4");
    skinny(kA4W4, 1, false, pre32, launch_skinny<kFp4, 1, true, false, true>, "a4w4");
    skinny(kA4W4, 2, false, pre32, launch_skinny<kFp4, 2, true, false, true>, "a4w4");
    skinny(kA4W4, 4, false, pre32, launch_skinny<kFp4, 4, true, false, true>, "a4w4");
    skinny(kA4W4, 1, true, pre32, launch_skinny<kFp4, 1, true, true, true>, "a4w4");
    skinny(kA4W4, 2, true, pre32, launch_skinny<kFp4, 2, true, true, true>, "a4w4");
    skinny(kA4W4, 4, true, pre32, launch_skinny<kFp4, 4, true, true, true>, "a4w4");
    tsplit(kA4W4, 64, 128, pre32, launch_t32<kFp4, true, 64, 128, 1, true, true>, "a4w4");
    persist(kA4W4, 256, pre32, launch_flat_persist<kFp4, 256, true>, "a4w4");
    // ---- skinny with 32 columns per workgroup (one A fragment serves two
    // B blocks); appended last so that earlier kernel ids stay put ----
    skinny(kA4W4, 1, false, pre, launch_skinny<kFp4, 1, true, false, false, 2>, "a4w4", 32);
    skinny(kA4W4, 2, false, pre, launch_skinny<kFp4, 2, true, false, false, 2>, "a4w4", 32);
    const Variant a8n{false, true, false};
    skinny(kA8W4, 1, false, a8n, launch_skinny<kFp8, 1, true, false, false, 2>, "a8w4", 32);
    skinny(kA8W4, 2, false, a8n, launch_skinny<kFp8, 2, true, false, false, 2>, "a8w4", 32);
    const Variant b16p{false, true, false}, b16r{false, false, false};
    skinny(kA16W16, 1, false, b16p, launch_skinny<kBf16, 1, true, false, false, 2>, "a16w16", 32);
    skinny(kA16W16, 2, false, b16p, launch_skinny<kBf16, 2, true, false, false, 2>, "a16w16", 32);
    skinny(kA16W16, 1, false, b16r, launch_skinny<kBf16, 1, false, false, false, 2>, "a16w16", 32);
    skinny(kA16W16, 2, false, b16r, launch_skinny<kBf16, 2, false, false, false, 2>, "a16w16", 32);
    // ---- bf16 256x256 persistent tiles with A and B both through LDS in
    // half-width ring slots (gemm_lds_persist.h) ----
    persist(kA16W16, 256, b16r, launch_lds_persist<false>, "a16w16");
    persist(kA16W16, 256, b16p, launch_lds_persist<true>, "a16w16");
    reg.back().name = "a16w16_tile_256x256_lds_persist";
    // ---- A4W4 64-row skinny with 32 columns per workgroup ----
    skinny(kA4W4, 4, false, pre, launch_skinny<kFp4, 4, true, false, false, 2>, "a4w4", 32);
    // ---- bf16 row-major B on the flat tiles: whole-line B copies into
    // wave-private LDS regions (gemm_flat.h, BLDS) ----
    tile(kA16W16, 256, 256, b16r, launch_flat<kBf16, 256, false, false>, "a16w16");
    reg.back().name += "_flat";
    // ---- skinny kernels with A (row-major bf16 B: A and B) copied
    // through LDS in whole lines (gemm_skinny_lds.h); rank 1: the
    // heuristic prefers them over the register-load forms above ----
    staged(kA16W16, 1, b16r, launch_skinny_alds<kBf16, 1, false, 2, 8, 2, true>, "a16w16", 32, "_lds");
    staged(kA16W16, 2, b16r, launch_skinny_alds<kBf16, 2, false, 2, 8, 2, true>, "a16w16", 32, "_lds");
    staged(kA16W16, 4, b16r, launch_skinny_alds<kBf16, 4, false, 2, 4, 2, true>, "a16w16", 32, "_lds");
    staged(kA16W16, 1, b16r, launch_skinny_alds<kBf16, 1, false, 1, 8, 2, true>, "a16w16", 16, "_lds");
    staged(kA16W16, 1, b16r, launch_skinny_alds<kBf16, 1, false, 1, 8, 3, true>, "a16w16", 16, "_lds_s3", 0);
    staged(kA16W16, 2, b16r, launch_skinny_alds<kBf16, 2, false, 1, 8, 2, true>, "a16w16", 16, "_lds");
    staged(kA16W16, 2, b16p, launch_skinny_alds<kBf16, 2, true, 2>, "a16w16", 32, "_alds");
    staged(kA16W16, 4, b16p, launch_skinny_alds<kBf16, 4, true, 2>, "a16w16", 32, "_alds");
    staged(kA4W4, 2, pre, launch_skinny_alds<kFp4, 2, true, 2>, "a4w4", 32, "_alds");
    staged(kA4W4, 4, pre, launch_skinny_alds<kFp4, 4, true, 2>, "a4w4", 32, "_alds");
    staged(kA4W4, 2, pre, launch_skinny_alds<kFp4, 2, true, 1>, "a4w4", 16, "_alds");
    staged(kA8W4, 2, a8n, launch_skinny_alds<kFp8, 2, true, 2>, "a8w4", 32, "_alds");
    // ---- split-K forms of the 256-row and 256-column bf16 row-major tiles
    // (M = 256 with long K: every B byte read once) ----
    tsplit(kA16W16, 256, 128, b16r, launch_t32<kBf16, false, 256, 128, 2, false, true>, "a16w16");
    tsplit(kA16W16, 128, 256, b16r, launch_t32<kBf16, false, 128, 256, 2, false, true>, "a16w16");
}

}  // namespace aiter_amd
