// Persistent 256x256 bf16 tile with A and B both staged through LDS, double
// buffered by whole stages.
//
// Why: with row-major B, the flat kernels' direct B loads touch 32 rows x 32
// bytes per instruction, four times the cache lines of a full-line copy.
// Here B is copied global -> LDS exactly like A, in full 128-byte lines.
// A stage (64 bf16 of K = 128 bytes of every A and B row, four k-steps of
// v_mfma_f32_32x32x16_bf16) takes 64 KiB, so the LDS holds two: the copies of
// stage t+1 are all issued at the start of stage t, into the buffer that
// every wave finished reading before the barrier that ended stage t-1.
//
// Layout of a stage buffer (1 KiB chunks):
//   * A, row-major B: chunk c holds tile rows 8c..8c+7 x 128 bytes; lane l of
//     the copy moves global piece (l%8) ^ ((r/2)%8) of row r = 8c + l/8 into
//     LDS piece l%8 (piece = 16 bytes), so the k-step reads (lane l: row l%32,
//     piece 2s + l/32) hit 16 different 16-byte bank groups per 16 lanes;
//   * preshuffled B (shuffle_weight(16,16)): chunks 2g, 2g+1 are the 2 KiB
//     run of 16-row group g for this stage, copied as is; it already holds
//     k-block s (512 bytes) as [k-half][row][16 bytes], the MFMA operand order.
// Waves form a 2x2 grid of 128x128 wave tiles (4x4 32x32 accumulators): per
// k-step a wave reads 4 A and 4 B fragments (ds_read_b128) for 16 MFMAs.
//
// Stage t: copies of stage t+1; then k-steps 0-2, each reading the next
// k-step's fragments while multiplying; wait for the own copies and LDS
// reads; barrier; read k-step 0 of stage t+1; multiply k-step 3.
//
// Persistence as in gemm_flat_persist.h: min(tiles, CUs) workgroups walk
// tiles b, b+G, ... (XCD-aware raster); a tile's last stage copies the next
// tile's stage 0, and the epilogue goes through the other buffer (free after
// the tile's last barrier; the next copies into it follow the barrier after
// the epilogue).  K is padded with a zero stage to an even stage count; rows
// past M / N read zeros through range-checked descriptors.  bf16 output,
// alpha applied unless SCALED is false (alpha == 1); no bias, batch or
// split-K (the host takes the one-tile-per-workgroup twin for those).
#pragma once
#include <type_traits>

#include "mfma32.h"

namespace aiter_amd {

struct LdsPersistCfg {
    static constexpr int A_CH = 32, B_CH = 32;           // 1 KiB chunks per stage buffer
    static constexpr int STAGE_BYTES = (A_CH + B_CH) * 1024;
    static constexpr int K_STAGE = 64;                   // bf16 elements of K per stage
};

template <bool BPRE, bool SCALED>
__global__ __launch_bounds__(256, 1) void gemm_lds_persist_kernel(GemmParams p) {
    using Cfg = LdsPersistCfg;
    constexpr int MA = 4, NB = 4;
    constexpr int A_CH = Cfg::A_CH;
    constexpr int STAGE_BYTES = Cfg::STAGE_BYTES;
    constexpr int NA = A_CH / 4, NBW = Cfg::B_CH / 4;   // copies per wave per stage
    constexpr int NDMA = NA + NBW;
    static_assert(2 * STAGE_BYTES <= 160 * 1024, "two stages fit the LDS");

    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    const int wm = wave >> 1, wn = wave & 1;

    const int n_tiles = p.tiles_m * p.tiles_n;
    const int G = gridDim.x, blk = blockIdx.x;
    const int my_tiles = (n_tiles - blk + G - 1) / G;
    const int nstages = p.K / Cfg::K_STAGE;
    const int nst = (nstages + 1) & ~1;   // even: the buffer parity is the same at every tile start

    // copy lane offsets (tile origin and stage added per copy)
    int a_off[NA], b_off[NBW];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int r = 8 * (wave + 4 * q) + (lane >> 3);
        a_off[q] = r * (int)p.lda + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
    }
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
        const int c = wave + 4 * q;
        if constexpr (BPRE) {
            b_off[q] = (c >> 1) * 16 * (int)p.ldb + (c & 1) * 1024 + lane * 16;
        } else {
            const int r = 8 * c + (lane >> 3);
            b_off[q] = r * (int)p.ldb + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
        }
    }
    constexpr int B_STAGE_OFF = BPRE ? 2048 : 128;   // bytes per stage along a B row (group)
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.A, (int64_t)p.M * p.lda);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(p.B, (int64_t)p.N * p.ldb);
    const __amdgpu_buffer_rsrc_t null_rsrc = make_rsrc(p.A, 0);

    // per-tile scalars: origin, byte offsets of the tile in A / B, live stage
    // count (0 for a tile past this workgroup's stream)
    auto tile_of = [&](int it, int& m0, int& n0, int& abase, int& bbase, int& live) {
        int tm, tn;
        tile_coords(min(it * G + blk, n_tiles - 1), n_tiles, p.tiles_m, p.tiles_n, tm, tn);
        m0 = tm * 256;
        n0 = tn * 256;
        abase = m0 * (int)p.lda;
        bbase = n0 * (int)p.ldb;
        live = it < my_tiles ? nstages : 0;
    };

    // copies of stage dt of the tile at (abase, bbase) into buffer `buf`
    auto dma = [&](int abase, int bbase, int dlive, int dt, int buf) {
        const bool live = dt < dlive;
        const __amdgpu_buffer_rsrc_t ra = live ? a_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rb = live ? b_rsrc : null_rsrc;
        uint8_t* base = smem + buf * STAGE_BYTES;
#pragma unroll
        for (int q = 0; q < NA; ++q) dma16(ra, base + (wave + 4 * q) * 1024, a_off[q] + abase, dt * 128);
#pragma unroll
        for (int q = 0; q < NBW; ++q)
            dma16(rb, base + (A_CH + wave + 4 * q) * 1024, b_off[q] + bbase, dt * B_STAGE_OFF);
    };

    // buffer offsets as opaque scalars (one LDS address register per operand
    // instead of one per buffer)
    auto buf_off = [&](auto buf_c) {
        int v;
        asm("s_mov_b32 %0, %1" : "=s"(v) : "i"(decltype(buf_c)::value * STAGE_BYTES));
        return v;
    };
    i32x4_t af[2][MA], bf[2][NB];
    // k-step s reads: row-major (row l%32 of a 32-row block, piece 2s + l/32
    // swizzled by the row), preshuffled (group 2j + (l/16)%2, chunk s/2,
    // 512 (s%2) + 256 (l/32) + 16 (l%16))
    const int ar = lane & 31;
    const int rd_row = (ar >> 3) * 1024 + (ar & 7) * 128;
    const int rd_swz = (ar >> 1) & 7;
    const int rd_pre = ((lane >> 4) & 1) * 2048 + (lane >> 5) * 256 + (lane & 15) * 16;
    auto read_ops = [&](auto buf_c, int s, int reg) {
        const uint8_t* base = smem + buf_off(buf_c);
        const int pc = ((2 * s + (lane >> 5)) ^ rd_swz) * 16;
#pragma unroll
        for (int i = 0; i < MA; ++i)
            af[reg][i] = *reinterpret_cast<const i32x4_t*>(base + (wm * 16 + 4 * i) * 1024 + rd_row + pc);
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if constexpr (BPRE)
                bf[reg][j] = *reinterpret_cast<const i32x4_t*>(base + (A_CH + 2 * (wn * 8 + 2 * j) + (s >> 1)) * 1024 +
                                                               rd_pre + (s & 1) * 512);
            else
                bf[reg][j] = *reinterpret_cast<const i32x4_t*>(base + (A_CH + wn * 16 + 4 * j) * 1024 + rd_row + pc);
        }
    };

    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    constexpr int RD = MA + NB;
    constexpr int MF = MA * NB;
    auto pace = [&](int vmem) {
#pragma unroll
        for (int k = 0; k < MF; ++k) {
            if (k < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (k < vmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
    };

    int cm0, cn0, ca, cb, clive;   // current tile
    int xm0, xn0, xa, xb, xlive;   // next tile
    tile_of(0, cm0, cn0, ca, cb, clive);
    tile_of(1, xm0, xn0, xa, xb, xlive);

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    dma(ca, cb, clive, 0, 0);
    fence();
    wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    fence();
    read_ops(B0{}, 0, 0);

    for (int it = 0; it < my_tiles; ++it) {
        f32x16v_t acc[MA][NB];
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[i][j] = f32x16v_t{};
        auto mma = [&](int reg) {
#pragma unroll
            for (int i = 0; i < MA; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j) acc[i][j] = mma32<kBf16, 0>(bf[reg][j], af[reg][i], af[reg][i], acc[i][j], 0, 0);
        };
        // stage in buffer BUF; copies of stage dt of tile (da, db, dlive) into the other buffer
        auto stage = [&](auto buf_c, int da, int db, int dlive, int dt) {
            constexpr int BUF = decltype(buf_c)::value;
            using NX = std::integral_constant<int, BUF ^ 1>;
            dma(da, db, dlive, dt, BUF ^ 1);
            read_ops(buf_c, 1, 1);
            mma(0);
            pace(NDMA);
            fence();
            read_ops(buf_c, 2, 0);
            mma(1);
            pace(0);
            fence();
            read_ops(buf_c, 3, 1);
            mma(0);
            pace(0);
            fence();
            wait_vmcnt_lgkm0<0>();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            fence();
            read_ops(NX{}, 0, 0);
            mma(1);
            pace(0);
            fence();
        };

        for (int t = 0; t < nst - 2; t += 2) {
            stage(B0{}, ca, cb, clive, t + 1);
            stage(B1{}, ca, cb, clive, t + 2);
        }
        stage(B0{}, ca, cb, clive, nst - 1);
        stage(B1{}, xa, xb, xlive, 0);

        // epilogue through buffer 1 (a quarter per wave): every wave finished
        // reading it before the last barrier; the next copies into it follow
        // the barrier below
        store_block<MA, NB, 2, false, SCALED, false, true>(p, acc, smem + STAGE_BYTES + wave * (STAGE_BYTES / 4),
                                                           lane, cm0 + wm * 128, cn0 + wn * 128);
        wait_vmcnt_lgkm0<63>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        cm0 = xm0; cn0 = xn0; ca = xa; cb = xb; clive = xlive;
        tile_of(it + 2, xm0, xn0, xa, xb, xlive);
    }
    wait_vmcnt<0>();
}

}  // namespace aiter_amd
