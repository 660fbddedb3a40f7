// Persistent form of the flat-B tile kernel (gemm_flat.h holds the tile
// itself: 4 waves side by side along N, B straight to VGPRs two stages ahead,
// A and the e8m0 scales through a 4-slot LDS ring).
//
// Why: with one workgroup per tile, every round of tiles ends with all CUs
// writing their outputs at once (32 MiB per round at 8192^3, at HBM write
// speed) while no MFMA runs, and the next round starts by waiting for its
// first copies.  Here min(tiles, CUs) workgroups each walk tiles b, b+G,
// b+2G, ... (the same XCD-aware raster as one launch per tile) as one stream
// of stages through the ring: the last three stages of a tile already issue
// the copies of the next tile's stages 0-2 and its B for stages 0-1, the
// epilogue's stores go out behind them, and the next tile starts multiplying
// at once.  vmcnt counts loads and stores in issue order, so the waits of the
// next tile's first two stages are raised by the number of epilogue stores
// (NST) to leave those outstanding; the prologue issues NST stores that the
// range check drops, so that the first tile's waits count the same way.
// The wait constants are exact for this issue order, so the first four and
// the last four stages of a tile are peeled out of the stage loop (a wait
// picked at run time inside the loop costs the register allocation dearly).
//
// Scope: no bias (the host uses the one-tile-per-workgroup kernel then),
// alpha applied, K padded with zero stages to a multiple of 4 stages: 4, or
// at least 8.  Results are bit-identical to gemm_flat_kernel: same MFMAs in the
// same order per tile.
#pragma once
#include <type_traits>

#include "mfma32.h"

namespace aiter_amd {

template <int KA, int BM>
struct FlatPersistCfg {
    static constexpr bool MX = KA != kBf16;
    static constexpr int FA = (KA == kFp8) ? 2 : 1;
    static constexpr int A_CH = (BM / 8) * FA;
    static constexpr int STAGE_KB = A_CH + (MX ? 4 : 0);
    static constexpr int NS = 4;
    static constexpr int K_STAGE = MX ? 256 : 64;
};

// BPRE = false: row-major B, loaded straight into VGPRs as in gemm_flat_kernel.
// SCALED = false: alpha == 1 (the epilogue skips the multiply).
// SHORT4 = true: every tile is one 4-stage group (K <= 4 stages), so its first
// four stages are its last four.  A separate instance: one body carrying both
// stage sequences spills hundreds of VGPRs on the 256-row tiles.
template <int KA, int BM, bool OUT_F32, bool BPRE = true, bool OUT_FP4 = false, bool SCALED = true, bool SHORT4 = false>
__global__ __launch_bounds__(256, 1) void gemm_flat_persist_kernel(GemmParams p) {
    using Cfg = FlatPersistCfg<KA, BM>;
    constexpr int NS = 4;
    constexpr int FA = Cfg::FA;
    constexpr int MA = BM / 32;
    constexpr int NB = 2;
    constexpr int A_CH = Cfg::A_CH;
    constexpr bool MX = Cfg::MX;
    constexpr int AG = BM / 32;
    constexpr int SCA = (AG + 3) / 4;
    static_assert(SCA + 2 <= 4, "scale chunks: one per wave");
    static_assert(A_CH % 4 == 0, "A chunks split over 4 waves");
    static_assert(NS * Cfg::STAGE_KB <= 160, "ring fits the LDS");
    constexpr int NA = A_CH / 4;
    constexpr int NDMA = NA + (MX ? 1 : 0);
    constexpr int NBL = NB * 4;
    constexpr int STAGE_BYTES = Cfg::STAGE_KB * 1024;
    constexpr int A_ROW_BYTES = 128 * FA;
    constexpr int EB2 = OUT_FP4 ? 1 : (OUT_F32 ? 8 : 4);   // output bytes per two elements
    // MX: the paired tile layout (swap45 in mfma32.h): MFMA tile 2p+b of a
    // wave takes rows 16b..16b+15 of the 32-row groups 2p and 2p+1 (B: columns
    // 16j..16j+15 of the wave's two 32-column groups), so every lane of a tile
    // uses byte b (+2) of the same two shuffled-scale dwords and a tile pair
    // shares them: two dword reads per pair and stage, no byte shuffle
    constexpr bool PAIRED = MX;
    static_assert(!PAIRED || MA % 2 == 0, "tile pairs");

    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;

    const int n_tiles = p.tiles_m * p.tiles_n;
    const int G = gridDim.x, blk = blockIdx.x;
    const int my_tiles = (n_tiles - blk + G - 1) / G;
    const int nstages = p.K / Cfg::K_STAGE;
    // stages per tile: a multiple of 4 (zero stages past K); 4 (SHORT4) or at least 8
    const int nst4 = SHORT4 ? 4 : (nstages <= 8 ? 8 : (nstages + 3) & ~3);

    // tile-independent lane offsets; the tile origin is added per tile
    int a_off[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int c = wave + 4 * q;
        const int half = c / (BM / 8), rb = c % (BM / 8);
        const int r = rb * 8 + (lane >> 3);
        a_off[q] = r * (int)p.lda + half * 128 + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
    }
    int b_off[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int b16 = 4 * wave + (PAIRED ? 2 * ((lane >> 4) & 1) + j : 2 * j + ((lane >> 4) & 1));
        const int col = 64 * wave + (PAIRED ? swap45(32 * j + (lane & 31)) : 32 * j + (lane & 31));
        if constexpr (BPRE)
            b_off[j] = b16 * 16 * (int)p.ldb + (lane >> 5) * 256 + (lane & 15) * 16;
        else
            b_off[j] = col * (int)p.ldb + (lane >> 5) * 16;
    }
    // whole-tensor descriptors: rows past M / N and groups past the scale
    // tensors read zeros
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.A, (int64_t)p.M * p.lda);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(p.B, (int64_t)p.N * p.ldb);
    const __amdgpu_buffer_rsrc_t null_rsrc = make_rsrc(p.A, 0);
    const bool sc_is_a = wave < SCA;
    const bool sc_is_b = wave >= SCA && wave < SCA + 2;
    const int sc_chunk = sc_is_a ? wave : (sc_is_b ? wave - SCA : 0);
    const int sc_stride = sc_is_b ? (int)p.sb_stride : (int)p.sa_stride;
    // chunk = 4 groups x 256 B (paired: the image of sc_pair_group / _granule)
    const int sc_off = PAIRED ? (4 * sc_chunk + sc_pair_group(lane)) * 32 * sc_stride + sc_pair_granule(lane) * 16
                              : (4 * sc_chunk + (lane >> 4)) * 32 * sc_stride + (lane & 15) * 16;
    const __amdgpu_buffer_rsrc_t sc_rsrc =
        sc_is_a ? make_rsrc(p.As, (int64_t)p.sa_groups * 32 * p.sa_stride)
                : (sc_is_b ? make_rsrc(p.Bs, (int64_t)p.sb_groups * 32 * p.sb_stride) : null_rsrc);

    // per-tile scalars: origin, byte offsets of the tile in A / B / this
    // wave's scale tensor, live stage count (0 for a tile past the stream)
    auto tile_of = [&](int it, int& m0, int& n0, int& abase, int& bbase, int& scbase, int& nst) {
        int tm, tn;
        tile_coords(min(it * G + blk, n_tiles - 1), n_tiles, p.tiles_m, p.tiles_n, tm, tn);
        m0 = tm * BM;
        n0 = tn * 256;
        abase = m0 * (int)p.lda;
        bbase = n0 * (int)p.ldb;
        scbase = sc_is_a ? (m0 / 32) * 32 * (int)p.sa_stride : (n0 / 32) * 32 * (int)p.sb_stride;
        nst = it < my_tiles ? nstages : 0;
    };

    const int pos0 = PAIRED ? sc_pair_read_off(lane) : ((lane & 15) + 16 * (lane >> 5)) * 4;
    const unsigned sc_perm = 0x06040200u + ((lane >> 4) & 1) * 0x01010101u;

    i32x4_t af[2][MA][FA];
    i32x4_t bq[2][NB][4];
    int sa_pk[MA] = {}, sb_pk[NB] = {};

    // ring slot offsets as opaque scalars: folded into constants, the reads of
    // slots past the 64 KiB ds_read offset range would each get an address
    // register of their own, live across the whole loop
    auto slot_off = [&](auto slot_c) {
        int v;
        asm("s_mov_b32 %0, %1" : "=s"(v) : "i"(decltype(slot_c)::value * STAGE_BYTES));
        return v;
    };
    const int ar = lane & 31;
    // paired: MFMA row ar of tile 2p+b is row swap45(32(2p+b) + ar), in 8-row
    // chunk 8p + 2b + 4(ar>>4) + ((ar>>3)&1); the swizzle (row>>1)&7 is the same
    const int a_lane_off = PAIRED ? (4 * ((ar >> 4) & 1) + ((ar >> 3) & 1)) * 1024 + (ar & 7) * 128
                                  : (ar >> 3) * 1024 + (ar & 7) * 128;
    const int a_swz = (ar >> 1) & 7;
    auto read_a = [&](auto slot_c, int s, int reg) {
        const uint8_t* base = smem + slot_off(slot_c);
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int h = 0; h < FA; ++h) {
                const int piece = (FA == 1) ? (2 * s + (lane >> 5)) : ((4 * s + 2 * h + (lane >> 5)) & 7);
                const int hh = (FA == 1) ? 0 : ((4 * s + 2 * h) >> 3);
                af[reg][i][h] = *reinterpret_cast<const i32x4_t*>(
                    base + (hh * (BM / 8) + (PAIRED ? (i >> 1) * 8 + (i & 1) * 2 : i * 4)) * 1024 + a_lane_off +
                    ((piece ^ a_swz) * 16));
            }
    };
    auto read_scales = [&](auto slot_c, int (&pa)[MA], int (&pb)[NB]) {
        if constexpr (!MX) return;
        const uint8_t* base = smem + slot_off(slot_c) + A_CH * 1024 + pos0;
        if constexpr (PAIRED) {
            // pair p: dwords d0 (k-steps 0, 2) and d1 (1, 3) -> pa[2p], pa[2p+1]
#pragma unroll
            for (int q = 0; q < MA / 2; ++q) {
                pa[2 * q] = *reinterpret_cast<const int*>(base + q * 512);
                pa[2 * q + 1] = *reinterpret_cast<const int*>(base + q * 512 + 256);
            }
            pb[0] = *reinterpret_cast<const int*>(base + SCA * 1024 + wave * 512);
            pb[1] = *reinterpret_cast<const int*>(base + SCA * 1024 + wave * 512 + 256);
            return;
        }
#pragma unroll
        for (int i = 0; i < MA; ++i) {
            const unsigned d0 = *reinterpret_cast<const unsigned*>(base + i * 256);
            const unsigned d1 = *reinterpret_cast<const unsigned*>(base + i * 256 + 128);
            pa[i] = (int)__builtin_amdgcn_perm(d1, d0, sc_perm);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint8_t* g = base + SCA * 1024 + (2 * wave + j) * 256;
            const unsigned d0 = *reinterpret_cast<const unsigned*>(g);
            const unsigned d1 = *reinterpret_cast<const unsigned*>(g + 128);
            pb[j] = (int)__builtin_amdgcn_perm(d1, d0, sc_perm);
        }
    };
    // B of stage bt of the tile at bbase (live stages < bnst), k-step s
    auto prefetch_b = [&](int bbase, int bnst, int bt, int bpar, int s) {
        const __amdgpu_buffer_rsrc_t rb = bt < bnst ? b_rsrc : null_rsrc;
#pragma unroll
        for (int j = 0; j < NB; ++j)
            bq[bpar][j][s] = __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[j] + bbase + s * (BPRE ? 512 : 32),
                                                                   bt * (BPRE ? 2048 : 128), 0);
    };
    constexpr int DMA_PART = (NDMA + 2) / 3;
    // third `part` of the copies of stage dt of the tile at (abase, scbase)
    // into ring slot `slot`
    auto dma_part = [&](int abase, int scbase, int dnst, int dt, int slot, int part) {
        const bool live = dt < dnst;
        const __amdgpu_buffer_rsrc_t ra = live ? a_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rs = live ? sc_rsrc : null_rsrc;
        uint8_t* base = smem + slot * STAGE_BYTES;
#pragma unroll
        for (int q = part * DMA_PART; q < (part + 1) * DMA_PART && q < NDMA; ++q) {
            if (q < NA) dma16(ra, base + (wave + 4 * q) * 1024, a_off[q] + abase, dt * A_ROW_BYTES);
            else dma16(rs, base + (A_CH + wave) * 1024, sc_off + scbase, dt * 256);
        }
    };
    constexpr int LOADS_ITER = NDMA + NBL;
    constexpr int WAIT_N = (NS - 3) * LOADS_ITER + NDMA + 3 * NB;
    // epilogue store instructions per wave
    constexpr int NST = BM * 64 * EB2 / 2048;
    // the first two waits of a tile after an epilogue: the stores were issued
    // after the copies waited for and may stay outstanding
    constexpr int WAIT_T = (WAIT_N + NST) > 63 ? 63 : (WAIT_N + NST);
    static_assert(WAIT_N < 64, "vmcnt range");
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    constexpr int RD = MA * FA;
    constexpr int MF = MA * NB;
    auto pace = [&](int vmem) {
#pragma unroll
        for (int k = 0; k < MF; ++k) {
            if (k < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (k >= MF - vmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        }
    };

    int cm0, cn0, ca, cb, csc, cnst;   // current tile
    int xm0, xn0, xa, xb, xsc, xnst;   // next tile
    tile_of(0, cm0, cn0, ca, cb, csc, cnst);
    tile_of(1, xm0, xn0, xa, xb, xsc, xnst);

    // prologue: copies of stages 0 and 1, B of stages 0 and 1, copies of
    // stage 2, then NST stores that the range check drops: the issue order of
    // a tile transition, so that every tile's first waits count alike
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int part = 0; part < 3; ++part) dma_part(ca, csc, cnst, t, t, part);
#pragma unroll
    for (int s = 0; s < 4; ++s) prefetch_b(cb, cnst, 0, 0, s);
#pragma unroll
    for (int s = 0; s < 4; ++s) prefetch_b(cb, cnst, 1, 1, s);
#pragma unroll
    for (int part = 0; part < 3; ++part) dma_part(ca, csc, cnst, 2, 2, part);
#pragma unroll
    for (int q = 0; q < NST; ++q) __builtin_amdgcn_raw_buffer_store_b32(0, null_rsrc, 0, 0, 0);
    fence();
    constexpr int WAIT_P = (2 * NDMA + 2 * NBL + NST) > 63 ? 63 : (2 * NDMA + 2 * NBL + NST);
    wait_vmcnt<WAIT_P>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    fence();

    // epilogue row tiles per pass: a quarter ring slot per wave
    constexpr int EP_ROW_TILE = 32 * 32 * EB2;
    constexpr int EP_MP = (MA * EP_ROW_TILE <= STAGE_BYTES / 4)         ? MA
                          : ((MA / 2) * EP_ROW_TILE <= STAGE_BYTES / 4) ? MA / 2
                          : ((MA / 4) * EP_ROW_TILE <= STAGE_BYTES / 4) ? MA / 4
                                                                         : 1;
    static_assert(MA % EP_MP == 0 && EP_MP * EP_ROW_TILE <= STAGE_BYTES / 4, "epilogue pass fits a quarter slot");

    for (int it = 0; it < my_tiles; ++it) {
        f32x16v_t acc[MA][NB];
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[i][j] = f32x16v_t{};
        auto mma = [&](int areg, int bpar, auto sel) {
            constexpr int s = decltype(sel)::value;
            constexpr int osel = (s == 0) ? 0 : (s == 1) ? 2 : (s == 2) ? 1 : 3;
            if constexpr (PAIRED) {
                // tile 2q+b: byte b + 2(s/2) of dword d(s%2) of pair q (B: tile j, byte j + 2(s/2))
                constexpr int o = 2 * (s >> 1);
#pragma unroll
                for (int i = 0; i < MA; ++i) {
                    const int sa = sa_pk[2 * (i >> 1) + (s & 1)], sb = sb_pk[s & 1];
                    const i32x4_t &a0 = af[areg][i][0], &a1 = af[areg][i][FA - 1];
                    if (i & 1) {
                        acc[i][0] = mma32x<KA, 1 + o, 0 + o>(bq[bpar][0][s], a0, a1, acc[i][0], sa, sb);
                        acc[i][1] = mma32x<KA, 1 + o, 1 + o>(bq[bpar][1][s], a0, a1, acc[i][1], sa, sb);
                    } else {
                        acc[i][0] = mma32x<KA, 0 + o, 0 + o>(bq[bpar][0][s], a0, a1, acc[i][0], sa, sb);
                        acc[i][1] = mma32x<KA, 0 + o, 1 + o>(bq[bpar][1][s], a0, a1, acc[i][1], sa, sb);
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < MA; ++i)
#pragma unroll
                    for (int j = 0; j < NB; ++j)
                        acc[i][j] = mma32<KA, osel>(bq[bpar][j][s], af[areg][i][0], af[areg][i][FA - 1], acc[i][j],
                                                    sa_pk[i], sb_pk[j]);
            }
        };
        // stage t (ring slot SLOT = t % 4) of the current tile; look-ahead: copies
        // of stage dt of tile (da, dsc, dnst) into slot SLOT+3, B of stage bt of
        // tile (bb, bnst); W: vmcnt of the wait that publishes stage t+1
        auto stage = [&](auto slot_c, auto w_c, int da, int dsc, int dnst, int dt, int bb, int bnst, int bt) {
            constexpr int SLOT = decltype(slot_c)::value;
            constexpr int W = decltype(w_c)::value;
            constexpr int NSLOT = (SLOT + 1) & 3;
            constexpr int DSLOT = (SLOT + 3) & 3;
            const int bpar = SLOT & 1;
            using S0 = std::integral_constant<int, 0>;
            using S1 = std::integral_constant<int, 1>;
            using S2 = std::integral_constant<int, 2>;
            using S3 = std::integral_constant<int, 3>;
            using CS = std::integral_constant<int, SLOT>;
            using CN = std::integral_constant<int, NSLOT>;
            read_a(CS{}, 1, 1);
            dma_part(da, dsc, dnst, dt, DSLOT, 0);
            mma(0, bpar, S0{});
            prefetch_b(bb, bnst, bt, bpar, 0);
            pace(NB + DMA_PART);
            fence();
            read_a(CS{}, 2, 0);
            dma_part(da, dsc, dnst, dt, DSLOT, 1);
            mma(1, bpar, S1{});
            prefetch_b(bb, bnst, bt, bpar, 1);
            pace(NB + DMA_PART);
            fence();
            read_a(CS{}, 3, 1);
            dma_part(da, dsc, dnst, dt, DSLOT, 2);
            mma(0, bpar, S2{});
            prefetch_b(bb, bnst, bt, bpar, 2);
            pace(NB + NDMA - 2 * DMA_PART);
            fence();
            wait_vmcnt_lgkm0<W>();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            fence();
            read_a(CN{}, 0, 0);
            int na[MA], nb[NB];
            read_scales(CN{}, na, nb);
            mma(1, bpar, S3{});
            prefetch_b(bb, bnst, bt, bpar, 3);
            if constexpr (MX) {
#pragma unroll
                for (int i = 0; i < MA; ++i) sa_pk[i] = na[i];
#pragma unroll
                for (int j = 0; j < NB; ++j) sb_pk[j] = nb[j];
            }
            pace(NB);
            fence();
        };
        using L0 = std::integral_constant<int, 0>;
        using L1 = std::integral_constant<int, 1>;
        using L2 = std::integral_constant<int, 2>;
        using L3 = std::integral_constant<int, 3>;
        using WN = std::integral_constant<int, WAIT_N>;
        using WT = std::integral_constant<int, WAIT_T>;

        read_scales(L0{}, sa_pk, sb_pk);
        read_a(L0{}, 0, 0);
        if constexpr (SHORT4) {
            // a 4-stage tile (K <= 4 stages): its first four stages are its
            // last four; the waits of stages 0 and 1 span the previous
            // epilogue's stores, the look-ahead moves on to the next tile
            stage(L0{}, WT{}, ca, csc, cnst, 3, cb, cnst, 2);
            stage(L1{}, WT{}, xa, xsc, xnst, 0, cb, cnst, 3);
            stage(L2{}, WN{}, xa, xsc, xnst, 1, xb, xnst, 0);
            stage(L3{}, WN{}, xa, xsc, xnst, 2, xb, xnst, 1);
        } else {
            // first four stages: the waits of stages 0 and 1 span the previous
            // epilogue's stores (or the prologue's stand-ins)
            stage(L0{}, WT{}, ca, csc, cnst, 3, cb, cnst, 2);
            stage(L1{}, WT{}, ca, csc, cnst, 4, cb, cnst, 3);
            stage(L2{}, WN{}, ca, csc, cnst, 5, cb, cnst, 4);
            stage(L3{}, WN{}, ca, csc, cnst, 6, cb, cnst, 5);
            for (int t = 4; t < nst4 - 4; t += 4) {
                stage(L0{}, WN{}, ca, csc, cnst, t + 3, cb, cnst, t + 2);
                stage(L1{}, WN{}, ca, csc, cnst, t + 4, cb, cnst, t + 3);
                stage(L2{}, WN{}, ca, csc, cnst, t + 5, cb, cnst, t + 4);
                stage(L3{}, WN{}, ca, csc, cnst, t + 6, cb, cnst, t + 5);
            }
            // last four stages: the look-ahead moves on to the next tile
            const int t4 = nst4 - 4;
            stage(L0{}, WN{}, ca, csc, cnst, t4 + 3, cb, cnst, t4 + 2);
            stage(L1{}, WN{}, xa, xsc, xnst, 0, cb, cnst, t4 + 3);
            stage(L2{}, WN{}, xa, xsc, xnst, 1, xb, xnst, 0);
            stage(L3{}, WN{}, xa, xsc, xnst, 2, xb, xnst, 1);
        }

        // epilogue through ring slot 3: every wave finished reading it before
        // the last stage's barrier, and its next copy is issued in the next
        // tile's first stage, after the barrier below
        store_block<MA, NB, EP_MP, false, SCALED, OUT_F32, true, OUT_FP4, false, PAIRED ? 3 : 0>(p, acc, smem + 3 * STAGE_BYTES + wave * (STAGE_BYTES / 4),
                                                              lane, cm0, cn0 + wave * 64);
        wait_vmcnt_lgkm0<63>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        cm0 = xm0; cn0 = xn0; ca = xa; cb = xb; csc = xsc; cnst = xnst;
        tile_of(it + 2, xm0, xn0, xa, xb, xsc, xnst);
    }
    wait_vmcnt<0>();
}

}  // namespace aiter_amd
