// Tile kernel on the 32x32 MFMAs of gfx950 with A and B both staged through
// LDS: e2m1 / e4m3 A with e2m1 B (v_mfma_scale_f32_32x32x64_f8f6f4, e8m0
// block scales) and bf16 A with bf16 B (v_mfma_f32_32x32x16_bf16).
//
// In bytes the two MFMA families have the same operand layout: lane l holds
// row l%32 and 16 bytes at 16*(l/32) of a 32-byte K window (64 e2m1 or 16
// bf16 elements; e4m3 A takes two such windows).  A k-step is one window, a
// stage is four k-steps: 256 MX or 64 bf16 elements, 128 bytes of every A and
// B row.  So one staging scheme serves all element types:
//   * A, and row-major B, are copied global -> LDS with buffer_load ... lds in
//     1 KiB chunks of 8 rows x 128 B, 16-byte pieces XOR-swizzled by row
//     ((r>>1)&7): full cache lines per copy, bank-conflict-free reads;
//   * preshuffled B (shuffle_weight (16,16), same byte layout for e2m1 and
//     bf16) is already in operand order: a chunk is four 256-byte runs;
//   * MX scales: one 1 KiB chunk of 4 row groups x 256 B per wave, read as two
//     dwords per group and packed per lane with v_perm so that k-step s takes
//     byte {0,2,1,3}[s] through the MFMA op_sel.
// A ring of NS stages (as many as fit 160 KiB, at most 4): the copies of
// stage t+NS-1 are issued during stage t; one vmcnt wait + barrier per stage
// (no workgroup memory fence: it would wait for the later stages' copies too).
// Each k-step is its own scheduling region: the LDS reads of the next k-step
// are interleaved with this k-step's MFMAs.  Loads past M, N or K go through
// range-checked buffer descriptors and return zeros (a stage past K
// contributes exactly zero), so the loop has no bounds branches.  Epilogue
// through LDS (store_block): whole output rows per store.
#pragma once
#include <type_traits>

#include "mfma32.h"

namespace aiter_amd {

template <int KA, bool BPRE, int BM, int BN>
struct T32Cfg {
    static constexpr bool MX = KA != kBf16;
    static constexpr int FA = (KA == kFp8) ? 2 : 1;           // 128-byte halves of an A row per stage
    static constexpr int A_CH = (BM / 8) * FA;                // A chunks per stage
    static constexpr int B_CH = BPRE ? (BN / 32) * 4 : BN / 8;
    static constexpr int SC_CH = MX ? 4 : 0;
    static constexpr int STAGE_KB = A_CH + B_CH + SC_CH;
    static constexpr int NS = (160 / STAGE_KB) > 4 ? 4 : (160 / STAGE_KB);
    static constexpr int K_STAGE = MX ? 256 : 64;             // K elements per stage
};

// SPLIT: blockIdx.y takes stages [y*S, y*S + S) of K (S = p.k_steps_per_split)
// and writes its fp32 partial tile to slice y of p.ws ([splits][M][N]); a
// second kernel sums the slices (fixed order, so results are deterministic).
// B_ONCE: the launch has one row of tiles (p.tiles_m == 1), so every B byte
// is read once and its copies carry the nt cache policy.
template <int KA, bool BPRE, int BM, int BN, int WAVES_M, bool OUT_F32, bool SPLIT = false, bool B_ONCE = false>
__global__ __launch_bounds__(256, 1) void gemm_t32_kernel(GemmParams p) {
    apply_batch(p);
    using Cfg = T32Cfg<KA, BPRE, BM, BN>;
    constexpr bool MX = Cfg::MX;
    constexpr int NS = Cfg::NS;
    constexpr int FA = Cfg::FA;
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int MA = WM / 32, NB = WN / 32;
    static_assert(MA >= 1 && NB >= 1, "wave tile must cover whole 32x32 MFMA tiles");
    static_assert(NS >= 2, "two LDS stages minimum");
    constexpr int AG = BM / 32, BG = BN / 32;
    constexpr int A_CH = Cfg::A_CH, B_CH = Cfg::B_CH;
    constexpr int SCA = MX ? (AG + 3) / 4 : 0, SCB = MX ? (BG + 3) / 4 : 0;
    static_assert(SCA + SCB <= 4, "one scale chunk per wave");
    static_assert(A_CH % 4 == 0 && B_CH % 4 == 0, "chunks split over 4 waves");
    constexpr int NA = A_CH / 4, NBW = B_CH / 4;   // copies per wave per stage
    constexpr int NDMA = NA + NBW + (MX ? 1 : 0);
    constexpr int WAIT_N = NS >= 3 ? (NS - 2) * NDMA : 0;
    static_assert(WAIT_N < 64, "vmcnt range");
    constexpr int STAGE_BYTES = Cfg::STAGE_KB * 1024;
    constexpr int A_ROW_BYTES = 128 * FA;
    // MX: the paired layout of mfma32.h (swap45) for the rows when a wave holds
    // an even number of 32-row tiles, for the columns when it holds an even
    // number of 32-column tiles; a paired tile's lanes share one scale byte
    constexpr bool PM = MX && MA % 2 == 0, PN = MX && NB % 2 == 0;

    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // stages of this workgroup: [t_base, t_base + nstages) of K
    const int t_base = SPLIT ? (int)blockIdx.y * p.k_steps_per_split : 0;
    const int nstages = SPLIT ? min(p.K / Cfg::K_STAGE - t_base, p.k_steps_per_split) : p.K / Cfg::K_STAGE;
    const __amdgpu_buffer_rsrc_t null_rsrc = make_rsrc(p.A, 0);

    // ---- A: chunk c = half*(BM/8) + 8-row block; lane l -> row l/8, stored piece l%8
    //      holding global 16-byte piece (l%8) ^ swz(row), swz(r) = (r>>1)&7
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (int64_t)(p.M - m0) * p.lda);
    int a_off[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int c = wave + 4 * q;
        const int half = c / (BM / 8), rb = c % (BM / 8);
        const int r = rb * 8 + (lane >> 3);
        a_off[q] = r * (int)p.lda + half * 128 + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
    }
    // ---- B: preshuffled chunk c = g*4 + s (four 256-byte runs), or row-major
    //      8-row block c staged like A
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(p.B + (int64_t)n0 * p.ldb, (int64_t)(p.N - n0) * p.ldb);
    int b_off[NBW];
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
        const int c = wave + 4 * q;
        if constexpr (BPRE) {
            const int s = c % 4, g = c / 4;
            // paired: tile g takes 16-row block g&1 of the groups 2(g>>1) + lane half
            const int b16 = PN ? 2 * (2 * (g >> 1) + ((lane >> 4) & 1)) + (g & 1) : 2 * g + ((lane >> 4) & 1);
            b_off[q] = b16 * 16 * (int)p.ldb + s * 512 + (lane >> 5) * 256 + (lane & 15) * 16;
        } else {
            const int r = c * 8 + (lane >> 3);
            b_off[q] = r * (int)p.ldb + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
        }
    }
    constexpr int B_STAGE_OFF = BPRE ? 2048 : 128;   // bytes per stage along a B row (block)
    // ---- MX scales: wave w copies chunk w (A groups, then B groups; spare chunks empty)
    int sc_off = 0;
    __amdgpu_buffer_rsrc_t sc_rsrc = null_rsrc;
    if constexpr (MX) {
        const int ga0 = m0 / 32, gb0 = n0 / 32;
        const __amdgpu_buffer_rsrc_t sa_rsrc =
            make_rsrc(p.As + (int64_t)ga0 * 32 * p.sa_stride, (int64_t)(p.sa_groups - ga0) * 32 * p.sa_stride);
        const __amdgpu_buffer_rsrc_t sb_rsrc =
            make_rsrc(p.Bs + (int64_t)gb0 * 32 * p.sb_stride, (int64_t)(p.sb_groups - gb0) * 32 * p.sb_stride);
        const bool sc_is_a = wave < SCA;
        const bool sc_is_b = wave >= SCA && wave < SCA + SCB;
        const int sc_chunk = sc_is_a ? wave : (sc_is_b ? wave - SCA : 0);
        const bool pair = sc_is_b ? PN : PM;   // chunk image of sc_pair_group / sc_pair_granule
        sc_off = (4 * sc_chunk + (pair ? sc_pair_group(lane) : (lane >> 4))) * 32 *
                     (int)(sc_is_b ? p.sb_stride : p.sa_stride) +
                 (pair ? sc_pair_granule(lane) : (lane & 15)) * 16;
        sc_rsrc = sc_is_a ? sa_rsrc : (sc_is_b ? sb_rsrc : null_rsrc);
    }

    // third `part` of the copies of stage t into its ring slot
    constexpr int DMA_PART = (NDMA + 2) / 3;
    auto dma_part = [&](int t, int part) {
        const bool live = t < nstages;
        const __amdgpu_buffer_rsrc_t ra = live ? a_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rb = live ? b_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rs = live ? sc_rsrc : null_rsrc;
        uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int q = part * DMA_PART; q < (part + 1) * DMA_PART && q < NDMA; ++q) {
            if (q < NA)
                dma16(ra, base + (wave + 4 * q) * 1024, a_off[q], (t_base + t) * A_ROW_BYTES);
            else if (q < NA + NBW) {
                dma16<B_ONCE ? kLoadNt : 0>(rb, base + (A_CH + wave + 4 * (q - NA)) * 1024, b_off[q - NA],
                                            (t_base + t) * B_STAGE_OFF);
            }
            else
                dma16(rs, base + (A_CH + B_CH + wave) * 1024, sc_off, (t_base + t) * 256);
        }
    };

    f32x16v_t acc[MA][NB];
#pragma unroll
    for (int i = 0; i < MA; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x16v_t{};

    i32x4_t af[2][MA][FA], bf[2][NB];
    int sa_pk[MA] = {}, sb_pk[NB] = {};   // packed scale bytes of the stage being multiplied

    // operand of k-step s: row r (32-row tile gi, lane row l%32), 16-byte piece
    // 2s + l/32 (+ 64 B for the second e4m3 half) stored at piece ^ swz(r)
    const int ar = lane & 31;
    const int row_off = (ar >> 3) * 1024 + (ar & 7) * 128;
    // paired: MFMA row ar of tile 2p+b is in 8-row chunk 8p + 2b + 4(ar>>4) + ((ar>>3)&1)
    const int prow_off = (4 * ((ar >> 4) & 1) + ((ar >> 3) & 1)) * 1024 + (ar & 7) * 128;
    const int swz = (ar >> 1) & 7;
    // 8-row chunk offset of 32-row tile I (paired: with the lane part prow_off)
    auto tile_chunks = [](int I, bool paired) { return paired ? (I >> 1) * 8 + (I & 1) * 2 : I * 4; };
    auto read_ops = [&](int t, int s, int slot) {
        const uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int h = 0; h < FA; ++h) {
                const int piece = (FA == 1) ? (2 * s + (lane >> 5)) : ((4 * s + 2 * h + (lane >> 5)) & 7);
                const int hh = (FA == 1) ? 0 : ((4 * s + 2 * h) >> 3);
                af[slot][i][h] = *reinterpret_cast<const i32x4_t*>(
                    base + (hh * (BM / 8) + tile_chunks(wm * MA + i, PM)) * 1024 + (PM ? prow_off : row_off) +
                    ((piece ^ swz) * 16));
            }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            if constexpr (BPRE)
                bf[slot][j] = *reinterpret_cast<const i32x4_t*>(base + (A_CH + (wn * NB + j) * 4 + s) * 1024 + lane * 16);
            else
                bf[slot][j] = *reinterpret_cast<const i32x4_t*>(
                    base + (A_CH + tile_chunks(wn * NB + j, PN)) * 1024 + (PN ? prow_off : row_off) +
                    (((2 * s + (lane >> 5)) ^ swz) * 16));
        }
    };
    // MX: lane l needs bytes h and 2+h (h = (l>>4)&1) of its group's two scale
    // dwords d0 (k-steps 0, 2) and d1 (k-steps 1, 3); packed [d0.h, d0.(2+h), d1.h, d1.(2+h)]
    // (paired: pair q's dwords d0 (k-steps 0, 2) and d1 (1, 3) as pa[2q], pa[2q+1])
    const int pos0 = ((lane & 15) + 16 * (lane >> 5)) * 4;
    const int ppos = sc_pair_read_off(lane);
    const unsigned sc_perm = 0x06040200u + ((lane >> 4) & 1) * 0x01010101u;
    auto read_scales = [&](int t, int (&pa)[MA], int (&pb)[NB]) {
        if constexpr (MX) {
            const uint8_t* base = smem + (t % NS) * STAGE_BYTES + (A_CH + B_CH) * 1024;
            if constexpr (PM) {
#pragma unroll
                for (int q = 0; q < MA / 2; ++q) {
                    const uint8_t* g = base + ppos + (wm * MA / 2 + q) * 512;
                    pa[2 * q] = *reinterpret_cast<const int*>(g);
                    pa[2 * q + 1] = *reinterpret_cast<const int*>(g + 256);
                }
            } else {
#pragma unroll
                for (int i = 0; i < MA; ++i) {
                    const uint8_t* g = base + pos0 + (wm * MA + i) * 256;
                    pa[i] = (int)__builtin_amdgcn_perm(*reinterpret_cast<const unsigned*>(g + 128),
                                                       *reinterpret_cast<const unsigned*>(g), sc_perm);
                }
            }
            if constexpr (PN) {
#pragma unroll
                for (int q = 0; q < NB / 2; ++q) {
                    const uint8_t* g = base + SCA * 1024 + ppos + (wn * NB / 2 + q) * 512;
                    pb[2 * q] = *reinterpret_cast<const int*>(g);
                    pb[2 * q + 1] = *reinterpret_cast<const int*>(g + 256);
                }
            } else {
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const uint8_t* g = base + SCA * 1024 + pos0 + (wn * NB + j) * 256;
                    pb[j] = (int)__builtin_amdgcn_perm(*reinterpret_cast<const unsigned*>(g + 128),
                                                       *reinterpret_cast<const unsigned*>(g), sc_perm);
                }
            }
        }
    };
    auto mma = [&](int slot, auto sel) {
        constexpr int s = decltype(sel)::value;
        constexpr int osel = (s == 0) ? 0 : (s == 1) ? 2 : (s == 2) ? 1 : 3;
        // paired: tile 2q+b uses byte b + 2(s/2) of dword d(s%2) of pair q
        constexpr int o0 = PM ? 2 * (s >> 1) : osel, o1 = PM ? 1 + 2 * (s >> 1) : osel;
        constexpr int p0 = PN ? 2 * (s >> 1) : osel, p1 = PN ? 1 + 2 * (s >> 1) : osel;
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int sa = PM ? sa_pk[2 * (i >> 1) + (s & 1)] : sa_pk[i];
                const int sb = PN ? sb_pk[2 * (j >> 1) + (s & 1)] : sb_pk[j];
                const i32x4_t &b = bf[slot][j], &a0 = af[slot][i][0], &a1 = af[slot][i][FA - 1];
                if (i & 1) {
                    if (j & 1) acc[i][j] = mma32x<KA, o1, p1>(b, a0, a1, acc[i][j], sa, sb);
                    else acc[i][j] = mma32x<KA, o1, p0>(b, a0, a1, acc[i][j], sa, sb);
                } else {
                    if (j & 1) acc[i][j] = mma32x<KA, o0, p1>(b, a0, a1, acc[i][j], sa, sb);
                    else acc[i][j] = mma32x<KA, o0, p0>(b, a0, a1, acc[i][j], sa, sb);
                }
            }
    };

    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    constexpr int RD = MA * FA + NB;   // ds_read_b128 per k-step
    constexpr int MF = MA * NB;        // MFMAs per k-step
    auto pace = [&](int vmem) {
#pragma unroll
        for (int k = 0; k < MF; ++k) {
            if (k < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);           // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // MFMA
            if (k >= MF - vmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;

    // prologue: stages 0 .. NS-2 in flight; wait for stage 0
#pragma unroll
    for (int t = 0; t < NS - 1; ++t)
#pragma unroll
        for (int part = 0; part < 3; ++part) dma_part(t, part);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<(NS - 2) * NDMA>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    read_scales(0, sa_pk, sb_pk);
    read_ops(0, 0, 0);

    for (int t = 0; t < nstages; ++t) {
        read_ops(t, 1, 1);
        dma_part(t + NS - 1, 0);
        mma(0, S0{});
        pace(DMA_PART);
        fence();
        read_ops(t, 2, 0);
        dma_part(t + NS - 1, 1);
        mma(1, S1{});
        pace(DMA_PART);
        fence();
        read_ops(t, 3, 1);
        dma_part(t + NS - 1, 2);
        mma(0, S2{});
        pace(NDMA - 2 * DMA_PART);
        fence();
        // stage t+1 published: own copies landed and own LDS reads of stage t
        // done, then everyone's (barrier)
        wait_vmcnt_lgkm0<WAIT_N>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        fence();
        read_ops(t + 1, 0, 0);
        int na[MA], nb[NB];
        read_scales(t + 1, na, nb);
        mma(1, S3{});
        if constexpr (MX) {
#pragma unroll
            for (int i = 0; i < MA; ++i) sa_pk[i] = na[i];
#pragma unroll
            for (int j = 0; j < NB; ++j) sb_pk[j] = nb[j];
        }
        pace(0);
        fence();
    }

    // ---- epilogue through LDS (the ring is free once every copy has landed)
    constexpr int EB = OUT_F32 ? 4 : 2;
    constexpr int WAVE_SCRATCH = NS * STAGE_BYTES / 4;
    constexpr int EP_MP = (MA * 32 * WN * EB <= WAVE_SCRATCH) ? MA
                          : (MA % 2 == 0 && MA / 2 * 32 * WN * EB <= WAVE_SCRATCH) ? MA / 2 : 1;
    static_assert(EP_MP * 32 * WN * EB <= WAVE_SCRATCH, "epilogue pass fits the ring");
    wait_vmcnt<0>();
    __syncthreads();
    if constexpr (SPLIT) {
        constexpr int EP_MP32 = (MA * 32 * WN * 4 <= WAVE_SCRATCH) ? MA
                                : (MA % 2 == 0 && MA / 2 * 32 * WN * 4 <= WAVE_SCRATCH) ? MA / 2 : 1;
        static_assert(EP_MP32 * 32 * WN * 4 <= WAVE_SCRATCH, "epilogue pass fits the ring");
        GemmParams q = p;
        q.D = p.ws + (int64_t)blockIdx.y * p.M * p.N;
        q.ldd = p.N;
        store_block<MA, NB, EP_MP32, false, false, true, false, false, false, (PM ? 1 : 0) | (PN ? 2 : 0)>(
            q, acc, smem + wave * WAVE_SCRATCH, lane, m0 + wm * WM, n0 + wn * WN);
    } else {
        store_block_any<MA, NB, EP_MP, OUT_F32, (PM ? 1 : 0) | (PN ? 2 : 0)>(p, acc, smem + wave * WAVE_SCRATCH, lane,
                                                                          m0 + wm * WM, n0 + wn * WN);
    }
}

}  // namespace aiter_amd
