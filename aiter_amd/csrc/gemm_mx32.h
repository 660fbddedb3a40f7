// MX tile kernel on v_mfma_scale_f32_32x32x64_f8f6f4 (gfx950).
//
// Why 32x32x64: on MI355X it issues once per 32 cycles for e2m1 (8 passes,
// 131072 FLOP), twice the e2m1 throughput of the 16x16x128 form, so it is the
// only shape that can approach the dense MXFP4 peak.
//
// Operand layout of one 32x32x64 MFMA (measured on gfx950):
//   e2m1 : lane l holds row (l % 32), bytes [16*(l/32), +16) of the 32-byte
//          K window (32 elements = one MX block per lane);
//   e4m3 : lane l holds row (l % 32), bytes [16*(l/32), +16) and
//          [32 + 16*(l/32), +16) of the 64-byte K window;
//   scale: lane l supplies the e8m0 of (row l%32, block 2s + l/32) for
//          k-step s of a 256-element window; result lane l holds
//          C[src1 col = l%32][src0 row = 8q + 4(l/32) + r], r<4, q<4.
//
// Data movement per 256-element K stage (4 k-steps):
//   * A and B are copied global -> LDS by buffer_load ... lds (no VGPR
//     staging).  One instruction moves one 1 KiB chunk: lane l's 16 bytes land
//     at chunk + 16*l.  A is staged as whole 128-byte row pieces (8 rows per
//     chunk, 16-byte pieces XOR-swizzled by row, bank-conflict-free reads);
//     preshuffled B is already in MFMA operand order (four 256-byte runs per
//     chunk).  Rows beyond M/N read as 0 (buffer range check).
//   * Scales: one chunk of 4 groups x 256 bytes per wave and stage, read as
//     two dwords per lane and group and shifted by 8*((l>>4)&1) + 16*(s>>1)
//     at use, so op_sel stays 0.
//   * A ring of NS stages (as many as fit 160 KiB, at most 4); one vmcnt wait
//     and barrier per stage; LDS reads of k-step s+1 overlap the MFMAs of s.
//   * Epilogue through LDS (store_block_bf16): whole output rows per store.
#pragma once
#include "gemm_kernels.h"

namespace aiter_amd {

typedef float f32x16v_t __attribute__((ext_vector_type(16)));
#define AA_LDS __attribute__((address_space(3)))

#define AA_MFMA32_SC(OA, OB)                                                                 \
    case (OA) * 4 + (OB):                                                                    \
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, FA, FB, OA, sa, OB, sb);

template <int FA, int FB>
AA_DEV f32x16v_t mfma32_scaled(i32x8_t a, i32x8_t b, f32x16v_t c, int sa, int oa, int sb, int ob) {
    switch (oa * 4 + ob) {
        AA_MFMA32_SC(0, 0) AA_MFMA32_SC(0, 2) AA_MFMA32_SC(2, 0) AA_MFMA32_SC(2, 2)
        default: __builtin_unreachable();
    }
}
#undef AA_MFMA32_SC

AA_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    // raw buffer, dword format; loads at offsets >= bytes return 0
    const int n = (int)(bytes > 0x7ffffff0LL ? 0x7ffffff0LL : (bytes < 0 ? 0 : bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

// global -> LDS copy of one 1 KiB chunk (16 bytes per lane, lane order)
AA_DEV void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_chunk, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (AA_LDS void*)lds_chunk, 16, voff, soff, 0, 0);
}

// s_waitcnt with only the vmcnt field constrained (expcnt/lgkmcnt left at max)
template <int N>
AA_DEV void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt vmcnt(N) lgkmcnt(0): own copies up to the N newest have landed and
// every LDS access of this wave has completed
template <int N>
AA_DEV void wait_vmcnt_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4));
}

// One k-step of a 32x32 MFMA tile: src0 = B fragment (16 bytes per lane),
// src1 = A fragment(s) (two 16-byte halves for e4m3), packed scale bytes with
// op_sel OSEL for the MX kinds.  Result lane l holds C[m = l%32][n = 8q + 4(l/32) + r].
template <int KA, int OSEL>
AA_DEV f32x16v_t mma32(const i32x4_t& b, const i32x4_t& a0, const i32x4_t& a1, f32x16v_t c, int sa, int sb) {
    if constexpr (KA == kBf16) {
        typedef __bf16 bf16x8v_t __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8v_t, b), __builtin_bit_cast(bf16x8v_t, a0),
                                                       c, 0, 0, 0);
    } else {
        i32x8_t bv, av;
        bv[0] = b[0]; bv[1] = b[1]; bv[2] = b[2]; bv[3] = b[3];
        bv[4] = 0; bv[5] = 0; bv[6] = 0; bv[7] = 0;
        av[0] = a0[0]; av[1] = a0[1]; av[2] = a0[2]; av[3] = a0[3];
        if constexpr (KA == kFp8) {
            av[4] = a1[0]; av[5] = a1[1]; av[6] = a1[2]; av[7] = a1[3];
        } else {
            av[4] = 0; av[5] = 0; av[6] = 0; av[7] = 0;
        }
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, c, 4, OpTraits<KA>::fmt, OSEL, sb, OSEL, sa);
    }
}

// Epilogue of a wave's (32*MA) x (32*NB) block of 32x32 MFMA accumulators
// (lane l holds C[m = l%32][n = 8q + 4(l/32) + r] of each tile) written as
// bf16 or f32, D = alpha*acc + beta*bias.  Stored directly, each global store
// would touch 32 rows; instead the block goes through the wave's own LDS
// scratch `cb`, MP row tiles (32*MP rows x 32*NB elements) per pass, 16-byte
// pieces XOR-swizzled by row so that both the writes and the 16-byte reads
// spread over the banks, and leaves as whole rows.  (mb, nb) is the block's
// global origin.  Branch-free: stores go through a range-checked descriptor
// of D (rows >= M fall outside it, columns >= N get an offset outside it) and
// bias reads are clamped into the bias tensor.  SCALED = false skips the
// alpha multiply (alpha == 1, no bias).
template <int MA, int NB, int MP, bool HAS_BIAS, bool SCALED = true, bool OUT_F32 = false>
AA_DEV void store_block(const GemmParams& p, f32x16v_t (&acc)[MA][NB], uint8_t* cb, int lane, int mb, int nb) {
    static_assert(MA % MP == 0, "whole passes");
    constexpr int EB = OUT_F32 ? 4 : 2;         // output bytes per element
    constexpr int RB = 32 * NB * EB;            // bytes per block row
    constexpr int P = RB / 16;                  // 16-byte pieces per row
    static_assert(P <= 64, "one row per read instruction at most");
    constexpr int SWM = (P < 8 ? P : 8) - 1;    // swizzle mask
    constexpr int RSH = RB < 128 ? 1 : 0;       // two 64-byte rows share a 128-byte bank line
    constexpr int ROWS_PER = 64 / P;            // rows per read instruction
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    // opaque copy of the lane index: keeps the compiler from hoisting this
    // epilogue's address arithmetic out of an enclosing loop
    asm volatile("" : "+v"(lane));
    const __amdgpu_buffer_rsrc_t d_rsrc = make_rsrc(p.D, (int64_t)p.M * p.ldd * EB);
    const int pc = lane % P;
    const int n_out = nb + pc * (16 / EB);
    const int col_off = n_out < p.N ? n_out * EB : 0x7fffffff;   // outside D when past N
#pragma unroll
    for (int i0 = 0; i0 < MA; i0 += MP) {
#pragma unroll
        for (int i = 0; i < MP; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = i * 32 + (lane & 31);
                    const int nl = j * 32 + 8 * q + 4 * (lane >> 5);
                    const f32x16v_t& a = acc[i0 + i][j];
                    float v[4] = {a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
                    if constexpr (SCALED) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] *= p.alpha;
                    }
                    if constexpr (HAS_BIAS) {
                        const int m = min(mb + i0 * 32 + r, p.M - 1), n = min(nb + nl, p.N - 4);
                        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p.bias + (int64_t)m * p.ld_bias + n);
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] += p.beta * b[e];
                    }
                    const int byte = nl * EB;
                    const int piece = (byte >> 4) ^ ((r >> RSH) & SWM);
                    if constexpr (OUT_F32) {
                        *reinterpret_cast<f32x4_t*>(cb + r * RB + piece * 16) = f32x4_t{v[0], v[1], v[2], v[3]};
                    } else {
                        *reinterpret_cast<u32x2_t*>(cb + r * RB + piece * 16 + (byte & 15)) =
                            u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    }
                }
        // the scratch is the wave's own: its LDS accesses complete in order
#pragma unroll
        for (int rr = 0; rr < 32 * MP; rr += ROWS_PER) {
            const int r = rr + lane / P;
            const i32x4_t v = *reinterpret_cast<const i32x4_t*>(cb + r * RB + ((pc ^ ((r >> RSH) & SWM)) * 16));
            const int m = mb + i0 * 32 + r;
            const int off = col_off == 0x7fffffff ? col_off : m * (int)p.ldd * EB + col_off;
            __builtin_amdgcn_raw_buffer_store_b128(v, d_rsrc, off, 0, 0);
        }
    }
}

// the three epilogue flavours picked at run time (uniform branch)
template <int MA, int NB, int MP, bool OUT_F32>
AA_DEV void store_block_any(const GemmParams& p, f32x16v_t (&acc)[MA][NB], uint8_t* cb, int lane, int mb, int nb) {
    if (p.bias)
        store_block<MA, NB, MP, true, true, OUT_F32>(p, acc, cb, lane, mb, nb);
    else if (p.alpha != 1.0f)
        store_block<MA, NB, MP, false, true, OUT_F32>(p, acc, cb, lane, mb, nb);
    else
        store_block<MA, NB, MP, false, false, OUT_F32>(p, acc, cb, lane, mb, nb);
}

// LDS ring depth that fits 160 KiB for a tile
template <int KA, int BM, int BN>
struct Mx32Cfg {
    static constexpr int FA = (KA == kFp8) ? 2 : 1;
    static constexpr int A_CH = (BM / 8) * FA;   // 8 rows x 128 B per chunk (per 128-byte half)
    static constexpr int B_CH = (BN / 32) * 4;   // 32-row group x k-step
    static constexpr int STAGE_KB = A_CH + B_CH + 4;
    static constexpr int NS = (160 / STAGE_KB) > 4 ? 4 : (160 / STAGE_KB);
};

template <int KA, int BM, int BN, int WAVES_M, bool OUT_F32>
__global__ __launch_bounds__(256, 1) void gemm_mx32_kernel(GemmParams p) {
    using Cfg = Mx32Cfg<KA, BM, BN>;
    constexpr int NS = Cfg::NS;                // LDS stages (ring)
    constexpr int FA = Cfg::FA;                // 128-byte halves of an A row per stage
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int MA = WM / 32, NB = WN / 32;
    static_assert(MA >= 1 && NB >= 1, "wave tile must cover whole 32x32 MFMA tiles");
    static_assert(NS >= 2, "two LDS stages minimum");
    constexpr int AG = BM / 32, BG = BN / 32;  // 32-row groups per block
    constexpr int A_CH = Cfg::A_CH, B_CH = Cfg::B_CH;
    constexpr int SCA = (AG + 3) / 4, SCB = (BG + 3) / 4;  // scale chunks (4 groups each)
    static_assert(SCA + SCB <= 4, "one scale chunk per wave");
    static_assert(A_CH % 4 == 0 && B_CH % 4 == 0, "chunks split over 4 waves");
    constexpr int NA = A_CH / 4, NBW = B_CH / 4;  // DMAs per wave per stage
    constexpr int NDMA = NA + NBW + 1;
    static_assert((NS - 2) * NDMA < 64, "vmcnt budget");
    constexpr int STAGE_BYTES = Cfg::STAGE_KB * 1024;
    constexpr int A_ROW_BYTES = 128 * FA;      // A bytes per row per stage (256 elements)

    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int nstages = p.K / 256;

    // ---- A: chunk c = half*(BM/8) + 8-row block; lane l -> row l/8, stored piece l%8
    //      holding global 16-byte piece (l%8) ^ swz(row), swz(r) = (r>>1)&7.
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.A + (int64_t)m0 * p.lda, (int64_t)(p.M - m0) * p.lda);
    int a_off[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int c = wave + 4 * q;
        const int half = c / (BM / 8), rb = c % (BM / 8);
        const int r = rb * 8 + (lane >> 3);
        a_off[q] = r * (int)p.lda + half * 128 + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
    }
    // ---- B (preshuffled): chunk c = g*4 + s, four 256-byte runs of the (16,16) layout
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(p.B + (int64_t)n0 * p.ldb, (int64_t)(p.N - n0) * p.ldb);
    int b_off[NBW];
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
        const int c = wave + 4 * q;
        const int s = c % 4, g = c / 4;
        const int blk = 2 * g + ((lane >> 4) & 1);
        b_off[q] = blk * 16 * (int)p.ldb + s * 512 + (lane >> 5) * 256 + (lane & 15) * 16;
    }
    // ---- scales: wave w copies chunk w = 4 groups x 256 bytes of the stage's window
    const int ga0 = m0 / 32, gb0 = n0 / 32;
    const __amdgpu_buffer_rsrc_t sa_rsrc =
        make_rsrc(p.As + (int64_t)ga0 * 32 * p.sa_stride, (int64_t)(p.sa_groups - ga0) * 32 * p.sa_stride);
    const __amdgpu_buffer_rsrc_t sb_rsrc =
        make_rsrc(p.Bs + (int64_t)gb0 * 32 * p.sb_stride, (int64_t)(p.sb_groups - gb0) * 32 * p.sb_stride);
    const bool sc_is_b = wave >= SCA && wave < SCA + SCB;
    const int sc_chunk = wave < SCA ? wave : (sc_is_b ? wave - SCA : 0);
    const int sc_off = (4 * sc_chunk + (lane >> 4)) * 32 * (int)(sc_is_b ? p.sb_stride : p.sa_stride) + (lane & 15) * 16;
    const __amdgpu_buffer_rsrc_t sc_rsrc = sc_is_b ? sb_rsrc : sa_rsrc;
    // zero-length descriptor: every load through it is out of range (no memory
    // traffic, LDS receives zeros); used for stages past the end so the loop body
    // stays a single basic block
    const __amdgpu_buffer_rsrc_t null_rsrc = make_rsrc(p.A, 0);

    auto dma_stage = [&](int t) {
        const bool live = t < nstages;
        const __amdgpu_buffer_rsrc_t ra = live ? a_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rb = live ? b_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rs = live ? sc_rsrc : null_rsrc;
        uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int q = 0; q < NA; ++q) dma16(ra, base + (wave + 4 * q) * 1024, a_off[q], t * A_ROW_BYTES);
#pragma unroll
        for (int q = 0; q < NBW; ++q) dma16(rb, base + (A_CH + wave + 4 * q) * 1024, b_off[q], t * 2048);
        dma16(rs, base + (A_CH + B_CH + wave) * 1024, sc_off, t * 256);
    };

    const int pos0 = ((lane & 15) + 16 * (lane >> 5)) * 4;
    const int sshift = 8 * ((lane >> 4) & 1);

    f32x16v_t acc[MA][NB];
#pragma unroll
    for (int i = 0; i < MA; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x16v_t{};

    i32x4_t af[2][MA][FA], bf[2][NB];
    int sa_raw[MA][2], sb_raw[NB][2];  // scale dwords of the current stage (window)

    // operand of k-step s: A row r = 32*gi + l%32, 16-byte piece 2s + l/32 (+ 64 B for the
    // second e4m3 half), stored at piece ^ swz(r); B chunk (gj, s), lane order
    const int ar = lane & 31;
    const int a_lane_off = (ar >> 3) * 1024 + (ar & 7) * 128;
    const int a_swz = (ar >> 1) & 7;
    auto read_ops = [&](int t, int s, int slot) {
        const uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int h = 0; h < FA; ++h) {
                const int piece = (FA == 1) ? (2 * s + (lane >> 5)) : ((4 * s + 2 * h + (lane >> 5)) & 7);
                const int hh = (FA == 1) ? 0 : ((4 * s + 2 * h) >> 3);
                af[slot][i][h] = *reinterpret_cast<const i32x4_t*>(
                    base + (hh * (BM / 8) + (wm * MA + i) * 4) * 1024 + a_lane_off + ((piece ^ a_swz) * 16));
            }
#pragma unroll
        for (int j = 0; j < NB; ++j)
            bf[slot][j] = *reinterpret_cast<const i32x4_t*>(base + (A_CH + (wn * NB + j) * 4 + s) * 1024 + lane * 16);
    };
    auto read_scales = [&](int t) {
        const uint8_t* base = smem + (t % NS) * STAGE_BYTES + (A_CH + B_CH) * 1024 + pos0;
#pragma unroll
        for (int i = 0; i < MA; ++i) {
            const uint8_t* g = base + (wm * MA + i) * 256;
            sa_raw[i][0] = *reinterpret_cast<const int*>(g);
            sa_raw[i][1] = *reinterpret_cast<const int*>(g + 128);
        }
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const uint8_t* g = base + SCA * 1024 + (wn * NB + j) * 256;
            sb_raw[j][0] = *reinterpret_cast<const int*>(g);
            sb_raw[j][1] = *reinterpret_cast<const int*>(g + 128);
        }
    };
    // k-step s of the window: dword (s & 1), byte 2*(s>>1) + r2 moved to position 0
    struct StepScales {
        int a[MA], b[NB];
    };
    auto step_scales = [&](int s) {
        StepScales sc;
        const int shift = sshift + 16 * (s >> 1);
#pragma unroll
        for (int i = 0; i < MA; ++i) sc.a[i] = sa_raw[i][s & 1] >> shift;
#pragma unroll
        for (int j = 0; j < NB; ++j) sc.b[j] = sb_raw[j][s & 1] >> shift;
        return sc;
    };
    auto mma = [&](int slot, const StepScales& sc) {
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                i32x8_t bv, av;
                bv[0] = bf[slot][j][0]; bv[1] = bf[slot][j][1]; bv[2] = bf[slot][j][2]; bv[3] = bf[slot][j][3];
                bv[4] = 0; bv[5] = 0; bv[6] = 0; bv[7] = 0;
                av[0] = af[slot][i][0][0]; av[1] = af[slot][i][0][1]; av[2] = af[slot][i][0][2]; av[3] = af[slot][i][0][3];
                if constexpr (FA == 2) {
                    av[4] = af[slot][i][1][0]; av[5] = af[slot][i][1][1]; av[6] = af[slot][i][1][2]; av[7] = af[slot][i][1][3];
                } else {
                    av[4] = 0; av[5] = 0; av[6] = 0; av[7] = 0;
                }
                acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, acc[i][j], 4, OpTraits<KA>::fmt,
                                                                            0, sc.b[j], 0, sc.a[i]);
            }
    };

    // interleave: per k-step, the next k-step's operand reads (and this
    // stage's DMA issues) are spread between the MFMAs so LDS latency hides
    // behind MFMA execution instead of stalling before each MFMA group
    constexpr int RD = MA * FA + NB;            // ds_read_b128 per k-step
    constexpr int MF = MA * NB;                 // MFMAs per k-step
    auto pace = [&](int dma_per_step) {
#pragma unroll
        for (int k = 0; k < MF; ++k) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);        // MFMA
            if (k < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            if (k < dma_per_step) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM
        }
    };
    constexpr int DMA_STEP = (NDMA + 2) / 3;    // DMAs spread over k-steps 0..2

    // prologue: stages 0 .. NS-2 in flight; wait for stage 0
#pragma unroll
    for (int t = 0; t < NS - 1; ++t) dma_stage(t);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<(NS - 2) * NDMA>();
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    read_scales(0);
    read_ops(0, 0, 0);

    // iteration t: DMA of stage t+NS-1 goes into the buffer of stage t-1 (all
    // reads of it ended before the barrier of iteration t-1); before k-step 3 the
    // wave waits for stage t+1 and a barrier publishes it, so its first operands
    // and scales are read while the MFMAs of k-step 3 run.  Past the last stage
    // the DMAs are out-of-range no-ops and the reads fetch unused data.
    for (int t = 0; t < nstages; ++t) {
        dma_stage(t + NS - 1);
        read_ops(t, 1, 1);
        mma(0, step_scales(0));
        pace(DMA_STEP);
        read_ops(t, 2, 0);
        mma(1, step_scales(1));
        pace(DMA_STEP);
        read_ops(t, 3, 1);
        mma(0, step_scales(2));
        pace(DMA_STEP);
        const StepScales sc3 = step_scales(3);  // before the next stage's scales land
        // nothing may be scheduled across the publication of stage t+1
        __builtin_amdgcn_sched_barrier(0);
        wait_vmcnt<(NS - 2) * NDMA>();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
        read_ops(t + 1, 0, 0);
        read_scales(t + 1);
        mma(1, sc3);
        pace(0);
    }

    // ---- epilogue through LDS (the ring is free once every copy has landed)
    static_assert(!OUT_F32, "the MX tile kernel writes bf16");
    static_assert(BM * BN * 2 <= NS * STAGE_BYTES, "epilogue fits the ring");
    wait_vmcnt<0>();
    __syncthreads();
    store_block_any<MA, NB, MA, false>(p, acc, smem + wave * (WM * WN * 2), lane, m0 + wm * WM, n0 + wn * WN);
}

}  // namespace aiter_amd
