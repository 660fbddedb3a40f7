// Shared pieces of the gfx950 32x32 MFMA tile kernels (gemm_flat.h,
// gemm_t32.h): the k-step MFMA wrapper for e2m1 / e4m3 (scaled, e8m0) and
// bf16, buffer descriptors with hardware range checks, global -> LDS copies,
// explicit wait counters and the LDS-staged epilogue.
//
// Measured on MI355X: v_mfma_scale_f32_32x32x64_f8f6f4 issues once per 32
// cycles for e2m1 x e2m1 (twice the e2m1 rate of the 16x16x128 form) and once
// per 64 cycles with an e4m3 operand; v_mfma_f32_32x32x16_bf16 once per 32.
// Operand layout (bytes are the same for all three): lane l holds row l%32
// and bytes [16*(l/32), +16) of a 32-byte K window (e4m3: also the same 16
// bytes of the following window); result lane l holds
// C[src1 row = l%32][src0 row = 8q + 4(l/32) + r], r < 4, q < 4.  Scales: lane
// l supplies the e8m0 byte of (row l%32, block 2s + l/32) for k-step s of a
// 256-element window, selected from a 32-bit register by op_sel (byte 0..3).
#pragma once
#include <type_traits>

#include "gemm_kernels.h"
#include "mx_quant.h"

namespace aiter_amd {

typedef float f32x16v_t __attribute__((ext_vector_type(16)));
#define AA_LDS __attribute__((address_space(3)))


AA_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    // raw buffer, dword format; loads at offsets >= bytes return 0
    const int n = (int)(bytes > 0x7ffffff0LL ? 0x7ffffff0LL : (bytes < 0 ? 0 : bytes));
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, n, 0x00020000);
}

// global -> LDS copy of one 1 KiB chunk (16 bytes per lane, lane order)
template <int AUX = 0>
AA_DEV void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_chunk, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (AA_LDS void*)lds_chunk, 16, voff, soff, 0, AUX);
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
template <int KA, int OSEL_A, int OSEL_B>
AA_DEV f32x16v_t mma32x(const i32x4_t& b, const i32x4_t& a0, const i32x4_t& a1, f32x16v_t c, int sa, int sb);

template <int KA, int OSEL>
AA_DEV f32x16v_t mma32(const i32x4_t& b, const i32x4_t& a0, const i32x4_t& a1, f32x16v_t c, int sa, int sb) {
    return mma32x<KA, OSEL, OSEL>(b, a0, a1, c, sa, sb);
}

// f(std::integral_constant<int, I>) for I = 0 .. N-1 (compile-time indices)
template <int N, typename F, int I = 0>
AA_DEV void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, F, I + 1>(static_cast<F&&>(f));
    }
}

// Row / column order of the "paired" tile layout: MFMA row (column) x of a
// 64-row (64-column) block holds row (column) swap45(x), i.e. bits 4 and 5 of
// the index exchanged.  Tile 2p+b then takes rows 16b..16b+15 of the 32-row
// groups 2p and 2p+1, so all its lanes read e8m0 byte b (+2) of the same
// shuffled-scale dwords (the scale of row r sits in byte (r%32)/16), and a
// pair of tiles shares one dword pair: no per-lane byte shuffle.
AA_DEV constexpr int swap45(int x) { return (x & ~48) | ((x & 16) << 1) | ((x & 32) >> 1); }

// e8m0 scales in the paired layout.  A ring slot's scale chunk holds 4 groups
// x 256 B (one K stage of 32 rows each).  The two groups of a pair interleave
// by 128-byte halves (even group's first half, odd group's first half, even's
// second, odd's second), the odd group's 64-byte quarters swapped.  A lane's
// two dwords (k-steps 0/2 and 1/3) are then 256 B apart for every lane, and
// a wave's reads spread over 32 or 64 banks.  Copy: lane l fetches 16-byte
// granule sc_pair_granule(l) of group sc_pair_group(l) of the chunk's four.
// Read: pair q's dwords at q*512 + sc_pair_read_off(l) and +256.
AA_DEV int sc_pair_group(int lane) { return 2 * (lane >> 5) + ((lane >> 3) & 1); }
AA_DEV int sc_pair_granule(int lane) { return ((lane >> 4) & 1) * 8 + ((lane & 7) ^ (((lane >> 3) & 1) * 4)); }
AA_DEV int sc_pair_read_off(int lane) {
    const int o = (lane >> 4) & 1;
    return o * 128 + ((((lane >> 5) * 64) + (lane & 15) * 4) ^ (o * 64));
}

// As mma32, with separate op_sel byte selections for the A and B scales.
template <int KA, int OSEL_A, int OSEL_B>
AA_DEV f32x16v_t mma32x(const i32x4_t& b, const i32x4_t& a0, const i32x4_t& a1, f32x16v_t c, int sa, int sb) {
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
        return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(bv, av, c, 4, OpTraits<KA>::fmt, OSEL_B, sb, OSEL_A, sa);
    }
}

// Buffer cache policy of split-K partials that one workgroup writes and the
// last-arriving split of the same tile (on any XCD) reads back: sc1, the
// agent-coherent form (past the XCD-private L2, to and from memory), so no
// L2 writeback or invalidate is needed between them (the MoE stage-1 split).
constexpr int kAgentCoherent = 16;

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
// alpha multiply (alpha == 1, no bias).  FENCED = true converts one 32x32
// block per scheduling region, for epilogues inside a loop where the other
// live registers leave no room for all accumulator reads at once.  OUT_FP4
// = true writes packed e2m1 (conversion scale 1, RNE, saturating: two values
// per byte, the lower column in the low nibble; p.ldd still counts elements).
// EPI = true adds, at run time, the bias and the fused output operation of
// p.epi (mul_add on the f32 values; split_cat sends each 16-byte piece to
// c1 or c2, which needs S1 and S2 to be multiples of a piece).  REMAP: the
// accumulators are in the paired layout, bit 0 for rows (swap45 of the row
// within each 64-row block; MA even), bit 1 for columns (NB even); (mb, nb)
// are then 64-aligned within the tile.
template <int MA, int NB, int MP, bool HAS_BIAS, bool SCALED = true, bool OUT_F32 = false, bool FENCED = false,
          bool OUT_FP4 = false, bool EPI = false, int REMAP = 0>
AA_DEV void store_block(const GemmParams& p, f32x16v_t (&acc)[MA][NB], uint8_t* cb, int lane, int mb, int nb) {
    static_assert(MA % MP == 0, "whole passes");
    static_assert(!(OUT_FP4 && OUT_F32), "one output format");
    static_assert(!(REMAP & 1) || MA % 2 == 0, "paired rows: 64-row blocks");
    static_assert(!(REMAP & 2) || NB % 2 == 0, "paired columns: 64-column blocks");
    constexpr bool RM = REMAP & 1, RN = REMAP & 2;
    constexpr int EB2 = OUT_FP4 ? 1 : (OUT_F32 ? 8 : 4);   // output bytes per two elements
    constexpr int RB = 16 * NB * EB2;           // bytes per block row
    constexpr int P = RB / 16;                  // 16-byte pieces per row
    static_assert(P <= 64, "one row per read instruction at most");
    constexpr int SWM = (P < 8 ? P : 8) - 1;    // swizzle mask
    constexpr int RSH = RB < 128 ? 1 : 0;       // two 64-byte rows share a 128-byte bank line
    constexpr int ROWS_PER = 64 / P;            // rows per read instruction
    typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
    // opaque copy of the lane index: keeps the compiler from hoisting this
    // epilogue's address arithmetic out of an enclosing loop
    asm volatile("" : "+v"(lane));
    const __amdgpu_buffer_rsrc_t d_rsrc = make_rsrc(p.D, (int64_t)p.M * p.ldd * EB2 / 2);
    const int pc = lane % P;
    const int n_out = nb + pc * (32 / EB2);
    const int col_off = n_out < p.N ? n_out * EB2 / 2 : 0x7fffffff;   // outside D when past N
    // lane parts of the paired row maps (swap45 permutes bits, and the
    // compile-time parts below hold the other bits)
    const int lrow1 = RM ? swap45(lane & 31) : (lane & 31);
    const int lrow2 = RM ? swap45(lane / P) : lane / P;
#pragma unroll
    for (int i0 = 0; i0 < MA; i0 += MP) {
#pragma unroll
        for (int i = 0; i < MP; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                if constexpr (FENCED) __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = i * 32 + (lane & 31);
                    // column: 4 adjacent ones; row within the block
                    const int nl = (RN ? swap45(j * 32 + 8 * q) : j * 32 + 8 * q) + 4 * (lane >> 5);
                    const int mr = (RM ? swap45((i0 + i) * 32) : (i0 + i) * 32) + lrow1;
                    const f32x16v_t& a = acc[i0 + i][j];
                    float v[4] = {a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]};
                    if constexpr (SCALED) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] *= p.alpha;
                    }
                    if constexpr (HAS_BIAS) {
                        const int m = min(mb + mr, p.M - 1), n = min(nb + nl, p.N - 4);
                        const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p.bias + (int64_t)m * p.ld_bias + n);
#pragma unroll
                        for (int e = 0; e < 4; ++e) v[e] += p.beta * b[e];
                    }
                    if constexpr (EPI) {
                        // values of rows >= M / columns >= N are computed at a
                        // clamped position and dropped by the store
                        const int m = min(mb + mr, p.M - 1), n = min(nb + nl, p.N - 4);
                        if (p.bias) {
                            const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p.bias + (int64_t)m * p.ld_bias + n);
#pragma unroll
                            for (int e = 0; e < 4; ++e) v[e] += p.beta * b[e];
                        }
                        if (p.epi.kind == 1) epi_mul_add(p, v, m, n);
                    }
                    const int byte = nl * EB2 / 2;
                    const int piece = (byte >> 4) ^ ((r >> RSH) & SWM);
                    if constexpr (OUT_FP4) {
                        uint32_t w = mx::cvt_fp4_pair<float>(0u, 0u, v[0], v[1], 1.0f, 0);
                        w = mx::cvt_fp4_pair<float>(w, 0u, v[2], v[3], 1.0f, 1);
                        *reinterpret_cast<uint16_t*>(cb + r * RB + piece * 16 + (byte & 15)) = (uint16_t)w;
                    } else if constexpr (OUT_F32) {
                        *reinterpret_cast<f32x4_t*>(cb + r * RB + piece * 16) = f32x4_t{v[0], v[1], v[2], v[3]};
                    } else {
                        *reinterpret_cast<u32x2_t*>(cb + r * RB + piece * 16 + (byte & 15)) =
                            u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                    }
                }
            }
        if constexpr (FENCED) __builtin_amdgcn_sched_barrier(0);
        // the scratch is the wave's own: its LDS accesses complete in order
#pragma unroll
        for (int rr = 0; rr < 32 * MP; rr += ROWS_PER) {
            const int r = rr + lane / P;
            const i32x4_t v = *reinterpret_cast<const i32x4_t*>(cb + r * RB + ((pc ^ ((r >> RSH) & SWM)) * 16));
            const int m = mb + (RM ? swap45(i0 * 32 + rr) : i0 * 32 + rr) + lrow2;
            if constexpr (EPI) {
                if (p.epi.kind == 2) {
                    if (m < p.M && n_out < p.N)
                        *reinterpret_cast<i32x4_t*>(epi_split_dst(p, m, n_out, EB2 / 2)) = v;
                    continue;
                }
            }
            const int off = col_off == 0x7fffffff ? col_off : m * (int)p.ldd * EB2 / 2 + col_off;
            __builtin_amdgcn_raw_buffer_store_b128(v, d_rsrc, off, 0, 0);
        }
    }
}

// the epilogue flavours picked at run time (uniform branch)
template <int MA, int NB, int MP, bool OUT_F32, int REMAP = 0>
AA_DEV void store_block_any(const GemmParams& p, f32x16v_t (&acc)[MA][NB], uint8_t* cb, int lane, int mb, int nb) {
    if (p.epi.kind)
        store_block<MA, NB, MP, false, true, OUT_F32, false, false, true, REMAP>(p, acc, cb, lane, mb, nb);
    else if (p.bias)
        store_block<MA, NB, MP, true, true, OUT_F32, false, false, false, REMAP>(p, acc, cb, lane, mb, nb);
    else if (p.alpha != 1.0f)
        store_block<MA, NB, MP, false, true, OUT_F32, false, false, false, REMAP>(p, acc, cb, lane, mb, nb);
    else
        store_block<MA, NB, MP, false, false, OUT_F32, false, false, false, REMAP>(p, acc, cb, lane, mb, nb);
}

}  // namespace aiter_amd
