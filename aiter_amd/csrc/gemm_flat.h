// Tile kernel with B read straight into registers ("flat" B), for tiles 256
// columns wide: MX (v_mfma_scale_f32_32x32x64_f8f6f4, e8m0 scales) and bf16
// (v_mfma_f32_32x32x16_bf16).  In bytes both have the same operand layout and
// the same preshuffled-B layout, so a stage is 128 bytes of every row either
// way (256 MX or 64 bf16 elements); bf16 simply has no scales.
//
// Why: aiter's preshuffled B (shuffle_weight (16,16)) stores every 16-row
// block so that one 16-byte load per lane is exactly the B operand of one
// 32x32x64 MFMA (rows l%32, bytes [16*(l/32), +16) of a 32-byte K window).
// B therefore needs no LDS staging: each wave loads its own 64 columns into
// VGPRs two 256-element stages ahead of use.  Only A (row-major, so it needs
// re-laying) and the e8m0 scales pass through LDS, in a ring of up to 4
// stages, which leaves up to 3 stages (~6000 MFMA cycles) to hide the
// global-memory latency of A.
//
// Work split: 4 waves side by side along N (1 x 4), wave w owns columns
// [64w, 64w+64) of the tile and every row, so no B byte is loaded twice and
// every wave reads the same A fragments from LDS.
//
// Per 256-element stage and workgroup:
//   A  : BM rows x 128 B (fp4) or 256 B (fp8), copied global -> LDS with
//        buffer_load ... lds in 1 KiB chunks of 8 rows x 128 B; 16-byte pieces
//        XOR-swizzled by row so the reads of one k-step are bank-conflict free;
//   B  : per wave 2 tiles x 4 k-steps of buffer_load_dwordx4 into VGPRs;
//   scales: 4 chunks of 4 groups x 256 B (A groups, then B groups), one
//        chunk per wave (a spare chunk is filled with zeros).
// Loads past the end of A, B or K go through range-checked buffer descriptors
// and return zeros, so the loop is a single basic block with no bounds
// branches (which keeps the accumulators in AGPRs); a stage past the end of K
// contributes exactly zero (zero operands, scale byte 0).
#pragma once
#include <type_traits>

#include "mfma32.h"

namespace aiter_amd {

template <int KA, int BM>
struct FlatCfg {
    static constexpr bool MX = KA != kBf16;
    static constexpr int FA = (KA == kFp8) ? 2 : 1;   // 128-byte halves of an A row per stage
    static constexpr int A_CH = (BM / 8) * FA;        // A chunks per stage
    static constexpr int STAGE_KB = A_CH + (MX ? 4 : 0);   // + 4 scale chunks (MX)
    static constexpr int NS = (160 / STAGE_KB) > 4 ? 4 : (160 / STAGE_KB);
    static constexpr int K_STAGE = MX ? 256 : 64;     // K elements per stage (128 bytes of a row)
};

// MoE stages (the two grouped GEMMs of fused_moe) on the same main loop.
// Row block b of the sorted routing list (see moe_sorting.hip) belongs to
// expert sorted_eids[b]: B and its scales are that expert's slices, and the
// A rows are gathered through sorted_ids (slot << 24 | token; padding entries
// point past the end of A, whose range check returns zeros).  A's scales are
// already in sorted order.  Stage 1 pairs gate and up rows of B in one tile
// (wave w: gate rows n0 + 32w.., up rows inter + n0 + 32w..), so one lane
// holds gate and up of the same output element and the epilogue writes
// act(gate) * up as bf16 to row token * topk + slot.  Stage 2 scales by the
// routing weight and adds into the token's output row with packed bf16
// atomics (the order of the topk additions is not fixed).
enum MoeStage : int { kMoeNone = 0, kMoeStage1 = 1, kMoeStage2 = 2 };
enum MoeAct : int { kActSilu = 0, kActGelu = 1 };

struct MoeParams {
    const int* sorted_ids;
    const int* sorted_eids;
    const int* num_valid;       // [0]: entries of the sorted list incl. padding
    const float* sorted_w;      // routing weight per sorted entry (null: 1)
    uint16_t* out;              // bf16
    int64_t out_stride;         // elements per output row
    int64_t b_expert_bytes;     // bytes of one expert's B / B scales
    int64_t bs_expert_bytes;
    int64_t a_rows;             // rows of A (gathered rows must stay below)
    int sorted_len;             // entries of sorted_ids (later positions are padding)
    int token_num, topk, inter, n_experts, act;
    int per_pair;               // stage 2: store rows token * topk + slot instead of adding into token rows
    int sort_bs;                // row block of the sort (a multiple of BM): expert of row r = sorted_eids[r / sort_bs]
    int k_splits;               // stage 1 split-K: > 1 -> raw f32 gate/up partials into GemmParams::ws
    int64_t ws_rows;            //   rows per split slice of ws (grid row blocks * BM)
    // split-K arrival counters, one per tile (row block * tiles_n + N tile),
    // zero before the launch (needed whenever k_splits > 1): the split that
    // arrives last sums the tile's partials in split order, applies weight,
    // activation (and the output quant) and sets its counter back to zero
    int* tile_cnt;
    // stage 1 with its output quantised in the epilogue (q_out null: bf16
    // rows into `out`): each act(gate) * up row, rounded to bf16 as the plain
    // store would, goes out as MXFP4 (RoundUp e8m0 from a running max of
    // 1e-10): 16 code bytes per 32-column block into row token * topk + slot
    // of q_out, the scale byte at the row's sorted position of the sorted,
    // shuffled scale layout; a zero q_w (sorted routing weight) gives a zero
    // block and byte, an invalid entry byte 0 (the sorted quantiser's rules)
    uint8_t* q_out;
    uint8_t* q_scale;
    const float* q_w;
    int64_t q_stride;           // bytes per q_out row
    int q_scale_n_pad;          // scale columns of the sorted layout (pad8 of inter / 32)
};

// The MXFP4 block of 32 bf16 values given as 16 element pairs (RoundUp,
// running max from 1e-10, the sorted quantiser's constants).
AA_DEV uint32_t moe_quant_block(const uint32_t (&raw)[16], i32x4_t& o) {
    float v[32];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        v[2 * i] = __builtin_bit_cast(float, raw[i] << 16);
        v[2 * i + 1] = __builtin_bit_cast(float, raw[i] & 0xffff0000u);
    }
    return mx::quant32_fp4<uint16_t, mx::kRoundUp>(v, raw, 1e-10f, 1.0f / 6.0f, 0.25f, 0u, 2u, o);
}

AA_DEV void atomic_add_bf16x2(uint16_t* addr, uint32_t v) {
    asm volatile("global_atomic_pk_add_bf16 %0, %1, off" : : "v"(addr), "v"(v) : "memory");
}

AA_DEV float moe_act(float g, int act) {
    if (act == kActGelu) return 0.5f * g * (1.0f + erff(g * 0.70710678118654752f));
    return g / (1.0f + __expf(-g));
}

// Stage-1 split-K sum of one item of a tile: sorted position pos (entry id,
// routing weight w), output columns c .. c+3.  The f32 gate / up partials of
// every split are loaded together (up to 8 splits in flight) and added in
// split order; then weight and act(gate) * up, rounded to bf16, go to row
// token * topk + slot, as bf16 or (q_out) as MXFP4.  With q_out the 8 items
// of one 32-column block must be 8 consecutive lanes (same pos, c = 32y + 4
// sub): they take the block's amax by lane exchange; each converts its 4
// values with the block's scale into 2 code bytes (the bytes quant32_fp4
// gives) and the first writes the scale byte.  Every exit is taken by all 8
// lanes of a block or none.
// Split-K partials are written and read in the agent-coherent form
// (kAgentCoherent), so the split that sums a tile sees what splits on other
// XCDs wrote; ws_rsrc covers the partials (byte offsets below 2^31).
template <bool QUANT>
AA_DEV void moe_fold_item(__amdgpu_buffer_rsrc_t ws_rsrc, int splits, const MoeParams& mq, int64_t pos, int id,
                          float w, int c) {
    const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
    const bool valid = tok < mq.token_num && slot < mq.topk;
    const int y = c / 32, sub = (c % 32) / 4;
    if constexpr (QUANT) {
        uint8_t* sc = mq.q_scale + mx::scale_shuffle_idx(mq.q_scale_n_pad, (int)pos, y);
        if (!valid) {
            if (sub == 0) *sc = 0;
            return;
        }
        if (mq.q_w && mq.q_w[pos] == 0.0f) {
            *reinterpret_cast<uint16_t*>(mq.q_out + ((int64_t)tok * mq.topk + slot) * mq.q_stride + y * 16 + 2 * sub) =
                0;
            if (sub == 0) *sc = 0;
            return;
        }
    } else {
        if (!valid) return;
    }
    f32x4_t g = {0.f, 0.f, 0.f, 0.f}, u = {0.f, 0.f, 0.f, 0.f};
    const int slice = (int)(mq.ws_rows * 2 * mq.inter * 4);      // bytes per split
    const int off = (int)((pos * 2 * mq.inter + c) * 4);
    for (int s0 = 0; s0 < splits; s0 += 8) {
        f32x4_t gb[8], ub[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (s0 + k < splits) {
                const int o = off + (s0 + k) * slice;
                gb[k] = __builtin_bit_cast(f32x4_t,
                                           __builtin_amdgcn_raw_buffer_load_b128(ws_rsrc, o, 0, kAgentCoherent));
                ub[k] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(ws_rsrc, o + mq.inter * 4,
                                                                                          0, kAgentCoherent));
            }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (s0 + k < splits) {
                g += gb[k];
                u += ub[k];
            }
    }
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = moe_act(g[r] * w, mq.act) * (u[r] * w);
    const uint32_t raw0 = pack_bf16x2(v[0], v[1]), raw1 = pack_bf16x2(v[2], v[3]);
    if constexpr (!QUANT) {
        *reinterpret_cast<uint2*>(mq.out + ((int64_t)tok * mq.topk + slot) * mq.out_stride + c) = uint2{raw0, raw1};
    } else {
        // the bf16 values the plain path stores, as f32
        const float b[4] = {__builtin_bit_cast(float, raw0 << 16), __builtin_bit_cast(float, raw0 & 0xffff0000u),
                            __builtin_bit_cast(float, raw1 << 16), __builtin_bit_cast(float, raw1 & 0xffff0000u)};
        float amax = 1e-10f;
#pragma unroll
        for (int r = 0; r < 4; ++r) amax = __builtin_fmaxf(amax, __builtin_fabsf(b[r]));
#pragma unroll
        for (int d = 1; d < 8; d <<= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, d));
        const uint32_t byte = mx::e8m0_byte<mx::kRoundUp>(amax, 1.0f / 6.0f, 0.25f, 0u, 2u);
        uint32_t wq = 0;
        if (byte != 0u && byte != 255u) {
            const float ds = __builtin_bit_cast(float, byte << 23);
            wq = mx::cvt_fp4_pair<uint16_t>(wq, raw0, 0.f, 0.f, ds, 0);
            wq = mx::cvt_fp4_pair<uint16_t>(wq, raw1, 0.f, 0.f, ds, 1);
        } else {
            const float inv = mx::inv_scale_from_byte(byte);
#pragma unroll
            for (int r = 0; r < 4; ++r) wq |= mx::f32_to_e2m1(b[r] * inv) << (4 * r);
        }
        *reinterpret_cast<uint16_t*>(mq.q_out + ((int64_t)tok * mq.topk + slot) * mq.q_stride + y * 16 + 2 * sub) =
            (uint16_t)wq;
        if (sub == 0) *(mq.q_scale + mx::scale_shuffle_idx(mq.q_scale_n_pad, (int)pos, y)) = (uint8_t)byte;
    }
}

// BPRE = false: B row-major [N, K].  The 32x32 MFMA's B operand is then 16
// contiguous bytes of one row per lane (row l%32, bytes 16*(l/32) of the
// k-step's 32-byte window), so row-major B also loads straight into VGPRs;
// one load touches 32 rows (32 bytes each), and the four k-steps of a stage
// consume each row's 128-byte line.
template <int KA, int BM, bool OUT_F32, bool BPRE, int MOE>
AA_DEV void flat_body(GemmParams p, const MoeParams& mq) {
    static_assert(MOE == kMoeNone || (BPRE && !OUT_F32), "MoE stages: preshuffled B, bf16 output");
    using Cfg = FlatCfg<KA, BM>;
    constexpr int BN = 256;
    constexpr int FA = Cfg::FA;
    constexpr int MA = BM / 32;           // 32-row A tiles per wave (all rows of the tile)
    constexpr int NB = 2;                 // 32-column B tiles per wave
    constexpr int A_CH = Cfg::A_CH;
    constexpr bool MX = Cfg::MX;
    constexpr int AG = BM / 32;           // A scale groups in the tile
    constexpr int SCA = (AG + 3) / 4;     // A scale chunks
    static_assert(SCA + 2 <= 4, "scale chunks: one per wave");
    static_assert(A_CH % 4 == 0, "A chunks split over 4 waves");
    constexpr int NA = A_CH / 4;          // A DMAs per wave per stage
    constexpr int NDMA = NA + (MX ? 1 : 0);   // + one scale chunk (MX)
    constexpr int NBL = NB * 4;           // B loads per wave per stage
    constexpr int STAGE_BYTES = Cfg::STAGE_KB * 1024;
    constexpr int A_ROW_BYTES = 128 * FA;
    // MX GEMM (not MoE): the paired tile layout of mfma32.h (swap45): MFMA
    // tile 2p+b takes rows 16b..16b+15 of the 32-row groups 2p and 2p+1, the
    // wave's B tile j columns 16j..16j+15 of its two 32-column groups, so each
    // tile's lanes share one scale byte (op_sel) and a tile pair one dword pair
    constexpr bool PAIRED = MX && MOE == kMoeNone;
    static_assert(!PAIRED || MA % 2 == 0, "tile pairs");
    // bf16 with row-major B (BLDS): B is copied global -> LDS in whole
    // 128-byte row lines (8 rows per copy, like A) into two wave-private 8 KiB
    // regions used in turn (stage t in region t % 2), and the MFMA operands
    // are read from there.  A direct operand load of row-major B touches 32
    // rows x 32 bytes per instruction and runs at a quarter of the full-line
    // rate in the memory pipeline.  The A ring gives the regions its fourth
    // slot (NS = 3 for BM = 256).
    constexpr bool BLDS = !MX && !BPRE && MOE == kMoeNone;
    constexpr int BPRIV = 8192;   // 64 rows x 128 B per wave
    constexpr int NPRIV = BLDS ? 2 : 0;
    constexpr int NS = (Cfg::NS * Cfg::STAGE_KB + 4 * NPRIV * BPRIV / 1024 <= 160)
                           ? Cfg::NS
                           : (160 - 4 * NPRIV * BPRIV / 1024) / Cfg::STAGE_KB;
    static_assert(NS >= (BLDS ? 3 : 2), "LDS ring depth");
    static_assert(NS * Cfg::STAGE_KB + 4 * NPRIV * BPRIV / 1024 <= 160, "ring + private B fit the LDS");

    __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * STAGE_BYTES + 4 * NPRIV * BPRIV];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;

    int tm, tn;
    int kt0 = 0;   // first K stage of this workgroup (MoE stage-1 split-K)
    const uint8_t* b_base = p.B;
    const uint8_t* bs_base = p.Bs;
    if constexpr (MOE != kMoeNone) {
        // 1-D grid, tiles in (row block, N tile) order with N fastest; the
        // workgroups of one row block (and the neighbouring blocks of the same
        // expert) share B, so consecutive tiles go to the same XCD (workgroup
        // ids are dealt round-robin over the 8 XCDs, each with its own L2)
        // (the host pads the grid to a multiple of 8; the extra ids leave)
        int bid = blockIdx.x;
        bid = (bid % 8) * (gridDim.x / 8) + bid / 8;
        if (bid >= p.tiles_n * p.tiles_m * ((MOE == kMoeStage1 && mq.k_splits > 1) ? mq.k_splits : 1)) return;
        if constexpr (MOE == kMoeStage1) {
            const int per_split = p.tiles_n * p.tiles_m;
            const int sp = bid / per_split;
            bid -= sp * per_split;
            kt0 = sp * p.k_steps_per_split;
        }
        tn = bid % p.tiles_n;
        tm = bid / p.tiles_n;
        if (tm * BM >= mq.num_valid[0]) return;   // whole workgroup: past the sorted list
        const int e = mq.sorted_eids[tm * BM / mq.sort_bs];
        if (e < 0 || e >= mq.n_experts) return;
        b_base += (int64_t)e * mq.b_expert_bytes;
        bs_base += (int64_t)e * mq.bs_expert_bytes;
    } else {
        apply_batch(p);
        tile_coords(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, tm, tn);
    }
    // stage 1: 128 output columns per tile (128 gate + 128 up rows of B)
    const int m0 = tm * BM, n0 = (MOE == kMoeStage1) ? tn * (BN / 2) : tn * BN;
    const int nstages = (MOE == kMoeStage1 && mq.k_splits > 1) ? min(p.k_steps_per_split, p.K / Cfg::K_STAGE - kt0)
                                                                : p.K / Cfg::K_STAGE;
    // MoE: the block's sorted entries and routing weights, one per lane
    // (registers 0 / 1 = rows 0-63 / 64-127), loaded once; later uses read
    // them with lane shuffles instead of a dependent global load per row
    constexpr int IDR = (BM + 63) / 64;
    int ids_r[IDR];
    float w_r[IDR];
    if constexpr (MOE != kMoeNone) {
#pragma unroll
        for (int k = 0; k < IDR; ++k) {
            const int pos = m0 + 64 * k + lane;
            const bool in = 64 * k + lane < BM && pos < mq.sorted_len;
            ids_r[k] = in ? mq.sorted_ids[pos] : mq.token_num;
            w_r[k] = (in && mq.sorted_w) ? mq.sorted_w[pos] : 1.0f;
        }
    }
    // entry of tile row r (any lane pattern; rows in one 64-row half when uniform)
    auto row_entry = [&](int r) -> int {
        const int lo = __shfl(ids_r[0], r & 63);
        return (IDR == 1 || r < 64) ? lo : __shfl(ids_r[IDR - 1], r & 63);
    };

    // ---- A: chunk c = half*(BM/8) + 8-row block; lane l -> row l/8, stored piece l%8
    //      holding global 16-byte piece (l%8) ^ swz(row), swz(r) = (r>>1)&7
    const __amdgpu_buffer_rsrc_t a_rsrc = (MOE != kMoeNone)
                                              ? make_rsrc(p.A, mq.a_rows * p.lda)
                                              : make_rsrc(p.A + (int64_t)m0 * p.lda, (int64_t)(p.M - m0) * p.lda);
    int a_off[NA];
#pragma unroll
    for (int q = 0; q < NA; ++q) {
        const int c = wave + 4 * q;
        const int half = c / (BM / 8), rb = c % (BM / 8);
        const int r = rb * 8 + (lane >> 3);
        int row = r;
        if constexpr (MOE != kMoeNone) {
            // A row of sorted entry m0 + r; padding -> a_rows (reads zeros)
            const int id = row_entry(r);
            const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
            row = (tok >= mq.token_num || slot >= mq.topk) ? (int)mq.a_rows
                                                           : (MOE == kMoeStage1 ? tok : tok * mq.topk + slot);
        }
        a_off[q] = row * (int)p.lda + half * 128 + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
    }
    // ---- B preshuffled (16,16): tile j of wave w = 16-row blocks 4w+2j, 4w+2j+1;
    //      k-step s of stage t at blk*16*ldb + (4t+s)*512 + (l/32)*256 + (l%16)*16
    //      B row-major: row 64w+32j+l%32 at (4t+s)*32 + (l/32)*16
    const __amdgpu_buffer_rsrc_t b_rsrc = (MOE != kMoeNone)
                                              ? make_rsrc(b_base, (int64_t)p.N * p.ldb)
                                              : make_rsrc(p.B + (int64_t)n0 * p.ldb, (int64_t)(p.N - n0) * p.ldb);
    int b_off[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        int blk = 4 * wave + (PAIRED ? 2 * ((lane >> 4) & 1) + j : 2 * j + ((lane >> 4) & 1));
        if constexpr (MOE == kMoeStage1) blk = ((j ? mq.inter : 0) + n0 + 32 * wave) / 16 + ((lane >> 4) & 1);
        if constexpr (MOE == kMoeStage2) blk += n0 / 16;
        if constexpr (BPRE)
            b_off[j] = blk * 16 * (int)p.ldb + (lane >> 5) * 256 + (lane & 15) * 16;
        else
            b_off[j] = (64 * wave + (PAIRED ? swap45(32 * j + (lane & 31)) : 32 * j + (lane & 31))) * (int)p.ldb +
                       (lane >> 5) * 16;
    }
    // BLDS: copy q = the wave's B rows 8q..8q+7 (lane: row 8q + l/8), lane l
    // fetching 16-byte piece (l%8) ^ swz(row) so that its granule 64q + l of
    // the region holds row r's piece p at r*128 + ((p ^ swz(r)) * 16), the
    // layout of the A copies (swz(r) = (r>>1)&7)
    int braw_off[BLDS ? 8 : 1];
    if constexpr (BLDS) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int r = 8 * q + (lane >> 3);
            braw_off[q] = (64 * wave + r) * (int)p.ldb + (((lane & 7) ^ ((r >> 1) & 7)) * 16);
        }
    }
    // ---- scales: wave w copies chunk w (A chunks first, then the 2 B chunks)
    const int ga0 = m0 / 32, gb0 = n0 / 32;
    const __amdgpu_buffer_rsrc_t sa_rsrc =
        make_rsrc(p.As + (int64_t)ga0 * 32 * p.sa_stride, (int64_t)(p.sa_groups - ga0) * 32 * p.sa_stride);
    const __amdgpu_buffer_rsrc_t sb_rsrc =
        (MOE != kMoeNone)
            ? make_rsrc(bs_base, (int64_t)p.sb_groups * 32 * p.sb_stride)
            : make_rsrc(p.Bs + (int64_t)gb0 * 32 * p.sb_stride, (int64_t)(p.sb_groups - gb0) * 32 * p.sb_stride);
    const __amdgpu_buffer_rsrc_t null_rsrc = make_rsrc(p.A, 0);
    const bool sc_is_a = wave < SCA;
    const bool sc_is_b = wave >= SCA && wave < SCA + 2;
    const int sc_chunk = sc_is_a ? wave : (sc_is_b ? wave - SCA : 0);
    int sc_group = 4 * sc_chunk + (lane >> 4);
    if constexpr (MOE == kMoeStage1) {
        if (sc_is_b) sc_group = (sc_chunk ? mq.inter / 32 : 0) + gb0 + (lane >> 4);   // chunk 0 gate, 1 up
    }
    if constexpr (MOE == kMoeStage2) {
        if (sc_is_b) sc_group += gb0;
    }
    // paired: the chunk image of sc_pair_group / sc_pair_granule
    int sc_gran = lane & 15;
    if constexpr (PAIRED) {
        sc_group = 4 * sc_chunk + sc_pair_group(lane);
        sc_gran = sc_pair_granule(lane);
    }
    const int sc_off = sc_group * 32 * (int)(sc_is_b ? p.sb_stride : p.sa_stride) + sc_gran * 16;
    const __amdgpu_buffer_rsrc_t sc_rsrc = sc_is_a ? sa_rsrc : (sc_is_b ? sb_rsrc : null_rsrc);

    auto dma_stage = [&](int t) {
        const bool live = t < nstages;
        const __amdgpu_buffer_rsrc_t ra = live ? a_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rs = live ? sc_rsrc : null_rsrc;
        uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int q = 0; q < NA; ++q) dma16(ra, base + (wave + 4 * q) * 1024, a_off[q], (kt0 + t) * A_ROW_BYTES);
        if constexpr (MX) dma16(rs, base + (A_CH + wave) * 1024, sc_off, (kt0 + t) * 256);
    };
    auto load_b = [&](int t, int j, int s) -> i32x4_t {
        const __amdgpu_buffer_rsrc_t rb = t < nstages ? b_rsrc : null_rsrc;
        return __builtin_amdgcn_raw_buffer_load_b128(rb, b_off[j] + s * (BPRE ? 512 : 32),
                                                     (kt0 + t) * (BPRE ? 2048 : 128), 0);
    };

    const int pos0 = PAIRED ? sc_pair_read_off(lane) : ((lane & 15) + 16 * (lane >> 5)) * 4;
    // per group, lane l needs bytes h and 2+h (h = (l>>4)&1) of the window's
    // two scale dwords d0 (k-steps 0, 2) and d1 (k-steps 1, 3); v_perm packs
    // them as [d0.h, d0.(2+h), d1.h, d1.(2+h)] so that k-step s takes byte
    // {0, 2, 1, 3}[s] through the MFMA's op_sel, the same for every lane
    const unsigned sc_perm = 0x06040200u + ((lane >> 4) & 1) * 0x01010101u;

    f32x16v_t acc[MA][NB];
#pragma unroll
    for (int i = 0; i < MA; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x16v_t{};

    i32x4_t af[2][MA][FA];
    i32x4_t bq[2][NB][4];          // [stage parity][tile][k-step]
    i32x4_t bfr[2][NB];            // BLDS: operands of the current / next k-step
    int sa_pk[MA] = {}, sb_pk[NB] = {};   // packed scale bytes of the stage being multiplied

    const int ar = lane & 31;
    // paired: MFMA row ar of tile 2p+b is in 8-row chunk 8p + 2b + 4(ar>>4) + ((ar>>3)&1)
    const int a_lane_off = PAIRED ? (4 * ((ar >> 4) & 1) + ((ar >> 3) & 1)) * 1024 + (ar & 7) * 128
                                  : (ar >> 3) * 1024 + (ar & 7) * 128;
    const int a_swz = (ar >> 1) & 7;
    auto read_a = [&](int t, int s, int slot) {
        const uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int h = 0; h < FA; ++h) {
                const int piece = (FA == 1) ? (2 * s + (lane >> 5)) : ((4 * s + 2 * h + (lane >> 5)) & 7);
                const int hh = (FA == 1) ? 0 : ((4 * s + 2 * h) >> 3);
                af[slot][i][h] = *reinterpret_cast<const i32x4_t*>(
                    base + (hh * (BM / 8) + (PAIRED ? (i >> 1) * 8 + (i & 1) * 2 : i * 4)) * 1024 + a_lane_off +
                    ((piece ^ a_swz) * 16));
            }
    };
    auto read_scales = [&](int t, int (&pa)[MA], int (&pb)[NB]) {
        if constexpr (!MX) return;
        const uint8_t* base = smem + (t % NS) * STAGE_BYTES + A_CH * 1024 + pos0;
        if constexpr (PAIRED) {
            // pair q: d0 (k-steps 0, 2) and d1 (1, 3) -> pa[2q], pa[2q+1]; B: the wave's pair
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
            const int bg = (MOE == kMoeStage1) ? 4 * j + wave : 2 * wave + j;
            const uint8_t* g = base + SCA * 1024 + bg * 256;
            const unsigned d0 = *reinterpret_cast<const unsigned*>(g);
            const unsigned d1 = *reinterpret_cast<const unsigned*>(g + 128);
            pb[j] = (int)__builtin_amdgcn_perm(d1, d0, sc_perm);
        }
    };
    // k-step S of the stage; scale byte {0, 2, 1, 3}[S] of the packed scales
    auto mma = [&](int aslot, int bpar, auto sel, const int (&pa)[MA], const int (&pb)[NB]) {
        constexpr int s = decltype(sel)::value;
        constexpr int osel = (s == 0) ? 0 : (s == 1) ? 2 : (s == 2) ? 1 : 3;
        if constexpr (PAIRED) {
            // tile 2q+b: byte b + 2(s/2) of dword d(s%2) of pair q (B: tile j, byte j + 2(s/2))
            constexpr int o = 2 * (s >> 1);
#pragma unroll
            for (int i = 0; i < MA; ++i) {
                const int sa = pa[2 * (i >> 1) + (s & 1)], sb = pb[s & 1];
                const i32x4_t &a0 = af[aslot][i][0], &a1 = af[aslot][i][FA - 1];
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
                    acc[i][j] = mma32<KA, osel>(BLDS ? bfr[s & 1][j] : bq[bpar][j][s], af[aslot][i][0],
                                                af[aslot][i][FA - 1], acc[i][j], pa[i], pb[j]);
        }
    };
    // B of stage t+2, k-step s, into the registers k-step s of stage t just used
    auto prefetch_b = [&](int t, int bpar, int s) {
#pragma unroll
        for (int j = 0; j < NB; ++j) bq[bpar][j][s] = load_b(t + 2, j, s);
    };
    // BLDS: the operand of k-step s (tile j: rows 32j + l%32, piece 2s +
    // l/32) of a stage of parity par into bfr[slot]
    uint8_t* const bpriv0 = smem + NS * STAGE_BYTES + wave * BPRIV;         // even stages
    uint8_t* const bpriv1 = smem + NS * STAGE_BYTES + (4 + wave) * BPRIV;   // odd stages
    auto read_bfr = [&](int s, int slot, int par) {
        const uint8_t* reg = par ? bpriv1 : bpriv0;
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int rr = 32 * j + (lane & 31);
            bfr[slot][j] = *reinterpret_cast<const i32x4_t*>(reg + rr * 128 + (((2 * s + (lane >> 5)) ^ a_swz) * 16));
        }
    };
    // BLDS: the copies of B stage t (8 rows x 128 B each) into its region
    auto dma_b = [&](int t, int q0, int q1) {
        const __amdgpu_buffer_rsrc_t r = t < nstages ? b_rsrc : null_rsrc;
        uint8_t* reg = (t & 1) ? bpriv1 : bpriv0;
#pragma unroll
        for (int q = q0; q < q1; ++q) dma16(r, reg + q * 1024, braw_off[q], (kt0 + t) * 128);
    };

    // Each k-step is its own scheduling region (sched_barrier fences): the LDS
    // reads of the next k-step, this k-step's MFMAs, a third of the next-but-two
    // stage's A copies and the B loads of stage t+2 into the registers this
    // k-step has just consumed.  The LDS reads therefore have a whole k-step
    // (16 MFMAs) of latency budget and the compiler's lgkmcnt waits never stall.
    constexpr int DMA_PART = (NDMA + 2) / 3;
    auto dma_part = [&](int t, int part) {
        const bool live = t < nstages;
        const __amdgpu_buffer_rsrc_t ra = live ? a_rsrc : null_rsrc;
        const __amdgpu_buffer_rsrc_t rs = live ? sc_rsrc : null_rsrc;
        uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int q = part * DMA_PART; q < (part + 1) * DMA_PART && q < NDMA; ++q) {
            if (q < NA) dma16(ra, base + (wave + 4 * q) * 1024, a_off[q], (kt0 + t) * A_ROW_BYTES);
            else dma16(rs, base + (A_CH + wave) * 1024, sc_off, (kt0 + t) * 256);
        }
    };
    // BLDS issue order per stage: the A copies in k-steps 1 and 2 (D3, then
    // the rest), the B copies in k-step 3
    constexpr int D3 = (NDMA + 1) / 2;
    auto dma_half = [&](int t, int h) {
        const bool live = t < nstages;
        const __amdgpu_buffer_rsrc_t ra = live ? a_rsrc : null_rsrc;
        uint8_t* base = smem + (t % NS) * STAGE_BYTES;
#pragma unroll
        for (int q = h * D3; q < (h ? NDMA : D3); ++q)
            dma16(ra, base + (wave + 4 * q) * 1024, a_off[q], (kt0 + t) * A_ROW_BYTES);
    };
    // loads issued after the last A copy of stage t+1 and before the wait at
    // the end of iteration t (all of them from later iterations): the loads of
    // NS-3 whole stages, then those of stage t before its wait
    constexpr int LOADS_ITER = NDMA + NBL;
    // BLDS: the copies of B stage t+1 go out in k-step 3 of stage t-1, and
    // after them only the A copies of stage t+NS-1 (k-steps 1, 2 of stage t)
    // before the wait that publishes stage t+1: WAIT_N = NDMA
    constexpr int PRE_WAIT = BLDS ? NDMA : NDMA + 3 * NB;
    constexpr int WAIT_N = BLDS ? NDMA : (NS >= 3 ? (NS - 3) * LOADS_ITER + PRE_WAIT : 0);
    static_assert(WAIT_N < 64, "vmcnt range");
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    // order inside a k-step region: one LDS read after each of the first RD
    // MFMAs, the region's global loads after the last MFMAs
    constexpr int RD = MA * FA;
    constexpr int MF = MA * NB;
    auto pace2 = [&](int ds, int vmem) {
#pragma unroll
        for (int k = 0; k < MF; ++k) {
            if (k < ds) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);           // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                       // MFMA
            if (k >= MF - vmem) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // VMEM
        }
    };
    auto pace = [&](int vmem) { pace2(RD, vmem); };

    // stage t of the main loop; bpar = t & 1 selects the B registers
    auto stage = [&](int t, int bpar) {
        using S0 = std::integral_constant<int, 0>;
        using S1 = std::integral_constant<int, 1>;
        using S2 = std::integral_constant<int, 2>;
        using S3 = std::integral_constant<int, 3>;
        if constexpr (BLDS) {
            // k-steps 1, 2: the A copies of stage t+NS-1 (NS = 3: t+2);
            // k-step 3, after the barrier: the B copies of stage t+2 into the
            // region of stage t, whose last operand read (k-step 3's, issued
            // in k-step 2) the wait before the barrier has completed.
            // (Loading B into registers two stages ahead and writing it to
            // one region with ds_write instead, with a 4-slot A ring,
            // measured 3-5% slower on the large bf16 shapes.)
            read_a(t, 1, 1);
            read_bfr(1, 1, bpar);
            mma(0, bpar, S0{}, sa_pk, sb_pk);
            pace2(RD + NB, 0);
            fence();
            read_a(t, 2, 0);
            read_bfr(2, 0, bpar);
            dma_half(t + NS - 1, 0);
            mma(1, bpar, S1{}, sa_pk, sb_pk);
            pace2(RD + NB, D3);
            fence();
            read_a(t, 3, 1);
            read_bfr(3, 1, bpar);
            dma_half(t + NS - 1, 1);
            mma(0, bpar, S2{}, sa_pk, sb_pk);
            pace2(RD + NB, NDMA - D3);
            fence();
            wait_vmcnt_lgkm0<WAIT_N>();
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            fence();
            read_a(t + 1, 0, 0);
            read_bfr(0, 0, bpar ^ 1);
            dma_b(t + 2, 0, 8);
            mma(1, bpar, S3{}, sa_pk, sb_pk);
            pace2(RD + NB, NBL);
            fence();
            return;
        }
        read_a(t, 1, 1);
        dma_part(t + NS - 1, 0);
        mma(0, bpar, S0{}, sa_pk, sb_pk);
        prefetch_b(t, bpar, 0);
        pace(NB + DMA_PART);
        fence();
        read_a(t, 2, 0);
        dma_part(t + NS - 1, 1);
        mma(1, bpar, S1{}, sa_pk, sb_pk);
        prefetch_b(t, bpar, 1);
        pace(NB + DMA_PART);
        fence();
        read_a(t, 3, 1);
        dma_part(t + NS - 1, 2);
        mma(0, bpar, S2{}, sa_pk, sb_pk);
        prefetch_b(t, bpar, 2);
        pace(NB + NDMA - 2 * DMA_PART);
        fence();
        // stage t+1 published: own copies landed and own LDS reads of stage t
        // done (waitcnt), then everyone's (barrier).  No workgroup memory fence:
        // it would also wait for the copies of later stages still in flight.
        wait_vmcnt_lgkm0<WAIT_N>();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        fence();
        read_a(t + 1, 0, 0);
        int na[MA], nb[NB];
        read_scales(t + 1, na, nb);
        mma(1, bpar, S3{}, sa_pk, sb_pk);
        prefetch_b(t, bpar, 3);
        if constexpr (MX) {
#pragma unroll
            for (int i = 0; i < MA; ++i) sa_pk[i] = na[i];
#pragma unroll
            for (int j = 0; j < NB; ++j) sb_pk[j] = nb[j];
        }
        pace(NB);
        fence();
    };

    // prologue: B stages 0, 1 first (BLDS: copies), then A stages 0..NS-2 (so that at the loop
    // head at least as many loads follow each B load as in the steady state,
    // and the compiler's B waits there stay as loose as in the loop).
    // The wait at the end of stage t (vmcnt WAIT_N) publishes the copies of
    // stage t+1 only if at least WAIT_N loads were issued after them.  For a
    // copy issued here (stage t+1 <= NS-2) that is (NS-3-t)*NDMA later
    // prologue copies + t whole stages + the loads of stage t before its wait
    // (PRE_WAIT), fewer than WAIT_N for the first stages of a 4-slot ring.  Those copies are waited for here, with stage 0's: they
    // were issued right after it.
    constexpr int PRO_WAITED = [] {
        int d = 0;
        for (int t = 0; t + 1 <= NS - 2; ++t)
            if ((NS - 3 - t) * NDMA + t * LOADS_ITER + PRE_WAIT < WAIT_N) d = t + 1;
        return d;
    }();
    if constexpr (BLDS) {
        dma_b(0, 0, 8);
        dma_b(1, 0, 8);
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < NB; ++j) bq[0][j][s] = load_b(0, j, s);
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < NB; ++j) bq[1][j][s] = load_b(1, j, s);
    }
#pragma unroll
    for (int t = 0; t < NS - 1; ++t) dma_stage(t);
    __builtin_amdgcn_sched_barrier(0);
    wait_vmcnt<(NS - 2 - PRO_WAITED) * NDMA>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    read_scales(0, sa_pk, sb_pk);
    read_a(0, 0, 0);
    if constexpr (BLDS) read_bfr(0, 0, 0);

    // the loop runs an even number of stages; an odd last stage is a zero stage
    for (int t = 0; t < nstages; t += 2) {
        stage(t, 0);
        stage(t + 1, 1);
    }

    // ---- epilogue through LDS (the ring is free once every copy has landed)
    constexpr int EB = OUT_F32 ? 4 : 2;
    constexpr int WAVE_SCRATCH = NS * STAGE_BYTES / 4;
    // row tiles per epilogue pass: the most whose bytes fit the wave's scratch
    constexpr int EP_MP = (MA * 32 * 64 * EB <= WAVE_SCRATCH)         ? MA
                          : ((MA / 2) * 32 * 64 * EB <= WAVE_SCRATCH) ? MA / 2
                                                                      : MA / 4;
    static_assert(MA % EP_MP == 0 && EP_MP * 32 * 64 * EB <= WAVE_SCRATCH, "epilogue pass fits the ring");
    wait_vmcnt<0>();
    if constexpr (MOE == kMoeStage1) {
        if (mq.k_splits > 1) {
            // raw f32 gate / up partials [split][ws_rows][2 * inter]; the split
            // that finishes the tile last sums them and applies weight and activation
            // (rows of padding entries are never read: not stored)
            const __amdgpu_buffer_rsrc_t ws_rsrc = make_rsrc(p.ws, 0x7ffffff0LL);
            const int wsb = (int)((kt0 / p.k_steps_per_split) * mq.ws_rows * (2 * mq.inter));   // floats
            auto entry_of = [&](int r) -> int {   // any lane pattern
                const int lo = __shfl(ids_r[0], r & 63), hi = __shfl(ids_r[IDR - 1], r & 63);
                return r < 64 ? lo : hi;
            };
#pragma unroll
            for (int i = 0; i < MA; ++i) {
                const int id = entry_of(32 * i + (lane & 31));
                const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
                if (tok >= mq.token_num || slot >= mq.topk) continue;
                const int wrow = wsb + (m0 + 32 * i + (lane & 31)) * (2 * mq.inter) + n0 + 32 * wave + 4 * (lane >> 5);
#pragma unroll
                for (int j = 0; j < NB; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x16v_t& a = acc[i][j];
                        __builtin_amdgcn_raw_buffer_store_b128(
                            __builtin_bit_cast(i32x4_t, f32x4_t{a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]}),
                            ws_rsrc, (wrow + (j ? mq.inter : 0) + 8 * q) * 4, 0, kAgentCoherent);
                    }
            }
            // arrival: every thread's partial stores have reached memory before
            // the tile's counter is incremented
            wait_vmcnt<0>();
            __syncthreads();
            int* flag = reinterpret_cast<int*>(smem);   // the ring is idle
            if (threadIdx.x == 0) {
                int* cnt = mq.tile_cnt + (int64_t)tm * p.tiles_n + tn;
                const int last = atomicAdd(cnt, 1) == mq.k_splits - 1;
                if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                *flag = last;
            }
            __syncthreads();
            if (!*flag) return;
            // the last split sums the tile: rows m0 .., output columns n0 .. n0 + BN/2
            // (entries and weights from the registers loaded at the start)
            constexpr int IPR = BN / 8;   // items per row, 4 columns each
            for (int it = threadIdx.x; it < BM * IPR; it += 256) {
                const int row = it / IPR;
                const int id = entry_of(row);
                const float wl = __shfl(w_r[0], row & 63), wh = __shfl(w_r[IDR - 1], row & 63);
                const float wgt = row < 64 ? wl : wh;
                const int c = n0 + 4 * (it % IPR);
                if (mq.q_out)
                    moe_fold_item<true>(ws_rsrc, mq.k_splits, mq, m0 + row, id, wgt, c);
                else
                    moe_fold_item<false>(ws_rsrc, mq.k_splits, mq, m0 + row, id, wgt, c);
            }
            return;
        }
    }
    if constexpr (MOE != kMoeNone) {
        // Through LDS, so that every store / atomic instruction covers whole
        // output rows instead of one 8-byte piece of 32 rows: the tile goes to
        // the (now idle) ring as [BM][OC] bf16 (OC = 128 for stage 1, act(gate) *
        // up, or 256 for stage 2), 8-byte chunks XOR-swizzled by row; then
        // stage 1 stores two 256-byte rows per instruction and stage 2 adds
        // one 512-byte row per pair of packed-bf16 atomics.
        constexpr int OC = (MOE == kMoeStage1) ? 128 : 256;
        static_assert(BM * OC * 2 <= NS * STAGE_BYTES, "epilogue tile fits the ring");
        auto chunk = [&](int row, int c) -> uint2* {
            return reinterpret_cast<uint2*>(smem + row * (OC * 2) + ((c ^ (row & 31)) * 8));
        };
        __syncthreads();
#pragma unroll
        for (int i = 0; i < MA; ++i) {
            // lane: row 32i + l%32 of the tile, columns 8q + 4(l/32) + r of each 32-column tile
            const int row = 32 * i + (lane & 31);
            const float wgt = __shfl(w_r[i / 2], row & 63);
            if constexpr (MOE == kMoeStage1) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v[4];
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        v[r] = moe_act(acc[i][0][4 * q + r] * wgt, mq.act) * (acc[i][1][4 * q + r] * wgt);
                    *chunk(row, 8 * wave + 2 * q + (lane >> 5)) = uint2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                }
            } else {
#pragma unroll
                for (int j = 0; j < NB; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x16v_t& a = acc[i][j];
                        *chunk(row, 16 * wave + 8 * j + 2 * q + (lane >> 5)) =
                            uint2{pack_bf16x2(a[4 * q] * wgt, a[4 * q + 1] * wgt),
                                  pack_bf16x2(a[4 * q + 2] * wgt, a[4 * q + 3] * wgt)};
                    }
            }
        }
        __syncthreads();
        if constexpr (MOE == kMoeStage1) {
            if (mq.q_out) {
                // fused output quant: (row, 32-column block) items of the tile
                for (int it = threadIdx.x; it < BM * 4; it += 256) {
                    const int row = it >> 2, yb = it & 3;
                    const int pos = m0 + row;
                    if (pos >= mq.sorted_len) continue;
                    const int id = mq.sorted_ids[pos];
                    const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
                    const int y = n0 / 32 + yb;
                    uint8_t* sc = mq.q_scale + mx::scale_shuffle_idx(mq.q_scale_n_pad, pos, y);
                    if (tok >= mq.token_num || slot >= mq.topk) {
                        *sc = 0;
                        continue;
                    }
                    i32x4_t o = {0, 0, 0, 0};
                    uint32_t byte = 0;
                    if (!(mq.q_w && mq.q_w[pos] == 0.0f)) {
                        uint32_t raw[16];
#pragma unroll
                        for (int k = 0; k < 8; ++k) {
                            const uint2 c = *chunk(row, 8 * yb + k);
                            raw[2 * k] = c.x;
                            raw[2 * k + 1] = c.y;
                        }
                        byte = moe_quant_block(raw, o);
                    }
                    *reinterpret_cast<i32x4_t*>(mq.q_out + ((int64_t)tok * mq.topk + slot) * mq.q_stride + y * 16) = o;
                    *sc = (uint8_t)byte;
                }
                return;
            }
            // lane l: row r0 + l/32, columns 4(l%32) .. +3
            for (int r0 = 2 * wave; r0 < BM; r0 += 8) {
                const int row = r0 + (lane >> 5);
                const int id = __shfl((IDR == 1 || r0 < 64) ? ids_r[0] : ids_r[IDR - 1], row & 63);
                const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
                if (tok >= mq.token_num || slot >= mq.topk) continue;
                *reinterpret_cast<uint2*>(mq.out + ((int64_t)tok * mq.topk + slot) * mq.out_stride + n0 +
                                          4 * (lane & 31)) = *chunk(row, lane & 31);
            }
        } else {
            // one row per iteration (uniform over the wave); lane l: columns 4l .. 4l+3
            for (int row = wave; row < BM; row += 4) {
                const int id = __builtin_amdgcn_readlane((IDR == 1 || row < 64) ? ids_r[0] : ids_r[IDR - 1], row & 63);
                const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
                if (tok >= mq.token_num || slot >= mq.topk) continue;
                const uint2 v = *chunk(row, lane);
                if (mq.per_pair) {
                    // per-pair rows, summed over the slots afterwards (moe_sum): no atomics
                    *reinterpret_cast<uint2*>(mq.out + ((int64_t)tok * mq.topk + slot) * mq.out_stride + n0 +
                                              4 * lane) = v;
                } else {
                    uint16_t* o = mq.out + (int64_t)tok * mq.out_stride + n0 + 4 * lane;
                    atomic_add_bf16x2(o, v.x);
                    atomic_add_bf16x2(o + 2, v.y);
                }
            }
        }
        return;
    }
    __syncthreads();
    store_block_any<MA, NB, EP_MP, OUT_F32, PAIRED ? 3 : 0>(p, acc, smem + wave * WAVE_SCRATCH, lane, m0, n0 + wave * 64);
}

template <int KA, int BM, bool OUT_F32, bool BPRE = true>
__global__ __launch_bounds__(256, 1) void gemm_flat_kernel(GemmParams p) {
    flat_body<KA, BM, OUT_F32, BPRE, kMoeNone>(p, MoeParams{});
}

template <int KA, int BM, int MOE>
__global__ __launch_bounds__(256, 1) void moe_flat_kernel(GemmParams p, MoeParams mq) {
    flat_body<KA, BM, false, true, MOE>(p, mq);
}

}  // namespace aiter_amd
