// MoE stage 2 (down projection) for short K (K = inter_dim of 256 or 512): the
// row block's A fragments stay in registers and the workgroup streams a group
// of N tiles of its expert's w2, loading the next window of B while the MFMAs
// of the current one run.
//
// Why a second kernel: with K = 256 the flat tile kernel does one K stage per
// workgroup, so its time is the pipeline's fill and drain and the epilogue's
// barriers, and one workgroup in flight per CU cannot hide them (measured:
// about 8 us per 64 x 256 tile).  Here a workgroup loads A once (straight to
// registers: the MFMA operand layout of a row-major A row is 16 contiguous
// bytes per lane, so no LDS re-layout is needed) and then only streams B and
// stores output, with no barriers at all (the epilogue's LDS tile is private
// to each wave).
//
// Layout per wave (4 waves side by side over the 256 columns of an N tile):
// rows 0..BM of the row block (MA = BM / 32 MFMA tiles), columns 64w..64w+63
// (NB = 2 tiles).  Output: per-pair rows token * topk + slot (plain stores)
// or token rows (packed-bf16 atomics), scaled by the routing weight.
#pragma once
#include "gemm_flat.h"

namespace aiter_amd {

struct MoeS2Params {
    int tiles_per_group;   // N tiles per workgroup
    int groups;            // N-tile groups per row block
    int row_blocks;        // row blocks in the grid
    int64_t a_scale_rows;  // rows of the sorted A-scale buffer
};

template <int KA, int BM, int KW>
__global__ __launch_bounds__(256, 2) void moe_stage2_stream_kernel(GemmParams p, MoeParams mq, MoeS2Params sp) {
    constexpr int MA = BM / 32, NB = 2;
    constexpr int FA = (KA == kFp8) ? 2 : 1;    // 16-byte A pieces per lane and k-step
    constexpr int KS = KW * 4;                  // k-steps (64 elements each); KW 256-element windows
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
    const int h = lane >> 5;
    __shared__ __attribute__((aligned(16))) uint8_t ep_all[4][BM * 128];
    uint8_t* ep = ep_all[wave];   // this wave's epilogue tile

    // ---- workgroup -> (row block, N-tile group), XCD-ordered like the flat kernel
    int bid = blockIdx.x;
    bid = (bid % 8) * (gridDim.x / 8) + bid / 8;
    if (bid >= sp.row_blocks * sp.groups) return;
    const int tm = bid / sp.groups, gn = bid % sp.groups;
    const int m0 = tm * BM;
    if (m0 >= mq.num_valid[0]) return;
    const int e = mq.sorted_eids[m0 / mq.sort_bs];
    if (e < 0 || e >= mq.n_experts) return;
    const int tn0 = gn * sp.tiles_per_group;
    const int tn1 = min(tn0 + sp.tiles_per_group, p.tiles_n);

    // ---- the block's sorted entries / weights, one per lane
    constexpr int IDR = (BM + 63) / 64;
    int ids_r[IDR];
    float w_r[IDR];
#pragma unroll
    for (int k = 0; k < IDR; ++k) {
        const int pos = m0 + 64 * k + lane;
        const bool in = 64 * k + lane < BM && pos < mq.sorted_len;
        ids_r[k] = in ? mq.sorted_ids[pos] : mq.token_num;
        w_r[k] = (in && mq.sorted_w) ? mq.sorted_w[pos] : 1.0f;
    }

    // ---- A: row 32i + l%32 of the block, k-step s: bytes [32s (fp4) / 64s (fp8) + 16h, +16)
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(p.A, mq.a_rows * p.lda);
    i32x4_t af[MA][KS][FA];
    int sa[MA][KW];
#pragma unroll
    for (int i = 0; i < MA; ++i) {
        const int r = 32 * i + (lane & 31);
        const int id = __shfl(ids_r[i / 2], r & 63);
        const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
        const int row = (tok >= mq.token_num || slot >= mq.topk) ? (int)mq.a_rows : tok * mq.topk + slot;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int f = 0; f < FA; ++f)
                af[i][s][f] = __builtin_amdgcn_raw_buffer_load_b128(
                    a_rsrc, row * (int)p.lda + s * 32 * FA + 32 * f + 16 * h, 0, 0);
        // scale bytes of blocks 8w + 2s + h, s = 0..3, packed as byte s
        const int64_t x = m0 + r;
#pragma unroll
        for (int w = 0; w < KW; ++w) {
            uint32_t v = 0;
            if (x < sp.a_scale_rows) {
#pragma unroll
                for (int s = 0; s < 4; ++s)
                    v |= (uint32_t)p.As[(x / 32 * p.sa_stride) * 32 + w * 256 + ((2 * s + h) % 4) * 64 + (x % 16) * 4 +
                                        ((2 * s + h) % 8) / 4 * 2 + (x % 32) / 16]
                         << (8 * s);
            }
            sa[i][w] = (int)v;
        }
    }

    // ---- B of tile tn, window w: preshuffled (16, 16) rows 256 tn + 64 wave + 32 j + l%32
    const uint8_t* b_base = p.B + (int64_t)e * mq.b_expert_bytes;
    const uint8_t* bs_base = p.Bs + (int64_t)e * mq.bs_expert_bytes;
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(b_base, (int64_t)p.N * p.ldb);
    auto load_b = [&](int tn, int w, i32x4_t (&bq)[NB][4], int (&sb)[NB]) {
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int blk = (256 * tn) / 16 + 4 * wave + 2 * j + ((lane >> 4) & 1);
            const int off = blk * 16 * (int)p.ldb + h * 256 + (lane & 15) * 16;
#pragma unroll
            for (int s = 0; s < 4; ++s) bq[j][s] = __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, off + s * 512, w * 2048, 0);
            const int xn = 256 * tn + 64 * wave + 32 * j + (lane & 31);
            uint32_t v = 0;
#pragma unroll
            for (int s = 0; s < 4; ++s)
                v |= (uint32_t)bs_base[(xn / 32 * p.sb_stride) * 32 + w * 256 + ((2 * s + h) % 4) * 64 + (xn % 16) * 4 +
                                       ((2 * s + h) % 8) / 4 * 2 + (xn % 32) / 16]
                     << (8 * s);
            sb[j] = (int)v;
        }
    };

    auto mma_window = [&](int w, const i32x4_t (&bq)[NB][4], const int (&sb)[NB], f32x16v_t (&acc)[MA][NB]) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < MA; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    const i32x4_t& a0 = af[i][4 * w + s][0];
                    const i32x4_t& a1 = af[i][4 * w + s][FA - 1];
                    if (s == 0) acc[i][j] = mma32<KA, 0>(bq[j][s], a0, a1, acc[i][j], sa[i][w], sb[j]);
                    if (s == 1) acc[i][j] = mma32<KA, 1>(bq[j][s], a0, a1, acc[i][j], sa[i][w], sb[j]);
                    if (s == 2) acc[i][j] = mma32<KA, 2>(bq[j][s], a0, a1, acc[i][j], sa[i][w], sb[j]);
                    if (s == 3) acc[i][j] = mma32<KA, 3>(bq[j][s], a0, a1, acc[i][j], sa[i][w], sb[j]);
                }
    };

    // ---- stream (tile, window) pairs with one pair of B in flight ahead; the
    // buffer parity of every window is a compile-time constant (windows
    // unrolled per tile; with one window per tile, tiles go in pairs)
    i32x4_t bq[2][NB][4];
    int sbk[2][NB];
    load_b(tn0, 0, bq[0], sbk[0]);
    auto do_tile = [&](int tn, auto first_buf) {
        constexpr int P = decltype(first_buf)::value;   // buffer holding (tn, window 0)
        f32x16v_t acc[MA][NB];
#pragma unroll
        for (int i = 0; i < MA; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) acc[i][j] = f32x16v_t{};
        static_for<KW>([&](auto wc) {
            constexpr int w = decltype(wc)::value;
            constexpr int cur = (P + w) & 1;
            const int nt = (w + 1 < KW) ? tn : tn + 1;
            if (nt < tn1) load_b(nt, (w + 1 < KW) ? w + 1 : 0, bq[cur ^ 1], sbk[cur ^ 1]);
            mma_window(w, bq[cur], sbk[cur], acc);
        });
        // ---- epilogue: lane holds rows 32i + l%32, columns 64 wave + 32 j + 8 q + 4 h + r.
        // Per-pair rows go through the wave's own LDS tile [BM][64] bf16
        // (16-byte granules XOR-swizzled by row bits 1-3: two 128-byte rows
        // share a 256-byte bank line, so 32 rows of one granule spread over
        // all 16 granule positions, two rows each, the floor for 512 bytes)
        // so that each store writes 8 rows x 128 contiguous bytes; atomics
        // (decode) are stored directly.
        const int n0 = 256 * tn + 64 * wave;
        if (mq.per_pair) {
#pragma unroll
            for (int i = 0; i < MA; ++i) {
                const int r = 32 * i + (lane & 31);
                const float wgt = __shfl(w_r[i / 2], r & 63);
#pragma unroll
                for (int j = 0; j < NB; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x16v_t& a = acc[i][j];
                        const int cc = 8 * j + 2 * q + h;   // 8-byte chunk of the 128-byte row
                        *reinterpret_cast<uint2*>(ep + r * 128 + (((cc >> 1) ^ ((r >> 1) & 7)) * 16) + (cc & 1) * 8) =
                            uint2{pack_bf16x2(a[4 * q] * wgt, a[4 * q + 1] * wgt),
                                  pack_bf16x2(a[4 * q + 2] * wgt, a[4 * q + 3] * wgt)};
                    }
            }
#pragma unroll
            for (int r0 = 0; r0 < BM; r0 += 8) {
                const int r = r0 + (lane >> 3);
                const int id = __shfl(ids_r[r0 / 64], r & 63);
                const i32x4_t v = *reinterpret_cast<const i32x4_t*>(ep + r * 128 + (((lane & 7) ^ ((r >> 1) & 7)) * 16));
                const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
                if (tok >= mq.token_num || slot >= mq.topk) continue;
                *reinterpret_cast<i32x4_t*>(mq.out + ((int64_t)tok * mq.topk + slot) * mq.out_stride + n0 +
                                            8 * (lane & 7)) = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < MA; ++i) {
                const int r = 32 * i + (lane & 31);
                const int id = __shfl(ids_r[i / 2], r & 63);
                const float wgt = __shfl(w_r[i / 2], r & 63);
                const int tok = id & 0xffffff, slot = (int)((unsigned)id >> 24);
                if (tok >= mq.token_num || slot >= mq.topk) continue;
                uint16_t* orow = mq.out + (int64_t)tok * mq.out_stride + n0 + 4 * h;
#pragma unroll
                for (int j = 0; j < NB; ++j)
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const f32x16v_t& a = acc[i][j];
                        atomic_add_bf16x2(orow + 32 * j + 8 * q, pack_bf16x2(a[4 * q] * wgt, a[4 * q + 1] * wgt));
                        atomic_add_bf16x2(orow + 32 * j + 8 * q + 2,
                                          pack_bf16x2(a[4 * q + 2] * wgt, a[4 * q + 3] * wgt));
                    }
            }
        }
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    if constexpr (KW % 2 == 0) {
        for (int tn = tn0; tn < tn1; ++tn) do_tile(tn, B0{});
    } else {
        for (int tn = tn0; tn < tn1; tn += 2) {
            do_tile(tn, B0{});
            if (tn + 1 < tn1) do_tile(tn + 1, B1{});
        }
    }
}

}  // namespace aiter_amd
