// Skinny (decode) GEMM with A staged through LDS.
//
// Same work split as gemm_skinny_kernel (gemm_kernels.h): one workgroup per
// 16*NB output columns, NW waves over the k-pairs of its K range, 16x16 MFMAs,
// the waves' partial sums reduced through LDS.  The difference is how A
// reaches the MFMAs.  A 16x16 fragment load puts 16 different rows in 16
// consecutive lanes; measured on MI355X, such a load moves 17 B/clk per CU
// out of L2, against 50 B/clk when 8 consecutive lanes read one 128-byte
// line.  Every workgroup reads all of A, so at M = 32 with bf16 the fragment
// loads of A cost as much load-unit time as B's.  Here each wave copies the
// A rows of its k-pair into a wave-private LDS buffer with whole-line copies
// (`buffer_load ... lds`, 64 lanes = 1024/ROWB rows x ROWB bytes) and reads
// the fragments from LDS.  The LDS image is row-major with the 16-byte pieces
// of row r XOR-swizzled by swz(r), so a fragment read (16 rows, one piece
// each, per 16 lanes) touches 16 different 16-byte bank groups.  Rows at or
// past M come back as zeros from the buffer range check.
#pragma once
#include "mfma32.h"

namespace aiter_amd {

template <int KA, int MF, int NW, bool B_PRE, bool SPLIT, bool OUT_F32, int NB, int S, bool BL>
struct SkinnyLdsCfg {
    static constexpr bool SCALED = OpTraits<KA>::scaled;
    static constexpr int FA = OpTraits<KA>::frags_per_step;
    static constexpr int KPAIR = SCALED ? 256 : 64;        // elements per k-pair
    static constexpr int A_STEP = KA == kFp8 ? 128 : 64;   // A bytes per row per k-step
    static constexpr int ROWB = 2 * A_STEP;                // A bytes per row per k-pair
    static constexpr int PPR = ROWB / 16;                  // 16-byte pieces per row
    static constexpr int RPI = 64 / PPR;                   // rows per copy instruction
    static constexpr int AROWS = 16 * MF;
    static constexpr int NCP = AROWS / RPI;                // copies per k-pair
    static constexpr int ABUF = AROWS * ROWB;              // A bytes per buffer
    static constexpr int BBUF = BL ? 16 * NB * 128 : 0;    // B bytes per buffer (128 B per row per k-pair)
    static constexpr int SET = ABUF + BBUF;
    static constexpr int SGRP = (MF + 1) / 2;              // 32-row A scale groups
    static constexpr int SBN = (NB + 1) / 2;               // 32-row B scale groups
    static constexpr int LP = NCP + 2 * NB + (SCALED ? SGRP + SBN : 0);   // vector-memory ops per k-pair
    static constexpr int RED = NW * MF * NB * 64 * 16;
    static constexpr int LDS = (NW * S * SET > RED) ? NW * S * SET : RED;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static_assert(AROWS % RPI == 0, "whole copies");
    static_assert((S - 1) * LP < 64, "vmcnt range");
    static_assert(S >= 2, "at least two k-pairs in flight");
    static_assert(!(BL && B_PRE), "B through LDS is for row-major B");
    // piece swizzle of row r: 16 rows at one logical piece land in 16
    // different 16-byte groups of a 256-byte bank line
    static AA_DEV int swz(int r) { return (ROWB == 128 ? (r >> 1) : r) & (PPR - 1); }
};

template <int KA, int MF, int NB, bool BL>
struct SkinnyLdsStage {
    static constexpr int SGRP = (MF + 1) / 2;
    static constexpr int SBN = (NB + 1) / 2;
    i32x4_t b[BL ? 1 : 2][NB];   // unused with B through LDS
    int sb[SBN];
    int sa[SGRP];
};

// NT: B and its scales are loaded with the nt cache policy (picked at launch
// for weights large enough to stream)
template <int KA, int MF, int NW, bool B_PRE, bool SPLIT, bool OUT_F32, int NB, int S = 2, bool BL = false,
          bool NT = false>
__global__ __launch_bounds__(64 * NW) void gemm_skinny_alds_kernel(GemmParams p) {
    static_assert(NB == 1 || NB == 2, "one or two column blocks per workgroup");
    using C = SkinnyLdsCfg<KA, MF, NW, B_PRE, SPLIT, OUT_F32, NB, S, BL>;
    using St = SkinnyLdsStage<KA, MF, NB, BL>;
    apply_batch(p);
    __shared__ __attribute__((aligned(1024))) uint8_t smem[C::LDS];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n0 = blockIdx.x * 16 * NB;
    const int total_pairs = p.K / C::KPAIR;
    const int p_begin = blockIdx.y * p.k_steps_per_split;   // k_steps_per_split counts pairs here
    const int p_end = min(total_pairs, p_begin + p.k_steps_per_split);

    const uint8_t* bsrc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        // a block past N (odd block count, NB = 2) reads the last valid rows;
        // its columns are never stored
        const int nb0 = min(n0 + 16 * j, (p.N - 1) / 16 * 16);
        if constexpr (B_PRE)
            bsrc[j] = p.B + (int64_t)nb0 * p.ldb + lane * 16;
        else
            bsrc[j] = p.B + (int64_t)min(nb0 + (lane & 15), p.N - 1) * p.ldb + (lane >> 4) * 16;
    }
    const uint8_t* sbp[C::SBN];
    const uint8_t* sap[C::SGRP];
    if constexpr (C::SCALED) {
#pragma unroll
        for (int g = 0; g < C::SBN; ++g) {
            const int nb0 = min(n0 + 32 * g, (p.N - 1) / 16 * 16);
            sbp[g] = p.Bs + (int64_t)(nb0 / 32) * 32 * p.sb_stride + lane * 4;
        }
#pragma unroll
        for (int g = 0; g < C::SGRP; ++g)
            sap[g] = p.As + (int64_t)min(g, p.sa_groups - 1) * 32 * p.sa_stride + lane * 4;
    }

    // A copies: instruction c covers rows c*RPI .. +RPI; lane l writes LDS
    // piece l % PPR of row c*RPI + l / PPR and fetches the logical piece that
    // the swizzle puts there
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(p.A, (int64_t)p.M * p.lda);
    int a_voff[C::NCP];
#pragma unroll
    for (int c = 0; c < C::NCP; ++c) {
        const int r = c * C::RPI + lane / C::PPR;
        a_voff[c] = r * (int)p.lda + ((lane % C::PPR) ^ C::swz(r)) * 16;
    }
    uint8_t* const abase = smem + wave * S * C::SET;
    // row-major B through LDS: the same whole-line copies over the
    // workgroup's 16*NB rows (128 bytes each per k-pair); rows past N read
    // as zeros and their columns are never stored
    const __amdgpu_buffer_rsrc_t br =
        make_rsrc(p.B + (BL ? (int64_t)n0 * p.ldb : 0), BL ? (int64_t)min(16 * NB, p.N - n0) * p.ldb : 0);
    int b_voff[BL ? 2 * NB : 1];
    if constexpr (BL) {
#pragma unroll
        for (int c = 0; c < 2 * NB; ++c) {
            const int r = c * 8 + lane / 8;
            b_voff[c] = r * (int)p.ldb + ((lane % 8) ^ ((r >> 1) & 7)) * 16;
        }
    }
    const int rd_rowb = (lane & 15) * 128;
    const int rd_swb = ((lane & 15) >> 1) & 7;
    // fragment reads: lane l, row i*16 + l%16, logical piece Q + l/16
    const int rd_row = (lane & 15) * C::ROWB;
    const int rd_sw = C::swz(lane & 15);
    const int rd_q = lane >> 4;

    f32x4_t acc[MF][NB];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };
    auto issue = [&](St& d, int pr, int buf) {
        uint8_t* dst = abase + buf * C::SET;
#pragma unroll
        for (int c = 0; c < C::NCP; ++c) dma16(ar, dst + c * 1024, a_voff[c], pr * C::ROWB);
        if constexpr (BL) {
#pragma unroll
            for (int c = 0; c < 2 * NB; ++c) dma16<NT ? kLoadNt : 0>(br, dst + C::ABUF + c * 1024, b_voff[c], pr * 128);
        } else {
            constexpr int BSTEP = B_PRE ? 1024 : 64;
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    d.b[h][j] = load_b<NT, i32x4_t>(bsrc[j] + (int64_t)(2 * pr + h) * BSTEP);
        }
        if constexpr (C::SCALED) {
#pragma unroll
            for (int g = 0; g < C::SBN; ++g) d.sb[g] = load_b<NT, int>(sbp[g] + (int64_t)pr * 256);
#pragma unroll
            for (int g = 0; g < C::SGRP; ++g) d.sa[g] = *reinterpret_cast<const int*>(sap[g] + (int64_t)pr * 256);
        }
    };
    // BHALF0: which 16-column half of its 32-row B scale group the first
    // column block covers (block j covers half BHALF0 + j)
    auto mma = [&](const St& d, int buf, auto bh) {
        constexpr int BHALF0 = decltype(bh)::value;
        const uint8_t* src = abase + buf * C::SET + rd_row;
        const uint8_t* bsl = abase + buf * C::SET + C::ABUF + rd_rowb;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            i32x4_t a[MF][C::FA];
#pragma unroll
            for (int i = 0; i < MF; ++i)
#pragma unroll
                for (int f = 0; f < C::FA; ++f) {
                    const int q = (h * C::A_STEP + f * 64) / 16 + rd_q;
                    a[i][f] = *reinterpret_cast<const i32x4_t*>(src + i * 16 * C::ROWB + ((q ^ rd_sw) * 16));
                }
            i32x4_t bl[NB];
            if constexpr (BL) {
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    bl[j] = *reinterpret_cast<const i32x4_t*>(bsl + j * 16 * 128 + (((h * 4 + rd_q) ^ rd_swb) * 16));
            }
            const i32x4_t* bf = BL ? bl : d.b[BL ? 0 : h];
#pragma unroll
            for (int i = 0; i < MF; ++i)
#pragma unroll
                for (int j = 0; j < NB; ++j) {
                    if constexpr (C::SCALED) {
                        const int bhj = (BHALF0 + j) & 1;
                        const int g = (BHALF0 + j) >> 1;
                        if (bhj)
                            acc[i][j] = mma_step<KA, kFp4>(&bf[j], a[i], acc[i][j], d.sb[g], h * 2 + 1,
                                                           d.sa[i >> 1], h * 2 + (i & 1));
                        else
                            acc[i][j] = mma_step<KA, kFp4>(&bf[j], a[i], acc[i][j], d.sb[g], h * 2,
                                                           d.sa[i >> 1], h * 2 + (i & 1));
                    } else {
                        acc[i][j] = mma_step<KA, KA>(&bf[j], a[i], acc[i][j], 0, 0, 0, 0);
                    }
                }
        }
    };
    // S k-pairs in flight per wave, in S register sets and S LDS buffers
    // used in turn (no register copies, which would wait for the loads).
    // The copies of the pair being multiplied have landed once at most the
    // operations of the pairs issued after it (LP each) are outstanding.
    St st[S];
    auto consume = [&](auto set, auto after, auto bh) {
        fence();
        wait_vmcnt<decltype(after)::value * C::LP>();
        fence();
        mma(st[decltype(set)::value], decltype(set)::value, bh);
    };
    auto run = [&](auto bh) {
        const int pr = p_begin + wave;
        if (pr >= p_end) return;
        const int npairs = (p_end - pr + NW - 1) / NW;   // pair t of this wave: pr + t*NW
        if (npairs < S) {
            // at most S-1 pairs: all issued up front
            static_for<S - 1>([&](auto nn) {
                constexpr int N = decltype(nn)::value + 1;
                if (npairs == N) {
                    static_for<N>([&](auto u) { issue(st[u], pr + decltype(u)::value * NW, decltype(u)::value); });
                    static_for<N>([&](auto u) {
                        consume(u, std::integral_constant<int, N - 1 - decltype(u)::value>{}, bh);
                    });
                }
            });
            return;
        }
        static_for<S - 1>([&](auto u) { issue(st[u], pr + decltype(u)::value * NW, decltype(u)::value); });
        int t = 0;   // pairs consumed; t % S == 0 at the top of the loop
        for (; t + 2 * S - 2 < npairs; t += S) {
            static_for<S>([&](auto u) {
                constexpr int U = decltype(u)::value, I = (U + S - 1) % S;
                fence();
                issue(st[I], pr + (t + U + S - 1) * NW, I);
                consume(u, std::integral_constant<int, S - 1>{}, bh);
            });
        }
        // pairs t .. t+S-2 are in flight in sets 0 .. S-2; R more to issue
        const int rem = npairs - t - (S - 1);
        static_for<S>([&](auto rr) {
            constexpr int R = decltype(rr)::value;
            if (rem == R) {
                static_for<S - 1 + R>([&](auto u) {
                    constexpr int U = decltype(u)::value;
                    if constexpr (U < R) {
                        constexpr int I = (U + S - 1) % S;
                        fence();
                        issue(st[I], pr + (t + U + S - 1) * NW, I);
                        consume(std::integral_constant<int, U % S>{}, std::integral_constant<int, S - 1>{}, bh);
                    } else {
                        consume(std::integral_constant<int, U % S>{}, std::integral_constant<int, S - 2 + R - U>{},
                                bh);
                    }
                });
            }
        });
    };
    // NB = 2 starts on a 32-row group boundary; NB = 1 on either half
    if (NB == 1 && ((n0 / 16) & 1)) run(std::integral_constant<int, 1>{});
    else run(std::integral_constant<int, 0>{});

    // every copy has landed (the last pair waited for vmcnt 0); the
    // reduction reuses the A buffers once all waves have read theirs
    __syncthreads();
    f32x4_t* red = reinterpret_cast<f32x4_t*>(smem);   // [NW][MF*NB][64]
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) red[(wave * MF * NB + i * NB + j) * 64 + lane] = acc[i][j];
    __syncthreads();
    for (int t = threadIdx.x; t < MF * NB * 64; t += 64 * NW) {
        const int ij = t / 64, l = t % 64;
        const int i = ij / NB, j = ij % NB;
        f32x4_t s = red[ij * 64 + l];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[(w * MF * NB + ij) * 64 + l];
        const int m = i * 16 + (l & 15);
        const int n = n0 + 16 * j + 4 * (l >> 4);
        if constexpr (SPLIT) {
            if (m < p.M && n < p.N) {
                float* w = p.ws + (int64_t)m * p.N + n;
#pragma unroll
                for (int r = 0; r < 4; ++r) atomicAdd(w + r, s[r]);
            }
        } else {
            store_frag<OUT_F32>(p, s, m, n);
        }
    }
}

// Stream-K form of the row-major bf16 staged kernel (A and B through LDS).
// A decode shape with fewer 32-column blocks than CUs leaves CUs idle (N =
// 7168: 224 blocks on 256 CUs), and splitting every block in two leaves the
// same longest share per CU.  Here gridDim.x workgroups (one per CU) share
// the U = blocks x k-pairs units evenly: workgroup g takes units
// [g*U/G, (g+1)*U/G).  It walks its range in windows of at most two column
// blocks; the waves take the window's units in turn (wave w: units w, w+NW,
// ...), each accumulating the units of the window's first block, then
// those of its second, in two register sets.  A block whose units all lie in
// one range is stored directly.  A block split over ranges leaves one f32
// partial per range in that range's slot (workgroup g, slot 0 for the
// range's first segment, 1 for its last), written with agent-coherent
// stores (past the XCD-private L2); after they have landed one thread
// increments the block's arrival counter, and the range that arrives last
// loads the block's slots with agent-coherent loads, adds them in range
// order (the result does not depend on the arrival order), stores the block
// and sets the counter back to zero.  p.ws: 2 * G slots of 16*MF x 16*NB
// floats; p.cnt: one zeroed counter per column block.  The host caps G at
// 8 workgroups per block: each range beyond that adds one more partial to
// load for the range that sums the block.
template <int MF, int NW, bool OUT_F32, int NB, int S, bool NT>
__global__ __launch_bounds__(64 * NW) void gemm_skinny_sk_kernel(GemmParams p) {
    static_assert(NB == 1 || NB == 2, "one or two column blocks per workgroup");
    using C = SkinnyLdsCfg<kBf16, MF, NW, false, false, OUT_F32, NB, S, true>;
    using St = SkinnyLdsStage<kBf16, MF, NB, true>;
    constexpr int ITEMS = MF * NB * 64;                    // f32x4 items of one block's sum
    constexpr int LDS = C::LDS > 2 * NW * ITEMS * 16 ? C::LDS : 2 * NW * ITEMS * 16;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    __shared__ __attribute__((aligned(1024))) uint8_t smem[LDS];
    __shared__ int last_flag[2];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int BW = 16 * NB;   // columns per block
    const int T = p.K / C::KPAIR;
    const int nblk = (p.N + BW - 1) / BW;
    const int64_t U = (int64_t)nblk * T, G = gridDim.x, g = blockIdx.x;
    const int64_t lo0 = g * U / G, hi = (g + 1) * U / G;
    // the range that holds unit x: the largest g with g*U/G <= x
    auto owner = [&](int64_t x) -> int64_t { return ((x + 1) * G - 1) / U; };

    const __amdgpu_buffer_rsrc_t ar = make_rsrc(p.A, (int64_t)p.M * p.lda);
    // the whole of B: rows past N read as zeros, their columns are never stored
    const __amdgpu_buffer_rsrc_t br = make_rsrc(p.B, (int64_t)p.N * p.ldb);
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.ws, 2 * G * ITEMS * 16);
    int a_voff[C::NCP];
#pragma unroll
    for (int c = 0; c < C::NCP; ++c) {
        const int r = c * C::RPI + lane / C::PPR;
        a_voff[c] = r * (int)p.lda + ((lane % C::PPR) ^ C::swz(r)) * 16;
    }
    int b_voff[2 * NB];
#pragma unroll
    for (int c = 0; c < 2 * NB; ++c) {
        const int r = c * 8 + lane / 8;
        b_voff[c] = r * (int)p.ldb + ((lane % 8) ^ ((r >> 1) & 7)) * 16;
    }
    uint8_t* const abase = smem + wave * S * C::SET;
    const int rd_rowb = (lane & 15) * 128;
    const int rd_swb = ((lane & 15) >> 1) & 7;
    const int rd_row = (lane & 15) * C::ROWB;
    const int rd_sw = C::swz(lane & 15);
    const int rd_q = lane >> 4;
    auto fence = [] { __builtin_amdgcn_sched_barrier(0); };

    for (int64_t x = lo0; x < hi;) {
        const int b0 = (int)(x / T);
        const int64_t xe = min(hi, (int64_t)(b0 + 2) * T);   // window [x, xe): blocks b0 and b0 + 1
        const int64_t xb = min(xe, (int64_t)(b0 + 1) * T);   // first unit of block b0 + 1
        const int64_t ubase = x + wave;                       // unit t of this wave: ubase + t*NW
        const int npairs = ubase < xe ? (int)((xe - ubase + NW - 1) / NW) : 0;
        // consumed units before tsw are block b0's
        const int tsw = xb > ubase ? (int)((xb - ubase + NW - 1) / NW) : 0;

        f32x4_t acc[MF][NB], acc0[MF][NB];
#pragma unroll
        for (int i = 0; i < MF; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                acc0[i][j] = acc[i][j];
            }

        auto issue = [&](int t, int buf) {
            const int64_t u = ubase + (int64_t)t * NW;
            const int blk = u < xb ? b0 : b0 + 1;
            const int pr = (int)(u - (int64_t)blk * T);
            uint8_t* dst = abase + buf * C::SET;
#pragma unroll
            for (int c = 0; c < C::NCP; ++c) dma16(ar, dst + c * 1024, a_voff[c], pr * C::ROWB);
            // the block's row offset goes into the range-checked lane offset
            const int brow = blk * BW * (int)p.ldb;
#pragma unroll
            for (int c = 0; c < 2 * NB; ++c)
                dma16<NT ? kLoadNt : 0>(br, dst + C::ABUF + c * 1024, b_voff[c] + brow, pr * 128);
        };
        auto mma = [&](int buf) {
            const uint8_t* src = abase + buf * C::SET + rd_row;
            const uint8_t* bsl = abase + buf * C::SET + C::ABUF + rd_rowb;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                i32x4_t a[MF][C::FA];
#pragma unroll
                for (int i = 0; i < MF; ++i)
#pragma unroll
                    for (int f = 0; f < C::FA; ++f) {
                        const int q = (h * C::A_STEP + f * 64) / 16 + rd_q;
                        a[i][f] = *reinterpret_cast<const i32x4_t*>(src + i * 16 * C::ROWB + ((q ^ rd_sw) * 16));
                    }
                i32x4_t bl[NB];
#pragma unroll
                for (int j = 0; j < NB; ++j)
                    bl[j] = *reinterpret_cast<const i32x4_t*>(bsl + j * 16 * 128 + (((h * 4 + rd_q) ^ rd_swb) * 16));
#pragma unroll
                for (int i = 0; i < MF; ++i)
#pragma unroll
                    for (int j = 0; j < NB; ++j) acc[i][j] = mma_step<kBf16, kBf16>(&bl[j], a[i], acc[i][j], 0, 0, 0, 0);
            }
        };
        // unit t (consumed in order): the first unit of block b0 + 1 moves
        // the first block's sum aside
        auto consume = [&](int t, auto set, auto after) {
            fence();
            wait_vmcnt<decltype(after)::value * (C::NCP + 2 * NB)>();
            fence();
            if (t == tsw) {
#pragma unroll
                for (int i = 0; i < MF; ++i)
#pragma unroll
                    for (int j = 0; j < NB; ++j) {
                        acc0[i][j] = acc[i][j];
                        acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
                    }
            }
            mma(decltype(set)::value);
        };
        if (npairs > 0 && npairs < S) {
            static_for<S - 1>([&](auto nn) {
                constexpr int N = decltype(nn)::value + 1;
                if (npairs == N) {
                    static_for<N>([&](auto u) { issue(decltype(u)::value, decltype(u)::value); });
                    static_for<N>([&](auto u) {
                        constexpr int UU = decltype(u)::value;
                        consume(UU, u, std::integral_constant<int, N - 1 - UU>{});
                    });
                }
            });
        } else if (npairs >= S) {
            static_for<S - 1>([&](auto u) { issue(decltype(u)::value, decltype(u)::value); });
            int t = 0;   // units consumed; t % S == 0 at the top of the loop
            for (; t + 2 * S - 2 < npairs; t += S) {
                static_for<S>([&](auto u) {
                    constexpr int UU = decltype(u)::value, I = (UU + S - 1) % S;
                    fence();
                    issue(t + UU + S - 1, I);
                    consume(t + UU, u, std::integral_constant<int, S - 1>{});
                });
            }
            const int rem = npairs - t - (S - 1);
            static_for<S>([&](auto rr) {
                constexpr int R = decltype(rr)::value;
                if (rem == R) {
                    static_for<S - 1 + R>([&](auto u) {
                        constexpr int UU = decltype(u)::value;
                        if constexpr (UU < R) {
                            constexpr int I = (UU + S - 1) % S;
                            fence();
                            issue(t + UU + S - 1, I);
                            consume(t + UU, std::integral_constant<int, UU % S>{}, std::integral_constant<int, S - 1>{});
                        } else {
                            consume(t + UU, std::integral_constant<int, UU % S>{},
                                    std::integral_constant<int, S - 2 + R - UU>{});
                        }
                    });
                }
            });
        }
        // register set of each block: a wave that switched holds block b0's
        // sum in acc0 and block b0 + 1's in acc; one that did not, b0's in acc
        const bool switched = tsw < npairs;

        // every copy has landed; the reduction reuses the buffers once all
        // waves have read theirs
        __syncthreads();
        f32x4_t* red = reinterpret_cast<f32x4_t*>(smem);   // [2][NW][MF*NB][64]
#pragma unroll
        for (int i = 0; i < MF; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int ij = i * NB + j;
                red[(wave * MF * NB + ij) * 64 + lane] = switched ? acc0[i][j] : acc[i][j];
                red[((NW + wave) * MF * NB + ij) * 64 + lane] = switched ? acc[i][j] : f32x4_t{0.f, 0.f, 0.f, 0.f};
            }
        __syncthreads();
        // segment of each set in this window: [s_lo, s_hi) within its block
        auto seg_lo = [&](int st) { return st ? xb : x; };
        auto seg_hi = [&](int st) { return st ? xe : xb; };
        bool any_partial = false;
        constexpr int PER = 2 * ITEMS / (64 * NW) > 0 ? 2 * ITEMS / (64 * NW) : 1;
        static_assert(2 * ITEMS % (64 * NW) == 0 || 2 * ITEMS < 64 * NW, "items per thread");
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int it = threadIdx.x + k * 64 * NW;
            if (it >= 2 * ITEMS) continue;
            const int st = it / ITEMS, ij = (it % ITEMS) / 64, l = it % 64;
            f32x4_t s = red[(st * NW * MF * NB + ij) * 64 + l];
#pragma unroll
            for (int w = 1; w < NW; ++w) s += red[((st * NW + w) * MF * NB + ij) * 64 + l];
            const int64_t slo = seg_lo(st), shi = seg_hi(st);
            if (slo >= shi) continue;   // no second block in this window
            const int blk = b0 + st;
            const bool whole = slo == (int64_t)blk * T && shi == (int64_t)(blk + 1) * T;
            if (whole) {
                const int i = ij / NB, j = ij % NB;
                store_frag<OUT_F32>(p, s, i * 16 + (l & 15), blk * BW + 16 * j + 4 * (l >> 4));
            } else {
                const int which = slo == lo0 ? 0 : 1;
                const int off = (int)(((g * 2 + which) * ITEMS + (it % ITEMS)) * 16);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(i32x4_t, s), wr, off, 0, kAgentCoherent);
            }
        }
        // arrival of the partial blocks (uniform: depends on the window only)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
            const int64_t slo = seg_lo(st), shi = seg_hi(st);
            const int blk = b0 + st;
            if (slo < shi && !(slo == (int64_t)blk * T && shi == (int64_t)(blk + 1) * T)) any_partial = true;
        }
        if (any_partial) {
            wait_vmcnt<0>();
            __syncthreads();
            if (threadIdx.x < 2) {
                const int st = threadIdx.x;
                const int64_t slo = seg_lo(st), shi = seg_hi(st);
                const int blk = b0 + st;
                int last = 0;
                if (slo < shi && !(slo == (int64_t)blk * T && shi == (int64_t)(blk + 1) * T)) {
                    const int np = (int)(owner((int64_t)(blk + 1) * T - 1) - owner((int64_t)blk * T) + 1);
                    last = atomicAdd(p.cnt + blk, 1) == np - 1;
                    if (last) __hip_atomic_store(p.cnt + blk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                last_flag[st] = last;
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < PER; ++k) {
                const int it = threadIdx.x + k * 64 * NW;
                if (it >= 2 * ITEMS) continue;
                const int st = it / ITEMS;
                if (!last_flag[st]) continue;
                const int blk = b0 + st, ij = (it % ITEMS) / 64, l = it % 64;
                const int64_t x0 = (int64_t)blk * T;
                const int64_t gf = owner(x0), gl = owner(x0 + T - 1);
                // up to 8 slots in flight; slots past the last range read as
                // zeros (an offset past the descriptor) and add nothing
                f32x4_t s = f32x4_t{0.f, 0.f, 0.f, 0.f};
                for (int64_t g0 = gf; g0 <= gl; g0 += 8) {
                    f32x4_t v[8];
#pragma unroll
                    for (int q = 0; q < 8; ++q) {
                        const int64_t gg = g0 + q;
                        const int which = gg * U / G < x0 ? 1 : 0;
                        const int off = gg <= gl ? (int)(((gg * 2 + which) * ITEMS + (it % ITEMS)) * 16) : 0x7ffffff0;
                        v[q] = __builtin_bit_cast(f32x4_t,
                                                  __builtin_amdgcn_raw_buffer_load_b128(wr, off, 0, kAgentCoherent));
                    }
#pragma unroll
                    for (int q = 0; q < 8; ++q) s += v[q];
                }
                const int i = ij / NB, j = ij % NB;
                store_frag<OUT_F32>(p, s, i * 16 + (l & 15), blk * BW + 16 * j + 4 * (l >> 4));
            }
        }
        x = xe;
        // the next window's waits count its own loads only; the buffers and
        // flags are reused by it
        wait_vmcnt<0>();
        __syncthreads();
    }
}

}  // namespace aiter_amd
