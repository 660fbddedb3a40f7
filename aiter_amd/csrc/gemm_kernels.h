// Device code of the scaled-GEMM family (gfx950, wave64).
//
// Operand staging unit: the "byte-fragment" — 16 rows x 64 bytes = 1 KiB,
// stored so that lane l holds row (l % 16), bytes [16*(l/16), 16*(l/16)+16).
// That is exactly:
//   * the A/B operand of v_mfma_scale_f32_16x16x128_f8f6f4 for e2m1
//     (32 contiguous fp4 = one MX block per lane, one e8m0 scale per lane),
//   * the A/B operand of v_mfma_f32_16x16x32_bf16 (8 contiguous bf16),
//   * one 64-byte K window of aiter's preshuffled weight layout
//     (shuffle_weight((16,16)): per 16-row block, 32-byte K chunks of
//     [2 halves][16 rows][16 B]; aiter/ops/shuffle.py:192-204), which is
//     therefore a contiguous 1 KiB read.
// e4m3 operands use two consecutive byte-fragments per MFMA: lane l holds
// bytes [16g, 16g+16) and [64+16g, 64+16g+16) of the 128-byte k-step
// window (g = l/16) -- the K pairing the scaled MFMA applies between an e4m3
// operand and an e2m1 operand laid out as above (measured on gfx950 with
// one-hot operands).
//
// Scales use aiter's shuffled e8m0 layout (aiter/ops/shuffle.py:339-365):
// one dword per lane covers rows (l%16, l%16+16) of a 32-row group and MX
// blocks (l/16, l/16+4) of a 256-element K window; byte 2*k2+r2 is the scale
// for K half k2 and row half r2, which is the op_sel byte of the scaled MFMA.
#pragma once
#include "common.h"

namespace aiter_amd {

enum OpKind : int { kFp4 = 4, kFp8 = 0, kBf16 = 16 };

// cache-policy operand of a buffer load: nt, for data that one launch reads
// exactly once (weights at decode sizes), so it does not displace what the
// other workgroups re-read from L2
constexpr int kLoadNt = 2;

// plain load of data read once per launch (nt)
template <typename T>
AA_DEV T load_once(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const T*>(p));
}

// B-operand load, nt when NT
template <bool NT, typename T>
AA_DEV T load_b(const uint8_t* p) {
    if constexpr (NT)
        return load_once<T>(p);
    else
        return *reinterpret_cast<const T*>(p);
}

// Weights read once per launch stream from HBM faster with the nt policy
// (a 470 MB row-major matrix: 6.6 TB/s against 5.7 TB/s), but decode
// launches over a few MB ran slower with it; launchers pick nt from this size.
constexpr int64_t kNtMinBytes = 16LL << 20;

template <int KIND> struct OpTraits;
template <> struct OpTraits<kFp4> {
    static constexpr int frags_per_step = 1;   // byte-fragments per MFMA k-step
    static constexpr int fmt = 4;
    static constexpr bool scaled = true;
};
template <> struct OpTraits<kFp8> {
    static constexpr int frags_per_step = 2;
    static constexpr int fmt = 0;
    static constexpr bool scaled = true;
};
template <> struct OpTraits<kBf16> {
    static constexpr int frags_per_step = 1;
    static constexpr int fmt = -1;
    static constexpr bool scaled = false;
};

// Output operation fused into the epilogue (fused_gemm_afp4wfp4_mul_add /
// _split_cat of aiter/ops/triton/gemm/fused/), applied to the f32 result
// after alpha and bias:
//   kind 1 (mul_add): out = a * acc + b (fuse 0) or a * b + acc (fuse 1),
//     a and b each a scalar or an [M, N] tensor (f32 or bf16, element strides);
//   kind 2 (split_cat): column n of the [M, D*(S1+S2)] product goes to
//     c1[m, d, s] (s < S1) or c2[m, d, s-S1] (d = n / (S1+S2), s = n % (S1+S2));
//     p.D is c1 ([M, D, S1+S3] rows of ld1 elements), c2 has rows of ld2.
struct EpiOp {
    int kind;
    int fuse;
    const void* ta;   // mul_add tensors (null: the scalar sa / sb)
    const void* tb;
    int ta_bf16, tb_bf16;
    int64_t ta_sm, ta_sn, tb_sm, tb_sn;
    float sa, sb;
    void* c2;
    int s1, s2, s3;
    int64_t ld1, ld2;
};

struct GemmParams {
    const uint8_t* A;
    const uint8_t* B;
    const uint8_t* As;  // shuffled e8m0 (scaled kinds)
    const uint8_t* Bs;
    void* D;
    const float* bias;
    float* ws;           // split-K f32 partial sums: [M, N] (skinny), [splits][M][N] (tiles)
    int* cnt;            // stream-K: one zeroed arrival counter per column block
    int64_t lda, ldb;    // bytes per row (row-major) / per row of the preshuffled matrix
    int64_t ldd;         // elements per output row
    int64_t ld_bias;     // elements per bias row (0 = broadcast one row)
    int64_t sa_stride, sb_stride;  // bytes per row of the scale buffers (pad8(K/32))
    int M, N, K;
    int sa_groups, sb_groups;      // 32-row groups present in the scale buffers
    int tiles_m, tiles_n;
    int k_steps_per_split;         // split-K: k-pairs (skinny) or stages (tiles) per split
    float alpha, beta;
    // batched launches (gridDim.z = batch): per-batch offsets of A, B, D in
    // bytes and of the bias in elements (0: shared by every batch)
    int64_t bs_a, bs_b, bs_d, bs_bias;
    EpiOp epi;
};

// element (m, n) of a mul_add operand
AA_DEV float epi_operand(const void* t, int bf16, int64_t sm, int64_t sn, float scalar, int m, int n) {
    if (!t) return scalar;
    const int64_t off = (int64_t)m * sm + (int64_t)n * sn;
    return bf16 ? bf16_bits_to_f32(static_cast<const uint16_t*>(t)[off]) : static_cast<const float*>(t)[off];
}

// mul_add on the four f32 values of row m, columns n..n+3 (all inside the output)
AA_DEV void epi_mul_add(const GemmParams& p, float (&v)[4], int m, int n) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float a = epi_operand(p.epi.ta, p.epi.ta_bf16, p.epi.ta_sm, p.epi.ta_sn, p.epi.sa, m, n + r);
        const float b = epi_operand(p.epi.tb, p.epi.tb_bf16, p.epi.tb_sm, p.epi.tb_sn, p.epi.sb, m, n + r);
        v[r] = p.epi.fuse == 0 ? a * v[r] + b : a * b + v[r];
    }
}

// split_cat destination of output element (m, n), in elements of `elem` bytes:
// a run of columns that stays inside one S1 or S2 segment is contiguous there
AA_DEV uint8_t* epi_split_dst(const GemmParams& p, int m, int n, int elem) {
    const int seg = p.epi.s1 + p.epi.s2;
    const int d = n / seg, s = n - d * seg;
    if (s < p.epi.s1)
        return static_cast<uint8_t*>(p.D) + ((int64_t)m * p.epi.ld1 + (int64_t)d * (p.epi.s1 + p.epi.s3) + s) * elem;
    return static_cast<uint8_t*>(p.epi.c2) + ((int64_t)m * p.epi.ld2 + (int64_t)d * p.epi.s2 + (s - p.epi.s1)) * elem;
}

// moves the operand pointers to batch blockIdx.z (no-op for unbatched grids)
AA_DEV void apply_batch(GemmParams& p) {
    const int64_t z = blockIdx.z;
    if (z == 0) return;
    p.A += z * p.bs_a;
    p.B += z * p.bs_b;
    p.D = static_cast<uint8_t*>(p.D) + z * p.bs_d;
    if (p.bias) p.bias += z * p.bs_bias;
}

// ---------------------------------------------------------------------------
// MFMA wrappers.  op_sel bytes must be immediates: the switch folds away once
// the caller's loops are unrolled.
// ---------------------------------------------------------------------------
#define AA_MFMA_SC(OA, OB)                                                                 \
    case (OA) * 4 + (OB):                                                                  \
        return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FA, FB, OA, sa, OB, sb);

template <int FA, int FB>
AA_DEV f32x4_t mfma_scaled(i32x8_t a, i32x8_t b, f32x4_t c, int sa, int oa, int sb, int ob) {
    switch (oa * 4 + ob) {
        AA_MFMA_SC(0, 0) AA_MFMA_SC(0, 1) AA_MFMA_SC(0, 2) AA_MFMA_SC(0, 3)
        AA_MFMA_SC(1, 0) AA_MFMA_SC(1, 1) AA_MFMA_SC(1, 2) AA_MFMA_SC(1, 3)
        AA_MFMA_SC(2, 0) AA_MFMA_SC(2, 1) AA_MFMA_SC(2, 2) AA_MFMA_SC(2, 3)
        AA_MFMA_SC(3, 0) AA_MFMA_SC(3, 1) AA_MFMA_SC(3, 2) AA_MFMA_SC(3, 3)
        default: __builtin_unreachable();
    }
}
#undef AA_MFMA_SC

AA_DEV f32x4_t mfma_bf16(i32x4_t a, i32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// One MFMA k-step for a (B-fragment, A-fragment) pair.  src0 = B so that the
// 16x16 result lands transposed: lane l holds C[m = l%16][n = 4*(l/16)+r],
// i.e. four consecutive output columns of one row (an 8-byte bf16 store).
template <int KA, int KB>
AA_DEV f32x4_t mma_step(const i32x4_t* b, const i32x4_t* a, f32x4_t c, int sb, int ob, int sa,
                        int oa) {
    if constexpr (KA == kBf16) {
        return mfma_bf16(b[0], a[0], c);
    } else {
        i32x8_t bv, av;
        bv[0] = b[0][0]; bv[1] = b[0][1]; bv[2] = b[0][2]; bv[3] = b[0][3];
        if constexpr (KB == kFp8) {
            bv[4] = b[1][0]; bv[5] = b[1][1]; bv[6] = b[1][2]; bv[7] = b[1][3];
        } else {
            bv[4] = 0; bv[5] = 0; bv[6] = 0; bv[7] = 0;
        }
        av[0] = a[0][0]; av[1] = a[0][1]; av[2] = a[0][2]; av[3] = a[0][3];
        if constexpr (KA == kFp8) {
            av[4] = a[1][0]; av[5] = a[1][1]; av[6] = a[1][2]; av[7] = a[1][3];
        } else {
            av[4] = 0; av[5] = 0; av[6] = 0; av[7] = 0;
        }
        return mfma_scaled<OpTraits<KB>::fmt, OpTraits<KA>::fmt>(bv, av, c, sb, ob, sa, oa);
    }
}

// XCD-aware tile order: hardware dispatches workgroup i to XCD (i % 8); the
// remap gives each XCD a contiguous range of the grouped (GROUP_M rows)
// raster so tiles sharing A rows / B columns share one L2.
AA_DEV void tile_coords(int bid, int nblocks, int tiles_m, int tiles_n, int& tm, int& tn) {
    constexpr int kXcd = 8;
    constexpr int kGroupM = 8;
    int pid = bid;
    if (nblocks % kXcd == 0) pid = (bid % kXcd) * (nblocks / kXcd) + bid / kXcd;
    const int in_group = kGroupM * tiles_n;
    const int group = pid / in_group;
    const int first_m = group * kGroupM;
    const int gsize = min(tiles_m - first_m, kGroupM);
    const int r = pid % in_group;
    tm = first_m + r % gsize;
    tn = r / gsize;
}

// ---------------------------------------------------------------------------
// Epilogue store of one 16x16 fragment (transposed accumulator layout).
// ---------------------------------------------------------------------------
template <bool OUT_F32>
AA_DEV void store_frag(const GemmParams& p, f32x4_t acc, int m, int n) {
    if (m >= p.M || n >= p.N) return;
    float v[4] = {acc[0] * p.alpha, acc[1] * p.alpha, acc[2] * p.alpha, acc[3] * p.alpha};
    if (p.bias) {
        const float* bp = p.bias + (int64_t)m * p.ld_bias + n;
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] += p.beta * bp[r];
    }
    if (p.epi.kind == 1) epi_mul_add(p, v, m, n);
    if constexpr (OUT_F32) {
        float* d = p.epi.kind == 2 ? reinterpret_cast<float*>(epi_split_dst(p, m, n, 4))
                                   : static_cast<float*>(p.D) + (int64_t)m * p.ldd + n;
        *reinterpret_cast<f32x4_t*>(d) = f32x4_t{v[0], v[1], v[2], v[3]};
    } else {
        uint16_t* d = p.epi.kind == 2 ? reinterpret_cast<uint16_t*>(epi_split_dst(p, m, n, 2))
                                      : static_cast<uint16_t*>(p.D) + (int64_t)m * p.ldd + n;
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2_t*>(d) = u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    }
}

// ---------------------------------------------------------------------------
// Tile kernel: BM x BN block tile, 4 waves in 2x2, each (BM/2) x (BN/2).
// One stage = 2 MFMA k-steps (256 MX elements / 64 bf16 elements), double
// buffered in LDS through registers: global loads for stage t+1 are in
// flight while stage t is multiplied, then written to the other LDS buffer.
// ---------------------------------------------------------------------------
template <int KA, int KB, int BM, int BN, bool A_PRE, bool B_PRE, bool OUT_F32>
__global__ __launch_bounds__(256, 1) void gemm_tile_kernel(GemmParams p) {
    apply_batch(p);
    constexpr int FA = OpTraits<KA>::frags_per_step;
    constexpr int FB = OpTraits<KB>::frags_per_step;
    constexpr bool SCALED = OpTraits<KA>::scaled;
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int MI = WM / 16, NJ = WN / 16;
    constexpr int A_FRAGS = (BM / 16) * 2 * FA;  // byte-fragments of A per stage
    constexpr int B_FRAGS = (BN / 16) * 2 * FB;
    constexpr int TOT = A_FRAGS + B_FRAGS;
    static_assert(TOT % 4 == 0, "fragments must split evenly over 4 waves");
    constexpr int PER_WAVE = TOT / 4;
    constexpr int STAGE_BYTES = TOT * 1024;
    constexpr int A_KBYTES = 128 * FA;  // A bytes per row per stage
    constexpr int B_KBYTES = 128 * FB;

    __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * STAGE_BYTES];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, p.tiles_m, p.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    // ---- per-thread global source pointers of its PER_WAVE fragments
    const uint8_t* src[PER_WAVE];
    int64_t kstride[PER_WAVE];  // bytes to advance per stage
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
        const int f = wave + 4 * q;
        if (f < A_FRAGS) {
            const int rf = f / (2 * FA), kf = f % (2 * FA);
            int row = m0 + rf * 16;
            if constexpr (A_PRE) {
                row = min(row, p.M - 16);
                src[q] = p.A + (int64_t)row * p.lda + kf * 1024 + lane * 16;
                kstride[q] = A_KBYTES * 16;
            } else {
                row = min(row + (lane & 15), p.M - 1);
                src[q] = p.A + (int64_t)row * p.lda + kf * 64 + (lane >> 4) * 16;
                kstride[q] = A_KBYTES;
            }
        } else {
            const int g = f - A_FRAGS;
            const int rf = g / (2 * FB), kf = g % (2 * FB);
            int row = n0 + rf * 16;
            if constexpr (B_PRE) {
                row = min(row, p.N - 16);
                src[q] = p.B + (int64_t)row * p.ldb + kf * 1024 + lane * 16;
                kstride[q] = B_KBYTES * 16;
            } else {
                row = min(row + (lane & 15), p.N - 1);
                src[q] = p.B + (int64_t)row * p.ldb + kf * 64 + (lane >> 4) * 16;
                kstride[q] = B_KBYTES;
            }
        }
    }

    // ---- scale pointers: one dword per lane per 32-row group per stage
    constexpr int SA = SCALED ? (WM / 32) : 1;
    constexpr int SB = SCALED ? (WN / 32) : 1;
    const uint8_t* sa_ptr[SA];
    const uint8_t* sb_ptr[SB];
    if constexpr (SCALED) {
#pragma unroll
        for (int i = 0; i < SA; ++i) {
            const int grp = min((m0 + wm * WM) / 32 + i, p.sa_groups - 1);
            sa_ptr[i] = p.As + (int64_t)grp * 32 * p.sa_stride + lane * 4;
        }
#pragma unroll
        for (int j = 0; j < SB; ++j) {
            const int grp = min((n0 + wn * WN) / 32 + j, p.sb_groups - 1);
            sb_ptr[j] = p.Bs + (int64_t)grp * 32 * p.sb_stride + lane * 4;
        }
    }

    const int stage_k = SCALED ? 256 : 64;
    const int nstages = p.K / stage_k;

    f32x4_t acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    i32x4_t stg[PER_WAVE];
    int sa_cur[SA], sb_cur[SB], sa_nxt[SA], sb_nxt[SB];

    auto load_stage = [&](int t) {
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q)
            stg[q] = *reinterpret_cast<const i32x4_t*>(src[q] + (int64_t)t * kstride[q]);
        if constexpr (SCALED) {
#pragma unroll
            for (int i = 0; i < SA; ++i) sa_nxt[i] = *reinterpret_cast<const int*>(sa_ptr[i] + t * 256);
#pragma unroll
            for (int j = 0; j < SB; ++j) sb_nxt[j] = *reinterpret_cast<const int*>(sb_ptr[j] + t * 256);
        }
    };
    auto store_stage = [&](int buf) {
        uint8_t* base = smem + buf * STAGE_BYTES;
#pragma unroll
        for (int q = 0; q < PER_WAVE; ++q) {
            const int f = wave + 4 * q;
            *reinterpret_cast<i32x4_t*>(base + f * 1024 + lane * 16) = stg[q];
        }
    };

    load_stage(0);
    store_stage(0);
    if constexpr (SCALED) {
#pragma unroll
        for (int i = 0; i < SA; ++i) sa_cur[i] = sa_nxt[i];
#pragma unroll
        for (int j = 0; j < SB; ++j) sb_cur[j] = sb_nxt[j];
    }
    __syncthreads();

    for (int t = 0; t < nstages; ++t) {
        const int buf = t & 1;
        if (t + 1 < nstages) load_stage(t + 1);
        const uint8_t* abase = smem + buf * STAGE_BYTES;
        const uint8_t* bbase = abase + A_FRAGS * 1024;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            i32x4_t af[MI][FA], bf[NJ][FB];
#pragma unroll
            for (int i = 0; i < MI; ++i) {
                const int rf = wm * MI + i;
#pragma unroll
                for (int h = 0; h < FA; ++h)
                    af[i][h] = *reinterpret_cast<const i32x4_t*>(abase + ((rf * 2 + ks) * FA + h) * 1024 + lane * 16);
            }
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int cf = wn * NJ + j;
#pragma unroll
                for (int h = 0; h < FB; ++h)
                    bf[j][h] = *reinterpret_cast<const i32x4_t*>(bbase + ((cf * 2 + ks) * FB + h) * 1024 + lane * 16);
            }
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    if constexpr (SCALED)
                        acc[i][j] = mma_step<KA, KB>(bf[j], af[i], acc[i][j], sb_cur[j >> 1],
                                                     ks * 2 + (j & 1), sa_cur[i >> 1], ks * 2 + (i & 1));
                    else
                        acc[i][j] = mma_step<KA, KB>(bf[j], af[i], acc[i][j], 0, 0, 0, 0);
                }
        }
        if (t + 1 < nstages) {
            // buf^1 was last read in stage t-1; every wave has passed the
            // barrier that ended stage t-1, so it is free to overwrite.
            store_stage(buf ^ 1);
            if constexpr (SCALED) {
#pragma unroll
                for (int i = 0; i < SA; ++i) sa_cur[i] = sa_nxt[i];
#pragma unroll
                for (int j = 0; j < SB; ++j) sb_cur[j] = sb_nxt[j];
            }
            __syncthreads();
        }
    }

    // ---- epilogue
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int m = m0 + wm * WM + i * 16 + (lane & 15);
            const int n = n0 + wn * WN + j * 16 + 4 * (lane >> 4);
            store_frag<OUT_F32>(p, acc[i][j], m, n);
        }
}

// ---------------------------------------------------------------------------
// Skinny (decode) kernel: HBM-bound streaming of B for small M.
// Block = NW waves on one 16-column B fragment.  Work unit = a k-pair (two
// MFMA k-steps = 256 MX / 64 bf16 elements), which is exactly what one scale
// dword covers, so every op_sel is an immediate.  Wave w takes pairs
// w, w+NW, ... of its K split with the next pair's loads in flight while the
// current one is multiplied; at the decode shapes every wave owns one or two
// pairs, so all of B is requested in the first few hundred cycles.
// Partial sums are reduced across waves through LDS; with a K split over
// blocks (gridDim.y > 1) the block result is atomically added to an f32
// workspace that a second kernel converts.
// ---------------------------------------------------------------------------
template <int KA, int MF, int NB>
struct SkinnyPair {
    static constexpr int FA = OpTraits<KA>::frags_per_step;
    static constexpr bool SCALED = OpTraits<KA>::scaled;
    static constexpr int SGRP = (MF + 1) / 2;
    static constexpr int SBN = (NB + 1) / 2;   // 32-row B scale groups
    i32x4_t b[2][NB];
    i32x4_t a[2][MF][FA];
    int sb[SBN];
    int sa[SGRP];
};

template <int KA, int MF, int NB, bool B_PRE, bool NT>
AA_DEV void skinny_load(SkinnyPair<KA, MF, NB>& d, int pr, const uint8_t* const* bsrc, const uint8_t* const* asrc,
                        const bool* arow_ok, const uint8_t* const* sbp, const uint8_t* const* sap) {
    using P = SkinnyPair<KA, MF, NB>;
    constexpr int A_STEP_BYTES = KA == kFp8 ? 128 : 64;
    constexpr int BSTEP = B_PRE ? 1024 : 64;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int s = 2 * pr + h;
#pragma unroll
        for (int j = 0; j < NB; ++j) d.b[h][j] = load_b<NT, i32x4_t>(bsrc[j] + (int64_t)s * BSTEP);
#pragma unroll
        for (int i = 0; i < MF; ++i)
#pragma unroll
            for (int f = 0; f < P::FA; ++f) {
                const i32x4_t v = *reinterpret_cast<const i32x4_t*>(asrc[i] + (int64_t)s * A_STEP_BYTES + f * 64);
                d.a[h][i][f] = arow_ok[i] ? v : i32x4_t{0, 0, 0, 0};
            }
    }
    if constexpr (P::SCALED) {
#pragma unroll
        for (int g = 0; g < P::SBN; ++g) d.sb[g] = load_b<NT, int>(sbp[g] + (int64_t)pr * 256);
#pragma unroll
        for (int g = 0; g < P::SGRP; ++g) d.sa[g] = *reinterpret_cast<const int*>(sap[g] + (int64_t)pr * 256);
    }
}

// BHALF0: which 16-column half of its 32-row B scale group the first
// column block covers (block j covers half BHALF0 + j)
template <int KA, int MF, int NB, int BHALF0>
AA_DEV void skinny_mma(const SkinnyPair<KA, MF, NB>& d, f32x4_t (*acc)[NB]) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < MF; ++i)
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                if constexpr (OpTraits<KA>::scaled) {
                    const int bh = (BHALF0 + j) & 1;
                    const int g = (BHALF0 + j) >> 1;
                    if (bh)
                        acc[i][j] = mma_step<KA, kFp4>(&d.b[h][j], d.a[h][i], acc[i][j], d.sb[g], h * 2 + 1,
                                                       d.sa[i >> 1], h * 2 + (i & 1));
                    else
                        acc[i][j] = mma_step<KA, kFp4>(&d.b[h][j], d.a[h][i], acc[i][j], d.sb[g], h * 2,
                                                       d.sa[i >> 1], h * 2 + (i & 1));
                } else {
                    acc[i][j] = mma_step<KA, KA>(&d.b[h][j], d.a[h][i], acc[i][j], 0, 0, 0, 0);
                }
            }
}

// NB column blocks of 16 per workgroup share each A fragment (NB = 2: the
// two halves of one 32-row B scale group, so one scale dword serves both)
// The skinny GEMM of one workgroup: column blocks bx * NB .. +NB, K split
// `by` (the __global__ below; also one half of the fused pair kernel)
template <int KA, int MF, int NW, bool B_PRE, bool SPLIT, bool OUT_F32, int NB, bool NT>
AA_DEV void skinny_body(const GemmParams& p, int bx, int by) {
    static_assert(NB == 1 || NB == 2, "one or two column blocks per workgroup");
    constexpr bool SCALED = OpTraits<KA>::scaled;
    constexpr int KPAIR = SCALED ? 256 : 64;               // elements per k-pair
    constexpr int SGRP = (MF + 1) / 2;                     // 32-row A scale groups
    constexpr int SBN = (NB + 1) / 2;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = bx * 16 * NB;
    const int total_pairs = p.K / KPAIR;
    const int p_begin = by * p.k_steps_per_split;   // k_steps_per_split counts pairs here
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
    const uint8_t* asrc[MF];
    bool arow_ok[MF];
#pragma unroll
    for (int i = 0; i < MF; ++i) {
        const int row = i * 16 + (lane & 15);
        arow_ok[i] = row < p.M;
        asrc[i] = p.A + (int64_t)min(row, p.M - 1) * p.lda + (lane >> 4) * 16;
    }
    const uint8_t* sbp[SBN];
    const uint8_t* sap[SGRP];
    if constexpr (SCALED) {
#pragma unroll
        for (int g = 0; g < SBN; ++g) {
            const int nb0 = min(n0 + 32 * g, (p.N - 1) / 16 * 16);
            sbp[g] = p.Bs + (int64_t)(nb0 / 32) * 32 * p.sb_stride + lane * 4;
        }
#pragma unroll
        for (int g = 0; g < SGRP; ++g)
            sap[g] = p.As + (int64_t)min(g, p.sa_groups - 1) * 32 * p.sa_stride + lane * 4;
    }

    f32x4_t acc[MF][NB];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // software pipeline: the next pair's loads are in flight while the
    // current pair is multiplied (a deeper register ring measured slower on
    // the bf16 decode shapes)
    auto run = [&](auto bh) {
        constexpr int BH = decltype(bh)::value;
        int pr = p_begin + wave;
        if (pr < p_end) {
            SkinnyPair<KA, MF, NB> cur;
            skinny_load<KA, MF, NB, B_PRE, NT>(cur, pr, bsrc, asrc, arow_ok, sbp, sap);
            for (pr += NW; pr < p_end; pr += NW) {
                SkinnyPair<KA, MF, NB> nxt;
                skinny_load<KA, MF, NB, B_PRE, NT>(nxt, pr, bsrc, asrc, arow_ok, sbp, sap);
                skinny_mma<KA, MF, NB, BH>(cur, acc);
                cur = nxt;
            }
            skinny_mma<KA, MF, NB, BH>(cur, acc);
        }
    };
    // NB = 2 starts on a 32-row group boundary; NB = 1 on either half
    if (NB == 1 && ((n0 / 16) & 1)) run(std::integral_constant<int, 1>{});
    else run(std::integral_constant<int, 0>{});

    __shared__ f32x4_t red[NW][MF * NB][64];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) red[wave][i * NB + j][lane] = acc[i][j];
    __syncthreads();
    for (int t = threadIdx.x; t < MF * NB * 64; t += 64 * NW) {
        const int ij = t / 64, l = t % 64;
        const int i = ij / NB, j = ij % NB;
        f32x4_t s = red[0][ij][l];
#pragma unroll
        for (int w = 1; w < NW; ++w) s += red[w][ij][l];
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

template <int KA, int MF, int NW, bool B_PRE, bool SPLIT, bool OUT_F32, int NB = 1, bool NT = false>
__global__ __launch_bounds__(64 * NW) void gemm_skinny_kernel(GemmParams p) {
    apply_batch(p);
    skinny_body<KA, MF, NW, B_PRE, SPLIT, OUT_F32, NB, NT>(p, blockIdx.x, blockIdx.y);
}

// Two skinny GEMMs of the same M in one grid (fused_gemm_afp4wfp4_a16w16 at
// decode sizes): workgroups [0, nblk_a) compute the MXFP4 GEMM `pa`, the rest
// the bf16 GEMM `pb`, one pass over K each (16-column blocks, 8 waves).
template <int MF, bool BPRE_A>
__global__ __launch_bounds__(512) void skinny_pair_kernel(GemmParams pa, GemmParams pb, int nblk_a) {
    if ((int)blockIdx.x < nblk_a)
        skinny_body<kFp4, MF, 8, BPRE_A, false, false, 1, false>(pa, blockIdx.x, 0);
    else
        skinny_body<kBf16, MF, 8, false, false, false, 1, false>(pb, blockIdx.x - nblk_a, 0);
}

// Skinny (decode) GEMM for short K: every wave owns 16*NB output columns and
// the whole K range, at most KP k-pairs.  All of a wave's loads (B, A and
// both scale tensors, KP register sets) are issued before its first MFMA and
// the wave stores its own columns: no split-K, no reduction through LDS, no
// barrier, one launch.  With K = 2048 (8 k-pairs) a wave keeps 8 x 2 KiB of
// B in flight, so the 448 waves of N = 7168 hold the whole weight in flight
// at once.  NWC independent waves per workgroup (consecutive column blocks).
template <int KA, int MF, int NB, int KP, bool B_PRE, bool OUT_F32, bool NT, int NWC>
__global__ __launch_bounds__(64 * NWC) void gemm_skinny_direct_kernel(GemmParams p) {
    static_assert(NB == 1 || NB == 2, "one or two column blocks per wave");
    apply_batch(p);
    constexpr bool SCALED = OpTraits<KA>::scaled;
    constexpr int KPAIR = SCALED ? 256 : 64;
    constexpr int SGRP = (MF + 1) / 2;
    constexpr int SBN = (NB + 1) / 2;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int n0 = (blockIdx.x * NWC + wave) * 16 * NB;
    if (n0 >= p.N) return;
    const int npairs = p.K / KPAIR;   // <= KP (checked on the host)

    const uint8_t* bsrc[NB];
#pragma unroll
    for (int j = 0; j < NB; ++j) {
        const int nb0 = min(n0 + 16 * j, (p.N - 1) / 16 * 16);
        if constexpr (B_PRE)
            bsrc[j] = p.B + (int64_t)nb0 * p.ldb + lane * 16;
        else
            bsrc[j] = p.B + (int64_t)min(nb0 + (lane & 15), p.N - 1) * p.ldb + (lane >> 4) * 16;
    }
    const uint8_t* asrc[MF];
    bool arow_ok[MF];
#pragma unroll
    for (int i = 0; i < MF; ++i) {
        const int row = i * 16 + (lane & 15);
        arow_ok[i] = row < p.M;
        asrc[i] = p.A + (int64_t)min(row, p.M - 1) * p.lda + (lane >> 4) * 16;
    }
    const uint8_t* sbp[SBN];
    const uint8_t* sap[SGRP];
    if constexpr (SCALED) {
#pragma unroll
        for (int g = 0; g < SBN; ++g) {
            const int nb0 = min(n0 + 32 * g, (p.N - 1) / 16 * 16);
            sbp[g] = p.Bs + (int64_t)(nb0 / 32) * 32 * p.sb_stride + lane * 4;
        }
#pragma unroll
        for (int g = 0; g < SGRP; ++g)
            sap[g] = p.As + (int64_t)min(g, p.sa_groups - 1) * 32 * p.sa_stride + lane * 4;
    }

    SkinnyPair<KA, MF, NB> st[KP];
#pragma unroll
    for (int u = 0; u < KP; ++u)
        if (u < npairs) skinny_load<KA, MF, NB, B_PRE, NT>(st[u], u, bsrc, asrc, arow_ok, sbp, sap);

    f32x4_t acc[MF][NB];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto run = [&](auto bh) {
        constexpr int BH = decltype(bh)::value;
#pragma unroll
        for (int u = 0; u < KP; ++u)
            if (u < npairs) skinny_mma<KA, MF, NB, BH>(st[u], acc);
    };
    if (NB == 1 && ((n0 / 16) & 1)) run(std::integral_constant<int, 1>{});
    else run(std::integral_constant<int, 0>{});
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) store_frag<OUT_F32>(p, acc[i][j], i * 16 + (lane & 15), n0 + 16 * j + 4 * (lane >> 4));
}

// f32 workspace -> output (+alpha, +bias) for the split-K skinny path.
template <bool OUT_F32>
__global__ __launch_bounds__(256) void splitk_finish_kernel(GemmParams p) {
    const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int64_t total = (int64_t)p.M * p.N;
    if (idx >= total) return;
    const int m = (int)(idx / p.N), n = (int)(idx % p.N);
    const f32x4_t v = *reinterpret_cast<const f32x4_t*>(p.ws + idx);
    store_frag<OUT_F32>(p, v, m, n);
}

// Sum of the `splits` f32 partial slices [splits][M][N] of a split tile
// GEMM (slice order fixed) -> output (+alpha, +bias).
template <bool OUT_F32>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmParams p, int splits) {
    const int64_t idx = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    const int64_t total = (int64_t)p.M * p.N;
    if (idx >= total) return;
    f32x4_t v = *reinterpret_cast<const f32x4_t*>(p.ws + idx);
    for (int s = 1; s < splits; ++s) v += *reinterpret_cast<const f32x4_t*>(p.ws + s * total + idx);
    const int m = (int)(idx / p.N), n = (int)(idx % p.N);
    store_frag<OUT_F32>(p, v, m, n);
}

template <int = 0>
__global__ __launch_bounds__(256) void fill_zero_kernel(float* p, int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i + 4 <= n) *reinterpret_cast<f32x4_t*>(p + i) = f32x4_t{0.f, 0.f, 0.f, 0.f};
    else
        for (int64_t j = i; j < n; ++j) p[j] = 0.f;
}

}  // namespace aiter_amd
