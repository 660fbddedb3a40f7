// Kernel instance registry of the scaled-GEMM family, shared by gemm.hip
// (dispatch, C-ABI) and the gemm_reg_*.hip units that instantiate the
// kernels (split so that the instantiations compile in parallel).
//
// Every kernel instance has a stable name and integer id (the `kernelName` /
// `kernelId` the tuned CSVs refer to); ids are assigned in registration
// order, which the parts keep: part_mx, part_bf16<false>, part_bf16<true>,
// part_persist_split, part_rest, part_direct, part_late.
#pragma once

#include <string>
#include <vector>

#include "gemm_kernels.h"
#include "mfma32.h"
#include "gemm_flat.h"
#include "gemm_flat_persist.h"
#include "gemm_lds_persist.h"
#include "gemm_skinny_lds.h"
#include "gemm_t32.h"

namespace aiter_amd {

enum Family : int { kA4W4 = 0, kA8W4 = 1, kA16W16 = 2 };

struct Variant {
    bool a_pre, b_pre, out_f32;
};

using LaunchFn = void (*)(const GemmParams&, dim3, hipStream_t);

struct Instance {
    int id;
    std::string name;
    Family fam;
    bool skinny;
    int bm, bn;   // tile: block tile; skinny: bm = 16*MF rows covered, bn = 16
    bool split;   // skinny split-K over blocks
    Variant var;
    LaunchFn fn;
    bool persistent = false;   // grid of min(tiles, CUs) workgroups walking the tiles
    int rank = 0;              // among skinny forms of one shape the heuristic takes the highest
    bool stream_k = false;     // skinny stream-K form: one workgroup per CU, partial blocks summed in place
};

template <int KA, int KB, int BM, int BN, bool AP, bool BP, bool OF>
void launch_tile(const GemmParams& p, dim3 grid, hipStream_t s) {
    gemm_tile_kernel<KA, KB, BM, BN, AP, BP, OF><<<grid, 256, 0, s>>>(p);
}

constexpr int kSkinnyWaves = 8;


template <int KA, int BM, bool OF = false, bool BP = true>
void launch_flat(const GemmParams& p, dim3 grid, hipStream_t s) {
    gemm_flat_kernel<KA, BM, OF, BP><<<grid, 256, 0, s>>>(p);
}

template <int KA, int BM, bool OF = false, bool BP = true>
void launch_flat_persist(const GemmParams& p, dim3 grid, hipStream_t s) {
    const bool short4 = p.K / FlatPersistCfg<KA, BM>::K_STAGE <= 4;
    if (p.alpha == 1.0f) {
        if (short4)
            gemm_flat_persist_kernel<KA, BM, OF, BP, false, false, true><<<grid, 256, 0, s>>>(p);
        else
            gemm_flat_persist_kernel<KA, BM, OF, BP, false, false><<<grid, 256, 0, s>>>(p);
    } else {
        if (short4)
            gemm_flat_persist_kernel<KA, BM, OF, BP, false, true, true><<<grid, 256, 0, s>>>(p);
        else
            gemm_flat_persist_kernel<KA, BM, OF, BP><<<grid, 256, 0, s>>>(p);
    }
}

template <bool BP>
void launch_lds_persist(const GemmParams& p, dim3 grid, hipStream_t s) {
    if (p.alpha == 1.0f)
        gemm_lds_persist_kernel<BP, false><<<grid, 256, 0, s>>>(p);
    else
        gemm_lds_persist_kernel<BP, true><<<grid, 256, 0, s>>>(p);
}

// B (e2m1 for the MX families, bf16 otherwise) large enough for nt loads
template <int KA>
bool b_streams(const GemmParams& p) {
    const int64_t elems = (int64_t)p.N * p.K;
    return (KA == kBf16 ? elems * 2 : elems / 2) >= kNtMinBytes;
}

template <int KA, bool BP, int BM, int BN, int WMW, bool OF = false, bool SPLIT = false>
void launch_t32(const GemmParams& p, dim3 grid, hipStream_t s) {
    if (p.tiles_m == 1 && b_streams<KA>(p))
        gemm_t32_kernel<KA, BP, BM, BN, WMW, OF, SPLIT, true><<<grid, 256, 0, s>>>(p);
    else
        gemm_t32_kernel<KA, BP, BM, BN, WMW, OF, SPLIT, false><<<grid, 256, 0, s>>>(p);
}

template <int KA, int MF, bool BP, bool SPLIT, bool OF, int NB = 1>
void launch_skinny(const GemmParams& p, dim3 grid, hipStream_t s) {
    if (b_streams<KA>(p))
        gemm_skinny_kernel<KA, MF, kSkinnyWaves, BP, SPLIT, OF, NB, true><<<grid, 64 * kSkinnyWaves, 0, s>>>(p);
    else
        gemm_skinny_kernel<KA, MF, kSkinnyWaves, BP, SPLIT, OF, NB, false><<<grid, 64 * kSkinnyWaves, 0, s>>>(p);
}

template <int KA, int MF, bool BP, int NB, int NW = kSkinnyWaves, int S = 2, bool BL = false>
void launch_skinny_alds(const GemmParams& p, dim3 grid, hipStream_t s) {
    // A (and a workgroup's B rows) are addressed through buffer descriptors
    // with 32-bit offsets
    AA_CHECK((int64_t)p.M * p.lda < (1LL << 31) && (int64_t)32 * p.ldb < (1LL << 31),
             "skinny through-LDS kernel: A or a 32-row B panel larger than 2 GiB");
    if (b_streams<KA>(p))
        gemm_skinny_alds_kernel<KA, MF, NW, BP, false, false, NB, S, BL, true><<<grid, 64 * NW, 0, s>>>(p);
    else
        gemm_skinny_alds_kernel<KA, MF, NW, BP, false, false, NB, S, BL, false><<<grid, 64 * NW, 0, s>>>(p);
}

// stream-K skinny kernel (row-major bf16 B): grid = workgroups sharing the
// units; p.ws holds 2 * grid.x partial slots, p.cnt the block counters
template <int MF, int NB, int NW, int S = 2, bool OF = false>
void launch_skinny_sk(const GemmParams& p, dim3 grid, hipStream_t s) {
    AA_CHECK(p.ws && p.cnt, "stream-K skinny kernel: no workspace");
    // lane offsets reach the rows of the last block past N
    AA_CHECK((int64_t)p.M * p.lda < (1LL << 31) && (int64_t)(p.N + 32) * p.ldb < (1LL << 31),
             "stream-K skinny kernel: A or B larger than 2 GiB");
    if (b_streams<kBf16>(p))
        gemm_skinny_sk_kernel<MF, NW, OF, NB, S, true><<<grid, 64 * NW, 0, s>>>(p);
    else
        gemm_skinny_sk_kernel<MF, NW, OF, NB, S, false><<<grid, 64 * NW, 0, s>>>(p);
}

// the short-K direct skinny kernel: KP k-pairs at most (K <= KP * 256 for
// the MX families), NWC waves of one column block each per workgroup (one:
// N = 7168 gives 448 workgroups, spread over all CUs); the launcher's grid
// counts column blocks
template <int KA, int MF, int NB, int KP, bool BP = true, bool OF = false, int NWC = 1>
void launch_skinny_direct(const GemmParams& p, dim3 grid, hipStream_t s) {
    constexpr int KPAIR = OpTraits<KA>::scaled ? 256 : 64;
    AA_CHECK(p.K / KPAIR <= KP, "direct skinny kernel: K = ", p.K, " is longer than its ", KP, " k-pairs");
    const dim3 g((grid.x + NWC - 1) / NWC, 1, grid.z);
    if (b_streams<KA>(p))
        gemm_skinny_direct_kernel<KA, MF, NB, KP, BP, OF, true, NWC><<<g, 64 * NWC, 0, s>>>(p);
    else
        gemm_skinny_direct_kernel<KA, MF, NB, KP, BP, OF, false, NWC><<<g, 64 * NWC, 0, s>>>(p);
}

// Registration in id order (see the file comment).
struct RegBuilder {
    std::vector<Instance>& reg;
    int id = 0;

    void tile(Family f, int bm, int bn, Variant v, LaunchFn fn, const char* fam) {
        std::string nm = std::string(fam) + "_tile_" + std::to_string(bm) + "x" + std::to_string(bn);
        if (v.a_pre) nm += "_apre";
        if (!v.b_pre) nm += "_bplain";
        if (v.out_f32) nm += "_f32";
        reg.push_back({id++, nm, f, false, bm, bn, false, v, fn});
    }
    void skinny(Family f, int mf, bool split, Variant v, LaunchFn fn, const char* fam, int bn = 16) {
        std::string nm = std::string(fam) + "_skinny_m" + std::to_string(16 * mf);
        if (bn != 16) nm += "_n" + std::to_string(bn);
        if (split) nm += "_splitk";
        if (v.a_pre) nm += "_apre";
        if (!v.b_pre) nm += "_bplain";
        if (v.out_f32) nm += "_f32";
        reg.push_back({id++, nm, f, true, 16 * mf, bn, split, v, fn});
    }
    // persistent form of a 256-column tile (gemm_flat_persist.h, gemm_lds_persist.h)
    void persist(Family f, int bm, Variant v, LaunchFn fn, const char* fam) {
        tile(f, bm, 256, v, fn, fam);
        reg.back().name += "_persist";
        reg.back().persistent = true;
    }
    // split-K form of a t32 tile (K over gridDim.y, f32 slices summed by splitk_reduce_kernel)
    void tsplit(Family f, int bm, int bn, Variant v, LaunchFn fn, const char* fam) {
        std::string nm = std::string(fam) + "_tile_" + std::to_string(bm) + "x" + std::to_string(bn) + "_splitk";
        if (v.a_pre) nm += "_apre";
        if (!v.b_pre) nm += "_bplain";
        if (v.out_f32) nm += "_f32";
        reg.push_back({id++, nm, f, false, bm, bn, true, v, fn});
    }
    // skinny kernel with operands copied through LDS (gemm_skinny_lds.h); the
    // heuristic takes the highest rank among the skinny forms of a shape
    void staged(Family f, int mf, Variant v, LaunchFn fn, const char* fam, int bn, const char* tag, int rank = 1) {
        skinny(f, mf, false, v, fn, fam, bn);
        reg.back().name += tag;
        reg.back().rank = rank;
    }

    void part_mx();                    // gemm_reg_mx.hip
    template <bool OF> void part_bf16();   // gemm_reg_bf16.hip (OF = false), gemm_reg_bf16_f32.hip (true)
    void part_persist_split();         // gemm_reg_split.hip
    void part_rest();                  // gemm_reg_rest.hip
    void part_direct();                // gemm_reg_direct.hip
    void part_late();                  // gemm_reg_late.hip
};

constexpr Variant kPre{false, true, false}, kPlain{false, false, false}, kPre32{false, true, true};
constexpr Variant kA8Pre{true, true, false};

}  // namespace aiter_amd
