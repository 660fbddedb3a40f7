// MoE token sorting for gfx950: groups the (token, slot) routing entries by
// expert, pads every expert's run to a multiple of the GEMM row block, and
// records the expert of each row block (aiter's moe_sorting_fwd,
// aiter/ops/moe_sorting.py:12-27; output format restated from the reference
// CPU sort op_tests/test_moe_sorting.py:45-98):
//
//   sorted_ids[p]        = slot << 24 | token, experts in order, tokens in
//                          increasing (token, slot) order inside an expert;
//                          padding = topk << 24 | M
//   sorted_weights[p]    = topk_weights[token, slot] (padding: 0)
//   sorted_expert_ids[b] = expert of row block b, renumbered over the experts
//                          the mask keeps (unused blocks: -1)
//   num_valid_ids        = {padded entry count, token count}
//
// The order inside an expert is fixed (a stable counting sort), so the output
// is deterministic.  Entries are processed in chunks of 1024 (one workgroup
// of 16 waves): each wave ranks its 64 entries among equal experts with a
// ballot per distinct expert, and per-wave counts in LDS give each wave its
// offset inside the chunk.  Up to kSingleChunks chunks run in one workgroup
// (count, scan, place); more take three launches: per-chunk counts, one scan
// over chunks and experts, and one placement workgroup per chunk.
#include "common.h"
#include "mx_quant.h"

namespace {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxE = 1024;
constexpr int kSingleChunks = 4;

struct SortParams {
    const int* topk_ids;
    const float* topk_w;
    int* sorted_ids;
    float* sorted_w;
    int* sorted_eids;
    int* num_valid;
    const int* expert_mask;   // [E], 0 drops the expert (may be null)
    const int* num_local;     // device token count (may be null)
    int* ws;                  // chunk counts [nchunks][E], then expert offsets [E]
    int64_t ids_stride, w_stride;   // elements per row of topk_ids / topk_weights
    int M, topk, E, bs, max_padded, max_blocks, nchunks;
};

struct SortSmem {
    int cnt[kMaxE];        // entries per expert
    int off[kMaxE + 1];    // padded start of each expert, then the total
    int base[kMaxE];       // next output position of each expert
    int scan[kMaxE];
    int lid[kMaxE];        // renumbered expert id
    uint8_t wcnt[kWaves][kMaxE];
};

__device__ __forceinline__ int local_tokens(const SortParams& p) {
    return p.num_local ? min(max(*p.num_local, 0), p.M) : p.M;
}

// expert of entry i (token i / topk, slot i % topk), -1 if dropped
__device__ __forceinline__ int expert_of(const SortParams& p, int i, int n) {
    if (i >= n) return -1;
    const int t = i / p.topk, s = i - t * p.topk;
    const int e = p.topk_ids[(int64_t)t * p.ids_stride + s];
    if (e < 0 || e >= p.E) return -1;
    if (p.expert_mask && p.expert_mask[e] == 0) return -1;
    return e;
}

// exclusive scan of v over the workgroup's threads (one value per thread):
// shuffles inside each wave, then one wave scans the 16 wave totals
__device__ int block_exclusive_scan(int v, int* buf) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    if (lane == 63) buf[w] = x;
    __syncthreads();
    if (w == 0) {
        int t = lane < kWaves ? buf[lane] : 0;
#pragma unroll
        for (int d = 1; d < kWaves; d <<= 1) {
            const int y = __shfl_up(t, d);
            if (lane >= d) t += y;
        }
        if (lane < kWaves) buf[lane] = t;
    }
    __syncthreads();
    const int r = (w ? buf[w - 1] : 0) + x - v;
    __syncthreads();
    return r;
}

// from sm.cnt: expert offsets, block -> expert table, padding entries,
// num_valid_ids; leaves sm.off / sm.lid set
__device__ void scan_experts(const SortParams& p, SortSmem& sm, int n_tokens) {
    const int e = threadIdx.x;
    const bool live = e < p.E;
    const bool kept = live && !(p.expert_mask && p.expert_mask[e] == 0);
    const int c = live ? sm.cnt[e] : 0;
    const int padded = (c + p.bs - 1) / p.bs * p.bs;
    const int start = block_exclusive_scan(padded, sm.scan);
    const int lid = block_exclusive_scan(kept ? 1 : 0, sm.scan);
    if (live) {
        sm.off[e] = start;
        sm.lid[e] = lid;
    }
    if (e == p.E - 1) sm.off[p.E] = start + padded;
    __syncthreads();
    const int total = sm.off[p.E];
    const int pad_id = (p.topk << 24) | p.M;
    (void)c;
    (void)pad_id;
    // padding entries: the whole list was filled with the padding id before
    // (fill_padding); placement overwrites the real entries
    if (live)
        for (int b = start / p.bs; b < (start + padded) / p.bs && b < p.max_blocks; ++b) p.sorted_eids[b] = lid;
    for (int b = total / p.bs + threadIdx.x; b < p.max_blocks; b += kThreads) p.sorted_eids[b] = -1;
    if (threadIdx.x == 0) {
        p.num_valid[0] = total;
        p.num_valid[1] = n_tokens;
    }
}

// positions [q0, q1) of sorted_ids / sorted_weights <- padding id / 0
// (coalesced; threads of `nthreads` starting at `t`)
__device__ void fill_padding(const SortParams& p, int64_t q0, int64_t q1, int t, int nthreads) {
    const int pad_id = (p.topk << 24) | p.M;
    for (int64_t q = q0 + t; q < q1; q += nthreads) {
        p.sorted_ids[q] = pad_id;
        p.sorted_w[q] = 0.0f;
    }
}

// places entries [c0, c0 + 1024) at sm.base[e] onward and advances sm.base;
// e_in >= -1: this thread's entry already resolved (expert, weight w_in)
__device__ void place_chunk(const SortParams& p, SortSmem& sm, int c0, int n, int e_in = -2, float w_in = 0.0f) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    reinterpret_cast<i32x4_t*>(&sm.wcnt[0][0])[tid] = i32x4_t{0, 0, 0, 0};
    static_assert(sizeof(sm.wcnt) == kThreads * 16, "one 16-byte clear per thread");
    __syncthreads();
    const int i = c0 + tid;
    const int e = e_in >= -1 ? e_in : expert_of(p, i, n);
    // rank among the lanes of this wave with the same expert and a lower lane
    uint64_t act = __ballot(e >= 0);
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int rank = 0;
    while (act) {
        const int leader = __builtin_ctzll(act);
        const int le = __builtin_amdgcn_readlane(e, leader);
        const uint64_t m = __ballot(e == le);
        if (e == le) rank = __popcll(m & below);
        if (lane == leader) sm.wcnt[w][le] = (uint8_t)__popcll(m);
        act &= ~m;
    }
    __syncthreads();
    if (e >= 0) {
        int pos = sm.base[e] + rank;
        for (int v = 0; v < w; ++v) pos += sm.wcnt[v][e];
        const int t = i / p.topk, s = i - t * p.topk;
        if (pos < p.max_padded) {
            p.sorted_ids[pos] = (s << 24) | t;
            p.sorted_w[pos] = e_in >= -1 ? w_in : p.topk_w[(int64_t)t * p.w_stride + s];
        }
    }
    __syncthreads();
    for (int x = tid; x < p.E; x += kThreads) {
        int add = 0;
        for (int v = 0; v < kWaves; ++v) add += sm.wcnt[v][x];
        sm.base[x] += add;
    }
    __syncthreads();
}

__global__ __launch_bounds__(kThreads) void moe_sort_single(SortParams p, uint8_t* zero_buf, int64_t zero_bytes) {
    __shared__ SortSmem sm;
    const int nt = local_tokens(p);
    const int n = nt * p.topk;
    // every chunk's entries stay in registers from one round of loads
    // (expert ids and weights of all chunks issued together), so neither the
    // count nor the placement of a later chunk waits on another load
    const int tid = threadIdx.x;
    int ev[kSingleChunks];
    float wv[kSingleChunks];
#pragma unroll
    for (int k = 0; k < kSingleChunks; ++k) {
        const int i = tid + k * kThreads;
        ev[k] = expert_of(p, i, n);
        wv[k] = 0.0f;
        if (i < n) {
            const int t = i / p.topk, s = i - t * p.topk;
            wv[k] = p.topk_w[(int64_t)t * p.w_stride + s];
        }
    }
    // a small moe_buf is cleared here rather than by a second launch
    for (int64_t b = (int64_t)tid * 16; b + 16 <= zero_bytes; b += kThreads * 16)
        *reinterpret_cast<i32x4_t*>(zero_buf + b) = i32x4_t{0, 0, 0, 0};
    for (int64_t b = zero_bytes / 16 * 16 + tid; b < zero_bytes; b += kThreads) zero_buf[b] = 0;
    fill_padding(p, 0, p.max_padded, tid, kThreads);   // ordered before placement by the barriers below
    for (int x = tid; x < kMaxE; x += kThreads) sm.cnt[x] = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSingleChunks; ++k)
        if (ev[k] >= 0) atomicAdd(&sm.cnt[ev[k]], 1);
    __syncthreads();
    scan_experts(p, sm, nt);
    for (int x = tid; x < p.E; x += kThreads) sm.base[x] = sm.off[x];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kSingleChunks; ++k)
        if (k == 0 || k * kThreads < n) place_chunk(p, sm, k * kThreads, n, ev[k], wv[k]);
}

__global__ __launch_bounds__(kThreads) void moe_sort_count(SortParams p) {
    __shared__ int cnt[kMaxE];
    const int n = local_tokens(p) * p.topk;
    // this chunk's share of the padding fill (placement runs in a later launch)
    const int64_t share = ((int64_t)p.max_padded + gridDim.x - 1) / gridDim.x;
    fill_padding(p, blockIdx.x * share, min<int64_t>((int64_t)(blockIdx.x + 1) * share, p.max_padded), threadIdx.x,
                 kThreads);
    for (int x = threadIdx.x; x < p.E; x += kThreads) cnt[x] = 0;
    __syncthreads();
    const int e = expert_of(p, blockIdx.x * kThreads + threadIdx.x, n);
    if (e >= 0) atomicAdd(&cnt[e], 1);
    __syncthreads();
    for (int x = threadIdx.x; x < p.E; x += kThreads) p.ws[(int64_t)blockIdx.x * p.E + x] = cnt[x];
}

__global__ __launch_bounds__(kThreads) void moe_sort_scan(SortParams p) {
    __shared__ SortSmem sm;
    const int e = threadIdx.x;
    if (e < p.E) {
        // chunk counts -> exclusive prefix over chunks (the chunk's start inside the expert)
        // 16 loads in flight per batch (the stores of a batch would otherwise
        // order every load behind the previous store)
        int run = 0;
        for (int c0 = 0; c0 < p.nchunks; c0 += 16) {
            int v[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = c0 + k < p.nchunks ? p.ws[(int64_t)(c0 + k) * p.E + e] : 0;
#pragma unroll
            for (int k = 0; k < 16; ++k)
                if (c0 + k < p.nchunks) {
                    p.ws[(int64_t)(c0 + k) * p.E + e] = run;
                    run += v[k];
                }
        }
        sm.cnt[e] = run;
    }
    __syncthreads();
    scan_experts(p, sm, local_tokens(p));
    if (e < p.E) p.ws[(int64_t)p.nchunks * p.E + e] = sm.off[e];
}

__global__ __launch_bounds__(kThreads) void moe_sort_place(SortParams p) {
    __shared__ SortSmem sm;
    const int n = local_tokens(p) * p.topk;
    for (int x = threadIdx.x; x < p.E; x += kThreads)
        sm.base[x] = p.ws[(int64_t)p.nchunks * p.E + x] + p.ws[(int64_t)blockIdx.x * p.E + x];
    __syncthreads();
    place_chunk(p, sm, blockIdx.x * kThreads, n);
}

__global__ __launch_bounds__(256) void fill_zero_kernel(uint8_t* dst, int64_t bytes) {
    const int64_t n16 = bytes / 16;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        reinterpret_cast<i32x4_t*>(dst)[i] = i32x4_t{0, 0, 0, 0};
    for (int64_t i = n16 * 16 + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < bytes; i += stride) dst[i] = 0;
}


// ---- decode: routing sort and the stage-1 activation quant in one launch ----
// (the fusion of aiter/ops/flydsl/kernels/moe_fused_route_quant_scatter.py,
// route map + MX quant + scale scatter, for this library's sorted list.)
// For at most kSQMaxEntries routed entries (one per thread of a workgroup),
// every workgroup ranks all entries itself (no cross-workgroup step) and
// then handles sorted row group blockIdx.x (32 positions): its sorted ids and
// weights, the MXFP4 quant of the tokens its rows name, and the shuffled
// 256-byte scale blocks of its rows.  A token's MXFP4 codes are written by
// the workgroup holding the token's first sorted position (or, where every
// workgroup quantises every token, split over the workgroups); workgroup 0
// writes the block -> expert table and num_valid_ids; the moe_buf clear is
// split over the workgroups.  Outputs equal moe_sorting_fwd followed by
// fused_dynamic_mx_quant_moe_sort (stage 1, RoundUp e8m0 from 1e-10, sorted
// weights given) at positions below num_valid_ids[0] (plus the rest of its
// last 32-row group); later positions of sorted_ids / sorted_weights and
// later scale groups are left unwritten, as is the row of a token whose
// entries were all dropped (no reader goes there).  A zero routing weight
// gives scale byte 0 at its position with the token row quantised as usual.
constexpr int kSQMaxEntries = 256;

struct SortQuantParams {
    SortParams s;               // no expert mask, no device token count
    const uint16_t* x;          // bf16 [M, K]
    int64_t x_stride;           // elements per row
    uint8_t* q;                 // fp4x2 [M, K / 2]
    int64_t q_stride;           // bytes per row
    uint8_t* q_scale;           // [pad32(max_padded), scale_n_pad], sorted and shuffled
    int scale_n, scale_n_pad;   // K / 32 and its pad to 8
    uint8_t* zero_buf;          // moe_buf (may be null)
    int64_t zero_bytes;
};

// the MXFP4 block of 32 bf16 values given as 4 x 16 loaded bytes
AA_DEV uint32_t sq_quant_block(const i32x4_t (&raw)[4], i32x4_t& o) {
    float v[32];
    uint32_t pr[16];
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = (uint32_t)raw[q][j];
            pr[4 * q + j] = d;
            v[8 * q + 2 * j] = __builtin_bit_cast(float, d << 16);
            v[8 * q + 2 * j + 1] = __builtin_bit_cast(float, d & 0xffff0000u);
        }
    return aiter_amd::mx::quant32_fp4<uint16_t, aiter_amd::mx::kRoundUp>(v, pr, 1e-10f, 1.0f / 6.0f, 0.25f, 0u, 2u, o);
}

// Up to 64 entries (one wave holds them all): wave 0 ranks the entries with a
// ballot per distinct expert (no histogram, scan or extra barrier) while the
// other waves quantise every token row, whose loads are issued first.
constexpr int kSQWaveEntries = 64;

__global__ __launch_bounds__(256) void moe_sort_quant_wave(SortQuantParams p) {
    extern __shared__ uint8_t tok_sc[];   // [M][scale_n_pad] e8m0 bytes of the token rows
    __shared__ int row_id[32];            // sorted entry of each row of the group (padding: pad id)
    __shared__ float row_w[32];
    __shared__ int s_total;
    const SortParams& s = p.s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = s.M * s.topk;
    const int grp = blockIdx.x, ngrp = gridDim.x;
    const int pad_id = (s.topk << 24) | s.M;

    // wave 0: entry `lane` (expert -1: none or dropped)
    int e = -1;
    float w = 0.0f;
    if (wave == 0) {
        e = expert_of(s, lane, n);
        if (lane < n) w = s.topk_w[(int64_t)(lane / s.topk) * s.w_stride + lane % s.topk];
    }
    // this workgroup's share of the moe_buf clear
    if (p.zero_bytes > 0) {
        const int64_t units = p.zero_bytes / 16, per = (units + ngrp - 1) / ngrp;
        for (int64_t u = grp * per + tid; u < min(units, (int64_t)(grp + 1) * per); u += 256)
            reinterpret_cast<i32x4_t*>(p.zero_buf)[u] = i32x4_t{0, 0, 0, 0};
        if (grp == 0)
            for (int64_t b = units * 16 + tid; b < p.zero_bytes; b += 256) p.zero_buf[b] = 0;
    }
    // token rows: item (token, block y), up to 4 per thread with their loads in flight together
    const int items = s.M * p.scale_n;
    for (int b0 = 0; b0 < items; b0 += 4 * 256) {
        i32x4_t raw[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int it = b0 + 256 * k + tid;
            if (it < items) {
                const int t = it / p.scale_n, y = it - t * p.scale_n;
                const i32x4_t* src = reinterpret_cast<const i32x4_t*>(p.x + t * p.x_stride + (int64_t)y * 32);
#pragma unroll
                for (int c = 0; c < 4; ++c) raw[k][c] = src[c];
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int it = b0 + 256 * k + tid;
            if (it >= items) continue;
            const int t = it / p.scale_n, y = it - t * p.scale_n;
            float v[32];
            uint32_t pr[16];
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t d = (uint32_t)raw[k][c][j];
                    pr[4 * c + j] = d;
                    v[8 * c + 2 * j] = __builtin_bit_cast(float, d << 16);
                    v[8 * c + 2 * j + 1] = __builtin_bit_cast(float, d & 0xffff0000u);
                }
            i32x4_t o;
            const uint32_t byte =
                aiter_amd::mx::quant32_fp4<uint16_t, aiter_amd::mx::kRoundUp>(v, pr, 1e-10f, 1.0f / 6.0f, 0.25f, 0u, 2u, o);
            tok_sc[t * p.scale_n_pad + y] = (uint8_t)byte;
            if (it % ngrp == grp) *reinterpret_cast<i32x4_t*>(p.q + t * p.q_stride + (int64_t)y * 16) = o;
        }
    }
    for (int i = tid; i < s.M * (p.scale_n_pad - p.scale_n); i += 256) {
        const int t = i / (p.scale_n_pad - p.scale_n);
        tok_sc[t * p.scale_n_pad + p.scale_n + i % (p.scale_n_pad - p.scale_n)] = 0;
    }
    if (wave == 0) {
        // rank: position = padded counts of the smaller experts + entries of
        // the same expert on lower lanes (entry order = token, slot order)
        uint64_t act = __ballot(e >= 0);
        const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
        int before = 0, rank = 0, mine = 0, total = 0;
        while (act) {
            const int leader = __builtin_ctzll(act);
            const int le = __builtin_amdgcn_readlane(e, leader);
            const uint64_t m = __ballot(e == le);
            const int pc = (__popcll(m) + s.bs - 1) / s.bs * s.bs;
            if (e == le) {
                rank = __popcll(m & below);
                mine = pc;
            }
            if (e > le) before += pc;
            total += pc;
            act &= ~m;
        }
        const int pos = before + rank;
        if (lane < 32) {
            row_id[lane] = pad_id;
            row_w[lane] = 0.0f;
        }
        if (e >= 0 && pos >= 32 * grp && pos < 32 * grp + 32) {
            const int t = lane / s.topk;
            row_id[pos - 32 * grp] = ((lane - t * s.topk) << 24) | t;
            row_w[pos - 32 * grp] = w;
        }
        if (lane == 0) s_total = total;
        if (grp == 0) {
            // the expert's row blocks (the first entry of each expert writes them)
            if (e >= 0 && rank == 0)
                for (int b = before / s.bs; b < (before + mine) / s.bs && b < s.max_blocks; ++b) s.sorted_eids[b] = e;
            if (lane == 0) {
                s.num_valid[0] = total;
                s.num_valid[1] = s.M;
            }
        }
    }
    __syncthreads();
    const int total = s_total;
    if (grp == 0)
        for (int b = total / s.bs + tid; b < s.max_blocks; b += 256) s.sorted_eids[b] = -1;
    if (32 * grp >= total) return;
    if (tid < 32 && 32 * grp + tid < s.max_padded) {
        s.sorted_ids[32 * grp + tid] = row_id[tid];
        s.sorted_w[32 * grp + tid] = row_w[tid];
    }
    // the group's scale blocks: 16-byte piece w16 of column octet y8 holds
    // rows 4(w16 % 4) + (b >> 2) + 16(b & 1), columns 8 y8 + w16 / 4 + 4((b >> 1) & 1)
    // for its bytes b (the mx_scale_shuffle_idx layout)
    for (int c = tid; c < 2 * p.scale_n_pad; c += 256) {
        const int y8 = c >> 4, w16 = c & 15;
        uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const int xr = 4 * (w16 & 3) + (b >> 2) + 16 * (b & 1);
            const int yy = (w16 >> 2) + 4 * ((b >> 1) & 1);
            const int id = row_id[xr];
            const int t = id & 0xffffff, slot = (int)((unsigned)id >> 24);
            const bool valid = 32 * grp + xr < total && t < s.M && slot < s.topk && row_w[xr] != 0.0f;
            const uint32_t byte = valid ? tok_sc[t * p.scale_n_pad + 8 * y8 + yy] : 0u;
            d[b >> 2] |= byte << (8 * (b & 3));
        }
        *reinterpret_cast<i32x4_t*>(p.q_scale + (int64_t)grp * 32 * p.scale_n_pad + y8 * 256 + w16 * 16) =
            i32x4_t{(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
    }
}

// PRE: every workgroup loads and quantises all token rows, the loads issued
// before the ranking (tokens * K/32 <= 1024: at most 4 blocks per thread);
// otherwise a workgroup quantises the tokens of its rows after the ranking.
template <bool PRE>
__global__ __launch_bounds__(256) void moe_sort_quant_small(SortQuantParams p) {
    // e8m0 bytes of the quantised tokens: [M] (PRE) or [32] (the group's tokens) x scale_n_pad
    extern __shared__ uint8_t tok_sc[];
    __shared__ __attribute__((aligned(16))) uint8_t wcnt[4][kMaxE];   // entries per (wave, expert)
    __shared__ int off[kMaxE];                                        // padded start of each expert
    __shared__ int scan_buf[4];
    __shared__ int first_pos[kSQMaxEntries];                          // smallest sorted position of each token
    __shared__ int row_id[32];                                        // entry of each row of the group (padding: pad id)
    __shared__ float row_w[32];
    __shared__ int row_tix[32];                                       // index of the row's token in gtok
    __shared__ int gtok[32];                                          // distinct tokens of the group's rows
    __shared__ int s_ntok;
    const SortParams& s = p.s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = s.M * s.topk;
    const int grp = blockIdx.x, ngrp = gridDim.x;
    const int pad_id = (s.topk << 24) | s.M;

    // entry `tid` (expert -1: none or dropped)
    const int e = expert_of(s, tid, n);
    const float w = tid < n ? s.topk_w[(int64_t)(tid / s.topk) * s.w_stride + tid % s.topk] : 0.0f;
    // PRE: all token rows, item (token, block y) = tid + 256 k
    i32x4_t raw[PRE ? 4 : 1][4];
    const int pre_items = PRE ? s.M * p.scale_n : 0;
    if constexpr (PRE) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int it = 256 * k + tid;
            if (it < pre_items) {
                const int t = it / p.scale_n, y = it - t * p.scale_n;
                const i32x4_t* src = reinterpret_cast<const i32x4_t*>(p.x + t * p.x_stride + (int64_t)y * 32);
#pragma unroll
                for (int q = 0; q < 4; ++q) raw[k][q] = src[q];
            }
        }
    }
    // this workgroup's share of the moe_buf clear
    if (p.zero_bytes > 0) {
        const int64_t units = p.zero_bytes / 16, per = (units + ngrp - 1) / ngrp;
        for (int64_t u = grp * per + tid; u < min(units, (int64_t)(grp + 1) * per); u += 256)
            reinterpret_cast<i32x4_t*>(p.zero_buf)[u] = i32x4_t{0, 0, 0, 0};
        if (grp == 0)
            for (int64_t b = units * 16 + tid; b < p.zero_bytes; b += 256) p.zero_buf[b] = 0;
    }
    static_assert(sizeof(wcnt) == 256 * 16, "one 16-byte clear per thread");
    reinterpret_cast<i32x4_t*>(&wcnt[0][0])[tid] = i32x4_t{0, 0, 0, 0};
    if (tid < s.M) first_pos[tid] = 0x7fffffff;
    if (tid < 32) {
        row_id[tid] = pad_id;
        row_w[tid] = 0.0f;
        row_tix[tid] = 0;
    }
    __syncthreads();
    // in-wave rank among equal experts and per-wave counts: one ballot per
    // distinct expert of the wave
    int rank = 0;
    {
        uint64_t act = __ballot(e >= 0);
        const uint64_t below = lane ? (~0ull >> (64 - lane)) : 0ull;
        while (act) {
            const int leader = __builtin_ctzll(act);
            const int le = __builtin_amdgcn_readlane(e, leader);
            const uint64_t m = __ballot(e == le);
            if (e == le) rank = __popcll(m & below);
            if (lane == leader) wcnt[wave][le] = (uint8_t)__popcll(m);
            act &= ~m;
        }
    }
    __syncthreads();
    // padded count of experts 4 tid .. 4 tid + 3, exclusive scan over the
    // workgroup -> each expert's padded start
    int pc[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int x = 4 * tid + k;
        const int c = x < s.E ? wcnt[0][x] + wcnt[1][x] + wcnt[2][x] + wcnt[3][x] : 0;
        pc[k] = (c + s.bs - 1) / s.bs * s.bs;
        sum += pc[k];
    }
    int incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(incl, d);
        if (lane >= d) incl += y;
    }
    if (lane == 63) scan_buf[wave] = incl;
    __syncthreads();
    int base = 0;
    for (int v = 0; v < wave; ++v) base += scan_buf[v];
    const int total = scan_buf[0] + scan_buf[1] + scan_buf[2] + scan_buf[3];
    {
        int o = base + incl - sum;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int x = 4 * tid + k;
            if (x < s.E) off[x] = o;
            // workgroup 0: the expert's row blocks
            if (grp == 0 && x < s.E)
                for (int b = o / s.bs; b < (o + pc[k]) / s.bs && b < s.max_blocks; ++b) s.sorted_eids[b] = x;
            o += pc[k];
        }
    }
    if (grp == 0) {
        for (int b = total / s.bs + tid; b < s.max_blocks; b += 256) s.sorted_eids[b] = -1;
        if (tid == 0) {
            s.num_valid[0] = total;
            s.num_valid[1] = s.M;
        }
    }
    __syncthreads();
    if (e >= 0) {
        int pos = off[e] + rank;
        for (int v = 0; v < wave; ++v) pos += wcnt[v][e];
        atomicMin(&first_pos[tid / s.topk], pos);
        if (pos >= 32 * grp && pos < 32 * grp + 32) {
            const int t = tid / s.topk;
            row_id[pos - 32 * grp] = ((tid - t * s.topk) << 24) | t;
            row_w[pos - 32 * grp] = w;
        }
    }
    if constexpr (PRE) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int it = 256 * k + tid;
            if (it >= pre_items) continue;
            const int t = it / p.scale_n, y = it - t * p.scale_n;
            i32x4_t o;
            tok_sc[t * p.scale_n_pad + y] = (uint8_t)sq_quant_block(raw[k], o);
            if (it % ngrp == grp) *reinterpret_cast<i32x4_t*>(p.q + t * p.q_stride + (int64_t)y * 16) = o;
        }
        for (int i = tid; i < s.M * (p.scale_n_pad - p.scale_n); i += 256) {
            const int t = i / (p.scale_n_pad - p.scale_n);
            tok_sc[t * p.scale_n_pad + p.scale_n + i % (p.scale_n_pad - p.scale_n)] = 0;
        }
    }
    __syncthreads();
    if (32 * grp >= total) return;
    if (tid < 32 && 32 * grp + tid < s.max_padded) {
        s.sorted_ids[32 * grp + tid] = row_id[tid];
        s.sorted_w[32 * grp + tid] = row_w[tid];
    }
    if constexpr (!PRE) {
        // the group's distinct tokens (wave 0, lane = row): one ballot per
        // distinct token numbers them in order of first appearance
        if (wave == 0) {
            int tok = -1;
            if (lane < 32) {
                const int id = row_id[lane];
                const int t = id & 0xffffff, slot = (int)((unsigned)id >> 24);
                if (32 * grp + lane < total && t < s.M && slot < s.topk) tok = t;
            }
            uint64_t act = __ballot(tok >= 0);
            int nt = 0;
            while (act) {
                const int leader = __builtin_ctzll(act);
                const int lt = __builtin_amdgcn_readlane(tok, leader);
                const uint64_t m = __ballot(tok == lt);
                if (tok == lt) row_tix[lane] = nt;
                if (lane == leader) gtok[nt] = lt;
                ++nt;
                act &= ~m;
            }
            if (lane == 0) s_ntok = nt;
        }
        __syncthreads();
        // quantise the group's tokens: item (token index, block y), up to 4
        // per thread with their loads in flight together; a token's codes
        // come from the workgroup holding its first sorted position
        const int ntok = s_ntok;
        const int items = ntok * p.scale_n;
        for (int b0 = 0; b0 < items; b0 += 4 * 256) {
            i32x4_t rw[4][4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int it = b0 + 256 * k + tid;
                if (it < items) {
                    const int ti = it / p.scale_n, y = it - ti * p.scale_n;
                    const i32x4_t* src =
                        reinterpret_cast<const i32x4_t*>(p.x + gtok[ti] * p.x_stride + (int64_t)y * 32);
#pragma unroll
                    for (int q = 0; q < 4; ++q) rw[k][q] = src[q];
                }
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int it = b0 + 256 * k + tid;
                if (it >= items) continue;
                const int ti = it / p.scale_n, y = it - ti * p.scale_n;
                const int t = gtok[ti];
                i32x4_t o;
                tok_sc[ti * p.scale_n_pad + y] = (uint8_t)sq_quant_block(rw[k], o);
                if (first_pos[t] / 32 == grp) *reinterpret_cast<i32x4_t*>(p.q + t * p.q_stride + (int64_t)y * 16) = o;
            }
        }
        for (int i = tid; i < ntok * (p.scale_n_pad - p.scale_n); i += 256) {
            const int ti = i / (p.scale_n_pad - p.scale_n);
            tok_sc[ti * p.scale_n_pad + p.scale_n + i % (p.scale_n_pad - p.scale_n)] = 0;
        }
        __syncthreads();
    }
    // the group's scale blocks: 16-byte piece w16 of column octet y8 holds
    // rows 4(w16 % 4) + (b >> 2) + 16(b & 1), columns 8 y8 + w16 / 4 + 4((b >> 1) & 1)
    // for its bytes b (the mx_scale_shuffle_idx layout)
    for (int c2 = tid; c2 < 2 * p.scale_n_pad; c2 += 256) {
        const int y8 = c2 >> 4, w16 = c2 & 15;
        uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int b = 0; b < 16; ++b) {
            const int xr = 4 * (w16 & 3) + (b >> 2) + 16 * (b & 1);
            const int yy = (w16 >> 2) + 4 * ((b >> 1) & 1);
            const int id = row_id[xr];
            const int t = id & 0xffffff, slot = (int)((unsigned)id >> 24);
            const bool valid = 32 * grp + xr < total && t < s.M && slot < s.topk && row_w[xr] != 0.0f;
            const int ti = PRE ? t : row_tix[xr];
            const uint32_t byte = valid ? tok_sc[ti * p.scale_n_pad + 8 * y8 + yy] : 0u;
            d[b >> 2] |= byte << (8 * (b & 3));
        }
        *reinterpret_cast<i32x4_t*>(p.q_scale + (int64_t)grp * 32 * p.scale_n_pad + y8 * 256 + w16 * 16) =
            i32x4_t{(int)d[0], (int)d[1], (int)d[2], (int)d[3]};
    }
}
}  // namespace

// Checks the routing inputs and sorted outputs of a sort (the moe_sorting_fwd
// contract) and fills the kernel parameters.
static SortParams sort_params(aiter_tensor_t* topk_ids, aiter_tensor_t* topk_weights,
                              aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_weights,
                              aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids, int num_experts,
                              int unit_size, aiter_tensor_t* local_expert_mask, aiter_tensor_t* num_local_tokens) {
    using namespace aiter_amd;
    check_tensor(topk_ids, "topk_ids", 2);
    check_tensor(topk_weights, "topk_weights", 2);
    check_tensor(sorted_token_ids, "sorted_token_ids", 1);
    check_tensor(sorted_weights, "sorted_weights", 1);
    check_tensor(sorted_expert_ids, "sorted_expert_ids", 1);
    check_tensor(num_valid_ids, "num_valid_ids", 1);
    AA_CHECK(topk_ids->dtype == AITER_DTYPE_i32, "topk_ids must be int32");
    AA_CHECK(topk_weights->dtype == AITER_DTYPE_fp32, "topk_weights must be float32");
    AA_CHECK(sorted_token_ids->dtype == AITER_DTYPE_i32 && sorted_expert_ids->dtype == AITER_DTYPE_i32 &&
                 num_valid_ids->dtype == AITER_DTYPE_i32,
             "sorted_token_ids, sorted_expert_ids and num_valid_ids must be int32");
    AA_CHECK(sorted_weights->dtype == AITER_DTYPE_fp32, "sorted_weights must be float32");
    AA_CHECK(topk_ids->strides[1] == 1 && topk_weights->strides[1] == 1, "topk tensors need unit column stride");
    const int M = (int)topk_ids->shape[0], topk = (int)topk_ids->shape[1];
    AA_CHECK(topk_weights->shape[0] == M && topk_weights->shape[1] == topk, "topk_weights shape != topk_ids shape");
    AA_CHECK(num_experts >= 1 && num_experts <= kMaxE, "num_experts must be in [1, ", kMaxE, "], got ", num_experts);
    AA_CHECK(unit_size >= 1, "unit_size must be positive");
    AA_CHECK(topk >= 1 && topk < 128 && M < (1 << 24), "topk must be in [1, 127] and tokens < 2^24");
    const int64_t max_padded = (int64_t)M * topk + (int64_t)num_experts * unit_size - topk;
    const int64_t max_blocks = (max_padded + unit_size - 1) / unit_size;
    AA_CHECK(sorted_token_ids->numel >= (size_t)max_padded && sorted_weights->numel >= (size_t)max_padded,
             "sorted_token_ids / sorted_weights need ", max_padded, " entries");
    AA_CHECK(sorted_expert_ids->numel >= (size_t)max_blocks, "sorted_expert_ids needs ", max_blocks, " entries");
    AA_CHECK(num_valid_ids->numel >= 2, "num_valid_ids needs 2 entries");
    if (local_expert_mask) {
        AA_CHECK(local_expert_mask->dtype == AITER_DTYPE_i32 && local_expert_mask->numel >= (size_t)num_experts,
                 "local_expert_mask must be int32 with num_experts entries");
    }
    if (num_local_tokens) AA_CHECK(num_local_tokens->dtype == AITER_DTYPE_i32, "num_local_tokens must be int32");

    SortParams p{};
    p.topk_ids = static_cast<const int*>(topk_ids->ptr);
    p.topk_w = static_cast<const float*>(topk_weights->ptr);
    p.sorted_ids = static_cast<int*>(sorted_token_ids->ptr);
    p.sorted_w = static_cast<float*>(sorted_weights->ptr);
    p.sorted_eids = static_cast<int*>(sorted_expert_ids->ptr);
    p.num_valid = static_cast<int*>(num_valid_ids->ptr);
    p.expert_mask = local_expert_mask ? static_cast<const int*>(local_expert_mask->ptr) : nullptr;
    p.num_local = num_local_tokens ? static_cast<const int*>(num_local_tokens->ptr) : nullptr;
    p.ids_stride = topk_ids->strides[0];
    p.w_stride = topk_weights->strides[0];
    p.M = M;
    p.topk = topk;
    p.E = num_experts;
    p.bs = unit_size;
    p.max_padded = (int)max_padded;
    p.max_blocks = (int)max_blocks;
    return p;
}

extern "C" {

int moe_sorting_fwd(aiter_tensor_t* topk_ids, aiter_tensor_t* topk_weights, aiter_tensor_t* sorted_token_ids,
                    aiter_tensor_t* sorted_weights, aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                    aiter_tensor_t* moe_buf, int num_experts, int unit_size, aiter_tensor_t* local_expert_mask,
                    aiter_tensor_t* num_local_tokens, int dispatch_policy, aiter_stream_t stream) {
    using namespace aiter_amd;
    return safe_call([&] {
        check_tensor(topk_ids, "topk_ids", 2);
        DeviceGuard g(topk_ids->device_id);
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        AA_CHECK(dispatch_policy == 0, "only dispatch_policy 0 is supported");
        SortParams p = sort_params(topk_ids, topk_weights, sorted_token_ids, sorted_weights, sorted_expert_ids,
                                   num_valid_ids, num_experts, unit_size, local_expert_mask, num_local_tokens);
        const int M = p.M, topk = p.topk;
        const int64_t entries = (int64_t)M * topk;
        p.nchunks = (int)((entries + kThreads - 1) / kThreads);
        const int64_t buf_bytes =
            (moe_buf && moe_buf->numel > 0) ? (int64_t)moe_buf->numel * (int64_t)dtype_size(moe_buf->dtype) : 0;
        const bool zero_inside = p.nchunks <= kSingleChunks && buf_bytes <= (1 << 20);
        if (p.nchunks <= kSingleChunks) {
            moe_sort_single<<<1, kThreads, 0, st>>>(p, zero_inside && buf_bytes ? static_cast<uint8_t*>(moe_buf->ptr)
                                                                                  : nullptr,
                                                    zero_inside ? buf_bytes : 0);
        } else {
            p.ws = static_cast<int*>(
                lib_workspace(topk_ids->device_id, st, (size_t)(p.nchunks + 1) * num_experts * sizeof(int)));
            moe_sort_count<<<p.nchunks, kThreads, 0, st>>>(p);
            moe_sort_scan<<<1, kThreads, 0, st>>>(p);
            moe_sort_place<<<p.nchunks, kThreads, 0, st>>>(p);
        }
        AA_HIP(hipGetLastError());
        if (buf_bytes > 0 && !zero_inside) {
            const int64_t bytes = buf_bytes;
            const int64_t blocks = std::min<int64_t>((bytes / 16 + 255) / 256 + 1, 4096);
            fill_zero_kernel<<<(unsigned)blocks, 256, 0, st>>>(static_cast<uint8_t*>(moe_buf->ptr), bytes);
            AA_HIP(hipGetLastError());
        }
    });
}

int moe_sorting_mx_quant(aiter_tensor_t* topk_ids, aiter_tensor_t* topk_weights, aiter_tensor_t* hidden_states,
                         aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_weights,
                         aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids, aiter_tensor_t* moe_buf,
                         aiter_tensor_t* a_out, aiter_tensor_t* a_scale, int num_experts, int unit_size,
                         aiter_stream_t stream) {
    using namespace aiter_amd;
    return safe_call([&] {
        check_tensor(topk_ids, "topk_ids", 2);
        check_tensor(hidden_states, "hidden_states", 2);
        check_tensor(a_out, "a_out", 2);
        check_tensor(a_scale, "a_scale");
        DeviceGuard g(topk_ids->device_id);
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        SortQuantParams q{};
        q.s = sort_params(topk_ids, topk_weights, sorted_token_ids, sorted_weights, sorted_expert_ids, num_valid_ids,
                          num_experts, unit_size, nullptr, nullptr);
        const int M = q.s.M;
        const int64_t n = (int64_t)M * q.s.topk;
        AA_CHECK(n <= kSQMaxEntries, "moe_sorting_mx_quant: at most ", kSQMaxEntries, " routed entries, got ", n);
        AA_CHECK(hidden_states->dtype == AITER_DTYPE_bf16, "hidden_states must be bf16");
        const int64_t K = cols_2d(hidden_states);
        AA_CHECK(hidden_states->shape[0] == M, "hidden_states must have ", M, " rows");
        AA_CHECK(K > 0 && K % 32 == 0, "hidden_states columns must be a positive multiple of 32");
        AA_CHECK(hidden_states->strides[1] == 1 && hidden_states->strides[0] % 8 == 0 &&
                     ((uintptr_t)hidden_states->ptr & 15) == 0,
                 "hidden_states rows must be contiguous and 16-byte aligned");
        AA_CHECK(is_byte_type(a_out->dtype) && a_out->shape[0] == M && a_out->shape[1] == K / 2 &&
                     a_out->strides[1] == 1 && a_out->strides[0] % 16 == 0 && ((uintptr_t)a_out->ptr & 15) == 0,
                 "a_out must be fp4x2 [", M, ", ", K / 2, "] with 16-byte aligned rows");
        const int scale_n = (int)(K / 32), scale_n_pad = (scale_n + 7) / 8 * 8;
        const int64_t sorted_rows = ((int64_t)q.s.max_padded + 31) / 32 * 32;
        AA_CHECK(is_byte_type(a_scale->dtype) && (int64_t)a_scale->numel >= sorted_rows * scale_n_pad &&
                     ((uintptr_t)a_scale->ptr & 15) == 0,
                 "a_scale needs [pad32(len(sorted_token_ids)), ", scale_n_pad, "] bytes, 16-byte aligned");
        AA_CHECK(32 * (int64_t)scale_n_pad <= 65536, "moe_sorting_mx_quant: K must be at most 65536");
        // up to 64 entries: one wave ranks them, every workgroup quantises
        // all token rows; otherwise all token rows are loaded before the
        // ranking when they are at most 4 32-element blocks per thread
        const bool one_wave = n <= kSQWaveEntries && (int64_t)M * scale_n_pad <= 32768;
        const bool pre = (int64_t)M * scale_n <= 1024;
        const int64_t lds = (one_wave || pre ? M : 32) * (int64_t)scale_n_pad;
        q.x = static_cast<const uint16_t*>(hidden_states->ptr);
        q.x_stride = hidden_states->strides[0];
        q.q = static_cast<uint8_t*>(a_out->ptr);
        q.q_stride = a_out->strides[0];
        q.q_scale = static_cast<uint8_t*>(a_scale->ptr);
        q.scale_n = scale_n;
        q.scale_n_pad = scale_n_pad;
        if (moe_buf && moe_buf->numel > 0) {
            AA_CHECK(((uintptr_t)moe_buf->ptr & 15) == 0, "moe_buf must be 16-byte aligned");
            q.zero_buf = static_cast<uint8_t*>(moe_buf->ptr);
            q.zero_bytes = (int64_t)moe_buf->numel * (int64_t)dtype_size(moe_buf->dtype);
        }
        if (M == 0) {
            moe_sort_single<<<1, kThreads, 0, st>>>(q.s, q.zero_buf, q.zero_bytes);
            AA_HIP(hipGetLastError());
            return;
        }
        // every sorted position below num_valid_ids[0] is in one of these groups:
        // the padded count is at most entries * unit_size (and the list length)
        const int64_t bound = std::min<int64_t>(n * unit_size, q.s.max_padded);
        const unsigned groups = (unsigned)std::max<int64_t>(1, (bound + 31) / 32);
        if (one_wave)
            moe_sort_quant_wave<<<groups, 256, (size_t)lds, st>>>(q);
        else if (pre)
            moe_sort_quant_small<true><<<groups, 256, (size_t)lds, st>>>(q);
        else
            moe_sort_quant_small<false><<<groups, 256, (size_t)lds, st>>>(q);
        AA_HIP(hipGetLastError());
    });
}

}  // extern "C"
