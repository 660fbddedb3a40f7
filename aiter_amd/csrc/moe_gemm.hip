// Host side of the MoE grouped GEMMs (stage 1: gate/up GEMM + activation,
// stage 2: down GEMM + weighted scatter-add), MXFP4 weights with per-1x32 e8m0
// scales and MXFP4 (a4w4) or MXFP8 (a8w4) activations.  The kernels are the
// flat tile kernel's MoE stages (gemm_flat.h).  Entry points keep the argument
// lists of the reference's ck_moe_stage1 / ck_moe_stage2
// (aiter/ops/moe_op.py:350-394).
#include <cstdlib>
#include <string>

#include "gemm_kernels.h"
#include "mfma32.h"
#include "gemm_flat.h"
#include "moe_stage2.h"

namespace {

using namespace aiter_amd;

struct StageArgs {
    aiter_tensor_t *a, *w, *a_scale, *w_scale, *sorted_ids, *sorted_eids, *num_valid, *out, *sorted_w;
    int topk, block_m, activation, stage, splitk;
    int tile_m;   // GEMM row block (divides block_m; 0 = block_m)
    const char* kernel_name;
    // stage 1 with the fused MXFP4 output quant: `out` holds the e2m1 codes
    // [token_num * topk, inter / 2], q_scale the sorted shuffled scale bytes,
    // q_w the sorted routing weights of the zero-row rule (optional)
    aiter_tensor_t* q_scale = nullptr;
    aiter_tensor_t* q_w = nullptr;
};

template <int KA, int MOE>
void launch_bm(int bm, dim3 grid, const GemmParams& p, const MoeParams& mq, hipStream_t st) {
    switch (bm) {
        case 32: moe_flat_kernel<KA, 32, MOE><<<grid, 256, 0, st>>>(p, mq); break;
        case 64: moe_flat_kernel<KA, 64, MOE><<<grid, 256, 0, st>>>(p, mq); break;
        case 128: moe_flat_kernel<KA, 128, MOE><<<grid, 256, 0, st>>>(p, mq); break;
        default: fail("moe", "block_m must be 32, 64 or 128, got ", bm);
    }
}

// GEMM row block: kernelName "moe_m32" / "moe_m64" / "moe_m128" picks it
// (a "_flat" suffix keeps stage 2 on the flat tile kernel);
// otherwise the sort's block for stage 1 and at most 64 rows for stage 2
// (K is one or two stages there, so the tile is latency-bound and the smaller
// tile's lower register count lets two workgroups share a CU)
int tile_from_name(const char* name, int stage, int block_m) {
    if (name && name[0]) {
        const std::string n(name);
        AA_CHECK(n.rfind("moe_m", 0) == 0, "unknown MoE kernel name '", n,
                 "' (moe_m32 / moe_m64 / moe_m128, optional suffix _flat)");
        return std::atoi(n.c_str() + 5);
    }
    return stage == 1 ? block_m : std::min(block_m, 64);
}

// K = 256 or 512: one or two 256-element windows
template <int KA, int BM>
void launch_s2_kw(int kw, dim3 grid, const GemmParams& p, const MoeParams& mq, const MoeS2Params& sp, hipStream_t st) {
    if (kw == 1) {
        moe_stage2_stream_kernel<KA, BM, 1><<<grid, 256, 0, st>>>(p, mq, sp);
    } else if (kw == 2) {
        moe_stage2_stream_kernel<KA, BM, 2><<<grid, 256, 0, st>>>(p, mq, sp);
    } else {
        fail("moe", "stream stage 2: K / 256 must be 1 or 2");
    }
}

void run_stage(const StageArgs& s, hipStream_t st) {
    const char* fn = s.stage == 1 ? "ck_moe_stage1" : "ck_moe_stage2";
    check_tensor(s.a, "A", 2);
    check_tensor(s.w, "w", 3);
    check_tensor(s.sorted_ids, "sorted_token_ids", 1);
    check_tensor(s.sorted_eids, "sorted_expert_ids", 1);
    check_tensor(s.num_valid, "num_valid_ids", 1);
    check_tensor(s.out, "out", 2);
    AA_CHECK(s.a_scale && s.w_scale, fn, ": per-1x32 MX needs the activation and weight scales");
    check_tensor(s.a_scale, "a_scale");
    check_tensor(s.w_scale, "w_scale");
    AA_CHECK(s.sorted_ids->dtype == AITER_DTYPE_i32 && s.sorted_eids->dtype == AITER_DTYPE_i32 &&
                 s.num_valid->dtype == AITER_DTYPE_i32,
             "sorted ids must be int32");
    const bool fq = s.q_scale != nullptr;
    if (fq)
        AA_CHECK(s.stage == 1 && (s.out->dtype == AITER_DTYPE_fp4x2 || s.out->dtype == AITER_DTYPE_u8), fn,
                 ": the fused-quant output must be fp4x2");
    else
        AA_CHECK(s.out->dtype == AITER_DTYPE_bf16, fn, ": bf16 output only, got ", dtype_name(s.out->dtype));
    AA_CHECK(s.w->dtype == AITER_DTYPE_fp4x2 || s.w->dtype == AITER_DTYPE_u8, fn, ": MXFP4 (fp4x2) weights only");
    const bool a_fp8 = s.a->dtype == AITER_DTYPE_fp8;
    AA_CHECK(a_fp8 || s.a->dtype == AITER_DTYPE_fp4x2 || s.a->dtype == AITER_DTYPE_u8,
             fn, ": activations must be MXFP4 (fp4x2) or MXFP8 (fp8)");
    AA_CHECK(s.topk >= 1, "topk must be positive");

    const int64_t E = s.w->shape[0], wrows = s.w->shape[1], wbytes = s.w->shape[2];
    const int64_t K = wbytes * 2;                          // logical K of this stage
    AA_CHECK(s.w->strides[2] == 1 && s.w->strides[1] == wbytes && s.w->strides[0] == wrows * wbytes,
             "w must be contiguous [E, N, K/2]");
    AA_CHECK(K % 256 == 0, fn, ": K = ", K, " must be a multiple of 256");
    const int64_t lda = s.a->strides[0] * (int64_t)dtype_size(s.a->dtype);
    AA_CHECK(s.a->strides[1] == 1 && s.a->shape[1] * (a_fp8 ? 1 : 2) == K && lda % 16 == 0,
             "A must be [rows, K] with 16-byte aligned rows (K = ", K, ")");
    const int64_t arows = s.a->shape[0];
    AA_CHECK((arows + 1) * lda < ((int64_t)1 << 31), "A too large for 32-bit offsets");
    const int sn_pad = (int)((K / 32 + 7) / 8 * 8);
    const int64_t sorted_len = (int64_t)s.sorted_ids->numel;
    const int64_t sorted_rows = (sorted_len + 31) / 32 * 32;
    AA_CHECK((int64_t)s.a_scale->numel >= sorted_rows * sn_pad, "a_scale must be the sorted shuffled scale [",
             sorted_rows, ", ", sn_pad, "]");
    AA_CHECK(wrows % 32 == 0, "weight rows per expert must be a multiple of 32");
    AA_CHECK((int64_t)s.w_scale->numel >= E * wrows * sn_pad, "w_scale must hold [E * N, pad8(K/32)] shuffled");
    AA_CHECK(sorted_len < ((int64_t)1 << 31), "sorted_token_ids too long");
    const int64_t max_blocks = (sorted_len + s.block_m - 1) / s.block_m;
    AA_CHECK((int64_t)s.sorted_eids->numel >= max_blocks, "sorted_expert_ids needs ", max_blocks, " entries");
    const int bm = s.tile_m > 0 ? s.tile_m : s.block_m;
    AA_CHECK(bm == 32 || bm == 64 || bm == 128, "GEMM row block must be 32, 64 or 128, got ", bm);
    AA_CHECK(s.block_m % bm == 0, "the sort's block_m ", s.block_m, " must be a multiple of the GEMM row block ", bm);

    int64_t token_num = s.out->shape[0];
    MoeParams mq{};
    mq.sorted_ids = static_cast<const int*>(s.sorted_ids->ptr);
    mq.sorted_eids = static_cast<const int*>(s.sorted_eids->ptr);
    mq.num_valid = static_cast<const int*>(s.num_valid->ptr);
    mq.sorted_w = s.sorted_w ? static_cast<const float*>(s.sorted_w->ptr) : nullptr;
    mq.out = static_cast<uint16_t*>(s.out->ptr);
    mq.b_expert_bytes = wrows * wbytes;
    mq.bs_expert_bytes = wrows * sn_pad;
    mq.a_rows = arows;
    mq.sort_bs = s.block_m;
    mq.sorted_len = (int)sorted_len;
    mq.topk = s.topk;
    mq.n_experts = (int)E;
    mq.act = s.activation;
    if (s.sorted_w) {
        AA_CHECK(s.sorted_w->dtype == AITER_DTYPE_fp32 && (int64_t)s.sorted_w->numel >= sorted_len,
                 "sorted_weights must be float32 with len(sorted_token_ids) entries");
    }

    int tiles_n;
    if (s.stage == 1) {
        // out [token_num * topk, inter] (or [token_num, topk, inter] viewed as 2-D)
        const int64_t inter = wrows / 2;
        AA_CHECK(inter % 128 == 0, "ck_moe_stage1: inter_dim = ", inter, " must be a multiple of 128 (gate+up rows)");
        AA_CHECK(s.activation == kActSilu || s.activation == kActGelu, "activation must be Silu (0) or Gelu (1)");
        AA_CHECK(arows >= 1, "empty input");
        token_num = arows;
        if (fq) {
            AA_CHECK(inter % 256 == 0, "ck_moe_stage1_fuse_quant: inter_dim = ", inter,
                     " must be a multiple of 256 (whole 8-byte rows of scale bytes)");
            AA_CHECK(rows_2d(s.out) == token_num * s.topk && cols_2d(s.out) == inter / 2 &&
                         s.out->strides[s.out->ndim - 1] == 1,
                     "ck_moe_stage1_fuse_quant: out must be [token_num, topk, inter_dim / 2] fp4x2");
            mq.q_stride = s.out->ndim >= 2 ? s.out->strides[s.out->ndim - 2] : inter / 2;
            AA_CHECK(mq.q_stride % 16 == 0 && ((uintptr_t)s.out->ptr & 15) == 0, "out rows must be 16-byte aligned");
            check_tensor(s.q_scale, "out_scale");
            mq.q_scale_n_pad = (int)(inter / 32);
            const int64_t sorted_rows_q = ((int64_t)s.sorted_ids->numel + 31) / 32 * 32;
            AA_CHECK(is_byte_type(s.q_scale->dtype) && (int64_t)s.q_scale->numel >= sorted_rows_q * mq.q_scale_n_pad,
                     "out_scale must hold the sorted shuffled scales [", sorted_rows_q, ", ", mq.q_scale_n_pad, "]");
            mq.q_out = static_cast<uint8_t*>(s.out->ptr);
            mq.q_scale = static_cast<uint8_t*>(s.q_scale->ptr);
            if (s.q_w) {
                check_tensor(s.q_w, "quant_weights");
                AA_CHECK(s.q_w->dtype == AITER_DTYPE_fp32 && (int64_t)s.q_w->numel >= (int64_t)s.sorted_ids->numel,
                         "quant_weights must be float32 with len(sorted_token_ids) entries");
                mq.q_w = static_cast<const float*>(s.q_w->ptr);
            }
            mq.out = nullptr;
            mq.out_stride = 4;   // unused: no bf16 rows
        } else {
            AA_CHECK(rows_2d(s.out) == token_num * s.topk && cols_2d(s.out) == inter &&
                         s.out->strides[s.out->ndim - 1] == 1,
                     "ck_moe_stage1: out must be [token_num, topk, inter_dim] bf16");
            mq.out_stride = s.out->ndim >= 2 ? s.out->strides[s.out->ndim - 2] : inter;
        }
        mq.token_num = (int)token_num;
        mq.inter = (int)inter;
        tiles_n = (int)(inter / 128);
    } else {
        // out [token_num, model_dim]: packed-bf16 atomic adds into the token rows
        // (out starts at zero); out [token_num, topk, model_dim] (or its 2-D
        // view [token_num * topk, model_dim]): one row per routed pair, plain
        // stores, summed over the slots by moe_sum
        const int64_t model_dim = wrows;
        AA_CHECK(model_dim % 256 == 0, "ck_moe_stage2: model_dim = ", model_dim, " must be a multiple of 256");
        AA_CHECK(cols_2d(s.out) == model_dim && s.out->strides[s.out->ndim - 1] == 1,
                 "ck_moe_stage2: out must be [token_num, (topk,) ", model_dim, "] bf16");
        mq.per_pair = s.out->ndim == 3 ? 1 : 0;
        if (mq.per_pair) {
            AA_CHECK(s.out->shape[1] == s.topk, "ck_moe_stage2: out [token_num, topk, model_dim] needs topk = ",
                     s.topk);
            token_num = s.out->shape[0];
        }
        AA_CHECK(arows == token_num * s.topk, "ck_moe_stage2: inter_states must have token_num * topk rows");
        mq.out_stride = s.out->strides[s.out->ndim - 2];
        mq.token_num = (int)token_num;
        mq.inter = 0;
        tiles_n = (int)(model_dim / 256);
    }
    AA_CHECK(mq.out_stride % 4 == 0, "out rows must be 8-byte aligned");

    GemmParams p{};
    p.A = static_cast<const uint8_t*>(s.a->ptr);
    p.B = static_cast<const uint8_t*>(s.w->ptr);
    p.As = static_cast<const uint8_t*>(s.a_scale->ptr);
    p.Bs = static_cast<const uint8_t*>(s.w_scale->ptr);
    p.lda = lda;
    p.ldb = wbytes;
    p.sa_stride = sn_pad;
    p.sb_stride = sn_pad;
    p.M = (int)sorted_len;
    p.N = (int)wrows;
    p.K = (int)K;
    p.sa_groups = (int)(sorted_rows / 32);
    p.sb_groups = (int)(wrows / 32);
    p.tiles_n = tiles_n;
    p.alpha = 1.0f;

    // row blocks in use are at most ceil(entries / block_m) + (experts hit);
    // blocks past num_valid_ids[0] leave at once
    const int64_t entries = token_num * s.topk;
    const int64_t used_sort = std::min<int64_t>(max_blocks, (entries + s.block_m - 1) / s.block_m +
                                                              std::min<int64_t>(E, entries));
    const int64_t used = std::min<int64_t>(used_sort * (s.block_m / bm), (sorted_len + bm - 1) / bm);
    if (used == 0) return;
    p.tiles_m = (int)used;
    AA_CHECK((int64_t)tiles_n * used < ((int64_t)1 << 31), "grid too large");
    // stage-1 split-K while the tiles leave the CUs short of weight loads in
    // flight (decode and small batches; at least 2 K stages per split).  A
    // workgroup keeps one K stage of B ahead, so a CU with one tile streams
    // its weights far below its share of HBM.  Measured at the DeepSeek shape
    // (model_dim 7168, 257 experts, topk 9; 256 CUs): 1 token (20 tiles) is
    // fastest with ~120 workgroups (6 splits: 9.6 us, 10 splits 10.1, none
    // 14.9); 16-64 tokens (300-550 tiles) with 2 splits (16 tokens 53.6 ->
    // 42.7 us, 32 tokens 89.3 -> 74.5, 64 tokens 94.6 -> 90.1); from 128
    // tokens (590 tiles) one pass is faster.
    const int nst = (int)(K / 256);
    const int64_t tiles = (int64_t)tiles_n * used;
    int splits = 1;
    if (s.stage == 1) {
        // splitk: 1 = one pass over K (the reference's default), > 1 = that
        // many K slices, 0 = chosen here
        const int64_t cus = device_cu_count(s.out->device_id);
        int want = s.splitk;
        if (want == 0)
            want = tiles < cus / 2 ? (int)std::max<int64_t>(2, cus / 2 / tiles) : (tiles * 4 < cus * 9 ? 2 : 1);
        want = std::min(want, std::max(1, nst / 2));
        if (want > 1) {
            const int per = (nst + want - 1) / want;
            splits = (nst + per - 1) / per;
            p.k_steps_per_split = per;
        }
    }
    mq.k_splits = splits;
    mq.ws_rows = used * bm;
    if (splits > 1) {
        const size_t bytes = (size_t)splits * mq.ws_rows * 2 * mq.inter * sizeof(float);
        AA_CHECK(bytes <= 0x7ffffff0u, "stage-1 split-K partials need ", bytes,
                 " bytes (at most 2 GiB): ask for fewer splits (splitk)");
        p.ws = static_cast<float*>(lib_workspace(s.out->device_id, st, bytes));
        // the split that finishes a tile last sums it (no reduce launch)
        mq.tile_cnt = lib_counters(s.out->device_id, st, (size_t)tiles);
    }
    const dim3 grid((unsigned)((tiles * splits + 7) / 8 * 8));   // multiple of 8: XCD-aware tile order
    if (s.stage == 1) {
        if (a_fp8) launch_bm<kFp8, kMoeStage1>(bm, grid, p, mq, st);
        else launch_bm<kFp4, kMoeStage1>(bm, grid, p, mq, st);
    } else if ((bm == 32 || bm == 64) && (K == 256 || K == 512) &&
               !(s.kernel_name && std::string(s.kernel_name).find("flat") != std::string::npos)) {
        // short K: the streaming kernel (A in registers, a group of N tiles per
        // workgroup, about 2048 workgroups in all); "_flat" names keep the
        // flat tile kernel
        MoeS2Params sp{};
        const int64_t total_tiles = used * tiles_n;
        sp.tiles_per_group = (int)std::min<int64_t>(tiles_n, std::max<int64_t>(1, (total_tiles + 2047) / 2048));
        sp.groups = (tiles_n + sp.tiles_per_group - 1) / sp.tiles_per_group;
        sp.row_blocks = (int)used;
        sp.a_scale_rows = sorted_rows;
        const int64_t wgs = (int64_t)sp.row_blocks * sp.groups;
        const dim3 g2((unsigned)((wgs + 7) / 8 * 8));
        const int kw = (int)(K / 256);
        if (a_fp8) {
            if (bm == 32) launch_s2_kw<kFp8, 32>(kw, g2, p, mq, sp, st);
            else launch_s2_kw<kFp8, 64>(kw, g2, p, mq, sp, st);
        } else {
            if (bm == 32) launch_s2_kw<kFp4, 32>(kw, g2, p, mq, sp, st);
            else launch_s2_kw<kFp4, 64>(kw, g2, p, mq, sp, st);
        }
    } else {
        if (a_fp8) launch_bm<kFp8, kMoeStage2>(bm, grid, p, mq, st);
        else launch_bm<kFp4, kMoeStage2>(bm, grid, p, mq, st);
    }
    AA_HIP(hipGetLastError());
}

// out[t, c] = sum over slots s of in[t, s, c] (f32, slot order), bf16 in / out;
// 8 columns (16 bytes) per thread
__global__ __launch_bounds__(256) void moe_sum_kernel(const uint16_t* in, uint16_t* out, int64_t tokens, int topk,
                                                      int64_t dim, int64_t in_tok_stride, int64_t in_slot_stride,
                                                      int64_t out_stride) {
    const int64_t per_row = dim / 8;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= tokens * per_row) return;
    const int64_t t = gid / per_row, c = (gid % per_row) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint16_t* src = in + t * in_tok_stride + c;
    for (int s = 0; s < topk; ++s) {
        const i32x4_t v = *reinterpret_cast<const i32x4_t*>(src + s * in_slot_stride);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            acc[2 * k] += bf16_bits_to_f32((uint32_t)v[k] & 0xffffu);
            acc[2 * k + 1] += bf16_bits_to_f32((uint32_t)v[k] >> 16);
        }
    }
    i32x4_t o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = (int)pack_bf16x2(acc[2 * k], acc[2 * k + 1]);
    *reinterpret_cast<i32x4_t*>(out + t * out_stride + c) = o;
}

}  // namespace

extern "C" {

int moe_sum(aiter_tensor_t* input, aiter_tensor_t* output, aiter_stream_t stream) {
    return safe_call([&] {
        check_tensor(input, "input", 3);
        check_tensor(output, "output", 2);
        DeviceGuard g(input->device_id);
        AA_CHECK(input->dtype == AITER_DTYPE_bf16 && output->dtype == AITER_DTYPE_bf16, "moe_sum: bf16 only");
        AA_CHECK(input->ndim == 3 && output->ndim == 2, "moe_sum: input [M, topk, D], output [M, D]");
        const int64_t M = input->shape[0], topk = input->shape[1], D = input->shape[2];
        AA_CHECK(output->shape[0] == M && output->shape[1] == D, "moe_sum: output must be [M, D]");
        AA_CHECK(input->strides[2] == 1 && output->strides[1] == 1, "moe_sum: unit column stride needed");
        AA_CHECK(D % 8 == 0 && input->strides[1] % 8 == 0 && input->strides[0] % 8 == 0 && output->strides[0] % 8 == 0 &&
                     ((uintptr_t)input->ptr & 15) == 0 && ((uintptr_t)output->ptr & 15) == 0,
                 "moe_sum: rows must be 16-byte aligned and D a multiple of 8");
        const int64_t n = M * (D / 8);
        if (n == 0) return;
        moe_sum_kernel<<<(unsigned)((n + 255) / 256), 256, 0, reinterpret_cast<hipStream_t>(stream)>>>(
            static_cast<const uint16_t*>(input->ptr), static_cast<uint16_t*>(output->ptr), M, (int)topk, D,
            input->strides[0], input->strides[1], output->strides[0]);
        AA_HIP(hipGetLastError());
    });
}


int ck_moe_stage1(aiter_tensor_t* hidden_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                  aiter_tensor_t* out, int topk, const char* kernelName, aiter_tensor_t* w1_scale,
                  aiter_tensor_t* a1_scale, int block_m, aiter_tensor_t* sorted_weights, int quant_type,
                  int activation, int splitk, int use_non_temporal_load, const char* dst_type, int is_shuffled,
                  aiter_stream_t stream) {
    (void)w2;
    (void)use_non_temporal_load;
    (void)dst_type;
    return safe_call([&] {
        AA_CHECK(quant_type == 3, "ck_moe_stage1: only QuantType.per_1x32 (3) is implemented, got ", quant_type);
        AA_CHECK(is_shuffled != 0, "ck_moe_stage1: weights must be preshuffled (shuffle_weight (16,16))");
        DeviceGuard g(hidden_states ? hidden_states->device_id : -1);
        StageArgs s{hidden_states, w1, a1_scale, w1_scale, sorted_token_ids, sorted_expert_ids, num_valid_ids, out,
                    sorted_weights, topk, block_m, activation, 1, splitk, tile_from_name(kernelName, 1, block_m),
                    kernelName};
        run_stage(s, reinterpret_cast<hipStream_t>(stream));
    });
}

int ck_moe_stage1_fuse_quant(aiter_tensor_t* hidden_states, aiter_tensor_t* w1, aiter_tensor_t* sorted_token_ids,
                             aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids, aiter_tensor_t* out,
                             aiter_tensor_t* out_scale, int topk, const char* kernelName, aiter_tensor_t* w1_scale,
                             aiter_tensor_t* a1_scale, int block_m, aiter_tensor_t* sorted_weights,
                             aiter_tensor_t* quant_weights, int activation, int splitk, aiter_stream_t stream) {
    return safe_call([&] {
        AA_CHECK(out_scale, "ck_moe_stage1_fuse_quant: out_scale must be given");
        DeviceGuard g(hidden_states ? hidden_states->device_id : -1);
        StageArgs s{hidden_states, w1, a1_scale, w1_scale, sorted_token_ids, sorted_expert_ids, num_valid_ids, out,
                    sorted_weights, topk, block_m, activation, 1, splitk, tile_from_name(kernelName, 1, block_m),
                    kernelName, out_scale, quant_weights};
        run_stage(s, reinterpret_cast<hipStream_t>(stream));
    });
}

int ck_moe_stage2(aiter_tensor_t* inter_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                  aiter_tensor_t* out, int topk, const char* kernelName, aiter_tensor_t* w2_scale,
                  aiter_tensor_t* a2_scale, int block_m, aiter_tensor_t* sorted_weights, int quant_type,
                  int activation, int splitk, int use_non_temporal_load, const char* dst_type, int is_shuffled,
                  aiter_stream_t stream) {
    (void)w1;
    (void)use_non_temporal_load;
    (void)dst_type;
    (void)activation;
    return safe_call([&] {
        AA_CHECK(quant_type == 3, "ck_moe_stage2: only QuantType.per_1x32 (3) is implemented, got ", quant_type);
        AA_CHECK(splitk <= 1, "ck_moe_stage2: split-K is not implemented for per_1x32");
        AA_CHECK(is_shuffled != 0, "ck_moe_stage2: weights must be preshuffled (shuffle_weight (16,16))");
        DeviceGuard g(inter_states ? inter_states->device_id : -1);
        StageArgs s{inter_states, w2, a2_scale, w2_scale, sorted_token_ids, sorted_expert_ids, num_valid_ids, out,
                    sorted_weights, topk, block_m, 0, 2, 1, tile_from_name(kernelName, 2, block_m), kernelName};
        run_stage(s, reinterpret_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
