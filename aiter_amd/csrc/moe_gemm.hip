// Host side of the MoE grouped GEMMs (stage 1: gate/up GEMM + activation,
// stage 2: down GEMM + weighted scatter-add), MXFP4 weights with per-1x32 e8m0
// scales and MXFP4 (a4w4) or MXFP8 (a8w4) activations.  The kernels are the
// flat tile kernel's MoE stages (gemm_flat.h).  Entry points keep the argument
// lists of the reference's ck_moe_stage1 / ck_moe_stage2
// (aiter/ops/moe_op.py:350-394).
#include "gemm_kernels.h"
#include "mfma32.h"
#include "gemm_flat.h"

namespace {

using namespace aiter_amd;

struct StageArgs {
    aiter_tensor_t *a, *w, *a_scale, *w_scale, *sorted_ids, *sorted_eids, *num_valid, *out, *sorted_w;
    int topk, block_m, activation, stage;
    const char* kernel_name;
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
        AA_CHECK(rows_2d(s.out) == token_num * s.topk && cols_2d(s.out) == inter && s.out->strides[s.out->ndim - 1] == 1,
                 "ck_moe_stage1: out must be [token_num, topk, inter_dim] bf16");
        mq.out_stride = s.out->ndim >= 2 ? s.out->strides[s.out->ndim - 2] : inter;
        mq.token_num = (int)token_num;
        mq.inter = (int)inter;
        tiles_n = (int)(inter / 128);
    } else {
        const int64_t model_dim = wrows;
        AA_CHECK(model_dim % 256 == 0, "ck_moe_stage2: model_dim = ", model_dim, " must be a multiple of 256");
        AA_CHECK(cols_2d(s.out) == model_dim && s.out->strides[1] == 1, "ck_moe_stage2: out must be [token_num, ",
                 model_dim, "] bf16");
        AA_CHECK(arows == token_num * s.topk, "ck_moe_stage2: inter_states must have token_num * topk rows");
        mq.out_stride = s.out->strides[0];
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
    const int64_t used = std::min<int64_t>(max_blocks, (entries + s.block_m - 1) / s.block_m + std::min<int64_t>(E, entries));
    if (used == 0) return;
    p.tiles_m = (int)used;
    const dim3 grid((unsigned)tiles_n, (unsigned)used);
    if (s.stage == 1) {
        if (a_fp8) launch_bm<kFp8, kMoeStage1>(s.block_m, grid, p, mq, st);
        else launch_bm<kFp4, kMoeStage1>(s.block_m, grid, p, mq, st);
    } else {
        if (a_fp8) launch_bm<kFp8, kMoeStage2>(s.block_m, grid, p, mq, st);
        else launch_bm<kFp4, kMoeStage2>(s.block_m, grid, p, mq, st);
    }
    AA_HIP(hipGetLastError());
}

}  // namespace

extern "C" {

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
        AA_CHECK(splitk <= 1, "ck_moe_stage1: split-K is not implemented for per_1x32");
        AA_CHECK(is_shuffled != 0, "ck_moe_stage1: weights must be preshuffled (shuffle_weight (16,16))");
        DeviceGuard g(hidden_states ? hidden_states->device_id : -1);
        StageArgs s{hidden_states, w1, a1_scale, w1_scale, sorted_token_ids, sorted_expert_ids, num_valid_ids, out,
                    sorted_weights, topk, block_m, activation, 1, kernelName};
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
                    sorted_weights, topk, block_m, 0, 2, kernelName};
        run_stage(s, reinterpret_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
