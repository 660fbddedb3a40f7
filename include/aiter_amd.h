/*
 * aiter_amd — C ABI of the MI355X (gfx950) scaled-GEMM hot path.
 *
 * Every entry point is `extern "C"`, takes plain POD tensor descriptors
 * (`aiter_tensor_t*`), scalars and a trailing `hipStream_t`, returns 0 on
 * success and -1 on error (message via `aiter_get_last_error`).  No C++
 * exception crosses the boundary and the library never frees caller memory.
 * The argument order and meaning follow the reference's ctypes convention
 * (aiter/jit/core.py:1252-1555): Tensor -> aiter_tensor_t*, Optional[Tensor]
 * -> NULL, str -> const char* (Optional -> NULL), bool -> int, float -> float.
 *
 * Citations (file:line) name the reference entry point each symbol replaces.
 */
#ifndef AITER_AMD_H
#define AITER_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque HIP stream handle (hipStream_t). */
typedef struct ihipStream_t* aiter_stream_t;

/* Dtype ids, same order as AiterDtype in csrc/include/aiter_enum.h:40-56. */
typedef enum {
    AITER_DTYPE_fp8 = 0,      /* e4m3fn */
    AITER_DTYPE_fp8_e8m0 = 1, /* e8m0 block scale */
    AITER_DTYPE_fp16 = 2,
    AITER_DTYPE_bf16 = 3,
    AITER_DTYPE_fp32 = 4,
    AITER_DTYPE_i4x2 = 5,
    AITER_DTYPE_fp4x2 = 6,    /* two e2m1 per byte, even element low nibble */
    AITER_DTYPE_u32 = 7,
    AITER_DTYPE_i32 = 8,
    AITER_DTYPE_i16 = 9,
    AITER_DTYPE_i8 = 10,
    AITER_DTYPE_u8 = 11,
    AITER_DTYPE_i64 = 12,
    AITER_DTYPE_u64 = 13,
} AiterDtype;

/* POD tensor descriptor, layout of csrc/include/aiter_tensor.h:8-17
 * (aiter/utility/aiter_types.py:68-77).  Strides are in elements; for fp4x2
 * one element is one byte (two e2m1 values). */
typedef struct aiter_tensor_t {
    void* ptr;
    size_t numel;
    int ndim;
    int64_t shape[8];
    int64_t strides[8];
    int dtype; /* AiterDtype */
    int device_id;
} aiter_tensor_t;

/* ---- error ABI: csrc/include/aiter_ctypes_error.h:60-71 ---------------- */
int aiter_ctypes_abi_version(void); /* returns 2, as the reference */
const char* aiter_get_last_error(void);
void aiter_clear_last_error(void);

/* ---- dispatch helper: csrc/py_itfs_cu/gemm_common.cu:12-41 ------------- */
int getPaddedM(int M, int N, int K, int gl);

/* ---- A4W4: csrc/py_itfs_cu/asm_gemm_a4w4.cu:158-172 -------------------
 * D[M,N] bf16 = alpha * (A (x) A_scale) (B (x) B_scale)^T + beta * bias.
 * A [M,K/2] fp4x2 row-major; B [N,K/2] fp4x2 preshuffled (bpreshuffle=1,
 * shuffle_weight layout (16,16)) or row-major (bpreshuffle=0);
 * A_scale [>=pad32(M), >=K/32] / B_scale [>=pad32(N), >=K/32] e8m0 in the
 * shuffled MFMA layout; out [>=M, N] bf16 (aiter allocates pad32(M) rows);
 * bias optional f32 [N], [1,N] or [M,N].  kernelName: a name from this
 * library's table; or a reference kernel name (ASM "_ZN5aiter..._<tM>x<tN>E",
 * CK "a4w4_blockscale_<block>x<tM>x<tN>x<tK>_..."), which runs the tile of
 * the same shape here when there is one and M > 32, else the heuristic
 * choice; "" or NULL = heuristic; any other name is an error.
 * log2_k_split <= 0 lets the heuristic choose the split-K factor. */
int gemm_a4w4_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* A_scale,
                  aiter_tensor_t* B_scale, aiter_tensor_t* out, const char* kernelName,
                  aiter_tensor_t* bias, float alpha, float beta, int bpreshuffle,
                  int log2_k_split, aiter_stream_t stream);

/* ---- A4W4 without allocation.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments and
 * result as gemm_a4w4_asm; split-K partials go to a fixed per-GPU scratch
 * array of gemm_a4w4_noalloc_scratch_bytes() bytes (32 MiB) that the
 * library holds until the process ends, instead of the library workspace.
 * A call whose partials need more is an error; nothing is ever allocated.
 * Every call on a GPU shares that GPU's array, so calls that overlap on one
 * GPU (two streams or threads at once) race. */
int gemm_a4w4_asm_noalloc(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* A_scale,
                          aiter_tensor_t* B_scale, aiter_tensor_t* out, const char* kernelName,
                          aiter_tensor_t* bias, float alpha, float beta, int bpreshuffle,
                          int log2_k_split, aiter_stream_t stream);
size_t gemm_a4w4_noalloc_scratch_bytes(void);

/* ---- A4W4 blockscale (the CK-instance entry):
 * csrc/ck_gemm_a4w4_blockscale/gemm_a4w4_blockscale.cu:69-93 and the tune
 * entry csrc/ck_gemm_a4w4_blockscale/gemm_a4w4_blockscale_tune.cu:58-90.
 * Same tensors as gemm_a4w4_asm with B preshuffled; kernelId < 0 means the
 * heuristic choice, splitK is log2 of the K split. */
int gemm_a4w4_blockscale(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* x_scale,
                         aiter_tensor_t* w_scale, aiter_tensor_t* Y, int splitK,
                         int kernelId, aiter_stream_t stream);

/* ---- MXFP8 x MXFP4: aiter/ops/gemm_op_a8w4.py:18-31 (gfx1250 ASM entry
 * csrc/py_itfs_cu/asm_mxfp8fp4gemm.cu), implemented here for gfx950.
 * A [M,K] e4m3fn (row-major, or shuffle_weight layout when a_preshuffle=1),
 * B [N,K/2] fp4x2 preshuffled, ScaleA/ScaleB shuffled e8m0, out [M,N] bf16. */
int mxfp8_mxfp4_gemm_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* ScaleA,
                         aiter_tensor_t* ScaleB, aiter_tensor_t* out, const char* kernelName,
                         int a_preshuffle, aiter_stream_t stream);

/* ---- bf16 A16W16: csrc/py_itfs_cu/asm_gemm_a16w16.cu:192-205 ----------
 * out[M,N] (bf16 or f32) = A[M,K] @ B[N,K]^T (+ bias f32 [N]).  B row-major
 * or preshuffled (bpreshuffle=1, shuffle_weight (16,16)).  `semaphore` is
 * accepted for signature compatibility and unused (split-K partials go to a
 * library-owned per-stream workspace).  splitK is a literal split count,
 * capped at 16 (asm_gemm_a16w16.cu:111-114); <= 0 lets the launcher choose. */
int gemm_a16w16_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* out,
                    aiter_tensor_t* semaphore, aiter_tensor_t* bias, int splitK,
                    const char* kernelName, int bpreshuffle, aiter_stream_t stream);

/* ---- opus a16w16: csrc/opus_gemm/opus_gemm.cu:133-209 (heuristic) and
 * :294-350 (explicit kernel id).  XQ [b,M,K], WQ [b,N,K] bf16, Y [b,M,N]
 * bf16 or f32, bias f32 [N] or [b,N] or NULL.  kernelId is a reference opus
 * kid (csrc/opus_gemm/opus_gemm_common.py:238-513: 4-9, 200-223, 300-315,
 * 1400-1404 and their +1000 / +2000..+4000 / +5000 variants): the kernel of
 * the same tile here when there is one and M > 32, else the heuristic
 * choice; ids outside the gfx950 table are an error; < 0 = heuristic.
 * splitK is the literal KBatch of that kernel id, <= 1 one pass
 * (aiter/ops/opus/gemm_op_a16w16.py:488). */
int opus_gemm(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y,
              aiter_tensor_t* bias, aiter_stream_t stream);
int opus_gemm_a16w16_tune(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y,
                          aiter_tensor_t* bias, int kernelId, int splitK,
                          aiter_stream_t stream);

/* ---- quantisers ---------------------------------------------------------
 * dynamic_per_group_scaled_quant: csrc/kernels/quant_kernels.cu:837-962.
 * x [M,K] bf16/fp16/f32 -> out [M,K/2] fp4x2 or [M,K] fp8, scales e8m0
 * (RoundUp, [M,K/32] plain or shuffled [pad256(M), pad8(K/32)]).  num_rows
 * (optional i32 device scalar) limits the rows processed to
 * num_rows*num_rows_factor. */
int dynamic_per_group_scaled_quant(aiter_tensor_t* out, aiter_tensor_t* input,
                                   aiter_tensor_t* scales, int group_size, int shuffle_scale,
                                   aiter_tensor_t* num_rows, int num_rows_factor,
                                   aiter_stream_t stream);

/* quant_mxfp4: csrc/kernels/quant_mxfp4.cu:233-300 (4 round modes, optional
 * e8m0 shuffle and fused shuffle_weight of the packed output).  a16w4 /
 * gate_up layouts are MoE-only and rejected. */
int quant_mxfp4(aiter_tensor_t* x, aiter_tensor_t* out_packed, aiter_tensor_t* out_scale,
                int group_size, int round_mode, int e8m0_shuffle, int a16w4_shuffle,
                int gate_up, int shuffle_weight, aiter_stream_t stream);

/* dynamic_mxfp4_quant (Even mode, Triton kernel of
 * aiter/utility/fp4_utils.py:373-597) and dynamic_mxfp8_quant (Even mode,
 * aiter/ops/triton/quant/quant.py:235-297), as HIP kernels.  The fp4 scale
 * buffer is [pad256(M), pad8(K/32)] when shuffle=1 (rows pad32(M).. untouched,
 * rows M..pad32(M) and columns K/32..pad8 written as 0), else [M, K/32]. */
int dynamic_mxfp4_quant(aiter_tensor_t* x, aiter_tensor_t* x_fp4, aiter_tensor_t* scale,
                        int shuffle, aiter_stream_t stream);
int dynamic_mxfp8_quant(aiter_tensor_t* x, aiter_tensor_t* y, aiter_tensor_t* scale,
                        int shuffle, aiter_stream_t stream);

/* Fused RMSNorm -> MX quant prologue: the entry behind fused_rms_mxfp4_quant
 * (aiter/ops/triton/quant/fused_mxfp4_quant.py:23-147) and
 * fused_rms_mxfp8_quant (aiter/ops/triton/quant/fused_mxfp8_quant.py:22-76),
 * which launch Triton kernels in the reference.  x1 [M, N1] (N1 % 32 == 0,
 * N1 <= 32768) + optional res1 -> out_res1, RMSNorm with x1_weight / eps1 in
 * f32 -> optional out1, Even-scale MX quant into out_q ([M, N1/2] u8 e2m1
 * pairs, or [M, N1] fp8 e4m3) and out_scale ([M, N1/32], or shuffled
 * [pad256(M), pad8(N1/32)] when shuffle=1; pad_scale=1 writes 127 into the
 * padding columns of each row, as the reference does).  Optional x2 [M, N2]
 * with x2_weight / eps2 -> out2 (RMSNorm only).  NULL for every absent
 * tensor. */
int fused_rms_mx_quant(aiter_tensor_t* x1, aiter_tensor_t* x1_weight, float eps1, aiter_tensor_t* x2,
                       aiter_tensor_t* x2_weight, float eps2, aiter_tensor_t* res1, aiter_tensor_t* out_q,
                       aiter_tensor_t* out_scale, aiter_tensor_t* out1, aiter_tensor_t* out2,
                       aiter_tensor_t* out_res1, int shuffle, int pad_scale, aiter_stream_t stream);

/* Batched bf16: replace the CK ops batched_gemm_bf16 / batched_gemm_bf16_tune
 * (aiter/ops/batched_gemm_op_bf16.py:28-36,127-134): XQ [B, M, K], WQ [B, N, K]
 * (row-major per batch), Y [B, M, N] bf16 or fp32, bias [N] or [B, N] fp32;
 * any batch and row strides with a unit last-dimension stride.  One launch with
 * gridDim.z = B.  opus_gemm / opus_gemm_a16w16_tune use the same path. */
int batched_gemm_bf16(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y, aiter_tensor_t* bias, int splitK,
                      aiter_stream_t stream);
int batched_gemm_bf16_tune(aiter_tensor_t* XQ, aiter_tensor_t* WQ, aiter_tensor_t* Y, int kernelId, int splitK,
                           aiter_stream_t stream);

/* Low-precision outputs: replaces mxfp4_gemm_asm (aiter/ops/gemm_op_a4w4.py:290-304;
 * gfx1250-only in the reference, whose gemm_a4w4o4 / gemm_a4w4o8 call it).
 * out bf16 [M, N]: as gemm_a4w4_asm without bias; fp4x2 [M, N/2]: e2m1 of the
 * product with conversion scale 1, input scales ignored (the reference's
 * packed-fp4 kernel is scale-free, op_tests/test_f4gemm.py:213-215); fp8
 * [M, N] + out_scale (M * N/128 e8m0 bytes, packed (M/64, N/128, 16, 4)):
 * per-128-column RoundUp e8m0 and e4m3 data, M % 64 == 0, N % 128 == 0.
 * a_preshuffle must be 0 (row-major A on gfx950). */
int mxfp4_gemm_asm(aiter_tensor_t* A, aiter_tensor_t* B, aiter_tensor_t* ScaleA, aiter_tensor_t* ScaleB,
                   aiter_tensor_t* out, aiter_tensor_t* out_scale, const char* kernelName, int a_preshuffle,
                   aiter_stream_t stream);

/* ---- fused GEMM + output operation: the Triton ops of
 * aiter/ops/triton/gemm/fused/fused_gemm_afp4wfp4_{mul_add,split_cat,a16w16}.py
 * (no C entry in the reference; these are what their host code would bind).
 * x [M, K/2] e2m1; w [N, K/2] row-major, or (preshuffled != 0) the
 * shuffle_weight bytes in any shape (the Triton ops pass [N/16, K*8]).
 * Scales: plain [R, K/32] e8m0 when not preshuffled; when preshuffled, w's
 * are the shuffle_scale bytes in any shape (Triton: [N/32, K]) and x's too
 * when M >= 32, plain below.  Plain scales are shuffled into a library
 * workspace first (so a graph capture needs one eager call of the shape).
 * kernelName: an A4W4 instance of this library or NULL for the heuristic. */
/* fused_gemm_afp4wfp4_mul_add.py:63-236 and _preshuffle_add_mul :239-:
 * out [M, N] bf16 = a * (x w^T) + b (fuse_type 0) or a * b + x w^T (1) in f32;
 * a / b: f32 or bf16 tensors broadcastable to [M, N] (one element = scalar)
 * or NULL for a_scalar / b_scalar. */
int fused_gemm_afp4wfp4_mul_add(aiter_tensor_t* x, aiter_tensor_t* w, aiter_tensor_t* x_scale,
                                aiter_tensor_t* w_scale, aiter_tensor_t* a, float a_scalar, aiter_tensor_t* b,
                                float b_scalar, int fuse_type, aiter_tensor_t* out, int preshuffled,
                                const char* kernelName, aiter_stream_t stream);
/* fused_gemm_afp4wfp4_split_cat.py:19-196 and _preshuffle_split_cat :199-:
 * C = x w^T viewed [M, D, S1+S2]; c1 [M, D, S1+S3] = cat(C[..., :S1], y),
 * c2 [M, D, S2] = C[..., S1:]; y [M, D, S3]; bf16; c1, c2 contiguous;
 * S1, S2, S3 multiples of 8. */
int fused_gemm_afp4wfp4_split_cat(aiter_tensor_t* x, aiter_tensor_t* w, aiter_tensor_t* x_scale,
                                  aiter_tensor_t* w_scale, aiter_tensor_t* y, aiter_tensor_t* c1,
                                  aiter_tensor_t* c2, int S1, int S2, int preshuffled, const char* kernelName,
                                  aiter_stream_t stream);
/* fused_gemm_afp4wfp4_a16w16.py:23-254: y_fp4 = x_fp4 w_fp4^T (+ bias_fp4) and
 * y_bf16 = x_bf16 w_bf16^T (+ bias_bf16), same M and K, bf16 out, biases f32
 * [N] or NULL; w_bf16 row-major [N_bf16, K]; two launches on `stream`. */
int fused_gemm_afp4wfp4_a16w16(aiter_tensor_t* x_fp4, aiter_tensor_t* w_fp4, aiter_tensor_t* x_fp4_scale,
                               aiter_tensor_t* w_fp4_scale, aiter_tensor_t* bias_fp4, aiter_tensor_t* y_fp4,
                               const char* kernel_fp4, aiter_tensor_t* x_bf16, aiter_tensor_t* w_bf16,
                               aiter_tensor_t* bias_bf16, aiter_tensor_t* y_bf16, const char* kernel_bf16,
                               int preshuffled, aiter_stream_t stream);

/* ---- fused MoE (MXFP4 weights, per-1x32 e8m0 scales) ---------------------
 * Routing sort: replaces moe_sorting_fwd (aiter/ops/moe_sorting.py:12-27,
 * called from aiter/fused_moe.py:171-285).  topk_ids int32 [M, topk],
 * topk_weights fp32 [M, topk]; outputs sized as aiter/fused_moe.py:206-215:
 * sorted_token_ids int32 / sorted_weights fp32 [M*topk + E*unit - topk]
 * (slot << 24 | token, experts in order, tokens in order inside an expert,
 * padding topk << 24 | M), sorted_expert_ids int32 [ceil(len / unit)]
 * (unused: -1), num_valid_ids int32 [2] = {padded count, tokens};
 * moe_buf (optional) is zeroed.  local_expert_mask int32 [E] (0 drops an
 * expert; kept experts renumbered), num_local_tokens int32 [1] (device
 * count of tokens to route).  dispatch_policy must be 0. */
int moe_sorting_fwd(aiter_tensor_t* topk_ids, aiter_tensor_t* topk_weights, aiter_tensor_t* sorted_token_ids,
                    aiter_tensor_t* sorted_weights, aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                    aiter_tensor_t* moe_buf, int num_experts, int unit_size, aiter_tensor_t* local_expert_mask,
                    aiter_tensor_t* num_local_tokens, int dispatch_policy, aiter_stream_t stream);

/* Routing sort + stage-1 activation quant in one launch, for decode-sized
 * routing (at most 256 entries M * topk; no expert mask, no device token
 * count): the fusion of route map, MX quant and scale scatter of
 * aiter/ops/flydsl/kernels/moe_fused_route_quant_scatter.py:1-50 for this
 * library's sorted list.  Same arguments and outputs as moe_sorting_fwd
 * (dispatch_policy 0) followed by fused_dynamic_mx_quant_moe_sort_hip(a_out,
 * a_scale, hidden_states, ..., sorted_weights) at stage 1: hidden_states bf16
 * [M, K], a_out fp4x2 [M, K/2], a_scale u8 [pad32(len(sorted_token_ids)),
 * pad8(K/32)] sorted and shuffled.  Positions at or past num_valid_ids[0]
 * (beyond the last 32-row group) and the rows of tokens whose entries were
 * all dropped are left unwritten; a zero routing weight gives scale byte 0
 * at its position.  Needs K <= 65536. */
int moe_sorting_mx_quant(aiter_tensor_t* topk_ids, aiter_tensor_t* topk_weights, aiter_tensor_t* hidden_states,
                         aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_weights,
                         aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids, aiter_tensor_t* moe_buf,
                         aiter_tensor_t* a_out, aiter_tensor_t* a_scale, int num_experts, int unit_size,
                         aiter_stream_t stream);

/* Sorted MX quant: replaces fused_dynamic_mx_quant_moe_sort_hip
 * (aiter/ops/quant.py:895-911; kernel csrc/kernels/quant_kernels.cu:1733-1880).
 * input bf16/fp16/fp32 [token_num * t, K] (t = 1: stage 1, t = topk: stage
 * 2), out fp4x2 [rows, K/2] or fp8 [rows, K], scales u8 [pad32(len(sorted_ids)),
 * pad8(K/32)] in sorted shuffled order; RoundUp e8m0 from the running max
 * 1e-10; sorted_weights (optional) zero weight -> zero row. */
int fused_dynamic_mx_quant_moe_sort_hip(aiter_tensor_t* out, aiter_tensor_t* scales, aiter_tensor_t* input,
                                        aiter_tensor_t* sorted_ids, aiter_tensor_t* num_valid_ids, int token_num,
                                        int block_m, int group_size, aiter_tensor_t* sorted_weights,
                                        aiter_stream_t stream);

/* Scale byte sort: replaces mxfp4_moe_sort_hip (aiter/ops/quant.py:861-871):
 * per-row e8m0 [rows, K/32] -> sorted shuffled [pad32(len), pad8(K/32)]. */
int mxfp4_moe_sort_hip(aiter_tensor_t* out_scale, aiter_tensor_t* scale, aiter_tensor_t* sorted_ids,
                       aiter_tensor_t* num_valid_ids, int token_num, int cols, aiter_stream_t stream);

/* Grouped GEMM stages: replace ck_moe_stage1 / ck_moe_stage2
 * (aiter/ops/moe_op.py:350-394; numerics aiter/fused_moe.py:3437-3680).
 * quant_type must be 3 (per_1x32); weights fp4x2 [E, N, K/2] preshuffled
 * (is_shuffled = 1) with scales shuffled as one [E*N, K/32] matrix; A fp4x2
 * (a4w4) or fp8 (a8w4) with its sorted scale (fused_dynamic_mx_quant_moe_sort).
 * Stage 1: w1 [E, 2*inter, K/2] (gate rows then up rows), out bf16
 * [token_num, topk, inter] = act(gate) * up (activation 0 Silu, 1 Gelu;
 * sorted_weights, if given, scale gate and up first).  Stage 2: w2
 * [E, model_dim, inter/2], inter_states [token_num*topk, inter(/2)], out bf16
 * [token_num, model_dim] += weight * GEMM (packed bf16 atomics; out must start
 * at zero), or, with out [token_num, topk, model_dim], each pair's weighted
 * row stored (then moe_sum).  block_m (32, 64, 128) must equal the sort's
 * unit_size.  Stage-1 splitk: 1 one pass over K, n > 1 n K slices (f32
 * partials in the library workspace, summed by a second kernel), 0 chosen
 * here; stage 2 ignores it.  w2 (stage 1) and w1 (stage 2) may be NULL. */
int ck_moe_stage1(aiter_tensor_t* hidden_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                  aiter_tensor_t* out, int topk, const char* kernelName, aiter_tensor_t* w1_scale,
                  aiter_tensor_t* a1_scale, int block_m, aiter_tensor_t* sorted_weights, int quant_type,
                  int activation, int splitk, int use_non_temporal_load, const char* dst_type, int is_shuffled,
                  aiter_stream_t stream);
/* Stage 1 with its output quantised in the same launch: replaces the stage-1
 * call of a fuse_quant == "fp4" configuration (aiter/fused_moe.py:3125-3171:
 * stage 1 returns (a2, a2_scale) and the separate
 * fused_dynamic_mx_quant_moe_sort of the stage-1 output is skipped).  Same
 * GEMM as ck_moe_stage1 (a4w4 or a8w4 input, per_1x32, preshuffled w1);
 * out fp4x2 [token_num, topk, inter_dim / 2] and out_scale e8m0
 * [pad32(len(sorted_token_ids)), inter_dim / 32] get exactly the bytes
 * fused_dynamic_mx_quant_moe_sort_hip(out, out_scale, <ck_moe_stage1's bf16
 * out>, sorted_token_ids, num_valid_ids, token_num, block_m, 32,
 * quant_weights) would write.  inter_dim must be a multiple of 256. */
int ck_moe_stage1_fuse_quant(aiter_tensor_t* hidden_states, aiter_tensor_t* w1, aiter_tensor_t* sorted_token_ids,
                             aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids, aiter_tensor_t* out,
                             aiter_tensor_t* out_scale, int topk, const char* kernelName, aiter_tensor_t* w1_scale,
                             aiter_tensor_t* a1_scale, int block_m, aiter_tensor_t* sorted_weights,
                             aiter_tensor_t* quant_weights, int activation, int splitk, aiter_stream_t stream);
int ck_moe_stage2(aiter_tensor_t* inter_states, aiter_tensor_t* w1, aiter_tensor_t* w2,
                  aiter_tensor_t* sorted_token_ids, aiter_tensor_t* sorted_expert_ids, aiter_tensor_t* num_valid_ids,
                  aiter_tensor_t* out, int topk, const char* kernelName, aiter_tensor_t* w2_scale,
                  aiter_tensor_t* a2_scale, int block_m, aiter_tensor_t* sorted_weights, int quant_type,
                  int activation, int splitk, int use_non_temporal_load, const char* dst_type, int is_shuffled,
                  aiter_stream_t stream);

/* Slot reduction: replaces _moe_sum (aiter/ops/moe_op.py:87-98): output
 * bf16 [M, D] = sum over topk of input bf16 [M, topk, D], f32 sums in slot
 * order (the reduce form of stage 2: ck_moe_stage2 with out [M, topk, D]). */
int moe_sum(aiter_tensor_t* input, aiter_tensor_t* output, aiter_stream_t stream);

/* ---- library introspection and workspace --------------------------------
 * The reference keeps its kernel list in per-arch CSVs next to its ASM code
 * objects (hsa/gfx950/f4gemm/f4gemm_bf16_per1x32Fp4.csv) and the CK instance
 * list in generated headers; the tuner enumerates those.  Here the table is
 * compiled into the library and read through these two calls:
 * aiter_amd_num_kernels() -> number of kernel ids (ids are 0..n-1);
 * aiter_amd_kernel_info(id, buf, len) writes
 * "id,name,family,skinny,bm,bn,split,a_pre,b_pre,out_f32" (0 or -1). */
int aiter_amd_num_kernels(void);
int aiter_amd_kernel_info(int id, char* buf, int buflen);

/* Tuned-CSV name resolution, the lookup gemm_a4w4_asm / gemm_a16w16_asm /
 * mxfp8_mxfp4_gemm_asm apply to kernelName (the reference resolves names in
 * its dispatch maps, csrc/py_itfs_cu/asm_gemm_a4w4.cu:221-263 and
 * csrc/ck_gemm_a4w4_blockscale/gemm_a4w4_blockscale.cu:28-62), for an
 * M-row GEMM of family 0 (a4w4), 1 (a8w4) or 2 (a16w16) with the given
 * layout flags: returns the kernel id, -1 for the heuristic choice, -2 for a
 * name that is neither this library's nor a reference kernel name.
 * aiter_amd_resolve_opus_kid does the same for a reference opus kernel id
 * (row-major B).  No GPU call. */
int aiter_amd_resolve_kernel_name(const char* name, int family, int a_pre, int b_pre, int out_f32, int64_t M);
int aiter_amd_resolve_opus_kid(int kid, int out_f32, int64_t M);

/* Pre-sizes the split-K fp32 workspace owned by (device, stream) to at least
 * `bytes` (and allocates its split-K tile counters, 64K of them), so that a
 * later HIP-graph capture never needs to allocate.  The
 * reference's counterpart is the caller-provided semaphore / workspace
 * tensor of csrc/py_itfs_cu/asm_gemm_a16w16.cu:192-205 and
 * aiter/ops/opus/gemm_op_opus.py (opus_gemm_workspace_init). */
int gemm_workspace_reserve(int device, aiter_stream_t stream, size_t bytes);

/* Introspection, no counterpart in the reference: bytes of the split-K
 * workspace currently held for (device, stream), 0 if none.  Tests read it
 * to check the split count a call used (fp32 partials: splits * M * N * 4). */
int64_t aiter_amd_workspace_bytes(int device, aiter_stream_t stream);

/* No counterpart in the reference: frees every library workspace held for
 * (device, stream) once the stream's queued work has completed (a later call
 * that needs one allocates it again).  Not allowed during graph capture.
 * Returns 0 or -1 (message in aiter_get_last_error). */
int aiter_amd_workspace_release(int device, aiter_stream_t stream);

/* ---- calibration ---------------------------------------------------------
 * No counterpart in the reference: a plain streaming read of src (contiguous
 * 1-D, 16-byte aligned, any dtype) with `grid` workgroups of 256 threads and
 * nothing else in the kernel.  Its rate at a given byte count is the
 * attainable HBM read rate that the bandwidth-bound decode GEMMs are
 * compared against; sink (one int32) only keeps the reads live. */
int hbm_stream_read(aiter_tensor_t* src, aiter_tensor_t* sink, int grid, aiter_stream_t stream);

/* The same calibration read with its launch shape and cache policy chosen:
 * `unroll` 16-byte loads per thread in flight (1, 2, 4, 8), `block` threads
 * per workgroup (64..1024, powers of two), `policy` the buffer-load cache
 * bits (0, 1 sc0, 2 nt, 3, 16 sc1, 17, 18, 19) or -1 for the plain
 * nontemporal load of hbm_stream_read; -2 (block 256) launches the same grid
 * of empty workgroups: the launch floor.  No counterpart in the reference. */
int hbm_stream_read_cfg(aiter_tensor_t* src, aiter_tensor_t* sink, int grid, int block, int unroll, int policy,
                        aiter_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* AITER_AMD_H */
