"""Fused MoE with MX weights: routing sort, sorted MX activation quant and the
two grouped GEMM stages, on this library's HIP kernels.

Mirrors the reference's entry points with their arguments and return values:
  moe_sorting                         aiter/fused_moe.py:337-403 (outputs of
                                      aiter/ops/moe_sorting.py:12-27)
  fused_dynamic_mx_quant_moe_sort     aiter/ops/quant.py:1036-1149
  fused_dynamic_mxfp4_quant_moe_sort  aiter/ops/quant.py:1152-1180
  fused_dynamic_mxfp8_quant_moe_sort  aiter/ops/quant.py:1183-1215
  mxfp4_moe_sort_fwd                  aiter/ops/quant.py:874-892
  ck_moe_stage1 / ck_moe_stage2       aiter/ops/moe_op.py:350-394
  ck_moe_stage1_fuse_quant            the stage-1 call of a fuse_quant == "fp4"
                                      configuration, aiter/fused_moe.py:3125-3171
  moe_sorting_mx_quant                moe_sorting + the stage-1 quant in one
                                      launch for decode-sized routing (the
                                      fusion of aiter/ops/flydsl/kernels/
                                      moe_fused_route_quant_scatter.py)
  fused_moe                           aiter/fused_moe.py:454-558 (the
                                      per_1x32 path of fused_moe_2stages,
                                      aiter/fused_moe.py:2892-3276)

Supported: QuantType.per_1x32 with MXFP4 (fp4x2) gate/up and down weights,
preshuffled with ``shuffle_weight`` and scales shuffled with ``shuffle_scale``;
MXFP4 activations (a4w4, the default) or MXFP8 activations (a8w4,
``q_dtype_a=dtypes.fp8`` on ``fused_moe_2stages``); gate+up weights
(w1 [E, 2 * inter_dim, model_dim / 2]); Silu and Gelu; routing weights applied
in stage 2 or, with ``doweight_stage1``, in stage 1; expert masks (EP).
Anything else raises.
"""
from __future__ import annotations

import enum
import functools

import torch

from . import dtypes
from ._lib import call
from .quant import QuantType, per_1x32_mx_quant_hip


class ActivationType(enum.IntEnum):
    """csrc/include/aiter_enum.h:7-14."""

    No = -1
    Silu = 0
    Gelu = 1
    Swiglu = 2
    Situv2 = 3


BLOCK_SIZE_M = 32


def _u8(t: torch.Tensor | None) -> torch.Tensor | None:
    if t is None or t.dtype == torch.uint8:
        return t
    return t.view(torch.uint8)


# ------------------------------------------------------------------ sorting
def moe_sorting_fwd(topk_ids, topk_weights, sorted_token_ids, sorted_weights, sorted_expert_ids, num_valid_ids,
                    moe_buf, num_experts: int, unit_size: int, local_expert_mask=None, num_local_tokens=None,
                    dispatch_policy: int = 0) -> None:
    """C entry of aiter/ops/moe_sorting.py:12-27."""
    call("moe_sorting_fwd", topk_ids, topk_weights, sorted_token_ids, sorted_weights, sorted_expert_ids,
         num_valid_ids, moe_buf, int(num_experts), int(unit_size), local_expert_mask, num_local_tokens,
         int(dispatch_policy))


def moe_sorting(topk_ids, topk_weights, num_experts, model_dim, moebuf_dtype, block_size=BLOCK_SIZE_M,
                expert_mask=None, num_local_tokens=None, dispatch_policy=0, accumulate=True):
    """-> (sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf).

    Sizes as aiter/fused_moe.py:206-215: ``max_num_tokens_padded = M * topk +
    E * block_size - topk``; ``moe_buf`` [M, model_dim] is zeroed (stage 2
    accumulates into it), or empty [0, 0] when ``accumulate`` is False and no
    expert mask is given (stage 2 then reduces per-pair rows instead)."""
    device = topk_ids.device
    M, topk = topk_ids.shape
    if topk_ids.dtype != torch.int32:
        topk_ids = topk_ids.to(torch.int32)
    if topk_weights.dtype != torch.float32:
        topk_weights = topk_weights.float()
    if expert_mask is not None and expert_mask.dtype != torch.int32:
        expert_mask = expert_mask.to(torch.int32)
    if num_local_tokens is not None and num_local_tokens.dtype != torch.int32:
        num_local_tokens = num_local_tokens.to(torch.int32)
    max_num_tokens_padded = int(topk_ids.numel() + num_experts * block_size - topk)
    max_num_m_blocks = int((max_num_tokens_padded + block_size - 1) // block_size)
    sorted_ids = torch.empty(max_num_tokens_padded, dtype=torch.int32, device=device)
    sorted_weights = torch.empty(max_num_tokens_padded, dtype=torch.float32, device=device)
    sorted_expert_ids = torch.empty(max_num_m_blocks, dtype=torch.int32, device=device)
    num_valid_ids = torch.empty(2, dtype=torch.int32, device=device)
    if expert_mask is not None or accumulate:
        moe_buf = torch.empty((M, model_dim), dtype=moebuf_dtype, device=device)
    else:
        moe_buf = torch.empty((0, 0), dtype=moebuf_dtype, device=device)
    moe_sorting_fwd(topk_ids.contiguous(), topk_weights.contiguous(), sorted_ids, sorted_weights, sorted_expert_ids,
                    num_valid_ids, moe_buf, num_experts, int(block_size), expert_mask, num_local_tokens,
                    dispatch_policy)
    return sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf


SORT_QUANT_MAX_ENTRIES = 256


def moe_sorting_mx_quant_fwd(topk_ids, topk_weights, hidden_states, sorted_token_ids, sorted_weights,
                             sorted_expert_ids, num_valid_ids, moe_buf, a_out, a_scale, num_experts: int,
                             unit_size: int) -> None:
    """C entry: the routing sort and the stage-1 MXFP4 activation quant in one
    launch (decode-sized routing; the fusion of
    aiter/ops/flydsl/kernels/moe_fused_route_quant_scatter.py)."""
    call("moe_sorting_mx_quant", topk_ids, topk_weights, hidden_states, sorted_token_ids, sorted_weights,
         sorted_expert_ids, num_valid_ids, moe_buf, _u8(a_out), _u8(a_scale), int(num_experts), int(unit_size))


def can_sort_quant(hidden_states, topk_ids, expert_mask=None, num_local_tokens=None, dispatch_policy=0) -> bool:
    """Whether moe_sorting_mx_quant takes this call: at most
    SORT_QUANT_MAX_ENTRIES routed entries, bf16 rows, no expert mask or
    device token count."""
    M, topk = topk_ids.shape
    K = hidden_states.shape[-1]
    return (expert_mask is None and num_local_tokens is None and dispatch_policy == 0 and
            M * topk <= SORT_QUANT_MAX_ENTRIES and hidden_states.dtype == dtypes.bf16 and hidden_states.dim() == 2 and
            K % 32 == 0 and K <= 65536)


def moe_sorting_mx_quant(topk_ids, topk_weights, hidden_states, num_experts, block_size=BLOCK_SIZE_M,
                         accumulate=True):
    """-> (sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf,
    a1, a1_scale): moe_sorting followed by fused_dynamic_mx_quant_moe_sort of
    ``hidden_states`` (fp4x2, sorted weights given) in one launch.  Sorted
    positions past num_valid_ids[0] (beyond its 32-row group) and the rows of
    tokens whose entries were all dropped stay unwritten.  Raises unless
    can_sort_quant holds."""
    if not can_sort_quant(hidden_states, topk_ids):
        raise ValueError("moe_sorting_mx_quant: needs at most %d routed entries, bf16 [M, K] rows with K %% 32 == 0 "
                         "and K <= 65536" % SORT_QUANT_MAX_ENTRIES)
    device = topk_ids.device
    M, topk = topk_ids.shape
    if topk_ids.dtype != torch.int32:
        topk_ids = topk_ids.to(torch.int32)
    if topk_weights.dtype != torch.float32:
        topk_weights = topk_weights.float()
    model_dim = hidden_states.shape[-1]
    max_num_tokens_padded = int(topk_ids.numel() + num_experts * block_size - topk)
    max_num_m_blocks = int((max_num_tokens_padded + block_size - 1) // block_size)
    sorted_ids = torch.empty(max_num_tokens_padded, dtype=torch.int32, device=device)
    sorted_weights = torch.empty(max_num_tokens_padded, dtype=torch.float32, device=device)
    sorted_expert_ids = torch.empty(max_num_m_blocks, dtype=torch.int32, device=device)
    num_valid_ids = torch.empty(2, dtype=torch.int32, device=device)
    moe_buf = torch.empty((M, model_dim) if accumulate else (0, 0), dtype=dtypes.bf16, device=device)
    a1 = torch.empty((M, model_dim // 2), dtype=dtypes.fp4x2, device=device)
    a1_scale = _sorted_scale(sorted_ids, model_dim, device)
    moe_sorting_mx_quant_fwd(topk_ids.contiguous(), topk_weights.contiguous(), hidden_states.contiguous(), sorted_ids,
                             sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf, a1, a1_scale, num_experts,
                             int(block_size))
    return sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf, a1, a1_scale


# ------------------------------------------------------------- sorted quant
def _sorted_scale(sorted_ids: torch.Tensor, cols: int, device) -> torch.Tensor:
    scale_n_pad = ((cols + 31) // 32 + 7) // 8 * 8
    return torch.empty(((sorted_ids.shape[0] + 31) // 32 * 32, scale_n_pad), dtype=torch.uint8,
                       device=device).view(dtypes.fp8_e8m0)


def fused_dynamic_mx_quant_moe_sort_hip(out, scales, input, sorted_ids, num_valid_ids, token_num: int,
                                        block_m: int, group_size: int = 32, sorted_weights=None) -> None:
    """C entry (aiter/ops/quant.py:895-911)."""
    call("fused_dynamic_mx_quant_moe_sort_hip", _u8(out) if out.dtype != dtypes.fp8 else out, _u8(scales), input,
         sorted_ids, num_valid_ids, int(token_num), int(block_m), int(group_size), sorted_weights)


def mxfp4_moe_sort_hip(out_scale, scale, sorted_ids, num_valid_ids, token_num: int, cols: int) -> None:
    """C entry (aiter/ops/quant.py:861-871): per-row e8m0 bytes -> sorted shuffled layout."""
    call("mxfp4_moe_sort_hip", _u8(out_scale), _u8(scale), sorted_ids, num_valid_ids, int(token_num), int(cols))


def mxfp4_moe_sort_fwd(scale, sorted_ids, num_valid_ids, token_num: int, cols: int):
    out_scale = _sorted_scale(sorted_ids, cols, scale.device)
    mxfp4_moe_sort_hip(out_scale, scale, sorted_ids, num_valid_ids, token_num, cols)
    return out_scale


def fused_dynamic_mx_quant_moe_sort(input, sorted_ids, num_valid_ids, token_num: int, topk: int, block_size: int,
                                    quant_dtype=dtypes.fp4x2, num_rows=None, group_size: int = 32,
                                    sorted_weights=None):
    """Per-1x32 MX quant (RoundUp e8m0) of the rows a sorted routing list
    names, with the scale bytes in sorted, shuffled order
    [pad32(len(sorted_ids)), pad8(cols/32)].  Stage 1 (input [token_num, K]):
    one row per token; stage 2 (input [token_num * topk, K]): one row per
    routed pair.  Small inputs take the fused kernel; larger ones quantise per
    row and then sort the scale bytes (the dispatch of
    aiter/ops/quant.py:1085-1149).  Rows whose sorted routing weight is 0 are
    written as zeros by the fused kernel."""
    if quant_dtype not in (dtypes.fp4x2, dtypes.fp8):
        raise ValueError(f"fused_dynamic_mx_quant_moe_sort: unsupported quant_dtype {quant_dtype}")
    if group_size != 32:
        raise ValueError("only group_size 32 (MX) is implemented")
    x = input.view(-1, input.shape[-1])
    M, N = x.shape
    out_cols = N // 2 if quant_dtype == dtypes.fp4x2 else N
    is_stage1 = M == token_num
    eff_topk = 1 if is_stage1 else topk
    scale = _sorted_scale(sorted_ids, N, x.device)
    # stage 2 names every input row once, so the fused kernel never re-reads
    # a row and is used at every size (the reference switches both stages to
    # the split path above 8 * 1024 rows, aiter/ops/quant.py:1085-1114);
    # stage 1 re-reads each token once per slot, so large inputs split
    use_fused = (not is_stage1) or M <= 8 * 256 / topk
    if use_fused:
        out = torch.empty(M, out_cols, dtype=quant_dtype, device=x.device)
        fused_dynamic_mx_quant_moe_sort_hip(out, scale, x, sorted_ids, num_valid_ids, token_num, block_size,
                                            group_size, sorted_weights)
    else:
        out, per_row = per_1x32_mx_quant_hip(x, quant_dtype=quant_dtype, shuffle=False, num_rows=num_rows,
                                             num_rows_factor=eff_topk,
                                             scale_type=dtypes.fp8_e8m0 if quant_dtype == dtypes.fp8 else None)
        mxfp4_moe_sort_hip(scale, per_row, sorted_ids, num_valid_ids, token_num, N)
    return out, scale


def fused_dynamic_mxfp4_quant_moe_sort(input, sorted_ids, num_valid_ids, token_num, topk, block_size, num_rows=None,
                                       group_size=32, sorted_weights=None):
    return fused_dynamic_mx_quant_moe_sort(input, sorted_ids, num_valid_ids, token_num, topk, block_size,
                                           dtypes.fp4x2, num_rows, group_size, sorted_weights)


def fused_dynamic_mxfp8_quant_moe_sort(input, sorted_ids, num_valid_ids, token_num, topk, block_size, num_rows=None,
                                       group_size=32, sorted_weights=None):
    return fused_dynamic_mx_quant_moe_sort(input, sorted_ids, num_valid_ids, token_num, topk, block_size,
                                           dtypes.fp8, num_rows, group_size, sorted_weights)


# ---------------------------------------------------------------- GEMM stages
def ck_moe_stage1(hidden_states, w1, w2, sorted_token_ids, sorted_expert_ids, num_valid_ids, out, topk: int,
                  kernelName: str | None = None, w1_scale=None, a1_scale=None, block_m: int | None = 32,
                  sorted_weights=None, quant_type: int = 0, activation: int = 0, splitk: int | None = 1,
                  use_non_temporal_load: bool = False, dst_type: str | None = None, is_shuffled: bool = True) -> None:
    """out [token_num, topk, inter_dim] bf16 = act(gate) * up of the expert
    GEMM over the sorted rows; ``sorted_weights`` (doweight_stage1) scales
    gate and up before the activation (aiter/fused_moe.py:3546-3573).
    ``splitk``: 1 = one pass over K, n > 1 = n K slices summed by a second
    kernel, 0 = chosen by the library (split when the tiles cannot fill the
    GPU, as in decode)."""
    a = hidden_states if hidden_states.dtype == dtypes.fp8 else _u8(hidden_states)
    call("ck_moe_stage1", a, _u8(w1), None, sorted_token_ids, sorted_expert_ids, num_valid_ids,
         out.view(-1, out.shape[-1]), int(topk), kernelName or "", _u8(w1_scale), _u8(a1_scale), int(block_m or 32),
         sorted_weights, int(quant_type), int(activation), int(1 if splitk is None else splitk),
         int(bool(use_non_temporal_load)),
         dst_type, int(bool(is_shuffled)))


def ck_moe_stage1_fuse_quant(hidden_states, w1, sorted_token_ids, sorted_expert_ids, num_valid_ids, token_num: int,
                             topk: int, block_m: int, w1_scale, a1_scale, sorted_weights=None, quant_weights=None,
                             activation: int = 0, splitk: int = 0, kernelName: str | None = None):
    """Stage 1 of a fuse_quant == "fp4" configuration (aiter/fused_moe.py:3125-3171):
    the GEMM of ck_moe_stage1 with its act(gate) * up rows quantised to MXFP4
    in the same launch.  Returns (a2 fp4x2 [token_num, topk, inter_dim / 2],
    a2_scale in the sorted, shuffled layout), the bytes that
    fused_dynamic_mx_quant_moe_sort(<ck_moe_stage1's bf16 output>, ...,
    sorted_weights=quant_weights) returns.  ``sorted_weights`` (doweight_stage1)
    scales gate and up before the activation, as in ck_moe_stage1."""
    inter_dim = w1.shape[1] // 2
    a2 = torch.empty((token_num, topk, inter_dim // 2), dtype=dtypes.fp4x2, device=hidden_states.device)
    a2_scale = _sorted_scale(sorted_token_ids, inter_dim, hidden_states.device)
    a = hidden_states if hidden_states.dtype == dtypes.fp8 else _u8(hidden_states)
    call("ck_moe_stage1_fuse_quant", a, _u8(w1), sorted_token_ids, sorted_expert_ids, num_valid_ids,
         _u8(a2.view(-1, a2.shape[-1])), _u8(a2_scale), int(topk), kernelName or "", _u8(w1_scale), _u8(a1_scale),
         int(block_m), sorted_weights, quant_weights, int(activation), int(splitk))
    return a2, a2_scale


def ck_moe_stage2(inter_states, w1, w2, sorted_token_ids, sorted_expert_ids, num_valid_ids, out, topk: int,
                  kernelName: str | None = None, w2_scale=None, a2_scale=None, block_m: int | None = 32,
                  sorted_weights=None, quant_type: int = 0, activation: int = 0, splitk: int = 1,
                  use_non_temporal_load: bool = False, dst_type: str | None = None, is_shuffled: bool = True) -> None:
    """out [token_num, model_dim] bf16 += sum over the routed pairs of
    weight * (a2 row @ w2[expert]^T) (aiter/fused_moe.py:3575-3680); ``out``
    must start at zero (moe_sorting zeroes its moe_buf).  With ``out``
    [token_num, topk, model_dim] each routed pair's weighted row is stored
    instead (no atomics) and ``moe_sum`` reduces the slots."""
    a = inter_states.view(-1, inter_states.shape[-1])
    a = a if a.dtype == dtypes.fp8 else _u8(a)
    call("ck_moe_stage2", a, None, _u8(w2), sorted_token_ids, sorted_expert_ids, num_valid_ids, out, int(topk),
         kernelName or "", _u8(w2_scale), _u8(a2_scale), int(block_m or 32), sorted_weights, int(quant_type),
         int(activation), int(splitk), int(bool(use_non_temporal_load)), dst_type, int(bool(is_shuffled)))


def moe_sum(input: torch.Tensor, output: torch.Tensor) -> None:
    """output [M, D] = sum over slots of input [M, topk, D] (bf16; f32 sums in
    slot order) (aiter/ops/moe_op.py:91-98)."""
    call("moe_sum", input, output)


# -------------------------------------------------------------------- fused
@functools.lru_cache(maxsize=2048)
def get_block_size_M(token: int, topk: int, expert: int, inter_dim: int) -> int:
    """Row block of the sorted list, from the average routed rows per expert:
    32 up to 16 rows, 64 up to 512, 128 above (measured end to end at the
    DeepSeek shape, 257 experts x topk 9: 32 is fastest up to 256 tokens,
    64 from 512 tokens (512: 232.5 against 238.3 us) to 8192, 128 slower
    everywhere there); the reference picks from its tuned table with the
    same candidates (aiter/fused_moe.py:1178-1193)."""
    per_expert = token * topk / max(expert, 1)
    if per_expert <= 16:
        return 32
    if per_expert <= 512:
        return 64
    return 128


def get_inter_dim(w1_shape, w2_shape):
    """(E, model_dim, inter_dim) from fp4x2 weight shapes (aiter/fused_moe.py:444-451)."""
    E, _, model_dim = w1_shape
    E, model_dim2, inter_dim = w2_shape
    return E, model_dim2, inter_dim * 2


def fused_moe_2stages(hidden_states, w1, w2, topk, sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids,
                      moe_out, block_size_M, activation=ActivationType.Silu, quant_type=QuantType.per_1x32,
                      doweight_stage1=False, q_dtype_a=dtypes.fp4x2, w1_scale=None, w2_scale=None,
                      num_local_tokens=None, expert_mask=None, a1=None, a1_scale=None):
    """The per_1x32 two-stage flow of aiter/fused_moe.py:2892-3276: quant +
    sort of the tokens, stage 1, quant + sort of the stage-1 output, stage 2
    accumulating into ``moe_out``.  ``a1`` / ``a1_scale``: the tokens already
    quantised with their scales in sorted order (moe_sorting_mx_quant)."""
    token_num = hidden_states.shape[0]
    E, model_dim, inter_dim = get_inter_dim(w1.shape, w2.shape)
    # per-pair rows miss the pairs routed to masked experts or past
    # num_local_tokens, so those cases accumulate (as in the reference)
    reduce = expert_mask is None and num_local_tokens is None and _use_reduce(token_num, topk)
    if moe_out.numel() == 0:
        moe_out = torch.empty((token_num, model_dim), dtype=dtypes.bf16, device=hidden_states.device)
    if a1 is None:
        a1, a1_scale = fused_dynamic_mx_quant_moe_sort(hidden_states, sorted_ids, num_valid_ids, token_num, topk,
                                                       block_size_M, q_dtype_a, num_rows=num_local_tokens,
                                                       sorted_weights=sorted_weights)
    if q_dtype_a == dtypes.fp4x2 and inter_dim % 256 == 0 and expert_mask is None and num_local_tokens is None:
        # fuse_quant "fp4": stage 1 writes its output already quantised (one
        # launch and one pass over the stage-1 output less)
        a2q, a2_scale = ck_moe_stage1_fuse_quant(a1, w1, sorted_ids, sorted_expert_ids, num_valid_ids, token_num,
                                                 topk, block_size_M, w1_scale, a1_scale,
                                                 sorted_weights if doweight_stage1 else None, sorted_weights,
                                                 int(activation))
    else:
        a2 = torch.empty((token_num, topk, inter_dim), dtype=dtypes.bf16, device=hidden_states.device)
        ck_moe_stage1(a1, w1, w2, sorted_ids, sorted_expert_ids, num_valid_ids, a2, topk, "", w1_scale, a1_scale,
                      block_size_M, sorted_weights if doweight_stage1 else None, int(quant_type), int(activation),
                      splitk=0)
        a2q, a2_scale = fused_dynamic_mx_quant_moe_sort(a2.view(-1, inter_dim), sorted_ids, num_valid_ids,
                                                        token_num, topk, block_size_M, q_dtype_a,
                                                        sorted_weights=sorted_weights)
    if reduce:
        # one row per routed pair, then a fixed-order sum over the slots: device-
        # wide atomics cost one memory-side operation per 4 bytes, which
        # dominates once there are more than a few hundred routed rows
        per_pair = torch.empty((token_num, topk, model_dim), dtype=moe_out.dtype, device=moe_out.device)
        ck_moe_stage2(a2q, w1, w2, sorted_ids, sorted_expert_ids, num_valid_ids, per_pair, topk, "", w2_scale,
                      a2_scale, block_size_M, None if doweight_stage1 else sorted_weights, int(quant_type))
        moe_sum(per_pair, moe_out)
    else:
        ck_moe_stage2(a2q, w1, w2, sorted_ids, sorted_expert_ids, num_valid_ids, moe_out, topk, "", w2_scale,
                      a2_scale, block_size_M, None if doweight_stage1 else sorted_weights, int(quant_type))
    return moe_out


REDUCE_MIN_ROWS = 128


def _use_reduce(token_num: int, topk: int) -> bool:
    """Per-pair rows + moe_sum instead of atomics: from REDUCE_MIN_ROWS routed rows."""
    return token_num * topk >= REDUCE_MIN_ROWS


def fused_moe(hidden_states, w1, w2, topk_weight, topk_ids, expert_mask=None, activation=ActivationType.Silu,
              quant_type=QuantType.No, doweight_stage1=False, w1_scale=None, w2_scale=None, a1_scale=None,
              a2_scale=None, block_size_M=None, num_local_tokens=None, moe_sorting_dispatch_policy=0, dtype=None,
              hidden_pad=0, intermediate_pad=0, bias1=None, bias2=None, splitk=0, swiglu_limit=None, beta=None,
              linear_beta=None, gate_mode=None):
    """Output [token_num, model_dim] (bf16 by default) of the routed experts,
    sum over slots of topk_weight * down(act(gate) * up)."""
    if QuantType(quant_type) != QuantType.per_1x32:
        raise NotImplementedError("fused_moe: only QuantType.per_1x32 (MXFP4 weights) is implemented")
    if w1.dtype not in (dtypes.fp4x2, torch.uint8) or w2.dtype not in (dtypes.fp4x2, torch.uint8):
        raise NotImplementedError("fused_moe: per_1x32 needs fp4x2 (MXFP4) weights")
    if ActivationType(activation) not in (ActivationType.Silu, ActivationType.Gelu):
        raise NotImplementedError(f"fused_moe: activation {activation} is not implemented")
    for name, v in (("hidden_pad", hidden_pad), ("intermediate_pad", intermediate_pad), ("splitk", splitk)):
        if v:
            raise NotImplementedError(f"fused_moe: {name} is not implemented")
    if any(v is not None for v in (bias1, bias2, swiglu_limit, beta, linear_beta, a1_scale, a2_scale)):
        raise NotImplementedError("fused_moe: biases, SwiGLU limits and static activation scales are not implemented")
    if w1_scale is None or w2_scale is None:
        raise ValueError("fused_moe: per_1x32 needs w1_scale and w2_scale")
    E, model_dim, inter_dim = get_inter_dim(w1.shape, w2.shape)
    if w1.shape[1] != 2 * inter_dim:
        raise NotImplementedError("fused_moe: w1 must hold gate and up rows ([E, 2 * inter_dim, model_dim / 2])")
    if not (getattr(w1, "is_shuffled", True) and getattr(w2, "is_shuffled", True)):
        raise ValueError("fused_moe: weights must be preshuffled (shuffle_weight)")
    token_num, topk = topk_ids.shape
    dtype = dtype or (hidden_states.dtype if hidden_states.dtype in (dtypes.bf16,) else dtypes.bf16)
    if dtype != dtypes.bf16:
        raise NotImplementedError("fused_moe: bf16 output only")
    # with an expert mask (EP) w1 / w2 hold the local experts only; topk_ids are
    # global ids and the sort renumbers them (aiter/fused_moe.py:703-705)
    global_E = expert_mask.numel() if expert_mask is not None else E
    bm = block_size_M if block_size_M and block_size_M > 0 else get_block_size_M(token_num, topk, global_E,
                                                                                 inter_dim)
    accumulate = not (expert_mask is None and num_local_tokens is None and _use_reduce(token_num, topk))
    a1 = a1_scale = None
    if can_sort_quant(hidden_states, topk_ids, expert_mask, num_local_tokens, moe_sorting_dispatch_policy):
        # decode: the sort and the token quant in one launch
        sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf, a1, a1_scale = moe_sorting_mx_quant(
            topk_ids, topk_weight, hidden_states, global_E, bm, accumulate=accumulate)
    else:
        sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids, moe_buf = moe_sorting(
            topk_ids, topk_weight, global_E, model_dim, dtype, bm, expert_mask, num_local_tokens,
            moe_sorting_dispatch_policy, accumulate=accumulate)
    return fused_moe_2stages(hidden_states, w1, w2, topk, sorted_ids, sorted_weights, sorted_expert_ids,
                             num_valid_ids, moe_buf, bm, activation, quant_type, doweight_stage1, dtypes.fp4x2,
                             w1_scale, w2_scale, num_local_tokens, expert_mask, a1=a1, a1_scale=a1_scale)
