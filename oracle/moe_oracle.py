"""CPU oracle for the fused-MoE path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
may import this module, and only as the checker; the product path
(``aiter_amd``) never calls into it.

numpy restatements of the reference, each citing the file:line it follows:
routing sort, quantisation of the sorted rows with the scale bytes in sorted
order, and the two grouped-GEMM stages.  How each function is checked
independently of its own formula is listed in ``PINNED`` at the bottom and
exercised by ``tests/test_oracle_moe.py``.
"""
from __future__ import annotations

import numpy as np
from scipy.special import erf

from . import mx_oracle as O

SILU, GELU = 0, 1


def moe_sorting_ref(topk_ids, topk_weights, num_experts: int, block_size: int, expert_mask=None,
                    num_local_tokens: int | None = None):
    """``run_torch_moe_sorting`` of op_tests/test_moe_sorting.py:45-98:
    experts in order; inside an expert the (token, slot) pairs in row-major
    order (torch.where); each expert padded to a multiple of block_size with
    ``topk << 24 | M``; block -> expert id renumbered over the kept experts.
    Returns (sorted_ids, sorted_weights, sorted_expert_ids, num_valid_ids);
    padding weights are 0 and unused blocks -1 (the reference leaves padding
    weights unset and fills unused blocks with -1)."""
    topk_ids = np.asarray(topk_ids)
    m, topk = topk_ids.shape
    max_padded = m * topk + num_experts * block_size - topk
    max_blocks = (max_padded + block_size - 1) // block_size
    sorted_ids = np.full(max_padded, (topk << 24) | m, dtype=np.int32)
    sorted_w = np.zeros(max_padded, dtype=np.float32)
    sorted_eids = np.full(max_blocks, -1, dtype=np.int32)
    ids = topk_ids[:num_local_tokens] if num_local_tokens is not None else topk_ids
    begin = eb = skip = 0
    for e in range(num_experts):
        if expert_mask is not None and expert_mask[e] == 0:
            skip += 1
            continue
        tok, slot = np.nonzero(ids == e)
        n = tok.size
        nb = (n + block_size - 1) // block_size
        sorted_ids[begin:begin + n] = (slot.astype(np.int32) << 24) | tok.astype(np.int32)
        sorted_w[begin:begin + n] = np.asarray(topk_weights, dtype=np.float32)[tok, slot]
        begin += nb * block_size
        sorted_eids[eb:eb + nb] = e - skip
        eb += nb
    return sorted_ids, sorted_w, sorted_eids, np.array([begin, ids.shape[0]], dtype=np.int32)


def sorted_source_rows(sorted_ids, num_valid: int, token_num: int, topk: int):
    """Input row of every sorted position and its validity
    (csrc/kernels/quant_kernels.cu:1788-1812): token (topk == 1, stage 1) or
    token * topk + slot (stage 2); positions >= num_valid are padding."""
    ids = np.asarray(sorted_ids, dtype=np.int64).copy()
    ids[num_valid:] = token_num
    tok, slot = ids & 0xFFFFFF, ids >> 24
    valid = tok < token_num
    row = tok if topk == 1 else tok * topk + slot
    return np.where(valid, row, 0), valid


def sort_scale_ref(scale_rows, sorted_ids, num_valid: int, token_num: int, topk: int):
    """e8m0 byte sort into the GEMM's A-scale layout: ``run_torch`` of
    op_tests/test_moe_sorting_mxfp4.py:42-67 (gather by sorted position,
    padding 0, pad to (32, 8), view (sm/32, 2, 16, sn/8, 2, 4), permute
    (0, 3, 5, 2, 4, 1))."""
    scale_rows = np.asarray(scale_rows, dtype=np.uint8)
    row, valid = sorted_source_rows(sorted_ids, num_valid, token_num, topk)
    s = np.where(valid[:, None], scale_rows[row], 0).astype(np.uint8)
    sm, sn = s.shape
    smp, snp = (sm + 31) // 32 * 32, (sn + 7) // 8 * 8
    p = np.zeros((smp, snp), dtype=np.uint8)
    p[:sm, :sn] = s
    v = p.reshape(smp // 32, 2, 16, snp // 8, 2, 4).transpose(0, 3, 5, 2, 4, 1)
    return np.ascontiguousarray(v).reshape(smp, snp)


def quant_sort_ref(x, sorted_ids, num_valid: int, token_num: int, fp8: bool = False, sorted_w=None):
    """fused_mx_quant_moe_sort_kernel (csrc/kernels/quant_kernels.cu:1733-1880):
    RoundUp e8m0 with the running max starting at 1e-10, per input row; scale
    bytes sorted by ``sort_scale_ref``; a sorted position whose routing weight
    is 0 writes a zero row and scale byte 0 (:1692-1731).
    Returns (q rows [R, K/2 or K] u8, written-row mask [R], sorted scale)."""
    x = np.asarray(x, dtype=np.float32)
    rows = x.shape[0]
    topk = rows // token_num
    if fp8:
        q, s = O.quant_mxfp8(x, O.ROUND_UP, amax_floor=1e-10)
    else:
        q, s = O.quant_mxfp4(x, O.ROUND_UP, amax_floor=1e-10)
    row, valid = sorted_source_rows(sorted_ids, num_valid, token_num, topk)
    written = np.zeros(rows, dtype=bool)
    written[row[valid]] = True
    s = s.copy()
    q = q.copy()
    if sorted_w is not None:
        zero = valid & (np.asarray(sorted_w)[: len(valid)] == 0)
        q[row[zero]] = 0
        s[row[zero]] = 0
    return q, written, sort_scale_ref(s, sorted_ids, num_valid, token_num, topk)


def act_ref(g: np.ndarray, act: int) -> np.ndarray:
    """torch F.silu / F.gelu (exact erf) in f32 (aiter.get_torch_act)."""
    g = np.asarray(g, dtype=np.float32)
    if act == GELU:
        return (0.5 * g * (1.0 + erf(g / np.sqrt(2.0)))).astype(np.float32)
    return (g / (1.0 + np.exp(-g))).astype(np.float32)


def moe_stage1_ref(a, w1, topk_ids, topk_w, act: int = SILU, doweight: bool = False, expert_mask=None):
    """torch_moe_stage1 (aiter/fused_moe.py:3437-3573) on dequantised f32
    operands: per routed pair (t, s) with expert e, h = a[t] @ w1[e]^T
    (* weight if doweight), gate/up split, act(gate) * up.  a [M, K], w1
    [E, 2I, K] -> [M, topk, I] f32 (pairs of masked experts stay 0)."""
    a = np.asarray(a, dtype=np.float32)
    M, topk = topk_ids.shape
    E, N2, _ = w1.shape
    inter = N2 // 2
    out = np.zeros((M, topk, inter), dtype=np.float32)
    for e in range(E):
        if expert_mask is not None and expert_mask[e] == 0:
            continue
        tok, slot = np.nonzero(topk_ids == e)
        if tok.size == 0:
            continue
        h = a[tok] @ w1[e].T
        if doweight:
            h = h * np.asarray(topk_w, dtype=np.float32)[tok, slot][:, None]
        out[tok, slot] = act_ref(h[:, :inter], act) * h[:, inter:]
    return out


def moe_stage2_ref(a2, w2, topk_ids, topk_w, doweight: bool = True, expert_mask=None):
    """torch_moe_stage2 (aiter/fused_moe.py:3575-3680): per routed pair,
    a2[t, s] @ w2[e]^T (* weight), summed over slots.  a2 [M, topk, I], w2
    [E, D, I] -> [M, D] f32."""
    a2 = np.asarray(a2, dtype=np.float32)
    M, topk = topk_ids.shape
    D = w2.shape[1]
    out = np.zeros((M, topk, D), dtype=np.float32)
    for e in range(w2.shape[0]):
        if expert_mask is not None and expert_mask[e] == 0:
            continue
        tok, slot = np.nonzero(topk_ids == e)
        if tok.size:
            out[tok, slot] = a2[tok, slot] @ w2[e].T
    if doweight:
        out = out * np.asarray(topk_w, dtype=np.float32)[:, :, None]
    return out.sum(axis=1)


def dequant_experts(wq, ws, fp8: bool = False):
    """[E, N, K/2] fp4x2 (or [E, N, K] e4m3) + plain scales [E * N, K/32] ->
    [E, N, K] f32 (fp4_utils.mxfp4_to_f32 * e8m0_to_f32 per 1x32 block,
    aiter/fused_moe.py:3519-3531)."""
    E, N = wq.shape[:2]
    flat = wq.reshape(E * N, -1)
    d = O.dequant_mxfp8(flat, ws) if fp8 else O.dequant_mxfp4(flat, ws)
    return d.reshape(E, N, -1)


def fused_moe_ref(x, w1, w2, topk_ids, topk_w, act: int = SILU, doweight_stage1: bool = False, a_fp8: bool = False,
                  expert_mask=None):
    """The per_1x32 two-stage flow (aiter/fused_moe.py:2892-3276) with the
    kernels' quantisation points: x -> RoundUp MX quant (running max 1e-10) ->
    stage 1 in f32 -> bf16 -> RoundUp MX quant -> stage 2 in f32 -> bf16 bits.
    x [M, K] f32 (bf16 values); w1 / w2 dequantised f32 [E, 2I, K] / [E, D, I]."""
    x = np.asarray(x, dtype=np.float32)
    M, topk = topk_ids.shape
    if a_fp8:
        q, s = O.quant_mxfp8(x, O.ROUND_UP, amax_floor=1e-10)
        a1 = O.dequant_mxfp8(q, s)
    else:
        q, s = O.quant_mxfp4(x, O.ROUND_UP, amax_floor=1e-10)
        a1 = O.dequant_mxfp4(q, s)
    h = moe_stage1_ref(a1, w1, topk_ids, topk_w, act, doweight_stage1, expert_mask)
    h = O.bf16_bits_to_f32(O.f32_to_bf16_bits(h)).reshape(M * topk, -1)
    if a_fp8:
        q2, s2 = O.quant_mxfp8(h, O.ROUND_UP, amax_floor=1e-10)
        a2 = O.dequant_mxfp8(q2, s2)
    else:
        q2, s2 = O.quant_mxfp4(h, O.ROUND_UP, amax_floor=1e-10)
        a2 = O.dequant_mxfp4(q2, s2)
    y = moe_stage2_ref(a2.reshape(M, topk, -1), w2, topk_ids, topk_w, not doweight_stage1, expert_mask)
    return O.f32_to_bf16_bits(y)


def logits_diff(x, y) -> float:
    """1 - cosine-style similarity of op_tests/test_moe_2stage.py:550-554."""
    x = np.asarray(x, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    return float(1.0 - 2.0 * (x * y).sum() / (x * x + y * y).sum())


PINNED = {
    "moe_sorting_ref": "invariants checked on random routings (every pair placed once, per-expert runs in "
                       "(token, slot) order, padding to block_size, block table) and a hand-worked known answer",
    "sorted_source_rows": "hand-worked known answer (stage 1 and stage 2 indexing)",
    "sort_scale_ref": "equals the closed-form index mx_scale_shuffle_idx (csrc/include/mx_quant_utils.h:212-216) "
                      "applied per sorted position",
    "quant_sort_ref": "composition of the pinned quant_mxfp4 / quant_mxfp8 and sort_scale_ref",
    "act_ref": "torch.nn.functional.silu / gelu (library routines)",
    "moe_stage1_ref": "float64 per-pair loop on tiny shapes (dense one-hot routing matrix formulation)",
    "moe_stage2_ref": "float64 per-pair loop on tiny shapes",
    "dequant_experts": "per-expert dequant_mxfp4 / dequant_mxfp8 (pinned in mx_oracle)",
    "fused_moe_ref": "composition of the pinned pieces; the end-to-end GPU test also reports logits_diff, the "
                     "reference test's acceptance metric (op_tests/test_moe_2stage.py:556-562)",
}
