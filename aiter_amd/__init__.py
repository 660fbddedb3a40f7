"""aiter_amd — MI355X (gfx950) scaled-GEMM hot path with aiter's API.

Ops (all backed by hand-written HIP kernels in libaiter_amd.so):
  gemm_a4w4, gemm_a4w4_asm, gemm_a4w4_blockscale(_tune)   MXFP4 x MXFP4
  gemm_a8w4_mxfp8, gemm_a8w4_mxfp8_dynamic                MXFP8 x MXFP4
  gemm_a16w16, tgemm.mm, gemm_a16w16_opus, gemm_a16w16_asm bf16
  get_hip_quant / get_triton_quant(QuantType.per_1x32), quant_mxfp4_hip,
  per_1x32_mx_quant_hip, dynamic_mxfp4_quant, dynamic_mxfp8_quant
  fused_rms_mxfp4_quant, fused_rms_mxfp8_quant            RMSNorm -> MX quant
  shuffle_weight, shuffle_scale
The GEMMs and quantisers are also torch custom ops, torch.ops.aiter_amd.<name>
(torch_ops.py), with fake implementations for torch.compile / torch.export.
"""
from . import dtypes
from .gemm_common import get_padded_m
from .gemm_op_a4w4 import (MXFP8_OUT_SCALE_BLOCK, gemm_a4w4o4, gemm_a4w4o8, gemm_mxfp4_asm, unpack_mxfp8_out_scale,
                           compute_gemm_SplitK, gemm_a4w4, gemm_a4w4_asm, gemm_a4w4_blockscale,
                           gemm_a4w4_blockscale_tune, get_GEMM_config)
from .batched_gemm_op_bf16 import batched_gemm_bf16, batched_gemm_bf16_CK, batched_gemm_bf16_tune
from .fused_quant import fused_rms_mxfp4_quant, fused_rms_mxfp8_quant
from .fused_gemm import (fused_gemm_afp4wfp4_a16w16, fused_gemm_afp4wfp4_mul_add,
                         fused_gemm_afp4wfp4_preshuffle_add_mul, fused_gemm_afp4wfp4_preshuffle_split_cat,
                         fused_gemm_afp4wfp4_split_cat)
from .fused_moe import (ActivationType, ck_moe_stage1, ck_moe_stage1_fuse_quant, ck_moe_stage2,
                        fused_dynamic_mx_quant_moe_sort, fused_dynamic_mxfp4_quant_moe_sort, fused_dynamic_mxfp8_quant_moe_sort, fused_moe,
                        fused_moe_2stages, get_block_size_M, moe_sorting, moe_sorting_fwd, moe_sorting_mx_quant,
                        moe_sum, mxfp4_moe_sort_fwd)
from .gemm_op_a8w4 import gemm_a8w4_mxfp8, gemm_a8w4_mxfp8_dynamic
from .gemm_op_a16w16 import gemm_a16w16_asm
from .opus import gemm_a16w16_opus, opus_gemm_a16w16_tune, opus_gemm_workspace_init
from .quant import (MxScaleRoundMode, QuantType, dynamic_mxfp4_quant, dynamic_mxfp8_quant, get_hip_quant,
                    get_triton_quant, per_1x32_f4_quant_hip, per_1x32_f4_quant_triton, per_1x32_mx_quant_hip,
                    quant_mxfp4_hip)
from .shuffle import e8m0_shuffle, shuffle_scale, shuffle_weight
from .tuned_gemm import TunedGemm, gemm_a16w16, get_GEMM_A16W16_config, tgemm
from . import torch_ops  # registers torch.ops.aiter_amd.*

__all__ = [n for n in dir() if not n.startswith("_")]
