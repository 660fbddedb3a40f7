"""Writes the golden fixtures of tests/golden/ from the CPU oracle on seeded
inputs: ``python tests/golden/make_golden.py``.

Each fixture holds the inputs and the expected outputs of one case (numpy
.npz, no pickles).  The HIP path is checked against them by
tests/test_gpu_golden.py; tests/test_golden.py checks that the oracle still
reproduces them.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import mx_oracle as O  # noqa: E402


def quant_cases():
    rs = np.random.default_rng(42)
    x = (rs.standard_normal((48, 256)) * 2.0 ** rs.integers(-4, 5, (48, 1))).astype(np.float32)
    x[0, :32] = 0.0                     # all-zero block
    x[1, :32] = -3.0                    # constant block
    x[2, 5] = 1e4                       # one large outlier
    xb = O.bf16_bits_to_f32(O.f32_to_bf16_bits(x))  # bf16-representable input
    out = {"x_bf16_bits": O.f32_to_bf16_bits(x)}
    for mode in (0, 1, 2, 3):
        q, s = O.quant_mxfp4(xb, mode)
        out[f"fp4_mode{mode}_q"] = q
        out[f"fp4_mode{mode}_s"] = s
        out[f"fp4_mode{mode}_s_shuf"] = O.shuffle_scale(s)
    q, s = O.quant_mxfp4(xb, O.ROUND_UP, amax_floor=1e-10)   # dynamic_per_group_scaled_quant
    out["fp4_prod_q"], out["fp4_prod_s"] = q, s
    q, s = O.quant_mxfp4_triton_even(xb)                      # dynamic_mxfp4_quant
    out["fp4_triton_q"], out["fp4_triton_s"] = q, s
    q, s = O.quant_mxfp8(xb, O.EVEN)                          # dynamic_mxfp8_quant
    out["fp8_even_q"], out["fp8_even_s"] = q, s
    np.savez_compressed(os.path.join(HERE, "quant_48x256.npz"), **out)


def gemm_cases():
    rs = np.random.default_rng(7)
    m, n, k = 40, 64, 512
    a = rs.standard_normal((m, k)).astype(np.float32)
    b = rs.standard_normal((n, k)).astype(np.float32)
    aq, as_ = O.quant_mxfp4_triton_even(a)
    bq, bs = O.quant_mxfp4_triton_even(b)
    a8, as8 = O.quant_mxfp8(a, O.EVEN)
    bias = rs.standard_normal(n).astype(np.float32)
    a16 = O.f32_to_bf16_bits(a)
    b16 = O.f32_to_bf16_bits(b)
    np.savez_compressed(
        os.path.join(HERE, "gemm_40x64x512.npz"),
        a_fp4=aq, a_scale=as_, b_fp4=bq, b_scale=bs, b_fp4_shuf=O.shuffle_weight(bq),
        a_scale_shuf=O.shuffle_scale(as_), b_scale_shuf=O.shuffle_scale(bs),
        a_fp8=a8, a8_scale=as8, a8_scale_shuf=O.shuffle_scale(as8),
        a_bf16=a16, b_bf16=b16, bias=bias,
        d_a4w4=O.gemm_a4w4_ref(aq, bq, as_, bs),
        d_a8w4=O.gemm_a8w4_ref(a8, bq, as8, bs),
        d_a16w16=O.gemm_a16w16_ref(a16, b16),
        d_a16w16_bias=O.gemm_a16w16_ref(a16, b16, bias),
    )


if __name__ == "__main__":
    quant_cases()
    gemm_cases()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
