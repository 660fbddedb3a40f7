"""HIP kernels (through the C-ABI) against the committed golden fixtures:
quantisers bit-exact, GEMMs within rtol = atol = 1e-2 of the fp32-accumulated
dequantised matmul."""
import os

import numpy as np
import pytest
import torch

from tests.conftest import announce

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
pytestmark = pytest.mark.gpu


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def dev_u8(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def bf16_from_bits(bits, dev):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(dev)


def test_quant_kernels_match_fixture(cuda):
    import aiter_amd
    from aiter_amd._lib import call

    g = load("quant_48x256.npz")
    x = bf16_from_bits(g["x_bf16_bits"], cuda)
    for mode in (0, 1, 2, 3):
        for shuf in (0, 1):
            announce(f"golden quant_mxfp4 mode={mode} shuffle={shuf}")
            q = torch.empty((48, 128), dtype=torch.uint8, device=cuda)
            s = torch.zeros((256, 8) if shuf else (48, 8), dtype=torch.uint8, device=cuda)
            call("quant_mxfp4", x, q, s, 32, mode, shuf, 0, 0, 0)
            np.testing.assert_array_equal(q.cpu().numpy(), g[f"fp4_mode{mode}_q"])
            want = g[f"fp4_mode{mode}_s_shuf"] if shuf else g[f"fp4_mode{mode}_s"]
            np.testing.assert_array_equal(s.cpu().numpy(), want)
    announce("golden per_1x32_mx_quant_hip (RoundUp production)")
    q, s = aiter_amd.per_1x32_mx_quant_hip(x, shuffle=False)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), g["fp4_prod_q"])
    np.testing.assert_array_equal(s.view(torch.uint8).cpu().numpy(), g["fp4_prod_s"])
    announce("golden dynamic_mxfp4_quant (Even)")
    q, s = aiter_amd.dynamic_mxfp4_quant(x, shuffle=False)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), g["fp4_triton_q"])
    np.testing.assert_array_equal(s.view(torch.uint8).cpu().numpy(), g["fp4_triton_s"])
    announce("golden dynamic_mxfp8_quant (Even)")
    q, s = aiter_amd.dynamic_mxfp8_quant(x)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), g["fp8_even_q"])
    np.testing.assert_array_equal(s.view(torch.uint8).cpu().numpy(), g["fp8_even_s"])


def _close(out, want_bits, what):
    from oracle.mx_oracle import bf16_bits_to_f32

    want = torch.from_numpy(bf16_bits_to_f32(want_bits))
    got = out.float().cpu()
    bad = ((got - want).abs() > 1e-2 + 1e-2 * want.abs()).float().mean().item()
    assert bad == 0.0, f"{what}: {bad:.4%} of elements outside rtol=atol=1e-2"


def test_gemms_match_fixture(cuda):
    import aiter_amd
    from aiter_amd._lib import kernel_table

    g = load("gemm_40x64x512.npz")
    aq, asf = dev_u8(g["a_fp4"], cuda), dev_u8(g["a_scale_shuf"], cuda)
    bq, bsf = dev_u8(g["b_fp4_shuf"], cuda), dev_u8(g["b_scale_shuf"], cuda)
    for kid, name, fam, skinny, bm, bn, split, a_pre, b_pre, of32 in kernel_table():
        # bf16-output kernels only (the f32-output ones feed gemm_a4w4o4 / o8,
        # tested in test_gpu_lowp_out.py)
        if fam != "a4w4" or not b_pre or of32 or (skinny and bm < 40):
            continue
        announce(f"golden a4w4 {name}")
        out = torch.zeros((64, 64), dtype=torch.bfloat16, device=cuda)
        aiter_amd.gemm_a4w4_blockscale_tune(aq, bq, asf, bsf, out, kernelId=kid, splitK=0)
        _close(out[:40], g["d_a4w4"], name)
    announce("golden gemm_a4w4 (dispatch)")
    _close(aiter_amd.gemm_a4w4(aq, bq, asf, bsf), g["d_a4w4"], "gemm_a4w4")
    announce("golden gemm_a8w4_mxfp8")
    a8 = dev_u8(g["a_fp8"], cuda).view(torch.float8_e4m3fn)
    out = aiter_amd.gemm_a8w4_mxfp8(a8, bq, dev_u8(g["a8_scale_shuf"], cuda), bsf, a_preshuffle=False)
    _close(out, g["d_a8w4"], "gemm_a8w4_mxfp8")
    announce("golden tgemm.mm bf16 (+bias)")
    a16 = bf16_from_bits(g["a_bf16"], cuda)
    b16 = bf16_from_bits(g["b_bf16"], cuda)
    _close(aiter_amd.tgemm.mm(a16, b16), g["d_a16w16"], "tgemm.mm")
    bias = torch.from_numpy(g["bias"]).to(cuda)
    _close(aiter_amd.tgemm.mm(a16, b16, bias=bias), g["d_a16w16_bias"], "tgemm.mm bias")
