"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py) are reproduced by the oracle, and satisfy the
properties that do not depend on the oracle."""
import os

import numpy as np
import pytest

from oracle import mx_oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def test_quant_fixture_reproduced_by_oracle():
    g = load("quant_48x256.npz")
    x = O.bf16_bits_to_f32(g["x_bf16_bits"])
    for mode in (0, 1, 2, 3):
        q, s = O.quant_mxfp4(x, mode)
        np.testing.assert_array_equal(q, g[f"fp4_mode{mode}_q"])
        np.testing.assert_array_equal(s, g[f"fp4_mode{mode}_s"])
        np.testing.assert_array_equal(O.shuffle_scale(s), g[f"fp4_mode{mode}_s_shuf"])
    q, s = O.quant_mxfp4_triton_even(x)
    np.testing.assert_array_equal(q, g["fp4_triton_q"])
    np.testing.assert_array_equal(s, g["fp4_triton_s"])
    q, s = O.quant_mxfp8(x, O.EVEN)
    np.testing.assert_array_equal(q, g["fp8_even_q"])
    np.testing.assert_array_equal(s, g["fp8_even_s"])


def test_quant_fixture_edge_rows():
    g = load("quant_48x256.npz")
    for mode in (0, 1, 2, 3):
        q = g[f"fp4_mode{mode}_q"]
        assert not q[0, :16].any()                       # zero block -> zero codes
        deq = O.dequant_mxfp4(q[1:2, :16], g[f"fp4_mode{mode}_s"][1:2, :1])
        np.testing.assert_array_equal(deq, np.full((1, 32), -3.0, np.float32))
    assert g["fp4_prod_s"][0, 0] == 127 - 35              # production running-max floor 1e-10


@pytest.mark.parametrize("kind", ["a4w4", "a8w4", "a16w16", "a16w16_bias"])
def test_gemm_fixture_reproduced_by_oracle(kind):
    g = load("gemm_40x64x512.npz")
    if kind == "a4w4":
        d = O.gemm_a4w4_ref(g["a_fp4"], g["b_fp4"], g["a_scale"], g["b_scale"])
    elif kind == "a8w4":
        d = O.gemm_a8w4_ref(g["a_fp8"], g["b_fp4"], g["a8_scale"], g["b_scale"])
    elif kind == "a16w16":
        d = O.gemm_a16w16_ref(g["a_bf16"], g["b_bf16"])
    else:
        d = O.gemm_a16w16_ref(g["a_bf16"], g["b_bf16"], g["bias"])
    np.testing.assert_array_equal(d, g[f"d_{kind}"])


def test_gemm_fixture_layouts_invert():
    g = load("gemm_40x64x512.npz")
    np.testing.assert_array_equal(O.unshuffle_weight(g["b_fp4_shuf"]), g["b_fp4"])
    np.testing.assert_array_equal(O.unshuffle_scale(g["a_scale_shuf"], 40, 16), g["a_scale"])


def test_bf16_plumbing_config_oracle_vs_torch():
    """BASELINE configs[0] (A[128,4096] x B[4096,4096]^T bf16, torch seed 0):
    the oracle's bf16 GEMM against torch's CPU fp32 matmul of the same bf16
    operands (a library routine), rounded to bf16."""
    import torch

    g = torch.Generator().manual_seed(0)
    a = torch.randn(128, 4096, generator=g).to(torch.bfloat16)
    b = torch.randn(4096, 4096, generator=g).to(torch.bfloat16)
    want = (a.float() @ b.float().T).bfloat16().float().numpy()
    got = O.bf16_bits_to_f32(O.gemm_a16w16_ref(a.view(torch.int16).numpy().view(np.uint16),
                                               b.view(torch.int16).numpy().view(np.uint16)))
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)
    # the two f32 sums differ only in order: almost every bf16 result is equal
    assert (got == want).mean() > 0.99
