"""Fused RMSNorm -> MX quant (fused_rms_mxfp4_quant / fused_rms_mxfp8_quant,
aiter/ops/triton/quant/fused_mxfp4_quant.py:23-147, fused_mxfp8_quant.py:
22-76) against the CPU oracle.

* Exact case: rows of constant magnitude 2**e with eps = 0 make the norm
  factor exactly 2**-e, so every output is pinned bit for bit.
* Random case: the f32 sum of squares is reduced in a different order here
  than in numpy (and than in the reference's Triton kernel), so the norm
  factor may differ in its last bit; residual outputs are bit-exact, scale
  bytes and codes equal on all but a handful of elements sitting on a
  rounding boundary, where they differ by one step.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def _deq4(q, s):
    return O.dequant_mxfp4(q, s)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("fp8", [False, True])
def test_fused_rms_quant_exact(cuda, dtype, fp8):
    import aiter_amd

    m, k = 24, 3072
    announce(f"fused rms quant exact {dtype} fp8={fp8}")
    rs = np.random.default_rng(100)
    lo, hi = (-8, 8) if dtype == torch.float16 else (-30, 30)
    e = rs.integers(lo, hi, m)
    signs = rs.choice([-1.0, 1.0], (m, k)).astype(np.float32)
    x = signs * np.exp2(e.astype(np.float32))[:, None]
    w = torch.from_numpy((rs.standard_normal(k) * 2).astype(np.float32)).to(dtype)
    xt = torch.from_numpy(x).to(dtype)
    q_ref, s_ref, y_ref, _ = O.fused_rms_mx_quant_ref(xt.float().numpy(), w.float().numpy(), 0.0, fp8)
    if fp8:
        q, s = aiter_amd.fused_rms_mxfp8_quant(xt.to(cuda), w.to(cuda), 0.0)
    else:
        (q, s), _, _, _ = aiter_amd.fused_rms_mxfp4_quant(xt.to(cuda), w.to(cuda), 0.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(s), s_ref)
    np.testing.assert_array_equal(_u8(q), q_ref)


@pytest.mark.parametrize("m,k", [(1, 64), (7, 4096), (64, 7168), (33, 16384), (5, 32768)])
def test_fused_rms_mxfp4_random(cuda, m, k):
    import aiter_amd

    announce(f"fused rms mxfp4 random {m}x{k}")
    g = torch.Generator().manual_seed(101)
    x = (torch.randn((m, k), generator=g) * 3).to(torch.bfloat16)
    res = torch.randn((m, k), generator=g).to(torch.bfloat16)
    w = torch.randn(k, generator=g).to(torch.bfloat16)
    x2 = torch.randn((m, 1000), generator=g).to(torch.bfloat16)
    w2 = torch.randn(1000, generator=g).to(torch.bfloat16)
    (q, s), y1, y2, r1 = aiter_amd.fused_rms_mxfp4_quant(x.to(cuda), w.to(cuda), 1e-6, x2.to(cuda), w2.to(cuda),
                                                         1e-5, res.to(cuda), output_unquantized_inp1=True)
    torch.cuda.synchronize()
    q_ref, s_ref, y_ref, xr_ref = O.fused_rms_mx_quant_ref(x.float().numpy(), w.float().numpy(), 1e-6, False,
                                                           res.float().numpy())
    # residual: the bf16 of the f32 sum, bit-exact
    np.testing.assert_array_equal(r1.view(torch.int16).cpu().numpy(), O.f32_to_bf16_bits(xr_ref).view(np.int16))
    # unquantised normalised x1 and the second input, within bf16 rounding
    np.testing.assert_allclose(y1.float().cpu().numpy(), y_ref, rtol=1e-2, atol=1e-2)
    y2_ref, _ = O.rms_norm_f32(x2.float().numpy(), w2.float().numpy(), 1e-5)
    np.testing.assert_allclose(y2.float().cpu().numpy(), y2_ref, rtol=1e-2, atol=1e-2)
    # scales and codes: equal except on rounding boundaries
    s_gpu = _u8(s)
    assert (s_gpu != s_ref).mean() <= 1e-3
    d_gpu, d_ref = _deq4(_u8(q), s_gpu), _deq4(q_ref, s_ref)
    same = d_gpu == d_ref
    assert same.mean() >= 0.999, same.mean()
    # where they differ: neighbours on the grid (within one e2m1 step of the block scale)
    step = np.repeat(np.exp2(s_ref.astype(np.float64) - 127), 32, axis=1) * 2.0
    assert np.all(np.abs(d_gpu - d_ref)[~same] <= step[~same] + 1e-30)


@pytest.mark.parametrize("shuffle,padding", [(True, True), (False, True)])
def test_fused_rms_mxfp4_scale_layouts(cuda, shuffle, padding):
    """Shuffled / padded scale buffers: valid bytes at their (shuffled)
    positions, padding columns of valid rows = 127 (the reference kernel's
    fill, fused_mxfp4_quant.py:175-194)."""
    import aiter_amd

    m, k = 40, 1120                     # 35 blocks per row: 5 padding columns
    announce(f"fused rms mxfp4 scale layout shuffle={shuffle}")
    rs = np.random.default_rng(102)
    e = rs.integers(-10, 10, m)
    x = rs.choice([-1.0, 1.0], (m, k)).astype(np.float32) * np.exp2(e.astype(np.float32))[:, None]
    w = torch.from_numpy(rs.standard_normal(k).astype(np.float32)).to(torch.bfloat16)
    xt = torch.from_numpy(x).to(torch.bfloat16)
    (q, s), _, _, _ = aiter_amd.fused_rms_mxfp4_quant(xt.to(cuda), w.to(cuda), 0.0, shuffle=shuffle,
                                                      scale_shuffle_padding=padding)
    torch.cuda.synchronize()
    q_ref, s_ref, _, _ = O.fused_rms_mx_quant_ref(xt.float().numpy(), w.float().numpy(), 0.0, False)
    np.testing.assert_array_equal(_u8(q), q_ref)
    ss = _u8(s)
    assert ss.shape == (256, 40)
    full = np.full((m, 40), 127, dtype=np.uint8)
    full[:, :35] = s_ref
    if shuffle:
        xs, ys = np.meshgrid(np.arange(m), np.arange(40), indexing="ij")
        np.testing.assert_array_equal(ss.reshape(-1)[O.mx_scale_shuffle_idx(40, xs, ys)], full)
    else:
        np.testing.assert_array_equal(ss[:m], full)


def test_fused_rms_mxfp8_random(cuda):
    import aiter_amd

    m, k = 48, 7168
    announce(f"fused rms mxfp8 random {m}x{k}")
    g = torch.Generator().manual_seed(103)
    x = (torch.randn((m, k), generator=g) * 2).to(torch.bfloat16)
    w = torch.randn(k, generator=g).to(torch.bfloat16)
    q, s = aiter_amd.fused_rms_mxfp8_quant(x.to(cuda), w.to(cuda), 1e-6)
    torch.cuda.synchronize()
    q_ref, s_ref, _, _ = O.fused_rms_mx_quant_ref(x.float().numpy(), w.float().numpy(), 1e-6, True)
    s_gpu = _u8(s)
    assert (s_gpu != s_ref).mean() <= 1e-3
    d_gpu = O.dequant_mxfp8(_u8(q), s_gpu)
    d_ref = O.dequant_mxfp8(q_ref, s_ref)
    same = d_gpu == d_ref
    assert same.mean() >= 0.999, same.mean()
    np.testing.assert_allclose(d_gpu, d_ref, rtol=0.07, atol=1e-3)   # one e4m3 step is <= 2^-3 relative


def test_fused_matches_unfused_path(cuda):
    """The fused prologue against torch RMSNorm (f32) + this library's
    dynamic_mxfp4_quant of the f32 result: same scale bytes and codes except
    on rounding boundaries."""
    import aiter_amd

    m, k = 256, 8192
    announce("fused vs unfused rms + mxfp4 quant")
    g = torch.Generator().manual_seed(104)
    x = torch.randn((m, k), generator=g).to(torch.bfloat16).to(cuda)
    w = torch.randn(k, generator=g).to(torch.bfloat16).to(cuda)
    (q, s), _, _, _ = aiter_amd.fused_rms_mxfp4_quant(x, w, 1e-6)
    y = torch.nn.functional.rms_norm(x.float(), (k,), w.float(), eps=1e-6)
    q2, s2 = aiter_amd.dynamic_mxfp4_quant(y, shuffle=False)
    torch.cuda.synchronize()
    assert (s.cpu() != s2.view(torch.uint8).cpu()).float().mean() <= 1e-3
    assert (q.cpu() == q2.view(torch.uint8).cpu()).float().mean() >= 0.998
