"""Low-precision GEMM outputs (gemm_a4w4o4 / gemm_a4w4o8, mxfp4_gemm_asm) on the
GPU against the oracle.

* e2m1 output: the reference kernel is scale-free, so the product of fp4
  codes is exact in f32 in any summation order (codes x 2 are small
  integers): every byte must match.
* MXFP8 output with unit input scales: the f32 product is again exact, so
  e4m3 bytes and packed e8m0 scale bytes must match exactly.
* MXFP8 output with random scales: the f32 sums depend on order, so the
  reference test's criterion (op_tests/test_f4gemm.py:381-400: scale bytes
  within +-1, dequantised data within rtol 0.1 / atol 1) is asserted, and in
  addition >= 99.9 % of scale bytes and codes equal.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def _operands(m, n, k, seed, scale_lo=127, scale_hi=128):
    rng = np.random.default_rng(seed)
    aq = rng.integers(0, 256, (m, k // 2), dtype=np.uint8)
    bq = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    a_s = rng.integers(scale_lo, scale_hi, (m, k // 32), dtype=np.uint8)
    b_s = rng.integers(scale_lo, scale_hi, (n, k // 32), dtype=np.uint8)
    return aq, bq, a_s, b_s


def _call(cuda, fn, aq, bq, a_s, b_s):
    return fn(_dev(aq, cuda), _dev(O.shuffle_weight(bq), cuda), _dev(O.shuffle_scale(a_s), cuda),
              _dev(O.shuffle_scale(b_s), cuda))


# the last two fill the CUs with 256x256 tiles: e2m1 straight from the
# persistent kernel's epilogue (the second ragged in M and in its last tile)
@pytest.mark.parametrize("m,n,k", [(1, 256, 256), (64, 512, 512), (200, 1008, 1024), (256, 4096, 2048),
                                   (4096, 4096, 256), (4000, 4128, 256)])
def test_a4w4o4_exact(cuda, m, n, k):
    import aiter_amd

    announce(f"gemm_a4w4o4 {m}x{n}x{k}")
    aq, bq, a_s, b_s = _operands(m, n, k, m + n + k, 110, 140)   # scales are ignored by the fp4-output form
    out = _call(cuda, aiter_amd.gemm_a4w4o4, aq, bq, a_s, b_s)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (m, n // 2)
    np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), O.gemm_a4w4o4_ref(aq, bq))


@pytest.mark.parametrize("m,n,k", [(64, 128, 256), (128, 512, 1024), (256, 2048, 512)])
def test_a4w4o8_unit_scales_exact(cuda, m, n, k):
    import aiter_amd

    announce(f"gemm_a4w4o8 unit scales {m}x{n}x{k}")
    aq, bq, a_s, b_s = _operands(m, n, k, 7 * m + n + k)
    q, s = _call(cuda, aiter_amd.gemm_a4w4o8, aq, bq, a_s, b_s)
    torch.cuda.synchronize()
    rq, rs = O.gemm_a4w4o8_ref(aq, bq, a_s, b_s)
    np.testing.assert_array_equal(q.view(torch.uint8).cpu().numpy(), rq)
    np.testing.assert_array_equal(s.view(torch.uint8).cpu().numpy().reshape(-1), O.pack_mxfp8_out_scale(rs))
    np.testing.assert_array_equal(aiter_amd.unpack_mxfp8_out_scale(s, m, n).view(torch.uint8).cpu().numpy(), rs)


@pytest.mark.parametrize("m,n,k", [(64, 256, 512), (192, 1024, 2048)])
def test_a4w4o8_random_scales(cuda, m, n, k):
    import aiter_amd

    announce(f"gemm_a4w4o8 random scales {m}x{n}x{k}")
    aq, bq, a_s, b_s = _operands(m, n, k, 11 * m + n + k, 118, 134)
    q, s = _call(cuda, aiter_amd.gemm_a4w4o8, aq, bq, a_s, b_s)
    torch.cuda.synchronize()
    rq, rs = O.gemm_a4w4o8_ref(aq, bq, a_s, b_s)
    gs = O.unpack_mxfp8_out_scale(s.view(torch.uint8).cpu().numpy(), m, n)
    gq = q.view(torch.uint8).cpu().numpy()
    ds = gs.astype(int) - rs.astype(int)
    assert np.abs(ds).max() <= 1 and np.mean(ds == 0) >= 0.999
    deq = lambda qq, ss: (O.e4m3_decode(qq).reshape(m, n // 128, 128)
                          * np.exp2(ss.astype(np.float64) - 127)[..., None]).reshape(m, n)
    got, ref = deq(gq, gs), deq(rq, rs)
    assert np.all(np.abs(got - ref) <= 1.0 + 0.1 * np.abs(ref))
    assert np.mean(gq == rq) >= 0.999


def test_bf16_form_matches_gemm_a4w4(cuda):
    """mxfp4_gemm_asm with a bf16 output is gemm_a4w4 (same kernels, same bytes)."""
    import aiter_amd

    m, n, k = 96, 512, 1024
    announce(f"gemm_mxfp4_asm bf16 {m}x{n}x{k}")
    aq, bq, a_s, b_s = _operands(m, n, k, 5, 120, 134)
    args = (_dev(aq, cuda), _dev(O.shuffle_weight(bq), cuda), _dev(O.shuffle_scale(a_s), cuda),
            _dev(O.shuffle_scale(b_s), cuda))
    o1 = aiter_amd.gemm_mxfp4_asm(*args, dtype=torch.bfloat16, a_preshuffle=False)
    o2 = aiter_amd.gemm_a4w4(*args)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2[:m])


@pytest.mark.parametrize("kname", ["a4w4_tile_128x256_f32", "a4w4_tile_256x256_f32_persist",
                                   "a4w4_tile_128x128_f32", "a4w4_tile_64x128_f32", "a4w4_tile_64x128_splitk_f32"])
def test_f32_tile_kernels_by_name(cuda, kname):
    """Each f32-output A4W4 kernel behind the low-precision forms, picked by name."""
    import aiter_amd
    from aiter_amd.gemm_op_a4w4 import _alloc_f4gemm_out, _mxfp4_gemm_asm

    m, n, k = 320, 768, 1024
    announce(f"mxfp4_gemm_asm fp4 out via {kname} {m}x{n}x{k}")
    aq, bq, a_s, b_s = _operands(m, n, k, 13)
    out = _alloc_f4gemm_out(m, n, aiter_amd.dtypes.fp4x2, cuda)
    _mxfp4_gemm_asm(_dev(aq, cuda), _dev(O.shuffle_weight(bq), cuda), _dev(O.shuffle_scale(a_s), cuda),
                    _dev(O.shuffle_scale(b_s), cuda), out, None, kname, 0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.view(torch.uint8).cpu().numpy(), O.gemm_a4w4o4_ref(aq, bq))
