"""Empty inputs (M = 0 rows): every entry point returns an empty result of
the right shape and dtype and launches nothing."""
import pytest
import torch

from tests.conftest import announce

pytestmark = pytest.mark.gpu


def test_empty_rows(cuda):
    import aiter_amd

    announce("empty inputs M=0")
    k, n = 512, 256
    x = torch.zeros((0, k), dtype=torch.bfloat16, device=cuda)
    q, s = aiter_amd.dynamic_mxfp4_quant(x)
    assert tuple(q.shape) == (0, k // 2) and tuple(s.shape) == (0, k // 32)
    q8, s8 = aiter_amd.dynamic_mxfp8_quant(x)
    assert tuple(q8.shape) == (0, k) and tuple(s8.shape) == (0, k // 32)
    b = torch.randn((n, k), device=cuda).to(torch.bfloat16)
    bq, bs = aiter_amd.dynamic_mxfp4_quant(b, shuffle=True)
    bq = aiter_amd.shuffle_weight(bq)
    out = aiter_amd.gemm_a4w4(q, bq, s, bs)
    assert tuple(out.shape) == (0, n) and out.dtype == torch.bfloat16
    o4 = aiter_amd.gemm_a4w4o4(q, bq, s, bs)
    assert tuple(o4.shape) == (0, n // 2)
    y = aiter_amd.gemm_a16w16(x, b)
    assert tuple(y.shape) == (0, n)
    torch.cuda.synchronize()
