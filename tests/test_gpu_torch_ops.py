"""torch.ops.aiter_amd.* on the GPU: torch.library.opcheck (schema, fake vs
real outputs, aliasing) and equality with the Python entry points."""
import pytest
import torch

from aiter_amd import dtypes
from tests.conftest import announce

pytestmark = pytest.mark.gpu


def _mx_operands(cuda, m=96, n=512, k=1024, seed=80):
    import aiter_amd

    g = torch.Generator().manual_seed(seed)
    a = torch.randn((m, k), generator=g).to(cuda)
    b = torch.randn((n, k), generator=g).to(cuda)
    aq, as_ = aiter_amd.dynamic_mxfp4_quant(a, shuffle=True)
    bq, bs = aiter_amd.dynamic_mxfp4_quant(b, shuffle=True)
    # byte views: opcheck compares inputs arithmetically, which torch does not
    # implement for the fp4x2 / e8m0 dtypes (the ops accept u8 as well)
    u8 = lambda t: t.view(torch.uint8)
    return a, u8(aq), u8(as_), u8(aiter_amd.shuffle_weight(bq)), u8(bs)


def test_opcheck_gemm_a4w4(cuda):
    import aiter_amd

    announce("opcheck gemm_a4w4")
    _, aq, as_, bq, bs = _mx_operands(cuda)
    torch.library.opcheck(torch.ops.aiter_amd.gemm_a4w4.default, (aq, bq, as_, bs))
    got = torch.ops.aiter_amd.gemm_a4w4(aq, bq, as_, bs)
    assert torch.equal(got, aiter_amd.gemm_a4w4(aq, bq, as_, bs))


def test_opcheck_gemm_a4w4_asm(cuda):
    announce("opcheck gemm_a4w4_asm")
    _, aq, as_, bq, bs = _mx_operands(cuda)
    out = torch.empty((96, 512), dtype=dtypes.bf16, device=cuda)
    torch.library.opcheck(torch.ops.aiter_amd.gemm_a4w4_asm.default, (aq, bq, as_, bs, out))


def test_opcheck_gemm_a8w4(cuda):
    import aiter_amd

    announce("opcheck gemm_a8w4_mxfp8")
    a, _, _, bq, bs = _mx_operands(cuda)
    a8, s8 = aiter_amd.dynamic_mxfp8_quant(a.to(dtypes.bf16), shuffle=True)
    torch.library.opcheck(torch.ops.aiter_amd.gemm_a8w4_mxfp8.default,
                          (a8.view(torch.uint8), bq, s8.view(torch.uint8), bs, False))


def test_opcheck_gemm_a16w16(cuda):
    import aiter_amd

    announce("opcheck gemm_a16w16 / opus")
    g = torch.Generator().manual_seed(81)
    x = torch.randn((40, 512), generator=g).to(dtypes.bf16).to(cuda)
    w = torch.randn((256, 512), generator=g).to(dtypes.bf16).to(cuda)
    torch.library.opcheck(torch.ops.aiter_amd.gemm_a16w16.default, (x, w))
    torch.library.opcheck(torch.ops.aiter_amd.gemm_a16w16_opus.default, (x, w))
    assert torch.equal(torch.ops.aiter_amd.gemm_a16w16(x, w), aiter_amd.gemm_a16w16(x, w))
    ws = aiter_amd.shuffle_weight(w)
    got = torch.ops.aiter_amd.gemm_a16w16(x, ws, None, None, True)
    torch.testing.assert_close(got.float(), aiter_amd.gemm_a16w16(x, w).float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("shuffle", [False, True])
def test_opcheck_quant(cuda, shuffle):
    import aiter_amd

    announce(f"opcheck quantisers shuffle={shuffle}")
    g = torch.Generator().manual_seed(82)
    # 256 rows: every byte of the shuffled scale buffer is written (rows past
    # pad32(M) are left untouched, so repeated runs could differ there)
    x256 = torch.randn((256, 1024), generator=g).to(dtypes.bf16).to(cuda)
    # outputs are fp4x2 / e4m3 / e8m0, which torch cannot compare numerically:
    # schema, autograd registration and fake-vs-real metadata only
    for name in ("dynamic_mxfp4_quant", "dynamic_mxfp8_quant", "per_1x32_f4_quant_hip"):
        torch.library.opcheck(getattr(torch.ops.aiter_amd, name).default, (x256, shuffle),
                              test_utils=("test_schema", "test_autograd_registration", "test_faketensor"))
    x = torch.randn((100, 1024), generator=g).to(dtypes.bf16).to(cuda)
    y, s = torch.ops.aiter_amd.dynamic_mxfp4_quant(x, shuffle)
    y2, s2 = aiter_amd.dynamic_mxfp4_quant(x, shuffle=shuffle)
    assert torch.equal(y.view(torch.uint8), y2.view(torch.uint8))
    rows = (100 + 31) // 32 * 32 if shuffle else 100      # rows past pad32(M) are never written
    assert torch.equal(s.view(torch.uint8)[:rows], s2.view(torch.uint8)[:rows])
