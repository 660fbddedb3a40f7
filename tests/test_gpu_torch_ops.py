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


META_ONLY = ("test_schema", "test_autograd_registration", "test_faketensor")


def test_opcheck_lowp_outputs(cuda):
    import aiter_amd

    announce("opcheck gemm_a4w4o4 / gemm_a4w4o8")
    _, aq, as_, bq, bs = _mx_operands(cuda, m=128)
    # fp4x2 / e4m3 / e8m0 outputs: metadata checks, then byte equality with the Python entry points
    torch.library.opcheck(torch.ops.aiter_amd.gemm_a4w4o4.default, (aq, bq, as_, bs), test_utils=META_ONLY)
    torch.library.opcheck(torch.ops.aiter_amd.gemm_a4w4o8.default, (aq, bq, as_, bs), test_utils=META_ONLY)
    o4 = torch.ops.aiter_amd.gemm_a4w4o4(aq, bq, as_, bs)
    assert torch.equal(o4.view(torch.uint8), aiter_amd.gemm_a4w4o4(aq, bq, as_, bs).view(torch.uint8))
    q, s = torch.ops.aiter_amd.gemm_a4w4o8(aq, bq, as_, bs)
    q2, s2 = aiter_amd.gemm_a4w4o8(aq, bq, as_, bs)
    assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8))
    assert torch.equal(s.view(torch.uint8), s2.view(torch.uint8))


def test_opcheck_batched_bf16(cuda):
    import aiter_amd

    announce("opcheck batched_gemm_bf16")
    g = torch.Generator().manual_seed(83)
    x = torch.randn((4, 40, 512), generator=g).to(dtypes.bf16).to(cuda)
    w = torch.randn((4, 256, 512), generator=g).to(dtypes.bf16).to(cuda)
    torch.library.opcheck(torch.ops.aiter_amd.batched_gemm_bf16.default, (x, w))
    assert torch.equal(torch.ops.aiter_amd.batched_gemm_bf16(x, w), aiter_amd.batched_gemm_bf16_CK(x, w))


def test_opcheck_moe(cuda):
    import numpy as np

    import aiter_amd
    from oracle import mx_oracle as O

    announce("opcheck moe_sorting / fused_moe")
    rng = np.random.default_rng(84)
    m, e, topk, dim, inter = 20, 8, 2, 256, 256
    ids = torch.from_numpy(np.stack([rng.choice(e, topk, replace=False) for _ in range(m)]).astype(np.int32)).to(cuda)
    wts = torch.from_numpy(rng.random((m, topk)).astype(np.float32)).to(cuda)
    # sorted lists hold unwritten tails past num_valid_ids: metadata checks only
    torch.library.opcheck(torch.ops.aiter_amd.moe_sorting.default, (ids, wts, e, dim, dtypes.bf16, 32),
                          test_utils=META_ONLY)
    s, sw, se, nv, _ = torch.ops.aiter_amd.moe_sorting(ids, wts, e, dim, dtypes.bf16, 32)
    s2, sw2, se2, nv2, _ = aiter_amd.moe_sorting(ids, wts, e, dim, dtypes.bf16, 32)
    n = int(nv[0])
    assert torch.equal(nv, nv2) and torch.equal(s[:n], s2[:n]) and torch.equal(sw[:n], sw2[:n])
    assert torch.equal(se[: n // 32], se2[: n // 32])

    def w_dev(rows, k):
        q = rng.integers(0, 256, (e * rows, k // 2), dtype=np.uint8)
        sc = rng.integers(119, 123, (e * rows, k // 32), dtype=np.uint8)
        return (torch.from_numpy(O.shuffle_weight(q).reshape(e, rows, k // 2)).to(cuda),
                torch.from_numpy(O.shuffle_scale(sc)).to(cuda))

    w1, s1 = w_dev(2 * inter, dim)
    w2, s2_ = w_dev(dim, inter)
    x = torch.from_numpy(rng.standard_normal((m, dim)).astype(np.float32)).to(dtypes.bf16).to(cuda)
    # stage 2 may sum slots in either order: metadata checks, then closeness
    torch.library.opcheck(torch.ops.aiter_amd.fused_moe.default, (x, w1, w2, wts, ids, s1, s2_), test_utils=META_ONLY)
    got = torch.ops.aiter_amd.fused_moe(x, w1, w2, wts, ids, s1, s2_)
    want = aiter_amd.fused_moe(x, w1, w2, wts, ids, quant_type=aiter_amd.QuantType.per_1x32, w1_scale=s1,
                               w2_scale=s2_)
    torch.testing.assert_close(got.float(), want.float(), rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("shuffle", [False, True])
def test_opcheck_fused_rms_quant(cuda, shuffle):
    import aiter_amd

    announce(f"opcheck fused_rms_mxfp4/8_quant shuffle={shuffle}")
    g = torch.Generator().manual_seed(85)
    x = torch.randn((256, 1024), generator=g).to(dtypes.bf16).to(cuda)
    w = torch.randn((1024,), generator=g).to(dtypes.bf16).to(cuda)
    torch.library.opcheck(torch.ops.aiter_amd.fused_rms_mxfp4_quant.default, (x, w, 1e-6, shuffle),
                          test_utils=META_ONLY)
    q, s = torch.ops.aiter_amd.fused_rms_mxfp4_quant(x, w, 1e-6, shuffle)
    (q2, s2), _, _, _ = aiter_amd.fused_rms_mxfp4_quant(x, w, 1e-6, shuffle=shuffle)
    assert torch.equal(q, q2) and torch.equal(s, s2)
    torch.library.opcheck(torch.ops.aiter_amd.fused_rms_mxfp8_quant.default, (x, w, 1e-6), test_utils=META_ONLY)
    y, s8 = torch.ops.aiter_amd.fused_rms_mxfp8_quant(x, w, 1e-6)
    y2, s82 = aiter_amd.fused_rms_mxfp8_quant(x, w, 1e-6)
    assert torch.equal(y.view(torch.uint8), y2.view(torch.uint8)) and torch.equal(s8, s82)
