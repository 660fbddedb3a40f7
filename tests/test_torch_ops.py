"""torch.ops.aiter_amd.*: schemas, fake implementations (shapes and dtypes on
meta tensors, no kernel run) and the loud failure on CPU tensors.  The GPU
half (real vs fake, torch.library.opcheck, equality with the Python entry
points) is in test_gpu_torch_ops.py."""
import pytest
import torch

import aiter_amd
from aiter_amd import dtypes
from aiter_amd.torch_ops import OPS

META = torch.device("meta")


def test_every_op_is_registered():
    for name in OPS:
        assert hasattr(torch.ops.aiter_amd, name), name


def test_fake_gemm_shapes():
    a = torch.empty(300, 512, dtype=torch.uint8, device=META)
    b = torch.empty(1024, 512, dtype=torch.uint8, device=META)
    sa = torch.empty(512, 32, dtype=torch.uint8, device=META)
    sb = torch.empty(1024, 32, dtype=torch.uint8, device=META)
    out = torch.ops.aiter_amd.gemm_a4w4(a, b, sa, sb)
    assert out.shape == (300, 1024) and out.dtype == dtypes.bf16
    a3 = torch.empty(2, 150, 512, dtype=torch.uint8, device=META)
    assert torch.ops.aiter_amd.gemm_a4w4(a3, b, sa, sb).shape == (2, 150, 1024)
    a8 = torch.empty(64, 1024, dtype=dtypes.fp8, device=META)
    assert torch.ops.aiter_amd.gemm_a8w4_mxfp8(a8, b, sa, sb).shape == (64, 1024)
    x = torch.empty(7, 256, dtype=dtypes.bf16, device=META)
    w = torch.empty(96, 256, dtype=dtypes.bf16, device=META)
    y = torch.ops.aiter_amd.gemm_a16w16(x, w, None, torch.float32)
    assert y.shape == (7, 96) and y.dtype == torch.float32
    assert torch.ops.aiter_amd.gemm_a16w16_opus(x, w).shape == (7, 96)


@pytest.mark.parametrize("shuffle", [False, True])
def test_fake_quant_shapes(shuffle):
    x = torch.empty(300, 1056, dtype=dtypes.bf16, device=META)
    y, s = torch.ops.aiter_amd.dynamic_mxfp4_quant(x, shuffle)
    assert y.shape == (300, 528) and y.dtype == dtypes.fp4x2
    assert s.shape == ((512, 40) if shuffle else (300, 33)) and s.dtype == dtypes.fp8_e8m0
    y, s = torch.ops.aiter_amd.dynamic_mxfp8_quant(x, shuffle)
    assert y.shape == (300, 1056) and y.dtype == dtypes.fp8
    assert s.shape == ((512, 40) if shuffle else (300, 33))


def test_cpu_tensors_fail_loudly():
    x = torch.zeros(4, 64, dtype=dtypes.bf16)
    with pytest.raises(NotImplementedError):
        torch.ops.aiter_amd.gemm_a16w16(x, torch.zeros(16, 64, dtype=dtypes.bf16))
    with pytest.raises(NotImplementedError):
        torch.ops.aiter_amd.dynamic_mxfp4_quant(x)


def test_fake_lowp_and_batched_shapes():
    a = torch.empty(128, 256, dtype=torch.uint8, device=META)
    b = torch.empty(512, 256, dtype=torch.uint8, device=META)
    sa = torch.empty(128, 16, dtype=torch.uint8, device=META)
    sb = torch.empty(512, 16, dtype=torch.uint8, device=META)
    o4 = torch.ops.aiter_amd.gemm_a4w4o4(a, b, sa, sb)
    assert o4.shape == (128, 256) and o4.dtype == dtypes.fp4x2
    q, s = torch.ops.aiter_amd.gemm_a4w4o8(a, b, sa, sb)
    assert q.shape == (128, 512) and q.dtype == dtypes.fp8
    assert s.shape == (128, 4) and s.dtype == dtypes.fp8_e8m0
    x = torch.empty(16, 7, 256, dtype=dtypes.bf16, device=META)
    w = torch.empty(16, 96, 256, dtype=dtypes.bf16, device=META)
    y = torch.ops.aiter_amd.batched_gemm_bf16(x, w)
    assert y.shape == (16, 7, 96) and y.dtype == dtypes.bf16


def test_fake_moe_shapes():
    ids = torch.empty(5, 9, dtype=torch.int32, device=META)
    wts = torch.empty(5, 9, dtype=torch.float32, device=META)
    s, sw, se, nv, buf = torch.ops.aiter_amd.moe_sorting(ids, wts, 257, 7168, dtypes.bf16, 32)
    padded = 5 * 9 + 257 * 32 - 9
    assert s.shape == (padded,) and sw.shape == (padded,) and se.shape == ((padded + 31) // 32,)
    assert nv.shape == (2,) and buf.shape == (5, 7168) and buf.dtype == dtypes.bf16
    h = torch.empty(5, 512, dtype=dtypes.bf16, device=META)
    w1 = torch.empty(8, 512, 256, dtype=torch.uint8, device=META)
    w2 = torch.empty(8, 512, 128, dtype=torch.uint8, device=META)
    s1 = torch.empty(8 * 512, 16, dtype=torch.uint8, device=META)
    s2 = torch.empty(8 * 512, 8, dtype=torch.uint8, device=META)
    out = torch.ops.aiter_amd.fused_moe(h, w1, w2, wts[:, :2], ids[:, :2], s1, s2)
    assert out.shape == (5, 512) and out.dtype == dtypes.bf16


@pytest.mark.parametrize("shuffle", [False, True])
def test_fake_fused_rms_quant_shapes(shuffle):
    x = torch.empty(300, 1056, dtype=dtypes.bf16, device=META)
    w = torch.empty(1056, dtype=dtypes.bf16, device=META)
    q, s = torch.ops.aiter_amd.fused_rms_mxfp4_quant(x, w, 1e-6, shuffle)
    assert q.shape == (300, 528) and s.shape == ((512, 40) if shuffle else (300, 33))
    y, s8 = torch.ops.aiter_amd.fused_rms_mxfp8_quant(x[:, :1024], w[:1024], 1e-6)
    assert y.shape == (300, 1024) and y.dtype == dtypes.fp8 and s8.shape == (300, 32)
