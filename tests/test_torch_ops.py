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
