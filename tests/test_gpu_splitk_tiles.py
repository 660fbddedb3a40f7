"""Split-K tile instances (``*_tile_*_splitk*``): K split over gridDim.y into
f32 partial slices, summed by splitk_reduce_kernel.  Checked against the
oracle (rtol = atol = 1e-2) with even and uneven splits (the last split
shorter), alpha / bias through the reduce kernel, bf16 and f32 outputs, and
row-major and preshuffled B.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, bf16_operand, mxfp4_operand, mxfp8_operand

pytestmark = pytest.mark.gpu


def _rows(family, **kw):
    try:
        from aiter_amd._lib import kernel_table

        return [r for r in kernel_table() if r[2] == family and "_splitk" in r[1] and not r[3]
                and all(r[{"b_pre": 8, "out_f32": 9}[k]] == v for k, v in kw.items())]
    except Exception:  # library not built: collected, then skipped by the cuda fixture
        return []


def _dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


A4W4_ROWS = _rows("a4w4", out_f32=False)   # the f32 form feeds gemm_a4w4o4 / o8 (test_gpu_lowp_out.py)


@pytest.mark.parametrize("row", A4W4_ROWS, ids=[r[1] for r in A4W4_ROWS])
@pytest.mark.parametrize("log2_split", [1, 2])
def test_a4w4_split_tiles(cuda, row, log2_split):
    import aiter_amd

    name, b_pre = row[1], row[8]
    m, n, k = 72, 1040, 2560          # 10 stages: 2 splits of 5, or 4 splits of 3,3,3,1
    announce(f"a4w4 split tile {name} 2^{log2_split} {m}x{n}x{k}")
    a_q, a_s, a_ss = mxfp4_operand(m, k, 70, "triton")
    b_q, b_s, b_ss = mxfp4_operand(n, k, 71, "triton")
    bias = np.random.default_rng(72).standard_normal((1, n)).astype(np.float32)
    a = O.dequant_mxfp4(a_q, a_s)
    b = O.dequant_mxfp4(b_q, b_s)
    ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(0.5 * (a @ b.T) + 1.5 * bias))
    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q) if b_pre else b_q, cuda),
                            _dev(a_ss, cuda), _dev(b_ss, cuda), out, kernelName=name, bias=_dev(bias, cuda),
                            alpha=0.5, beta=1.5, bpreshuffle=bool(b_pre), log2_k_split=log2_split)
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, f"{name}: {msg}"


A8W4_ROWS = _rows("a8w4", out_f32=False)


@pytest.mark.parametrize("row", A8W4_ROWS, ids=[r[1] for r in A8W4_ROWS])
def test_a8w4_split_tiles(cuda, row):
    """The MXFP8 entry has no split argument: the library picks 2 splits here."""
    import aiter_amd

    name = row[1]
    m, n, k = 64, 512, 4096           # 4 tiles of 64x128 (2 of 64x256), 16 stages
    announce(f"a8w4 split tile {name} {m}x{n}x{k}")
    a_q, a_s, a_ss = mxfp8_operand(m, k, 73)
    b_q, b_s, b_ss = mxfp4_operand(n, k, 74, "triton")
    ref = O.bf16_bits_to_f32(O.gemm_a8w4_ref(a_q, b_q, a_s, b_s))
    out = aiter_amd.gemm_a8w4_mxfp8(_dev(a_q, cuda).view(torch.float8_e4m3fn), _dev(O.shuffle_weight(b_q), cuda),
                                    _dev(a_ss, cuda), _dev(b_ss, cuda), a_preshuffle=False, kernelName=name)
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, f"{name}: {msg}"


BF16_ROWS = _rows("a16w16")


@pytest.mark.parametrize("row", BF16_ROWS, ids=[r[1] for r in BF16_ROWS])
@pytest.mark.parametrize("splits", [2, 4])
def test_a16w16_split_tiles(cuda, row, splits):
    import aiter_amd

    name, b_pre, out_f32 = row[1], row[8], row[9]
    m, n, k = 100, 400, 640           # 10 stages of 64
    announce(f"a16w16 split tile {name} x{splits} {m}x{n}x{k}")
    a = bf16_operand(m, k, 75)
    b = bf16_operand(n, k, 76)
    bias = np.random.default_rng(77).standard_normal(n).astype(np.float32)
    c = O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T + bias
    ref = c if out_f32 else O.bf16_bits_to_f32(O.f32_to_bf16_bits(c))
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev((O.shuffle_weight(b) if b_pre else b).view(np.int16), cuda).view(torch.bfloat16)
    out = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=cuda)
    aiter_amd.gemm_a16w16_asm(at, bt, out, bias=_dev(bias, cuda), splitK=splits, kernelName=name,
                              bpreshuffle=bool(b_pre))
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, f"{name}: {msg}"


def test_split_tile_deterministic(cuda):
    """Fixed summation order: two calls give the same bits."""
    import aiter_amd

    m, n, k = 48, 2048, 8192
    announce(f"a16w16 split tile determinism {m}x{n}x{k}")
    g = torch.Generator().manual_seed(78)
    a = torch.randn((m, k), generator=g).to(torch.bfloat16).to(cuda)
    b = torch.randn((n, k), generator=g).to(torch.bfloat16).to(cuda)
    outs = []
    for _ in range(2):
        out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
        aiter_amd.gemm_a16w16_asm(a, b, out, splitK=8, kernelName="a16w16_tile_64x64_splitk_bplain")
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
