"""Batched bf16 GEMM (batched_gemm_bf16 / _CK / _tune, and the opus API) as one
launch over the batch, against the oracle's f32-accumulated reference per batch
(rtol = atol = 1e-2; op_tests/test_batched_gemm_bf16.py:25-33 compares the same
way).  Covers bias [N] and [B, N], the reference test's [m, b, k] transposed
layout for X and Y, f32 output, and explicit kernel ids."""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, bf16_operand

pytestmark = pytest.mark.gpu


def _bf16(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).to(cuda).view(torch.bfloat16)


def _ref(a_bits, b_bits, bias=None, out_f32=False):
    c = O.bf16_bits_to_f32(a_bits) @ O.bf16_bits_to_f32(b_bits).T
    if bias is not None:
        c = c + bias
    return c if out_f32 else O.bf16_bits_to_f32(O.f32_to_bf16_bits(c))


@pytest.mark.parametrize("b,m,n,k", [(2, 1, 1024, 512), (16, 32, 256, 1024), (4, 200, 384, 640), (8, 64, 512, 4096)])
@pytest.mark.parametrize("bias_kind", ["none", "shared", "per_batch"])
def test_batched_gemm_bf16(cuda, b, m, n, k, bias_kind):
    import aiter_amd

    announce(f"batched bf16 b={b} {m}x{n}x{k} bias={bias_kind}")
    a = np.stack([bf16_operand(m, k, 10 * i + 1) for i in range(b)])
    w = np.stack([bf16_operand(n, k, 10 * i + 2) for i in range(b)])
    rng = np.random.default_rng(b + m)
    bias = None
    if bias_kind == "shared":
        bias = rng.standard_normal(n).astype(np.float32)
    elif bias_kind == "per_batch":
        bias = rng.standard_normal((b, n)).astype(np.float32)
    out = aiter_amd.batched_gemm_bf16_CK(_bf16(a, cuda), _bf16(w, cuda),
                                         None if bias is None else torch.from_numpy(bias).to(cuda))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    for i in range(b):
        bi = None if bias is None else (bias if bias.ndim == 1 else bias[i])
        ok, msg = allclose_report(got[i], _ref(a[i], w[i], bi))
        assert ok, f"batch {i}: {msg}"


def test_batched_transposed_layout_and_f32(cuda):
    """X and Y in the reference test's [m, b, *] memory order (op_tests/test_batched_gemm_bf16.py:39-44)."""
    import aiter_amd

    b, m, n, k = 6, 48, 256, 512
    announce(f"batched bf16 mbn layout b={b} {m}x{n}x{k}")
    a = np.stack([bf16_operand(m, k, 100 + i) for i in range(b)])
    w = np.stack([bf16_operand(n, k, 200 + i) for i in range(b)])
    x = _bf16(np.ascontiguousarray(a.transpose(1, 0, 2)), cuda).transpose(0, 1)      # [b, m, k], strides (k, b*k, 1)
    y = torch.empty((m, b, n), dtype=torch.float32, device=cuda).transpose(0, 1)
    aiter_amd.batched_gemm_bf16(x, _bf16(w, cuda), y)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    for i in range(b):
        ok, msg = allclose_report(got[i], _ref(a[i], w[i], out_f32=True))
        assert ok, f"batch {i}: {msg}"


def test_batched_tune_kernel_ids(cuda):
    import aiter_amd
    from aiter_amd._lib import kernel_table

    b, m, n, k = 3, 100, 256, 512
    a = np.stack([bf16_operand(m, k, 300 + i) for i in range(b)])
    w = np.stack([bf16_operand(n, k, 400 + i) for i in range(b)])
    rows = [r for r in kernel_table() if r[2] == "a16w16" and not r[8] and not r[9] and (not r[3] or r[4] >= m)]
    assert rows
    for kid, name, *_ in rows:
        announce(f"batched bf16 tune {name}")
        out = torch.empty((b, m, n), dtype=torch.bfloat16, device=cuda)
        aiter_amd.batched_gemm_bf16_tune(_bf16(a, cuda), _bf16(w, cuda), out, kid, 0)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        for i in range(b):
            ok, msg = allclose_report(got[i], _ref(a[i], w[i]))
            assert ok, f"{name} batch {i}: {msg}"
