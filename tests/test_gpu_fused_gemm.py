"""fused_gemm_afp4wfp4_{mul_add, preshuffle_add_mul, split_cat,
preshuffle_split_cat, a16w16} against the oracle
(op_tests/triton_tests/gemm/fused/test_fused_gemm_afp4wfp4_{mul_add,split_cat,a16w16}.py
check the same compositions against torch): the A4W4 product is the oracle's
f32 dequantised matmul, the fused operation its restatement in
oracle/mx_oracle.py (``mul_add_ref``, ``split_cat_ref``), the tolerance the
GEMM one (rtol = atol = 1e-2 on every element)."""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, bf16_operand, mxfp4_operand, randn, to_bf16_f32

pytestmark = pytest.mark.gpu


def _dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def _case(m, n, k, seed):
    a_q, a_s, a_ss = mxfp4_operand(m, k, seed, "triton")
    b_q, b_s, b_ss = mxfp4_operand(n, k, seed + 1, "triton")
    return a_q, a_s, a_ss, b_q, b_s, b_ss, O.gemm_a4w4_f32(a_q, b_q, a_s, b_s)


def _operands(cuda, preshuffled, m, n, k, a_q, a_s, a_ss, b_q, b_s, b_ss):
    """(x, w, x_scales, w_scales) in the layout the plain / preshuffled op
    takes: the preshuffled weight in the Triton view [N/16, K*8] and its
    scales as [rows/32, K]; x scales shuffled only for M >= 32."""
    x = _dev(a_q, cuda)
    if not preshuffled:
        return x, _dev(b_q, cuda), _dev(a_s, cuda), _dev(b_s, cuda)
    w = _dev(O.shuffle_weight(b_q), cuda).view(n // 16, k * 8)
    ws = _dev(b_ss, cuda).view(b_ss.shape[0] // 32, k)
    xs = _dev(a_ss, cuda).view(a_ss.shape[0] // 32, k) if m >= 32 else _dev(a_s, cuda)
    return x, w, xs, ws


def _mul_add_operand(kind, m, n, seed, cuda):
    """(value passed to the op, f32 value for the oracle)."""
    if kind == "float":
        v = float(np.random.default_rng(seed).standard_normal() * 3)
        return v, np.float32(v)
    if kind == "int":
        v = int(np.random.default_rng(seed).integers(-5, 6))
        return v, np.float32(v)
    if kind == "one":   # one-element device tensor, read in the epilogue
        v = np.float32(np.random.default_rng(seed).standard_normal())
        return torch.tensor([v], device=cuda), v
    if kind == "f32":
        v = randn((m, n), seed)
        return _dev(v, cuda), v
    v = to_bf16_f32(randn((m, n), seed))   # bf16 tensor
    return _dev(v, cuda).to(torch.bfloat16), v


@pytest.mark.parametrize("fuse_type", [0, 1])
@pytest.mark.parametrize("a_kind,b_kind", [("float", "int"), ("f32", "float"), ("one", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("preshuffled", [False, True])
@pytest.mark.parametrize("m", [1, 31, 32, 200])
def test_fused_gemm_mul_add(cuda, m, preshuffled, a_kind, b_kind, fuse_type):
    import aiter_amd

    n, k = 768, 512
    announce(f"fused mul_add m={m} pre={preshuffled} a={a_kind} b={b_kind} fuse={fuse_type}")
    a_q, a_s, a_ss, b_q, b_s, b_ss, c = _case(m, n, k, 3 + m)
    x, w, xs, ws = _operands(cuda, preshuffled, m, n, k, a_q, a_s, a_ss, b_q, b_s, b_ss)
    a, a_ref = _mul_add_operand(a_kind, m, n, 11, cuda)
    b, b_ref = _mul_add_operand(b_kind, m, n, 12, cuda)
    op = aiter_amd.fused_gemm_afp4wfp4_preshuffle_add_mul if preshuffled else aiter_amd.fused_gemm_afp4wfp4_mul_add
    out = op(x, w, xs, ws, a, b, torch.bfloat16, fuse_type=fuse_type)
    torch.cuda.synchronize()
    assert out.shape == (m, n) and out.dtype == torch.bfloat16
    ref = O.bf16_bits_to_f32(O.mul_add_ref(c, a_ref, b_ref, fuse_type))
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, msg


def test_fused_gemm_mul_add_into_given_output_and_broadcast_rows(cuda):
    """A preallocated ``y`` is written in place; a [1, N] operand broadcasts
    over the rows."""
    import aiter_amd

    m, n, k = 64, 512, 512
    a_q, a_s, a_ss, b_q, b_s, b_ss, c = _case(m, n, k, 41)
    x, w, xs, ws = _operands(cuda, False, m, n, k, a_q, a_s, a_ss, b_q, b_s, b_ss)
    row = randn((1, n), 42)
    y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    out = aiter_amd.fused_gemm_afp4wfp4_mul_add(x, w, xs, ws, _dev(row, cuda), 0.25, torch.bfloat16, y=y)
    torch.cuda.synchronize()
    assert out.data_ptr() == y.data_ptr()
    ok, msg = allclose_report(y.float().cpu().numpy(), O.bf16_bits_to_f32(O.mul_add_ref(c, row, 0.25, 0)))
    assert ok, msg


@pytest.mark.parametrize("preshuffled", [False, True])
@pytest.mark.parametrize("m,d,s1,s2,s3", [(1, 4, 64, 64, 32), (48, 2, 128, 128, 64), (300, 8, 16, 48, 8)])
def test_fused_gemm_split_cat(cuda, m, d, s1, s2, s3, preshuffled):
    import aiter_amd

    n, k = d * (s1 + s2), 512
    announce(f"fused split_cat m={m} D={d} S=({s1},{s2},{s3}) pre={preshuffled}")
    a_q, a_s, a_ss, b_q, b_s, b_ss, c = _case(m, n, k, 7 + m)
    x, w, xs, ws = _operands(cuda, preshuffled, m, n, k, a_q, a_s, a_ss, b_q, b_s, b_ss)
    y = to_bf16_f32(randn((m, d, s3), 13))
    op = aiter_amd.fused_gemm_afp4wfp4_preshuffle_split_cat if preshuffled else aiter_amd.fused_gemm_afp4wfp4_split_cat
    c1, c2 = op(x, w, _dev(y, cuda).to(torch.bfloat16), xs, ws, s1, s2, torch.bfloat16)
    torch.cuda.synchronize()
    assert c1.shape == (m, d, s1 + s3) and c2.shape == (m, d, s2)
    r1, r2 = O.split_cat_ref(O.bf16_bits_to_f32(O.f32_to_bf16_bits(c)), y, s1, s2)
    g1, g2 = c1.float().cpu().numpy(), c2.float().cpu().numpy()
    assert np.array_equal(g1[:, :, s1:], y), "y must be copied unchanged"
    for got, ref, what in ((g1[:, :, :s1], r1[:, :, :s1], "c1"), (g2, r2, "c2")):
        ok, msg = allclose_report(got, ref)
        assert ok, f"{what}: {msg}"


def _force_a4w4_row(monkeypatch, tmp_path, m, n, k, name):
    """A tuned A4W4 table holding one row, (m, n, k) -> kernel `name`."""
    import pandas as pd

    from aiter_amd import config, gemm_op_a4w4

    row = {"gfx": "gfx950", "cu_num": 256, "M": m, "N": n, "K": k, "kernelId": 0, "splitK": 0, "us": 1.0,
           "kernelName": name, "tflops": 1.0, "bw": 1.0, "errRatio": 0.0}
    p = tmp_path / "a4w4_one_row.csv"
    pd.DataFrame([row]).to_csv(p, index=False)
    monkeypatch.setenv("AITER_CONFIG_GEMM_A4W4", str(p))
    monkeypatch.setenv("GPU_ARCHS", "gfx950")
    monkeypatch.setenv("CU_NUM", "256")
    for f in (config.get_gfx, config.get_cu_num, gemm_op_a4w4._a4w4_table, gemm_op_a4w4.get_GEMM_config):
        f.cache_clear()


def _clear_tables():
    from aiter_amd import config, gemm_op_a4w4

    for f in (config.get_gfx, config.get_cu_num, gemm_op_a4w4._a4w4_table, gemm_op_a4w4.get_GEMM_config):
        f.cache_clear()


# the epilogue paths of the long-K decode shapes the Triton ops serve:
# * skinny split-K (heuristic at M = 16, N = 2048: 128 column blocks, half the
#   CUs) -> the fused operation in splitk_finish_kernel;
# * a split tile named by the tuned table, long K -> in splitk_reduce_kernel;
# * the persistent 256x256 tile named by the tuned table -> the host runs its
#   one-tile twin, which carries the operation.
EPI_PATHS = [
    ("skinny_splitk", 16, 2048, 8192, None),
    ("tile_splitk", 64, 1024, 8192, "a4w4_tile_64x128_splitk"),
    ("persistent_twin", 512, 2048, 1024, "a4w4_tile_256x256_persist"),
]


@pytest.mark.parametrize("path,m,n,k,name", EPI_PATHS)
@pytest.mark.parametrize("preshuffled", [True, False])
def test_fused_mul_add_epilogue_paths(cuda, monkeypatch, tmp_path, path, m, n, k, name, preshuffled):
    import aiter_amd

    if name is not None:
        if not preshuffled:
            pytest.skip("tuned rows name preshuffled-B kernels only; the plain form runs the heuristic")
        _force_a4w4_row(monkeypatch, tmp_path, m, n, k, name)
    announce(f"fused mul_add path={path} {m}x{n}x{k} pre={preshuffled}")
    try:
        a_q, a_s, a_ss, b_q, b_s, b_ss, c = _case(m, n, k, 61)
        x, w, xs, ws = _operands(cuda, preshuffled, m, n, k, a_q, a_s, a_ss, b_q, b_s, b_ss)
        a, a_ref = _mul_add_operand("bf16", m, n, 62, cuda)
        b, b_ref = _mul_add_operand("f32", m, n, 63, cuda)
        op = aiter_amd.fused_gemm_afp4wfp4_preshuffle_add_mul if preshuffled else aiter_amd.fused_gemm_afp4wfp4_mul_add
        y = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda)
        out = op(x, w, xs, ws, a, b, torch.bfloat16, y=y, fuse_type=0)
        torch.cuda.synchronize()
    finally:
        _clear_tables()
    ref = O.bf16_bits_to_f32(O.mul_add_ref(c, a_ref, b_ref, 0))
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, msg


@pytest.mark.parametrize("path,m,n,k,name", EPI_PATHS)
def test_fused_split_cat_epilogue_paths(cuda, monkeypatch, tmp_path, path, m, n, k, name):
    import aiter_amd

    d, s2, s3 = 4, 128, 32
    s1 = n // d - s2
    if name is not None:
        _force_a4w4_row(monkeypatch, tmp_path, m, n, k, name)
    announce(f"fused split_cat path={path} {m}x{n}x{k}")
    try:
        a_q, a_s, a_ss, b_q, b_s, b_ss, c = _case(m, n, k, 71)
        x, w, xs, ws = _operands(cuda, True, m, n, k, a_q, a_s, a_ss, b_q, b_s, b_ss)
        y = to_bf16_f32(randn((m, d, s3), 72))
        c1, c2 = aiter_amd.fused_gemm_afp4wfp4_preshuffle_split_cat(x, w, _dev(y, cuda).to(torch.bfloat16), xs, ws,
                                                                     s1, s2, torch.bfloat16)
        torch.cuda.synchronize()
    finally:
        _clear_tables()
    r1, r2 = O.split_cat_ref(O.bf16_bits_to_f32(O.f32_to_bf16_bits(c)), y, s1, s2)
    g1, g2 = c1.float().cpu().numpy(), c2.float().cpu().numpy()
    assert np.array_equal(g1[:, :, s1:], y), "y must be copied unchanged"
    for got, ref, what in ((g1[:, :, :s1], r1[:, :, :s1], "c1"), (g2, r2, "c2")):
        ok, msg = allclose_report(got, ref)
        assert ok, f"{what}: {msg}"


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("preshuffled", [True, False])
@pytest.mark.parametrize("m,n4,n16", [(1, 1024, 256), (16, 1024, 256), (17, 1040, 272), (32, 1024, 256),
                                      (33, 1040, 272), (64, 1024, 256), (300, 1024, 256)])
def test_fused_gemm_afp4wfp4_a16w16(cuda, m, n4, n16, preshuffled, bias):
    """M <= 32 (K short enough that neither GEMM splits): both GEMMs in one
    grid (skinny_pair_kernel; ragged column block counts at M = 17); larger
    M: two launches."""
    import aiter_amd

    k = 512
    announce(f"fused a16w16 m={m} pre={preshuffled} bias={bias}")
    a_q, a_s, a_ss, b_q, b_s, b_ss, c = _case(m, n4, k, 21 + m)
    x, w, xs, ws = _operands(cuda, preshuffled, m, n4, k, a_q, a_s, a_ss, b_q, b_s, b_ss)
    xb = bf16_operand(m, k, 23)
    wb = bf16_operand(n16, k, 24)
    b4 = randn((n4,), 25) if bias else None
    b16 = randn((n16,), 26) if bias else None
    y4, y16 = aiter_amd.fused_gemm_afp4wfp4_a16w16(
        x, w, xs, ws, _dev(xb.view(np.int16), cuda).view(torch.bfloat16),
        _dev(wb.view(np.int16), cuda).view(torch.bfloat16), is_fp4_preshuffled=preshuffled,
        bias_fp4=None if b4 is None else _dev(b4, cuda).to(torch.bfloat16),
        bias_bf16=None if b16 is None else _dev(b16, cuda))
    torch.cuda.synchronize()
    assert y4.shape == (m, n4) and y16.shape == (m, n16)
    ref4 = c + (to_bf16_f32(b4) if bias else 0.0)
    ok, msg = allclose_report(y4.float().cpu().numpy(), O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref4)))
    assert ok, f"fp4 part: {msg}"
    ref16 = O.bf16_bits_to_f32(O.gemm_a16w16_ref(xb, wb, b16))
    ok, msg = allclose_report(y16.float().cpu().numpy(), ref16)
    assert ok, f"bf16 part: {msg}"


def test_fused_gemm_rejections(cuda):
    import aiter_amd

    m, n, k = 8, 256, 512
    a_q, a_s, a_ss, b_q, b_s, b_ss, _ = _case(m, n, k, 1)
    x, w, xs, ws = _operands(cuda, False, m, n, k, a_q, a_s, a_ss, b_q, b_s, b_ss)
    with pytest.raises(NotImplementedError):
        aiter_amd.fused_gemm_afp4wfp4_mul_add(x, w, xs, ws, 1.0, 0.0, torch.float16)
    y = torch.zeros((m, 4, 8), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(RuntimeError, match="multiples of 8"):
        aiter_amd.fused_gemm_afp4wfp4_split_cat(x, w, y, xs, ws, 60, 4)
    with pytest.raises(ValueError):
        aiter_amd.fused_gemm_afp4wfp4_split_cat(x, w, y, xs, ws, 16, 16)
