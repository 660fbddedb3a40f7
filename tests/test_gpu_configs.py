"""Oracle parity on every workload the benchmark configurations name, at their
full sizes (one MI355X):

* decode A4W4, M in {1, 8, 16, 32, 64}, N = 7168, K = 2048 through
  ``gemm_a4w4`` and the tuned table: every output element;
* prefill A4W4 M = 8192, N = 2048, K = 16384 (the long-K variant);
* MXFP8 x MXFP4 with the dynamic activation quant from bf16 N(0, 1),
  M in {256, 4096}, N = 7168, K = 16384;
* the transformer-linear sweep (N, K) x M in bf16 (``gemm_a16w16``) and A4W4
  with on-the-fly activation quant (``gemm_a4w4``).

Large shapes are generated on the GPU from seeded torch generators.  For
sampled rows the quantiser's bytes are compared bit-exactly with the oracle's
quantisation of the same bf16 values, and the GEMM outputs at sampled rows x
sampled columns are compared with the oracle's f32-accumulated dequantised
matmul (op_tests/test_gemm_a4w4.py:23-39) at rtol = atol = 1e-2, every
sampled element (op_tests/test_gemm_a4w4.py:88-123 uses the same rule).
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, mxfp4_operand, tile_samples

pytestmark = pytest.mark.gpu


def _dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def _u8(t: torch.Tensor) -> np.ndarray:
    return t.view(torch.uint8).cpu().numpy()


def _randn_bf16(rows, cols, seed, cuda):
    g = torch.Generator(device=cuda).manual_seed(seed)
    return torch.randn((rows, cols), generator=g, device=cuda, dtype=torch.float32).to(torch.bfloat16)


def _sample(n, count, seed):
    if n <= count:
        return np.arange(n)
    return np.sort(np.random.default_rng(seed).choice(n, count, replace=False))


def _take_rows(t: torch.Tensor, rows: np.ndarray) -> torch.Tensor:
    return t[torch.from_numpy(rows).to(t.device)]


def _bf16_rows_f32(x: torch.Tensor, rows: np.ndarray) -> np.ndarray:
    return _take_rows(x, rows).float().cpu().numpy()


def _check_fp4_rows(x_bf16, q, s_shuf, rows, what):
    """GPU quant of the sampled rows == oracle Even-mode quant of the same bf16 rows."""
    m, k = x_bf16.shape
    q_ref, s_ref = O.quant_mxfp4_triton_even(_bf16_rows_f32(x_bf16, rows))
    assert np.array_equal(_take_rows(q.view(torch.uint8), rows).cpu().numpy(), q_ref), f"{what}: packed e2m1 bytes differ from the oracle"
    s_all = O.unshuffle_scale(_u8(s_shuf), m, k // 32)
    assert np.array_equal(s_all[rows], s_ref), f"{what}: e8m0 scales differ from the oracle"
    return q_ref, s_ref


def _check_out(out, rows, cols, ref, what):
    got = out[torch.from_numpy(rows).to(out.device)][:, torch.from_numpy(cols).to(out.device)].float().cpu().numpy()
    ok, msg = allclose_report(got, ref)
    assert ok, f"{what}: {msg}"


# ------------------------------------------------------------------ decode A4W4
@pytest.mark.parametrize("m", [1, 8, 16, 32, 64])
@pytest.mark.parametrize("mode", ["triton", O.ROUND_UP])
def test_decode_a4w4_all_elements(cuda, m, mode):
    """A and B fp32 N(0,1), quantised per row (Even and RoundUp scale rules),
    B preshuffled, bf16 out; all M x 7168 elements against the oracle."""
    import aiter_amd

    n, k = 7168, 2048
    announce(f"decode gemm_a4w4 {m}x{n}x{k} mode={mode} kernel={aiter_amd.get_GEMM_config(m, n, k)}")
    a_q, a_s, a_ss = mxfp4_operand(m, k, 100 + m, mode)
    b_q, b_s, b_ss = mxfp4_operand(n, k, 7, mode)
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q, b_q, a_s, b_s))
    out = aiter_amd.gemm_a4w4(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda),
                              _dev(b_ss, cuda))
    torch.cuda.synchronize()
    assert out.shape == (m, n)
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, msg


# ------------------------------------------------------------------ long-K prefill
def _grid(m, n, n_rows, n_cols, seed):
    """Sampled rows x columns: for M or N beyond 128, one index in every band
    of 128 (so the grid touches every output tile of every instance) plus
    random ones."""
    rows = _sample(m, n_rows, seed)
    cols = _sample(n, n_cols, seed + 1)
    if m > 128:
        rows = np.union1d(rows, tile_samples(m, 128, seed + 2))
    if n > 128:
        cols = np.union1d(cols, tile_samples(n, 128, seed + 3))
    return rows, cols


def _a4w4_on_the_fly(m, n, k, seed, cuda, n_rows=16, n_cols=256, what=""):
    """bf16 N(0,1) activations and weights quantised on the GPU
    (get_triton_quant(per_1x32)), weights preshuffled, the tuned dispatch of
    gemm_a4w4 into a NaN-filled output; every output element finite (every
    tile written), quant bytes and sampled outputs checked."""
    import aiter_amd
    from aiter_amd.gemm_op_a4w4 import _gemm_a4w4_into

    quant = aiter_amd.get_triton_quant(aiter_amd.QuantType.per_1x32)
    x = _randn_bf16(m, k, seed, cuda)
    w = _randn_bf16(n, k, seed + 1, cuda)
    xq, xs = quant(x, shuffle=True)
    wq, ws = quant(w, shuffle=True)
    out = torch.full(((m + 31) // 32 * 32, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    _gemm_a4w4_into(xq, aiter_amd.shuffle_weight(wq), xs, ws, out, None, 1.0, 0.0, True)
    out = out[:m]
    assert bool(torch.isfinite(out).all()), f"{what}: output elements left unwritten (NaN)"
    rows, cols = _grid(m, n, n_rows, n_cols, seed + 2)
    a_q, a_s = _check_fp4_rows(x, xq, xs, rows, f"{what} activation quant")
    b_q, b_s = _check_fp4_rows(w, wq, ws, cols, f"{what} weight quant")
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q, b_q, a_s, b_s))
    _check_out(out, rows, cols, ref, f"{what} gemm_a4w4")


def test_prefill_a4w4_long_k(cuda):
    m, n, k = 8192, 2048, 16384
    announce(f"prefill gemm_a4w4 {m}x{n}x{k}")
    _a4w4_on_the_fly(m, n, k, 11, cuda, n_rows=24, n_cols=512, what=f"{m}x{n}x{k}")


# ------------------------------------------------------------------ MXFP8 x MXFP4
@pytest.mark.parametrize("m", [256, 4096])
def test_a8w4_dynamic_quant_full_size(cuda, m):
    """bf16 N(0,1) activation -> dynamic MXFP8 (Even) -> gemm with MXFP4
    preshuffled weights: e4m3 bytes and scales bit-exact on sampled rows,
    sampled outputs against the dequantised f32 matmul."""
    import aiter_amd

    n, k = 7168, 16384
    announce(f"a8w4 dynamic {m}x{n}x{k}")
    x = _randn_bf16(m, k, 21, cuda)
    w = _randn_bf16(n, k, 22, cuda)
    wq, ws = aiter_amd.dynamic_mxfp4_quant(w, shuffle=True)
    out = aiter_amd.gemm_a8w4_mxfp8_dynamic(x, aiter_amd.shuffle_weight(wq), ws)
    # the quant the dynamic entry runs, for its bytes
    aq, as_ = aiter_amd.dynamic_mxfp8_quant(x, shuffle=True)
    torch.cuda.synchronize()
    assert out.shape == (m, n)
    rows = _sample(m, 24, 23)
    cols = _sample(n, 512, 24)
    a_ref, sa_ref = O.quant_mxfp8(_bf16_rows_f32(x, rows), O.EVEN)
    assert np.array_equal(_take_rows(aq.view(torch.uint8), rows).cpu().numpy(), a_ref), "e4m3 bytes differ from the oracle"
    sa_all = O.unshuffle_scale(_u8(as_), m, k // 32)
    assert np.array_equal(sa_all[rows], sa_ref), "MXFP8 scales differ from the oracle"
    b_q, b_s = _check_fp4_rows(w, wq, ws, cols, "a8w4 weight quant")
    ref = O.bf16_bits_to_f32(O.gemm_a8w4_ref(a_ref, b_q, sa_ref, b_s))
    _check_out(out, rows, cols, ref, "gemm_a8w4_mxfp8_dynamic")


# ------------------------------------------------------------------ dispatch sweep
SWEEP_NK = [(4096, 4096), (14336, 4096), (4096, 14336), (28672, 8192), (8192, 28672)]
SWEEP_M = [1, 32, 256, 2048, 8192]
SWEEP = [(m, n, k) for (n, k) in SWEEP_NK for m in SWEEP_M]


@pytest.mark.parametrize("m,n,k", SWEEP)
def test_sweep_a4w4_on_the_fly_quant(cuda, m, n, k):
    import aiter_amd

    announce(f"sweep a4w4 {m}x{n}x{k} kernel={aiter_amd.get_GEMM_config(m, n, k)}")
    _a4w4_on_the_fly(m, n, k, 1000 + m + n + k, cuda, what=f"a4w4 {m}x{n}x{k}")


@pytest.mark.parametrize("m,n,k", SWEEP)
def test_sweep_bf16(cuda, m, n, k):
    """gemm_a16w16 (row-major B, the reference rows' layout) through the tuned
    table; sampled outputs against the f32 matmul of the bf16 operands."""
    import aiter_amd

    from aiter_amd import tuned_gemm

    announce(f"sweep bf16 {m}x{n}x{k}")
    seed = 2000 + m + n + k
    x = _randn_bf16(m, k, seed, cuda)
    w = _randn_bf16(n, k, seed + 1, cuda)
    out = aiter_amd.gemm_a16w16(x, w)
    torch.cuda.synchronize()
    assert out.shape == (m, n) and out.dtype == torch.bfloat16
    # the same dispatch into a NaN-filled output: every tile written, same bits
    cfg = aiter_amd.get_GEMM_A16W16_config(m, n, k, False, str(x.dtype), str(x.dtype), False, False)
    poisoned = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    tuned_gemm._run(x, w, None, torch.bfloat16, False, cfg, out=poisoned)
    assert bool(torch.isfinite(poisoned).all()), "output elements left unwritten (NaN)"
    rows, cols = _grid(m, n, 16, 256, seed + 2)
    a_bits = _take_rows(x, rows).view(torch.int16).cpu().numpy().view(np.uint16)
    b_bits = _take_rows(w, cols).view(torch.int16).cpu().numpy().view(np.uint16)
    ref = O.bf16_bits_to_f32(O.gemm_a16w16_ref(a_bits, b_bits))
    _check_out(out, rows, cols, ref, "gemm_a16w16")
    _check_out(poisoned, rows, cols, ref, "gemm_a16w16 into a NaN-filled output")
