"""Pins of the CPU oracle (oracle/mx_oracle.py) against checks that do not
restate its own formulas: known answers from the reference's tests, brute-force
nearest-grid searches, a library routine (torch's float8_e4m3fn cast) and
mathematical properties of each e8m0 rounding mode."""
import itertools
import math

import numpy as np
import pytest
import torch

from oracle import mx_oracle as O

GRID = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


# ----------------------------------------------------------------------------- e2m1
def test_e2m1_decode_closed_form():
    """OCP e2m1: e=0 -> m*0.5, else 2**(e-1)*(1+m/2); sign bit 3."""
    for c in range(16):
        s, e, m = c >> 3, (c >> 1) & 3, c & 1
        v = m * 0.5 if e == 0 else 2.0 ** (e - 1) * (1 + m / 2)
        assert O.e2m1_decode(np.array([c]))[0] == (-v if s else v)


def test_fp4_grid_known_answer():
    """FP4 magnitudes of op_tests/opus/device/test_opus_device.py:843-853."""
    assert list(O.E2M1_VALUES[:8]) == GRID


def _brute_e2m1(x: float) -> int:
    """nearest magnitude on the grid, ties to the even code (mantissa bit 0),
    saturating at 6; sign kept (also for zero)."""
    a = abs(x)
    best = None
    for code, g in enumerate(GRID):
        d = abs(a - g)
        if best is None or d < best[0] - 1e-12 or (abs(d - best[0]) <= 1e-12 and code % 2 == 0):
            best = (d, code)
    code = best[1]
    sign = 8 if math.copysign(1.0, x) < 0 else 0
    return sign | code


def test_e2m1_encode_rne_brute_force():
    vals = [k / 64.0 for k in range(-8 * 64, 8 * 64 + 1)]
    mids = [(a + b) / 2 for a, b in zip(GRID, GRID[1:])]
    vals += mids + [-m for m in mids] + [m + 1e-6 for m in mids] + [m - 1e-6 for m in mids]
    vals += [7.0, 100.0, -1e4, 1e-30, -1e-30, -0.0, 0.26, 0.24]
    x = np.array(vals, dtype=np.float32)
    got = O.e2m1_encode_rne(x)
    want = np.array([_brute_e2m1(float(v)) for v in x], dtype=np.uint8)
    np.testing.assert_array_equal(got, want)


def test_e2m1_threshold_form():
    """Threshold restatement of csrc/kernels/quant_mxfp4.cu:38-55 (independent
    of the bit-trick encoder)."""
    rs = np.random.default_rng(0)
    x = (rs.standard_normal(20000) * 3).astype(np.float32)
    x = np.concatenate([x, np.array([5.0, 3.5, 2.5, 1.75, 1.25, 0.75, 0.25], np.float32)])

    def thr(v):
        a = abs(v)
        if a > 5.0: mag = 7
        elif a >= 3.5: mag = 6
        elif a > 2.5: mag = 5
        elif a >= 1.75: mag = 4
        elif a > 1.25: mag = 3
        elif a >= 0.75: mag = 2
        elif a > 0.25: mag = 1
        else: mag = 0
        return (8 if v < 0 else 0) | mag

    want = np.array([thr(float(v)) for v in x], dtype=np.uint8)
    got = O.e2m1_encode_rne(x)
    nz = x != 0  # the threshold form drops the sign of -0.0
    np.testing.assert_array_equal(got[nz], want[nz])


def test_pack_known_answer():
    """elem i -> byte i/2, nibble i%2 (op_tests/opus/test_opus_fp4_device.cu:88)."""
    assert list(O.pack_fp4(np.arange(8, dtype=np.uint8))) == [0x10, 0x32, 0x54, 0x76]
    codes = np.random.default_rng(1).integers(0, 16, (5, 64), dtype=np.uint8)
    np.testing.assert_array_equal(O.unpack_fp4(O.pack_fp4(codes)), codes)


# ----------------------------------------------------------------------------- e4m3
def test_e4m3_encode_matches_torch_cast():
    rs = np.random.default_rng(2)
    x = np.concatenate([
        (rs.standard_normal(50000) * 50).astype(np.float32),
        (rs.standard_normal(5000) * 1e-3).astype(np.float32),
        np.array([0.0, -0.0, 448.0, -448.0, 2 ** -9, 2 ** -10, 1.5 * 2 ** -9, 2 ** -6, 0.5 * 2 ** -6], np.float32),
    ])
    x = np.clip(x, -448, 448)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(O.e4m3_encode_rne(x), want)


def test_e4m3_decode_roundtrip_all_codes():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    v = O.e4m3_decode(codes)
    want = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    np.testing.assert_array_equal(v, want)
    back = O.e4m3_encode_rne(v)
    np.testing.assert_array_equal(O.e4m3_decode(back), v)


# ----------------------------------------------------------------------------- e8m0
def _amax_samples():
    rs = np.random.default_rng(3)
    a = np.abs(rs.standard_normal(20000)).astype(np.float32) * np.float32(2.0) ** rs.integers(-40, 40, 20000)
    special = [6.0 * 2.0 ** k for k in range(-20, 20)] + [4.0 * 2.0 ** k for k in range(-20, 20)]
    special += [1.75 * 2.0 ** k for k in range(-10, 10)] + [1.7499 * 2.0 ** k for k in range(-10, 10)]
    return np.concatenate([a.astype(np.float32), np.array(special, np.float32)])


def test_e8m0_round_up_property():
    """RoundUp: smallest power of two >= f32(amax * (1/6))."""
    a = _amax_samples()
    x = (a * np.float32(1.0) / np.float32(6.0)).astype(np.float64)
    x = (a * (np.float32(1.0) / np.float32(6.0))).astype(np.float32).astype(np.float64)
    s = np.exp2(O.e8m0_scale_hip(a, O.ROUND_UP).astype(np.float64) - 127)
    assert np.all(s >= x) and np.all(s / 2 < x)


def test_e8m0_round_down_and_ceil_property():
    a = _amax_samples().astype(np.float64)
    x = a / 4.0
    sd = np.exp2(O.e8m0_scale_hip(a.astype(np.float32), O.ROUND_DOWN).astype(np.float64) - 127)
    assert np.all(sd <= x) and np.all(2 * sd > x)
    sc = np.exp2(O.e8m0_scale_hip(a.astype(np.float32), O.CEIL).astype(np.float64) - 127)
    assert np.all(sc >= x) and np.all(sc / 2 < x)


def test_e8m0_even_property_and_log2_form():
    """Even (Quark): scale = 2**(e-2) when the significand of amax is < 1.75,
    else 2**(e-1) (round the significand to 1 bit of mantissa, half-up);
    the Triton floor(log2) formulation gives the same byte."""
    a = _amax_samples()
    m, e = np.frexp(a.astype(np.float64))  # a = m * 2**e, m in [0.5, 1)
    sig = 2 * m                             # [1, 2)
    ex = e - 1
    want = np.where(sig < 1.75, ex - 2, ex - 1) + 127
    got = O.e8m0_scale_hip(a, O.EVEN)
    np.testing.assert_array_equal(got.astype(np.int64), want)
    lg, _ = O.e8m0_scale_log2(a, "fp4")
    np.testing.assert_array_equal(lg, got)


def test_e8m0_zero_block():
    """All-zero block: 0x00 for the quant_mxfp4 modes and the Triton quant
    (log2(0) clamps to -127); the production RoundUp kernel starts its running
    max at 1e-10, giving ceil_pow2(1e-10/6) = 2**-35 -> 0x5C (read from
    csrc/kernels/quant_kernels.cu:89; not pinned by a reference test)."""
    z = np.zeros((1, 32), np.float32)
    for mode in (O.ROUND_DOWN, O.EVEN, O.CEIL, O.ROUND_UP):
        assert O.quant_mxfp4(z, mode)[1][0, 0] == 0
    assert O.quant_mxfp4(z, O.ROUND_UP, amax_floor=1e-10)[1][0, 0] == 127 - 35
    assert O.quant_mxfp4_triton_even(z)[1][0, 0] == 0


# ----------------------------------------------------------------------------- quantisers
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_quant_mxfp4_is_nearest_grid_point(mode):
    """Every element is the RNE grid point of x / scale (brute force), and the
    scale byte is the mode's e8m0 of the block amax."""
    rs = np.random.default_rng(4)
    x = (rs.standard_normal((8, 256)) * 2.0 ** rs.integers(-6, 6, (8, 1))).astype(np.float32)
    q, s = O.quant_mxfp4(x, mode)
    codes = O.unpack_fp4(q).reshape(8, 8, 32)
    g = x.reshape(8, 8, 32)
    for r, b in itertools.product(range(8), range(8)):
        amax = np.abs(g[r, b]).max()
        assert s[r, b] == O.e8m0_scale_hip(np.array([amax], np.float32), mode)[0]
        inv = 2.0 ** (127 - int(s[r, b]))
        for k in range(32):
            assert codes[r, b, k] == _brute_e2m1(float(np.float32(g[r, b, k] * np.float32(inv))))


def test_quant_edge_values():
    """op_tests/test_quant_mxfp4.py:352-375: zeros -> packed all zero; -3.0
    constant -> each element exactly representable."""
    for mode in (0, 1, 2, 3):
        q, _ = O.quant_mxfp4(np.zeros((32, 64), np.float32), mode)
        assert q.sum() == 0
        q, s = O.quant_mxfp4(np.full((32, 64), -3.0, np.float32), mode)
        dq = O.dequant_mxfp4(q, s)
        np.testing.assert_array_equal(dq, np.full((32, 64), -3.0, np.float32))
        q, _ = O.quant_mxfp4(np.full((32, 64), 1e4, np.float32), mode)
        assert q.max() > 0


def test_round_up_never_saturates_and_error_bound():
    """RoundUp keeps |x|/scale <= 6, so the dequantised error is at most half
    the local grid step (1 ulp of e2m1 = 2**(e-1) at magnitude >= 1) times the scale."""
    x = np.random.default_rng(5).standard_normal((64, 512)).astype(np.float32)
    q, s = O.quant_mxfp4(x, O.ROUND_UP)
    dq = O.dequant_mxfp4(q, s)
    sc = np.repeat(O.e8m0_to_f32(s), 32, axis=1).astype(np.float64)
    err = np.abs(dq - x) / sc
    assert np.all(np.abs(x) / sc <= 6.0 + 1e-6)
    assert np.all(err <= 1.0 + 1e-6)  # largest half-step of the grid (between 4 and 6)


def test_mxfp8_even_matches_torch_cast_of_scaled_values():
    """op_tests/triton_tests/quant/test_quant_mxfp8.py:24-49 computes the
    elements with torch's .to(float8_e4m3fn); the oracle must agree bit-exactly."""
    x = (np.random.default_rng(6).standard_normal((16, 256)) * 4).astype(np.float32)
    q, s = O.quant_mxfp8(x, O.EVEN)
    m, e = np.frexp(np.abs(x.reshape(16, 8, 32)).max(-1).astype(np.float64))
    want_s = np.where(2 * m < 1.75, e - 1 - 8, e - 1 - 7) + 127
    np.testing.assert_array_equal(s.astype(np.int64), want_s)
    qs = np.exp2(127 - s.astype(np.float64)).astype(np.float32)
    scaled = (x.reshape(16, 8, 32) * qs[..., None]).reshape(16, 256)
    want = torch.from_numpy(scaled).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(q, want)


# ----------------------------------------------------------------------------- layouts
def test_shuffle_weight_index_formula_and_inverse():
    """Element (n, byte kb) of B sits at
    n16*16*Kb + (kb//32)*512 + ((kb%32)//16)*256 + (n%16)*16 + kb%16."""
    N, Kb = 48, 96
    w = np.random.default_rng(7).integers(0, 256, (N, Kb), dtype=np.uint8)
    ws = O.shuffle_weight(w).reshape(-1)
    n, kb = np.meshgrid(np.arange(N), np.arange(Kb), indexing="ij")
    idx = (n // 16) * 16 * Kb + (kb // 32) * 512 + ((kb % 32) // 16) * 256 + (n % 16) * 16 + kb % 16
    np.testing.assert_array_equal(ws[idx], w)
    np.testing.assert_array_equal(O.unshuffle_weight(O.shuffle_weight(w)), w)


def test_shuffle_weight_is_mfma_operand_order():
    """For every 64-byte K window of a 16-row block, the 1 KiB at
    block + window*1024 holds, at lane*16, row lane%16 and bytes
    [16*(lane//16), +16) of the window: the 16x16x128 e2m1 operand."""
    N, Kb = 32, 128
    w = np.random.default_rng(8).integers(0, 256, (N, Kb), dtype=np.uint8)
    ws = O.shuffle_weight(w).reshape(-1)
    for blk in range(N // 16):
        for win in range(Kb // 64):
            frag = ws[blk * 16 * Kb + win * 1024: blk * 16 * Kb + (win + 1) * 1024].reshape(64, 16)
            for lane in range(64):
                np.testing.assert_array_equal(
                    frag[lane], w[blk * 16 + lane % 16, win * 64 + 16 * (lane // 16): win * 64 + 16 * (lane // 16) + 16])


def test_shuffle_weight_bf16_layout():
    """2-byte elements: 8-element (16-byte) inner chunks (aiter/ops/shuffle.py:192-204)."""
    N, K = 32, 64
    w = np.random.default_rng(9).integers(0, 2 ** 16, (N, K), dtype=np.uint16)
    ws = O.shuffle_weight(w).reshape(-1)
    n, k = np.meshgrid(np.arange(N), np.arange(K), indexing="ij")
    idx = (n // 16) * 16 * K + (k // 32) * 512 + ((k % 32) // 8) * 128 + (n % 16) * 8 + k % 8
    np.testing.assert_array_equal(ws[idx], w)


@pytest.mark.parametrize("rows,cols", [(1, 1), (33, 5), (256, 64), (300, 130)])
def test_shuffle_scale_three_formulations(rows, cols):
    s = np.random.default_rng(10).integers(0, 256, (rows, cols), dtype=np.uint8)
    ss = O.shuffle_scale(s)
    assert ss.shape == ((rows + 255) // 256 * 256, (cols + 7) // 8 * 8)
    x, y = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    i1 = O.mx_scale_shuffle_idx(ss.shape[1], x, y)
    i2 = O.triton_scale_store_offset(ss.shape[1], x, y)
    np.testing.assert_array_equal(i1, i2)
    np.testing.assert_array_equal(ss.reshape(-1)[i1], s)
    np.testing.assert_array_equal(O.unshuffle_scale(ss, rows, cols), s)


# ----------------------------------------------------------------------------- GEMM refs
def test_gemm_refs_vs_float64_brute_force():
    rs = np.random.default_rng(11)
    m, n, k = 3, 5, 64
    a = rs.standard_normal((m, k)).astype(np.float32)
    b = rs.standard_normal((n, k)).astype(np.float32)
    aq, as_ = O.quant_mxfp4(a, O.EVEN)
    bq, bs = O.quant_mxfp4(b, O.EVEN)
    got = O.bf16_bits_to_f32(O.gemm_a4w4_ref(aq, bq, as_, bs))
    ad = [[float(O.E2M1_VALUES[c]) * 2.0 ** (int(as_[i, j // 32]) - 127)
           for j, c in enumerate(O.unpack_fp4(aq)[i])] for i in range(m)]
    bd = [[float(O.E2M1_VALUES[c]) * 2.0 ** (int(bs[i, j // 32]) - 127)
           for j, c in enumerate(O.unpack_fp4(bq)[i])] for i in range(n)]
    want = np.array([[sum(x * y for x, y in zip(ad[i], bd[j])) for j in range(n)] for i in range(m)])
    np.testing.assert_allclose(got, want, rtol=8e-3, atol=1e-6)
    aq8, as8 = O.quant_mxfp8(a, O.EVEN)
    got8 = O.bf16_bits_to_f32(O.gemm_a8w4_ref(aq8, bq, as8, bs))
    a8 = O.e4m3_decode(aq8).astype(np.float64) * np.repeat(np.exp2(as8.astype(np.float64) - 127), 32, 1)
    np.testing.assert_allclose(got8, a8 @ np.array(bd).T, rtol=8e-3, atol=1e-6)


def test_bf16_rounding_matches_torch():
    x = np.random.default_rng(12).standard_normal(100000).astype(np.float32) * 1e3
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(O.f32_to_bf16_bits(x), want)


# ----------------------------------------------------------------------------- dispatch
def test_get_padded_m_known_answers():
    """csrc/py_itfs_cu/gemm_common.cu:12-41 by hand."""
    assert [O.get_padded_m(m, 4096, 4096, 0) for m in (1, 16, 17, 256, 257, 1024, 1025, 4097)] == \
        [16, 16, 32, 256, 288, 1024, 1088, 4224]
    assert [O.get_padded_m(m, 4096, 4096, 1) for m in (1, 3, 33, 1000, 9000)] == [1, 4, 64, 1024, 16384]
    assert O.get_padded_m(9000, 8192, 1024, 1) == 8192


def test_rms_norm_f32_vs_torch():
    """rms_norm_f32 against torch's own RMSNorm (a library routine), f32."""
    import torch

    rs = np.random.default_rng(11)
    x = rs.standard_normal((5, 1536)).astype(np.float32) * 3
    res = rs.standard_normal((5, 1536)).astype(np.float32)
    w = rs.standard_normal(1536).astype(np.float32)
    y, xr = O.rms_norm_f32(x, w, 1e-6, res)
    want = torch.nn.functional.rms_norm(torch.from_numpy(x + res), (1536,), torch.from_numpy(w), eps=1e-6)
    np.testing.assert_allclose(y, want.numpy(), rtol=2e-6, atol=2e-6)
    np.testing.assert_array_equal(xr, (x + res).astype(np.float32))


def test_fused_rms_quant_exact_case():
    """Rows of constant magnitude 2**e with eps = 0: the norm factor is
    exactly 2**-e, the normalised row is exactly +-weight, so the fused
    quant must equal the plain quant of +-weight bit for bit."""
    rs = np.random.default_rng(12)
    k = 1024
    e = rs.integers(-20, 20, 6)
    signs = rs.choice([-1.0, 1.0], (6, k)).astype(np.float32)
    x = signs * np.exp2(e.astype(np.float32))[:, None]
    w = (rs.standard_normal(k) * 2).astype(np.float32)
    for fp8 in (False, True):
        q, s, y, _ = O.fused_rms_mx_quant_ref(x, w, 0.0, fp8)
        np.testing.assert_array_equal(y, signs * w)
        q2, s2 = O.quant_mxfp8(signs * w, O.EVEN) if fp8 else O.quant_mxfp4_triton_even(signs * w)
        np.testing.assert_array_equal(q, q2)
        np.testing.assert_array_equal(s, s2)


# ---------------------------------------------------------------- low-precision outputs
def test_pack_mxfp8_out_scale_known_answer():
    m, n = 128, 256
    rm = np.arange(m * (n // 128), dtype=np.int64).reshape(m, n // 128).astype(np.uint8)
    packed = O.pack_mxfp8_out_scale(rm)
    # byte (row r, block b) at ((r/64 * N/128 + b) * 16 + r%16) * 4 + (r%64)/16
    for r in (0, 1, 15, 16, 17, 63, 64, 100, 127):
        for b in (0, 1):
            assert packed[((r // 64 * 2 + b) * 16 + r % 16) * 4 + (r % 64) // 16] == rm[r, b]
    np.testing.assert_array_equal(O.unpack_mxfp8_out_scale(packed, m, n), rm)


def test_quant_mxfp8_block_n_properties():
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((64, 384)) * np.exp2(rng.integers(-6, 7, (64, 1)))).astype(np.float32)
    q, s = O.quant_mxfp8_block_n(x)
    v = O.e4m3_decode(q).reshape(64, 3, 128)
    scale = np.exp2(s.astype(np.float64) - 127)[..., None]
    assert np.abs(v).max() <= 448
    xb = x.reshape(64, 3, 128) / scale
    # RNE: each value within half an e4m3 step (3 mantissa bits) of the scaled input
    step = np.exp2(np.floor(np.log2(np.maximum(np.abs(xb), 2.0 ** -6))) - 3)
    assert np.all(np.abs(v - xb) <= step / 2 + 1e-12)
    # RoundUp: the block amax fits, one power of two less would not
    amax = np.abs(x.reshape(64, 3, 128)).max(-1)
    assert np.all(amax / scale[..., 0] <= 448) and np.all(amax / (scale[..., 0] / 2) > 448)


def test_gemm_a4w4o4_ref_integer_brute_force():
    rng = np.random.default_rng(32)
    a = rng.integers(0, 256, (5, 16), dtype=np.uint8)
    b = rng.integers(0, 256, (8, 16), dtype=np.uint8)
    got = O.unpack_fp4(O.gemm_a4w4o4_ref(a, b))
    ai = (O.mxfp4_to_f32(a) * 2).astype(np.int64)      # codes * 2 are integers
    bi = (O.mxfp4_to_f32(b) * 2).astype(np.int64)
    exact = (ai @ bi.T) / 4.0
    np.testing.assert_array_equal(got, O.e2m1_encode_rne(exact.astype(np.float32)))
    # saturation: |c| > 6 maps to code 7 / 15
    big = np.abs(exact) > 6
    assert np.all((got[big] & 7) == 7)


# ---------------------------------------------------------------- torch restatement (CPU baseline)
def test_torch_ref_codecs_match_numpy_oracle():
    """oracle/torch_ref.py decodes every e2m1 byte and every e8m0 byte exactly
    as the pinned numpy oracle (bit patterns, -0.0 and NaN included)."""
    import torch

    from oracle import torch_ref as T

    allb = np.arange(256, dtype=np.uint8)
    got = T.mxfp4_to_f32(torch.from_numpy(allb[None, :])).numpy()
    ref = O.mxfp4_to_f32(allb[None, :])
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    gs = T.e8m0_to_f32(torch.from_numpy(allb)).numpy()
    rs = O.e8m0_to_f32(allb)
    assert np.array_equal(gs[:255].view(np.uint32), rs[:255].view(np.uint32))
    assert np.isnan(gs[255]) and np.isnan(rs[255])


def test_torch_ref_gemm_matches_numpy_oracle():
    import torch

    from oracle import torch_ref as T

    rs = np.random.default_rng(5)
    m, n, k = 24, 40, 256
    aq = rs.integers(0, 256, (m, k // 2), dtype=np.uint8)
    bq = rs.integers(0, 256, (n, k // 2), dtype=np.uint8)
    asc = rs.integers(118, 136, (m, k // 32), dtype=np.uint8)
    bsc = rs.integers(118, 136, (n, k // 32), dtype=np.uint8)
    da = T.dequant_mxfp4(torch.from_numpy(aq), torch.from_numpy(asc)).numpy()
    assert np.array_equal(da.view(np.uint32), O.dequant_mxfp4(aq, asc).view(np.uint32))
    tm = {}
    got = T.run_torch_a4w4(torch.from_numpy(aq), torch.from_numpy(bq), torch.from_numpy(asc), torch.from_numpy(bsc),
                           timings=tm).view(torch.int16).numpy().view(np.uint16)
    ref = O.gemm_a4w4_ref(aq, bq, asc, bsc)
    assert set(tm) == {"dequant_s", "mm_s"}
    # same dequantised operands; the f32 matmul may sum in another order: bf16
    # results equal or one bf16 step apart
    diff = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert diff.max() <= 1 and np.mean(diff == 0) > 0.99


def test_mul_add_ref_known_answers():
    """fused mul_add epilogue: hand-computed values of both fuse types with
    scalar and matrix operands (all exact in bf16)."""
    c = np.array([[1.0, 2.0], [3.0, 4.0]], dtype=np.float32)
    bm = np.array([[1.0, 1.0], [0.0, -1.0]], dtype=np.float32)
    got0 = O.bf16_bits_to_f32(O.mul_add_ref(c, 2.0, bm, 0))
    assert np.array_equal(got0, np.array([[3.0, 5.0], [6.0, 7.0]], dtype=np.float32))
    got1 = O.bf16_bits_to_f32(O.mul_add_ref(c, 2.0, 3.0, 1))
    assert np.array_equal(got1, np.array([[7.0, 8.0], [9.0, 10.0]], dtype=np.float32))
    am = np.array([[0.5, -1.0], [2.0, 0.0]], dtype=np.float32)
    got2 = O.bf16_bits_to_f32(O.mul_add_ref(c, am, bm, 0))
    assert np.array_equal(got2, np.array([[1.5, -1.0], [6.0, -1.0]], dtype=np.float32))
    # a = 1, b = 0 is the plain GEMM rounding
    r = np.random.default_rng(0).standard_normal((3, 5)).astype(np.float32)
    assert np.array_equal(O.mul_add_ref(r, 1.0, 0.0, 0), O.f32_to_bf16_bits(r))
    assert np.array_equal(O.mul_add_ref(r, 0.0, 7.0, 1), O.f32_to_bf16_bits(r))


def test_split_cat_ref_known_answer_and_inverse():
    """fused split_cat: a hand-worked [1, 2*(2+1)] case, then on random data
    the parts reassemble the product and carry y unchanged."""
    c = np.arange(6, dtype=np.float32).reshape(1, 6)
    y = np.array([[[10.0], [11.0]]], dtype=np.float32)
    c1, c2 = O.split_cat_ref(c, y, 2, 1)
    assert np.array_equal(c1, np.array([[[0, 1, 10], [3, 4, 11]]], dtype=np.float32))
    assert np.array_equal(c2, np.array([[[2], [5]]], dtype=np.float32))
    rs = np.random.default_rng(1)
    m, d, s1, s2, s3 = 3, 4, 8, 16, 8
    c = rs.standard_normal((m, d * (s1 + s2))).astype(np.float32)
    y = rs.standard_normal((m, d, s3)).astype(np.float32)
    c1, c2 = O.split_cat_ref(c, y, s1, s2)
    assert c1.shape == (m, d, s1 + s3) and c2.shape == (m, d, s2)
    assert np.array_equal(np.concatenate([c1[:, :, :s1], c2], axis=2).reshape(m, -1), c)
    assert np.array_equal(c1[:, :, s1:], y)
