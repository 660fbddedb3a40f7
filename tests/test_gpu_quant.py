"""GPU parity of the MX quantisers against the CPU oracle: bit-exact bytes.

Shapes and inputs follow the reference's own quant tests
(op_tests/test_quant_mxfp4.py:488-496 seed 42; op_tests/triton_tests/quant/
test_quant_mxfp4.py seed 20 incl. odd M; test_quant_mxfp8.py randn*4).
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import randn

pytestmark = pytest.mark.gpu

SHAPES = [(1, 32), (2, 64), (7, 256), (32, 512), (33, 1024), (128, 2048), (257, 4096), (16, 7168)]


def _input(m, k, seed, dtype, scale=1.0):
    x = randn((m, k), seed, scale)
    t = torch.from_numpy(x).to(dtype)
    return t, t.float().numpy()


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


@pytest.mark.parametrize("m,k", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_per_1x32_mx_quant_hip_fp4(cuda, m, k, dtype):
    import aiter_amd

    announce(f"per_1x32_mx_quant_hip fp4 {m}x{k} {dtype}")
    xt, xf = _input(m, k, 42, dtype)
    q_ref, s_ref = O.quant_mxfp4(xf, O.ROUND_UP, amax_floor=1e-10)
    q, s = aiter_amd.per_1x32_mx_quant_hip(xt.to(cuda), shuffle=False)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(q), q_ref)
    np.testing.assert_array_equal(_u8(s), s_ref)
    q2, s2 = aiter_amd.per_1x32_mx_quant_hip(xt.to(cuda), shuffle=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(q2), q_ref)
    # shuffled: compare the bytes of valid (row, block) positions
    ss = _u8(s2)
    assert ss.shape == ((m + 255) // 256 * 256, (k // 32 + 7) // 8 * 8)
    xs, ys = np.meshgrid(np.arange(m), np.arange(k // 32), indexing="ij")
    idx = O.mx_scale_shuffle_idx(ss.shape[1], xs, ys)
    np.testing.assert_array_equal(ss.reshape(-1)[idx], s_ref)


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("m,k", [(32, 64), (33, 1024), (128, 2048), (256, 7168)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_quant_mxfp4_hip_modes(cuda, mode, m, k, dtype):
    """op_tests/test_quant_mxfp4.py:209-230 (byte-equal for modes 0-3)."""
    import aiter_amd

    announce(f"quant_mxfp4_hip mode={mode} {m}x{k} {dtype}")
    xt, xf = _input(m, k, 42, dtype)
    floor = 1e-10 if mode == O.ROUND_UP else None
    q_ref, s_ref = O.quant_mxfp4(xf, mode, amax_floor=floor)
    q, s = aiter_amd.quant_mxfp4_hip(xt.to(cuda).contiguous(), round_mode=mode)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(q), q_ref)
    np.testing.assert_array_equal(_u8(s), s_ref)


@pytest.mark.parametrize("m,k", [(32, 256), (64, 1024), (256, 2048)])
def test_quant_mxfp4_fused_shuffle(cuda, m, k):
    """Fused weight + e8m0 shuffle equals shuffle_weight + shuffle_scale
    (op_tests/test_quant_mxfp4.py:233-268)."""
    import aiter_amd

    announce(f"quant_mxfp4_hip fused shuffle {m}x{k}")
    xt, xf = _input(m, k, 7, torch.bfloat16)
    q_ref, s_ref = O.quant_mxfp4(xf, O.EVEN)
    q, s = aiter_amd.quant_mxfp4_hip(xt.to(cuda), round_mode=2, e8m0_shuffle=True, shuffle_weight=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(q), O.shuffle_weight(q_ref))
    ss = _u8(s)
    ref = O.shuffle_scale(s_ref)
    valid = O.shuffle_scale(np.ones_like(s_ref)) == 1
    np.testing.assert_array_equal(ss[valid], ref[valid])


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_quant_edge_values(cuda, mode):
    """op_tests/test_quant_mxfp4.py:352-375: zeros -> all-zero packed bytes,
    large / tiny / negative constants byte-equal to the oracle."""
    import aiter_amd

    for val in (0.0, 1e4, 1e-10, -3.0):
        announce(f"edge value {val} mode={mode}")
        x = torch.full((32, 64), val, dtype=torch.bfloat16)
        q, s = aiter_amd.quant_mxfp4_hip(x.to(cuda), round_mode=mode)
        torch.cuda.synchronize()
        floor = 1e-10 if mode == O.ROUND_UP else None
        q_ref, s_ref = O.quant_mxfp4(x.float().numpy(), mode, amax_floor=floor)
        np.testing.assert_array_equal(_u8(q), q_ref)
        np.testing.assert_array_equal(_u8(s), s_ref)
        if val == 0.0:
            assert _u8(q).sum() == 0


@pytest.mark.parametrize("m,k", [(1, 32), (2, 64), (8, 256), (137, 64), (256, 2048), (33, 7168)])
@pytest.mark.parametrize("shuffle", [False, True])
def test_dynamic_mxfp4_quant_even(cuda, m, k, shuffle):
    """Even-mode quant of the A4W4 test/tuner path (Triton dynamic_mxfp4_quant
    layout, aiter/utility/fp4_utils.py:373-597), seed 20."""
    import aiter_amd

    announce(f"dynamic_mxfp4_quant {m}x{k} shuffle={shuffle}")
    xt, xf = _input(m, k, 20, torch.bfloat16)
    q_ref, s_ref = O.quant_mxfp4_triton_even(xf)
    q, s = aiter_amd.dynamic_mxfp4_quant(xt.to(cuda), shuffle=shuffle)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(q), q_ref)
    if not shuffle:
        np.testing.assert_array_equal(_u8(s), s_ref)
    else:
        ss = _u8(s)
        sn_pad = ss.shape[1]
        rows32 = (m + 31) // 32 * 32
        # rows < pad32(M) written: valid scale or 0 in the padding (fp4_utils.py:526-529)
        full = np.zeros((rows32, sn_pad), dtype=np.uint8)
        full[:m, : k // 32] = s_ref
        xs, ys = np.meshgrid(np.arange(rows32), np.arange(sn_pad), indexing="ij")
        idx = O.triton_scale_store_offset(sn_pad, xs, ys)
        np.testing.assert_array_equal(ss.reshape(-1)[idx], full)


@pytest.mark.parametrize("m,k", [(1, 32), (8, 64), (32, 256), (137, 64), (128, 1024), (256, 16384)])
def test_dynamic_mxfp8_quant(cuda, m, k):
    """op_tests/triton_tests/quant/test_quant_mxfp8.py:79-104 (x = randn*4):
    scales bit-exact, and here the e4m3 bytes too."""
    import aiter_amd

    announce(f"dynamic_mxfp8_quant {m}x{k}")
    xt, xf = _input(m, k, 20, torch.bfloat16, scale=4.0)
    q_ref, s_ref = O.quant_mxfp8(xf, O.EVEN)
    q, s = aiter_amd.dynamic_mxfp8_quant(xt.to(cuda))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(s), s_ref)
    np.testing.assert_array_equal(_u8(q), q_ref)


@pytest.mark.parametrize("m,k", [(4, 64), (64, 2048), (100, 4096)])
def test_per_1x32_mx_quant_hip_fp8(cuda, m, k):
    import aiter_amd

    announce(f"per_1x32_mx_quant_hip fp8 {m}x{k}")
    xt, xf = _input(m, k, 3, torch.bfloat16, scale=2.0)
    q_ref, s_ref = O.quant_mxfp8(xf, O.ROUND_UP, amax_floor=1e-10)
    q, s = aiter_amd.per_1x32_mx_quant_hip(xt.to(cuda), quant_dtype=torch.float8_e4m3fn,
                                            scale_type=aiter_amd.dtypes.fp8_e8m0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(s), s_ref)
    np.testing.assert_array_equal(_u8(q), q_ref)


def test_quant_fp32_input(cuda):
    import aiter_amd

    announce("quant fp32 input")
    x = randn((64, 1024), 11)
    q_ref, s_ref = O.quant_mxfp4(x, O.ROUND_UP, amax_floor=1e-10)
    q, s = aiter_amd.per_1x32_mx_quant_hip(torch.from_numpy(x).to(cuda))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(q), q_ref)
    np.testing.assert_array_equal(_u8(s), s_ref)


_EXP_RANGE = {torch.float32: (-140, 40), torch.bfloat16: (-130, 40), torch.float16: (-22, 12)}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("fp8", [False, True])
def test_quant_block_magnitudes(cuda, dtype, fp8):
    """Every input dtype into e2m1 and e4m3, each 32-block scaled by its own
    power of two across the dtype's whole range (down to subnormal inputs,
    whose Even scale byte is 0), plus all-zero blocks; Even (dynamic_*) and
    RoundUp (per_1x32_mx_quant_hip) scales, bytes equal to the oracle."""
    import aiter_amd

    m, k = 64, 1024
    announce(f"quant block magnitudes {dtype} fp8={fp8}")
    rs = np.random.default_rng(90)
    lo, hi = _EXP_RANGE[dtype]
    e = rs.integers(lo, hi, (m, k // 32))
    x = rs.standard_normal((m, k)).astype(np.float32) * np.repeat(np.exp2(e.astype(np.float64)), 32, axis=1)
    x[::7, 64:96] = 0.0                                     # all-zero blocks
    xt = torch.from_numpy(x.astype(np.float32)).to(dtype)
    xf = xt.float().numpy()
    xd = xt.to(cuda)
    if fp8:
        q, s = aiter_amd.dynamic_mxfp8_quant(xd, shuffle=False)
        q_ref, s_ref = O.quant_mxfp8(xf, O.EVEN)
    else:
        q, s = aiter_amd.dynamic_mxfp4_quant(xd, shuffle=False)
        q_ref, s_ref = O.quant_mxfp4_triton_even(xf)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(_u8(s), s_ref)
    np.testing.assert_array_equal(_u8(q), q_ref)
    assert (s_ref == 0).any() or dtype == torch.float16    # the subnormal-scale branch is exercised
    qd = aiter_amd.dtypes.fp8 if fp8 else aiter_amd.dtypes.fp4x2
    q, s = aiter_amd.per_1x32_mx_quant_hip(xd, quant_dtype=qd, shuffle=False)
    torch.cuda.synchronize()
    if fp8:
        q_ref, s_ref = O.quant_mxfp8(xf, O.ROUND_UP, amax_floor=1e-10)
    else:
        q_ref, s_ref = O.quant_mxfp4(xf, O.ROUND_UP, amax_floor=1e-10)
    np.testing.assert_array_equal(_u8(s), s_ref)
    np.testing.assert_array_equal(_u8(q), q_ref)
