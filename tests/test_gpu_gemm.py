"""GPU parity of the GEMMs against the CPU oracle (dequantise -> f32 matmul ->
bf16; op_tests/test_gemm_a4w4.py:23-39), tolerance rtol = atol = 1e-2 on every
element.  Inputs are quantised by the oracle so these tests exercise the GEMM
kernels alone; the quantisers have their own bit-exact tests.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, bf16_operand, mxfp4_operand, mxfp8_operand, tile_samples

pytestmark = pytest.mark.gpu


def _bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy()


def _a4w4_case(m, n, k, seed=0):
    a_q, a_s, a_ss = mxfp4_operand(m, k, seed, "triton")
    b_q, b_s, b_ss = mxfp4_operand(n, k, seed + 1, "triton")
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q, b_q, a_s, b_s))
    return a_q, a_ss, b_q, b_ss, ref


def _dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


A4W4_SHAPES = [(1, 256, 256), (5, 512, 512), (16, 1024, 1024), (32, 7168, 2048), (33, 640, 1280),
               (64, 7168, 2048), (65, 256, 512), (128, 1024, 1024), (256, 512, 2048), (300, 1040, 768),
               (512, 512, 512), (24, 8208, 512)]


@pytest.mark.parametrize("m,n,k", A4W4_SHAPES)
def test_gemm_a4w4_heuristic(cuda, m, n, k):
    import aiter_amd

    announce(f"gemm_a4w4 {m}x{n}x{k}")
    a_q, a_ss, b_q, b_ss, ref = _a4w4_case(m, n, k)
    out = aiter_amd.gemm_a4w4(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda),
                              _dev(b_ss, cuda))
    torch.cuda.synchronize()
    assert out.shape == (m, n)
    ok, msg = allclose_report(_bf16_np(out), ref)
    assert ok, msg


def _kernels(family, skinny=None, b_pre=True, a_pre=False, out_f32=False):
    from aiter_amd._lib import kernel_table

    return [r for r in kernel_table() if r[2] == family and r[8] == b_pre and r[7] == a_pre and r[9] == out_f32
            and (skinny is None or r[3] == skinny)]


def _kernel_names(family, **kw):
    try:
        return [r[1] for r in _kernels(family, **kw)]
    except RuntimeError:
        return []


@pytest.mark.parametrize("name", _kernel_names("a4w4") + _kernel_names("a4w4", b_pre=False))
def test_gemm_a4w4_every_instance(cuda, name):
    """Every A4W4 instance (tile and skinny, incl. split-K; preshuffled and
    row-major B) on a ragged shape."""
    import aiter_amd
    from aiter_amd._lib import kernel_table

    row = [r for r in kernel_table() if r[1] == name][0]
    skinny, bm, b_pre = row[3], row[4], row[8]
    m = min(bm, 48) if skinny else 200
    if skinny:
        m = max(1, bm - 3)
    n, k = 1024 + 48, 2048
    announce(f"a4w4 instance {name} {m}x{n}x{k}")
    a_q, a_ss, b_q, b_ss, ref = _a4w4_case(m, n, k, seed=3)
    out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q) if b_pre else b_q, cuda), _dev(a_ss, cuda),
                            _dev(b_ss, cuda), out, kernelName=name, log2_k_split=2 if row[6] else 0,
                            bpreshuffle=bool(b_pre))
    torch.cuda.synchronize()
    ok, msg = allclose_report(_bf16_np(out[:m]), ref)
    assert ok, msg


@pytest.mark.parametrize("m", [1, 32, 96, 600])
def test_gemm_a4w4_row_major_b(cuda, m):
    import aiter_amd

    n, k = 512, 1024
    announce(f"a4w4 bpreshuffle=0 {m}x{n}x{k}")
    a_q, a_ss, b_q, b_ss, ref = _a4w4_case(m, n, k, seed=9)
    out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(b_q, cuda), _dev(a_ss, cuda), _dev(b_ss, cuda), out,
                            bpreshuffle=False)
    torch.cuda.synchronize()
    ok, msg = allclose_report(_bf16_np(out[:m]), ref)
    assert ok, msg


def test_gemm_a4w4_bias_alpha_beta(cuda):
    """D = alpha * A B^T + beta * bias (csrc/py_itfs_cu/asm_gemm_a4w4.cu:154)."""
    import aiter_amd

    m, n, k = 64, 512, 512
    announce("a4w4 alpha/beta/bias")
    a_q, a_ss, b_q, b_ss, _ = _a4w4_case(m, n, k, seed=4)
    bias = np.random.default_rng(5).standard_normal((1, n)).astype(np.float32)
    a = O.dequant_mxfp4(a_q, O.unshuffle_scale(a_ss, m, k // 32))
    b = O.dequant_mxfp4(b_q, O.unshuffle_scale(b_ss, n, k // 32))
    ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(0.5 * (a @ b.T) + 2.0 * bias))
    for name in ("a4w4_tile_64x128", "a4w4_skinny_m64"):
        out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
        aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda),
                                _dev(b_ss, cuda), out, kernelName=name, bias=_dev(bias, cuda), alpha=0.5,
                                beta=2.0)
        torch.cuda.synchronize()
        ok, msg = allclose_report(_bf16_np(out), ref)
        assert ok, f"{name}: {msg}"


def test_gemm_a4w4_full_size_every_tile(cuda):
    """M=N=K=8192 (BASELINE prefill config) through the tuned dispatch into a
    NaN-filled output: every element finite (every tile written), and one
    element of every 128x128 block (64 x 64 samples: every tile of every
    instance) against the oracle's f32 dot products of the dequantised rows."""
    import aiter_amd
    from aiter_amd.gemm_op_a4w4 import _gemm_a4w4_into

    m = n = k = 8192
    announce(f"a4w4 8192^3 every tile, kernel={aiter_amd.get_GEMM_config(m, n, k)}")
    g = torch.Generator(device="cpu").manual_seed(0)
    x = torch.randn((m, k), generator=g, dtype=torch.float32).to(torch.bfloat16).to(cuda)
    w = torch.randn((n, k), generator=g, dtype=torch.float32).to(torch.bfloat16).to(cuda)
    xq, xs = aiter_amd.dynamic_mxfp4_quant(x, shuffle=True)
    wq, ws = aiter_amd.dynamic_mxfp4_quant(w, shuffle=True)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    _gemm_a4w4_into(xq, aiter_amd.shuffle_weight(wq), xs, ws, out, None, 1.0, 0.0, True)
    assert bool(torch.isfinite(out).all()), "output elements left unwritten (NaN)"
    rows = tile_samples(m, 128, 1)
    cols = tile_samples(n, 128, 2)
    a_q = xq.view(torch.uint8)[torch.from_numpy(rows).to(cuda)].cpu().numpy()
    b_q = wq.view(torch.uint8)[torch.from_numpy(cols).to(cuda)].cpu().numpy()
    xs_np = xs.view(torch.uint8).cpu().numpy()
    ws_np = ws.view(torch.uint8).cpu().numpy()
    a_s = O.unshuffle_scale(xs_np, m, k // 32)[rows]
    b_s = O.unshuffle_scale(ws_np, n, k // 32)[cols]
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q, b_q, a_s, b_s))
    got = out[torch.from_numpy(rows).to(cuda)][:, torch.from_numpy(cols).to(cuda)].float().cpu().numpy()
    ok, msg = allclose_report(got, ref)
    assert ok, msg


# ----------------------------------------------------------------------------- a8w4
A8W4_SHAPES = [(1, 256, 512), (17, 512, 1024), (64, 7168, 2048), (100, 640, 512), (256, 1024, 2048), (20, 8208, 512)]


def _a8w4_case(m, n, k, seed=0):
    a_q, a_s, a_ss = mxfp8_operand(m, k, seed)
    b_q, b_s, b_ss = mxfp4_operand(n, k, seed + 1, "triton")
    ref = O.bf16_bits_to_f32(O.gemm_a8w4_ref(a_q, b_q, a_s, b_s))
    return a_q, a_ss, b_q, b_ss, ref


@pytest.mark.parametrize("m,n,k", A8W4_SHAPES)
def test_gemm_a8w4(cuda, m, n, k):
    import aiter_amd

    announce(f"gemm_a8w4_mxfp8 {m}x{n}x{k}")
    a_q, a_ss, b_q, b_ss, ref = _a8w4_case(m, n, k)
    a = _dev(a_q, cuda).view(torch.float8_e4m3fn)
    out = aiter_amd.gemm_a8w4_mxfp8(a, _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda), _dev(b_ss, cuda),
                                    a_preshuffle=False)
    torch.cuda.synchronize()
    ok, msg = allclose_report(_bf16_np(out), ref)
    assert ok, msg


@pytest.mark.parametrize("name", _kernel_names("a8w4") + _kernel_names("a8w4", a_pre=True))
def test_gemm_a8w4_every_instance(cuda, name):
    import aiter_amd
    from aiter_amd._lib import kernel_table

    row = [r for r in kernel_table() if r[1] == name][0]
    skinny, bm, a_pre = row[3], row[4], row[7]
    m = max(1, bm - 5) if skinny else 192
    n, k = 768, 1024
    announce(f"a8w4 instance {name} {m}x{n}x{k}")
    a_q, a_ss, b_q, b_ss, ref = _a8w4_case(m, n, k, seed=2)
    a_in = O.shuffle_weight(a_q) if a_pre else a_q
    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
    from aiter_amd._lib import call

    call("mxfp8_mxfp4_gemm_asm", _dev(a_in, cuda).view(torch.float8_e4m3fn), _dev(O.shuffle_weight(b_q), cuda),
         _dev(a_ss, cuda), _dev(b_ss, cuda), out, name, int(a_pre))
    torch.cuda.synchronize()
    ok, msg = allclose_report(_bf16_np(out), ref)
    assert ok, msg


def test_gemm_a8w4_dynamic_quant(cuda):
    """bf16 activation -> fused dynamic MXFP8 quant -> GEMM."""
    import aiter_amd

    m, n, k = 256, 512, 2048
    announce("a8w4 dynamic quant")
    x = np.random.default_rng(0).standard_normal((m, k)).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    b_q, b_s, b_ss = mxfp4_operand(n, k, 1, "triton")
    aq, as_ = O.quant_mxfp8(xb.float().numpy(), O.EVEN)
    ref = O.bf16_bits_to_f32(O.gemm_a8w4_ref(aq, b_q, as_, b_s))
    out = aiter_amd.gemm_a8w4_mxfp8_dynamic(xb.to(cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(b_ss, cuda))
    torch.cuda.synchronize()
    ok, msg = allclose_report(_bf16_np(out), ref)
    assert ok, msg


# ----------------------------------------------------------------------------- bf16
BF16_SHAPES = [(1, 256, 256), (7, 512, 1024), (32, 1024, 512), (64, 4096, 1024), (100, 640, 320),
               (256, 512, 1024), (513, 1024, 768)]


@pytest.mark.parametrize("m,n,k", BF16_SHAPES)
def test_gemm_a16w16(cuda, m, n, k):
    import aiter_amd

    announce(f"gemm_a16w16 {m}x{n}x{k}")
    a = bf16_operand(m, k, 0)
    b = bf16_operand(n, k, 1)
    ref = O.bf16_bits_to_f32(O.gemm_a16w16_ref(a, b))
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev(b.view(np.int16), cuda).view(torch.bfloat16)
    out = aiter_amd.gemm_a16w16(at, bt)
    torch.cuda.synchronize()
    ok, msg = allclose_report(_bf16_np(out), ref)
    assert ok, msg


@pytest.mark.parametrize("name", _kernel_names("a16w16") + _kernel_names("a16w16", b_pre=False)
                         + _kernel_names("a16w16", out_f32=True) + _kernel_names("a16w16", b_pre=False, out_f32=True))
def test_gemm_a16w16_every_instance(cuda, name):
    import aiter_amd
    from aiter_amd._lib import kernel_table

    row = [r for r in kernel_table() if r[1] == name][0]
    skinny, bm, b_pre, out_f32 = row[3], row[4], row[8], row[9]
    m = max(1, bm - 7) if skinny else 150
    n, k = 528, 1024
    announce(f"a16w16 instance {name} {m}x{n}x{k}")
    a = bf16_operand(m, k, 5)
    b = bf16_operand(n, k, 6)
    bias = np.random.default_rng(8).standard_normal(n).astype(np.float32)
    af, bf = O.bf16_bits_to_f32(a), O.bf16_bits_to_f32(b)
    c = af @ bf.T + bias
    ref = c if out_f32 else O.bf16_bits_to_f32(O.f32_to_bf16_bits(c))
    bt_np = O.shuffle_weight(b) if b_pre else b
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev(bt_np.view(np.int16), cuda).view(torch.bfloat16)
    out = torch.empty((m, n), dtype=torch.float32 if out_f32 else torch.bfloat16, device=cuda)
    aiter_amd.gemm_a16w16_asm(at, bt, out, bias=_dev(bias, cuda), splitK=4 if row[6] else 0, kernelName=name,
                              bpreshuffle=b_pre)
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, msg


def _split_f32_names():
    try:
        return [r[1] for r in _kernels("a16w16", out_f32=True) + _kernels("a16w16", b_pre=False, out_f32=True)
                if r[3] and r[6]]
    except RuntimeError:
        return []


@pytest.mark.parametrize("name", _split_f32_names())
def test_gemm_a16w16_f32_split_sums_into_output(cuda, name):
    """f32 output, no bias, split over K: the partials add straight into the
    output, which the call clears first (NaN before the call, then a second
    call on the first call's result)."""
    import aiter_amd
    from aiter_amd._lib import kernel_table

    row = [r for r in kernel_table() if r[1] == name][0]
    bm, b_pre = row[4], row[8]
    m, n, k = max(1, bm - 3), 544, 2048
    announce(f"a16w16 f32 split {name} {m}x{n}x{k}")
    a = bf16_operand(m, k, 15)
    b = bf16_operand(n, k, 16)
    ref = O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T
    bt_np = O.shuffle_weight(b) if b_pre else b
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev(bt_np.view(np.int16), cuda).view(torch.bfloat16)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=cuda)
    for _ in range(2):
        aiter_amd.gemm_a16w16_asm(at, bt, out, splitK=4, kernelName=name, bpreshuffle=b_pre)
        torch.cuda.synchronize()
        ok, msg = allclose_report(out.cpu().numpy(), ref)
        assert ok, msg


def _persistent_a16w16():
    try:
        from aiter_amd._lib import kernel_table

        return [(r[1], bool(r[8])) for r in kernel_table() if r[2] == "a16w16" and r[1].endswith("_persist")]
    except RuntimeError:
        return []


@pytest.mark.parametrize("m,n,k", [(600, 528, 64), (600, 528, 1088), (4352, 4096, 256)])
@pytest.mark.parametrize("name,b_pre", _persistent_a16w16())
def test_gemm_a16w16_persistent_instances(cuda, name, b_pre, m, n, k):
    """The persistent bf16 tiles without bias (with a bias the host takes
    their one-tile-per-workgroup twins): ragged M and N, K of one stage and of
    an odd stage count, and more tiles than CUs (several tiles per workgroup)."""
    import aiter_amd

    announce(f"a16w16 persistent {name} {m}x{n}x{k}")
    a = bf16_operand(m, k, 11)
    b = bf16_operand(n, k, 12)
    ref = O.bf16_bits_to_f32(O.gemm_a16w16_ref(a, b))
    bt_np = O.shuffle_weight(b) if b_pre else b
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev(bt_np.view(np.int16), cuda).view(torch.bfloat16)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a16w16_asm(at, bt, out, kernelName=name, bpreshuffle=b_pre)
    torch.cuda.synchronize()
    ok, msg = allclose_report(_bf16_np(out), ref)
    assert ok, msg


def test_gemm_a16w16_opus_batched(cuda):
    import aiter_amd

    announce("gemm_a16w16_opus batched")
    b_, m, n, k = 3, 64, 256, 512
    rs = np.random.default_rng(3)
    A = torch.from_numpy(rs.standard_normal((b_, m, k)).astype(np.float32)).to(torch.bfloat16)
    B = torch.from_numpy(rs.standard_normal((b_, n, k)).astype(np.float32)).to(torch.bfloat16)
    bias = torch.from_numpy(rs.standard_normal((b_, n)).astype(np.float32))
    ref = torch.bmm(A.float(), B.float().transpose(1, 2).contiguous()) + bias[:, None, :]
    out = aiter_amd.gemm_a16w16_opus(A.to(cuda), B.to(cuda), bias.to(cuda))
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), O.bf16_bits_to_f32(O.f32_to_bf16_bits(ref.numpy())))
    assert ok, msg


TILE_K_CASES = [(300, 528, 256), (257, 512, 768), (64, 272, 2304), (520, 784, 1280)]


@pytest.mark.parametrize("m,n,k", TILE_K_CASES)
def test_tile_instances_odd_stage_counts(cuda, m, n, k):
    """Every A4W4 / A8W4 tile instance with K/256 = 1, 3, 9, 5 (odd stage
    counts, a single stage) on ragged M and N, called twice in a row with
    different data (stale LDS or registers from the first call must not leak
    into the second)."""
    import aiter_amd
    from aiter_amd._lib import call

    for fam in ("a4w4", "a8w4"):
        for row in _kernels(fam, skinny=False):
            name = row[1]
            for seed in (11, 12):
                announce(f"{fam} tile {name} {m}x{n}x{k} seed {seed}")
                if fam == "a4w4":
                    a_q, a_ss, b_q, b_ss, ref = _a4w4_case(m, n, k, seed=seed)
                    out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=cuda)
                    aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda),
                                            _dev(b_ss, cuda), out, kernelName=name)
                else:
                    a_q, a_ss, b_q, b_ss, ref = _a8w4_case(m, n, k, seed=seed)
                    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
                    call("mxfp8_mxfp4_gemm_asm", _dev(a_q, cuda).view(torch.float8_e4m3fn),
                         _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda), _dev(b_ss, cuda), out, name, 0)
                torch.cuda.synchronize()
                ok, msg = allclose_report(_bf16_np(out[:m]), ref)
                assert ok, f"{name}: {msg}"


BF16_K_CASES = [(300, 528, 64), (257, 512, 192), (64, 272, 576), (520, 784, 320)]


@pytest.mark.parametrize("m,n,k", BF16_K_CASES)
def test_bf16_tile_instances_odd_stage_counts(cuda, m, n, k):
    """Every bf16 tile instance (row-major and preshuffled B) with K/64 = 1,
    3, 9, 5 (a single stage, odd stage counts: the row-major flat tile uses
    two B regions by stage parity and pads to an even count) on ragged M and
    N, called twice in a row with different data."""
    import aiter_amd

    for b_pre in (False, True):
        for row in _kernels("a16w16", skinny=False, b_pre=b_pre):
            name, split = row[1], row[6]
            for seed in (31, 32):
                announce(f"bf16 tile {name} {m}x{n}x{k} seed {seed}")
                a = bf16_operand(m, k, seed)
                b = bf16_operand(n, k, seed + 100)
                ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T))
                bt_np = O.shuffle_weight(b) if b_pre else b
                at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
                bt = _dev(bt_np.view(np.int16), cuda).view(torch.bfloat16)
                out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
                aiter_amd.gemm_a16w16_asm(at, bt, out, splitK=2 if split else 0, kernelName=name, bpreshuffle=b_pre)
                torch.cuda.synchronize()
                ok, msg = allclose_report(out.float().cpu().numpy(), ref)
                assert ok, f"{name}: {msg}"


@pytest.mark.parametrize("k", [64, 192, 576, 2112])
def test_bf16_skinny_instances_k_pairs(cuda, k):
    """Every bf16 skinny instance with K/64 = 1, 3, 9, 33 k-pairs over its 8
    waves (waves with no pair, fewer pairs than the load pipeline's depth,
    odd counts), N = 272 (17 column blocks: a 32-column workgroup past N)."""
    import aiter_amd

    n = 272
    for b_pre in (False, True):
        for row in _kernels("a16w16", skinny=True, b_pre=b_pre):
            name, bm, split = row[1], row[4], row[6]
            m = max(1, bm - 3)
            announce(f"bf16 skinny {name} {m}x{n}x{k}")
            a = bf16_operand(m, k, 41)
            b = bf16_operand(n, k, 42)
            ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T))
            bt_np = O.shuffle_weight(b) if b_pre else b
            at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
            bt = _dev(bt_np.view(np.int16), cuda).view(torch.bfloat16)
            out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
            aiter_amd.gemm_a16w16_asm(at, bt, out, splitK=2 if split else 0, kernelName=name, bpreshuffle=b_pre)
            torch.cuda.synchronize()
            ok, msg = allclose_report(out.float().cpu().numpy(), ref)
            assert ok, f"{name}: {msg}"


@pytest.mark.parametrize("k", [256, 768, 2048, 2304, 4096, 8448])
def test_mx_skinny_instances_k_pairs(cuda, k):
    """Every A4W4 and A8W4 skinny instance (preshuffled B) with K/256 = 1, 3,
    8, 9, 16, 33 k-pairs over its waves, N = 272 (17 column blocks).  The
    direct instances (``_direct_kP``) hold at most P k-pairs: longer K is
    refused on the host."""
    import aiter_amd
    from aiter_amd._lib import call

    n = 272
    for fam in ("a4w4", "a8w4"):
        for row in _kernels(fam, skinny=True):
            name, bm, split = row[1], row[4], row[6]
            if split:
                continue   # the split forms: test_gpu_splitk_tiles and the every-instance sweep
            m = max(1, bm - 3)
            kp = int(name.rsplit("_k", 1)[1]) if "_direct_k" in name else None
            if kp is not None and k // 256 > kp:
                announce(f"{fam} skinny {name} {m}x{n}x{k}: refused")
                with pytest.raises(RuntimeError, match="longer than"):
                    if fam == "a4w4":
                        out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=cuda)
                        a_long = torch.zeros((m, k // 2), dtype=torch.uint8, device=cuda)
                        b_long = torch.zeros((n, k // 2), dtype=torch.uint8, device=cuda)
                        s_a = torch.zeros(((m + 255) // 256 * 256, k // 32), dtype=torch.uint8, device=cuda)
                        s_b = torch.zeros(((n + 255) // 256 * 256, k // 32), dtype=torch.uint8, device=cuda)
                        aiter_amd.gemm_a4w4_asm(a_long, b_long, s_a, s_b, out, kernelName=name)
                    else:
                        out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
                        call("mxfp8_mxfp4_gemm_asm",
                             torch.zeros((m, k), dtype=torch.uint8, device=cuda).view(torch.float8_e4m3fn),
                             torch.zeros((n, k // 2), dtype=torch.uint8, device=cuda),
                             torch.zeros(((m + 255) // 256 * 256, k // 32), dtype=torch.uint8, device=cuda),
                             torch.zeros(((n + 255) // 256 * 256, k // 32), dtype=torch.uint8, device=cuda),
                             out, name, 0)
                continue
            announce(f"{fam} skinny {name} {m}x{n}x{k}")
            if fam == "a4w4":
                a_q, a_ss, b_q, b_ss, ref = _a4w4_case(m, n, k, seed=51)
                out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=cuda)
                aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda),
                                        _dev(b_ss, cuda), out, kernelName=name)
            else:
                a_q, a_ss, b_q, b_ss, ref = _a8w4_case(m, n, k, seed=52)
                out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
                call("mxfp8_mxfp4_gemm_asm", _dev(a_q, cuda).view(torch.float8_e4m3fn),
                     _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda), _dev(b_ss, cuda), out, name, 0)
            torch.cuda.synchronize()
            ok, msg = allclose_report(_bf16_np(out[:m]), ref)
            assert ok, f"{name}: {msg}"


def test_streamed_weight_instances(cuda):
    """Launches whose weights reach the nt-load size (16 MiB): every bf16
    skinny instance and every bf16 tile with one row of tiles at
    16x4096x2048, every non-split A4W4 skinny instance at 16x8192x4096."""
    import aiter_amd

    m, n, k = 16, 4096, 2048
    a = bf16_operand(m, k, 61)
    b = bf16_operand(n, k, 62)
    ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T))
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    for b_pre in (False, True):
        bt = _dev((O.shuffle_weight(b) if b_pre else b).view(np.int16), cuda).view(torch.bfloat16)
        for row in _kernels("a16w16", b_pre=b_pre):
            name, skinny, bm, split = row[1], row[3], row[4], row[6]
            if not skinny and bm < m:
                continue
            announce(f"bf16 streamed-weight {name} {m}x{n}x{k}")
            out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
            aiter_amd.gemm_a16w16_asm(at, bt, out, splitK=2 if split else 0, kernelName=name, bpreshuffle=b_pre)
            torch.cuda.synchronize()
            ok, msg = allclose_report(out.float().cpu().numpy(), ref)
            assert ok, f"{name}: {msg}"
    n, k = 8192, 4096
    a_q, a_ss, b_q, b_ss, ref = _a4w4_case(m, n, k, seed=63)
    bq = _dev(O.shuffle_weight(b_q), cuda)
    for row in _kernels("a4w4", skinny=True):
        name, split = row[1], row[6]
        if split:
            continue
        if "_direct_k" in name and k // 256 > int(name.rsplit("_k", 1)[1]):
            continue   # K beyond the direct instance's k-pairs (refused: test_mx_skinny_instances_k_pairs)
        announce(f"a4w4 streamed-weight {name} {m}x{n}x{k}")
        out = torch.empty((32, n), dtype=torch.bfloat16, device=cuda)
        aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), bq, _dev(a_ss, cuda), _dev(b_ss, cuda), out, kernelName=name)
        torch.cuda.synchronize()
        ok, msg = allclose_report(_bf16_np(out[:m]), ref)
        assert ok, f"{name}: {msg}"


@pytest.mark.parametrize("m,n,k", [(8192, 2048, 512), (2048, 8192, 512), (4608, 4096, 256)])
def test_tile_instances_more_tiles_than_cus(cuda, m, n, k):
    """Every A4W4 tile instance on grids of 512-2304 tiles (more tiles than
    CUs, and tile counts that are multiples of the 8 XCDs, which turns on the
    XCD-aware tile order): every tile must be written."""
    import aiter_amd

    a_q, a_ss, b_q, b_ss, ref = _a4w4_case(m, n, k, seed=21)
    b_dev = _dev(O.shuffle_weight(b_q), cuda)
    for row in _kernels("a4w4", skinny=False):
        name = row[1]
        announce(f"a4w4 tile {name} {m}x{n}x{k} (many tiles)")
        out = torch.zeros(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=cuda)
        aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), b_dev, _dev(a_ss, cuda), _dev(b_ss, cuda), out, kernelName=name)
        torch.cuda.synchronize()
        ok, msg = allclose_report(_bf16_np(out[:m]), ref)
        assert ok, f"{name}: {msg}"


def test_bf16_cpu_plumbing_config(cuda):
    """BASELINE configs[0] on the GPU: A[128,4096] x B[4096,4096]^T, bf16 from
    N(0,1) with torch seed 0, against the CPU fp32 reference of that config
    (tgemm.mm and gemm_a16w16, row-major and preshuffled B)."""
    import aiter_amd

    announce("bf16 plumbing config 128x4096x4096")
    g = torch.Generator().manual_seed(0)
    a = torch.randn(128, 4096, generator=g).to(torch.bfloat16)
    b = torch.randn(4096, 4096, generator=g).to(torch.bfloat16)
    ref = (a.float() @ b.float().T).bfloat16().float().numpy()
    ad, bd = a.to(cuda), b.to(cuda)
    for got in (aiter_amd.tgemm.mm(ad, bd), aiter_amd.gemm_a16w16(ad, bd),
                aiter_amd.gemm_a16w16(ad, aiter_amd.shuffle_weight(bd))):
        torch.cuda.synchronize()
        ok, msg = allclose_report(got.float().cpu().numpy(), ref)
        assert ok, msg


def test_hbm_stream_read_calibration(cuda):
    """The calibration read runs over a buffer, leaves the sink alone (the
    xor of an even number of equal words is 0) and rejects a strided view."""
    from aiter_amd._lib import call

    announce("hbm_stream_read 1 MiB")
    buf = torch.ones(1 << 20, dtype=torch.uint8, device=cuda)
    sink = torch.zeros(1, dtype=torch.int32, device=cuda)
    call("hbm_stream_read", buf, sink, 64)
    torch.cuda.synchronize()
    assert int(sink.item()) == 0
    with pytest.raises(RuntimeError, match="contiguous"):
        call("hbm_stream_read", buf[::2], sink, 64)


def test_outputs_of_2gib_and_more_run_in_row_chunks(cuda):
    """An output of 2 GiB or more (the reference's M = 16384, N = 106496 rows)
    runs as row chunks (the kernels address out through 32-bit offsets):
    A4W4 with bf16 out [16640, 65536] (2.03 GiB, chunks of 16128 rows) and bf16
    with f32 out [8448, 65536] (2.06 GiB, chunks of 7936 rows); rows on both sides of the chunk
    boundary, written into NaN-filled outputs, against the oracle."""
    import aiter_amd

    m, n, k = 16640, 65536, 256
    announce(f"a4w4 {m}x{n}x{k}: 2 GiB output in row chunks")
    g = torch.Generator(device="cpu").manual_seed(31)
    x = torch.randn((m, k), generator=g).to(cuda)
    w = torch.randn((n, k), generator=g).to(cuda)
    xq, xs = aiter_amd.dynamic_mxfp4_quant(x, shuffle=True)
    wq, ws = aiter_amd.dynamic_mxfp4_quant(w, shuffle=True)
    out = torch.full(((m + 31) // 32 * 32, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a4w4_asm(xq, aiter_amd.shuffle_weight(wq), xs, ws, out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out[:m]).all()), "output rows left unwritten"
    rows = np.array([0, 5, 16127, 16128, 16129, m - 1])
    cols = np.sort(np.random.default_rng(3).choice(n, 64, replace=False))
    a_q = xq.view(torch.uint8)[torch.from_numpy(rows).to(cuda)].cpu().numpy()
    b_q = wq.view(torch.uint8)[torch.from_numpy(cols).to(cuda)].cpu().numpy()
    a_s = O.unshuffle_scale(xs.view(torch.uint8).cpu().numpy(), m, k // 32)[rows]
    b_s = O.unshuffle_scale(ws.view(torch.uint8).cpu().numpy(), n, k // 32)[cols]
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q, b_q, a_s, b_s))
    got = out[torch.from_numpy(rows).to(cuda)][:, torch.from_numpy(cols).to(cuda)].float().cpu().numpy()
    ok, msg = allclose_report(got, ref)
    assert ok, msg
    del out, xq, xs, wq, ws, x, w

    m, n, k = 8448, 65536, 128
    announce(f"bf16 {m}x{n}x{k} f32 out: 2 GiB output in row chunks")
    xb = torch.randn((m, k), generator=g).to(torch.bfloat16).to(cuda)
    wb = torch.randn((n, k), generator=g).to(torch.bfloat16).to(cuda)
    out = torch.full((m, n), float("nan"), dtype=torch.float32, device=cuda)
    aiter_amd.gemm_a16w16_asm(xb, wb, out)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "output rows left unwritten"
    rows = np.array([0, 7935, 7936, m - 1])
    a_bits = xb[torch.from_numpy(rows).to(cuda)].view(torch.int16).cpu().numpy().view(np.uint16)
    b_bits = wb[torch.from_numpy(cols).to(cuda)].view(torch.int16).cpu().numpy().view(np.uint16)
    ref = O.bf16_bits_to_f32(a_bits) @ O.bf16_bits_to_f32(b_bits).T
    got = out[torch.from_numpy(rows).to(cuda)][:, torch.from_numpy(cols).to(cuda)].cpu().numpy()
    ok, msg = allclose_report(got, ref)
    assert ok, msg
