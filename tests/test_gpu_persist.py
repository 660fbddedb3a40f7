"""The persistent tile instances (``*_persist``) against their one-tile-per-
workgroup twins: the same MFMAs in the same order per tile, so outputs must be
bit-identical.  Shapes cover fewer tiles than CUs, uneven tile counts over
the workgroups (some take one tile more), partial edge tiles in M and N, K
padded with zero stages, alpha != 1, and bias (which the host routes to the
twin).  Parity of the twins themselves with the oracle is tested elsewhere;
one small case per family here also checks the persistent kernel against
the oracle directly.
"""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, bf16_operand, mxfp4_operand

pytestmark = pytest.mark.gpu


def _persist_rows():
    try:
        from aiter_amd._lib import kernel_table

        # bf16-output forms (the f32-output one is tested by name in test_gpu_lowp_out.py)
        return [r for r in kernel_table() if r[1].endswith("_persist") and not r[9]]
    except Exception:  # library not built: collected, then skipped by the cuda fixture
        return []


ROWS = _persist_rows()
IDS = [r[1] for r in ROWS]


def _k_stage(fam):
    return 64 if fam == "a16w16" else 256


def _shapes(row):
    fam, bm = row[2], row[4]
    ks = _k_stage(fam)
    return [
        (bm * 20 - 40, 256 * 16 - 16, 5 * ks),  # 320 tiles (more than the CUs), 5 stages -> 8
        (bm * 3, 256 * 2, 10 * ks),              # 6 tiles, 10 stages -> 12
        (bm * 32, 256 * 16, 8 * ks),             # 512 tiles: two per workgroup
        (bm * 20 - 40, 256 * 16 - 16, 3 * ks),   # 320 tiles, 3 stages -> one 4-stage tile each
        (bm * 32, 256 * 16, 4 * ks),             # 512 tiles of 4 stages: two per workgroup
        (bm * 3, 256 * 2, 1 * ks),               # 6 tiles of 1 stage -> 4
    ]


def _operands(fam, m, n, k, cuda, seed):
    """Random operands in the kernels' layouts (any byte pattern is a valid
    e2m1 pair; e4m3 from a cast; e8m0 scales in a tame range)."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    if fam == "a16w16":
        a = torch.randn((m, k), generator=g).to(torch.bfloat16).to(cuda)
        b = torch.randn((n, k), generator=g).to(torch.bfloat16).to(cuda)
        return a, b, None, None
    if fam == "a4w4":
        a = torch.randint(0, 256, (m, k // 2), generator=g, dtype=torch.uint8).to(cuda)
    else:
        a = torch.randn((m, k), generator=g).clamp(-400, 400).to(torch.float8_e4m3fn).view(torch.uint8).to(cuda)
    b = torch.randint(0, 256, (n, k // 2), generator=g, dtype=torch.uint8).to(cuda)
    sa = torch.randint(118, 136, ((m + 255) // 256 * 256, k // 32), generator=g, dtype=torch.uint8).to(cuda)
    sb = torch.randint(118, 136, ((n + 255) // 256 * 256, k // 32), generator=g, dtype=torch.uint8).to(cuda)
    return a, b, sa, sb


def _run(fam, name, a, b, sa, sb, m, n, cuda, bias=None, alpha=1.0, b_pre=True):
    import aiter_amd

    if fam == "a4w4":
        out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
        aiter_amd.gemm_a4w4_asm(a, b, sa, sb, out, kernelName=name, bias=bias, alpha=alpha,
                                beta=1.0 if bias is not None else 0.0, bpreshuffle=b_pre)
    elif fam == "a8w4":
        out = aiter_amd.gemm_a8w4_mxfp8(a.view(torch.float8_e4m3fn), b, sa, sb, a_preshuffle=False, kernelName=name)
    else:
        out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
        aiter_amd.gemm_a16w16_asm(a, b, out, bias=bias, kernelName=name, bpreshuffle=b_pre)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("row", ROWS, ids=IDS)
def test_persist_matches_twin(cuda, row):
    name, fam, b_pre = row[1], row[2], bool(row[8])
    # the one-tile-per-workgroup kernel of the same tile (the LDS-staged bf16
    # tile's twin is the plain tile name of its B layout)
    twin = name[: -len("_persist")].replace("_lds", "")
    for i, (m, n, k) in enumerate(_shapes(row)):
        announce(f"persist {name} vs {twin} {m}x{n}x{k}")
        a, b, sa, sb = _operands(fam, m, n, k, cuda, seed=40 + i)
        got = _run(fam, name, a, b, sa, sb, m, n, cuda, b_pre=b_pre)
        want = _run(fam, twin, a, b, sa, sb, m, n, cuda, b_pre=b_pre)
        assert torch.equal(got, want), f"{name} {m}x{n}x{k}: differs from {twin}"
        # a second call reuses nothing: same result again
        assert torch.equal(_run(fam, name, a, b, sa, sb, m, n, cuda, b_pre=b_pre), want)


def test_persist_alpha_and_bias(cuda):
    """alpha != 1 goes through the persistent epilogue; a bias routes to the twin."""
    name, twin = "a4w4_tile_256x256_persist", "a4w4_tile_256x256"
    m, n, k = 256 * 18, 256 * 16, 2048
    announce(f"persist alpha/bias {name} {m}x{n}x{k}")
    a, b, sa, sb = _operands("a4w4", m, n, k, cuda, seed=50)
    got = _run("a4w4", name, a, b, sa, sb, m, n, cuda, alpha=0.375)
    want = _run("a4w4", twin, a, b, sa, sb, m, n, cuda, alpha=0.375)
    assert torch.equal(got, want)
    bias = torch.randn((1, n), generator=torch.Generator().manual_seed(51)).to(cuda)
    got = _run("a4w4", name, a, b, sa, sb, m, n, cuda, bias=bias, alpha=0.5)
    want = _run("a4w4", twin, a, b, sa, sb, m, n, cuda, bias=bias, alpha=0.5)
    assert torch.equal(got, want)


def _dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def test_persist_against_oracle_a4w4(cuda):
    import aiter_amd

    m, n, k = 600, 1008, 1280   # 3 x 4 tiles of 256x256, partial in both, 5 stages -> 8
    announce(f"persist a4w4 vs oracle {m}x{n}x{k}")
    a_q, a_s, a_ss = mxfp4_operand(m, k, 60, "triton")
    b_q, b_s, b_ss = mxfp4_operand(n, k, 61, "triton")
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q, b_q, a_s, b_s))
    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda), _dev(b_ss, cuda),
                            out, kernelName="a4w4_tile_256x256_persist")
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, msg


def test_persist_four_stage_tiles_against_oracle(cuda):
    """K = 1024 (4 stages: the tile's first four stages are its last four) with
    more tiles than workgroups, each workgroup walking several tiles."""
    import aiter_amd

    m, n, k = 4096 + 200, 4096 - 16, 1024
    announce(f"persist a4w4 4-stage tiles vs oracle {m}x{n}x{k}")
    a_q, a_s, a_ss = mxfp4_operand(m, k, 64, "triton")
    b_q, b_s, b_ss = mxfp4_operand(n, k, 65, "triton")
    rows = np.unique(np.concatenate([np.arange(0, m, 97), [m - 1]]))
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q[rows], b_q, a_s[rows], b_s))
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a4w4_asm(_dev(a_q, cuda), _dev(O.shuffle_weight(b_q), cuda), _dev(a_ss, cuda), _dev(b_ss, cuda),
                            out, kernelName="a4w4_tile_256x256_persist")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()), "output left unwritten"
    ok, msg = allclose_report(out[torch.from_numpy(rows).to(cuda)].float().cpu().numpy(), ref)
    assert ok, msg


def test_persist_against_oracle_a16w16(cuda):
    import aiter_amd

    m, n, k = 300, 592, 640    # 2 x 3 tiles of 256x256 (bf16), 10 stages -> 12
    announce(f"persist a16w16 vs oracle {m}x{n}x{k}")
    a = bf16_operand(m, k, 62)
    b = bf16_operand(n, k, 63)
    ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T))
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev(O.shuffle_weight(b).view(np.int16), cuda).view(torch.bfloat16)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a16w16_asm(at, bt, out, kernelName="a16w16_tile_256x256_persist", bpreshuffle=True)
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, msg
