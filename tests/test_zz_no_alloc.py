"""gemm_a4w4_asm_noalloc (the entry point that allocates nothing; split-K
partials in a fixed per-GPU scratch array) against gemm_a4w4_asm on the same
inputs: bit-identical outputs (same kernels, same split, same summation
order), on two calls in a row, the second with smaller shapes, for the
skinny split-K kernel (heuristic) and a split tile kernel; sizes beyond the
scratch raise."""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, mxfp4_operand

pytestmark = pytest.mark.gpu


def _case(m, n, k, seed, cuda):
    a_q, a_s, a_ss = mxfp4_operand(m, k, seed, "triton")
    b_q, b_s, b_ss = mxfp4_operand(n, k, seed + 1, "triton")
    ref = O.bf16_bits_to_f32(O.gemm_a4w4_ref(a_q, b_q, a_s, b_s))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(cuda)
    return dev(a_q), dev(O.shuffle_weight(b_q)), dev(a_ss), dev(b_ss), ref


def _both(cuda, m, n, k, seed, name, log2_split):
    from aiter_amd._lib import call

    A, B, As, Bs, ref = _case(m, n, k, seed, cuda)
    outs = []
    for fn in ("gemm_a4w4_asm", "gemm_a4w4_asm_noalloc"):
        out = torch.full(((m + 31) // 32 * 32, n), float("nan"), dtype=torch.bfloat16, device=cuda)
        call(fn, A, B, As, Bs, out, name or None, None, 1.0, 0.0, 1, log2_split)
        outs.append(out[:m])
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), f"{name or 'heuristic'} {m}x{n}x{k}: no-alloc output differs"
    ok, msg = allclose_report(outs[1].float().cpu().numpy(), ref)
    assert ok, msg


@pytest.mark.parametrize("name,log2_split,big,small", [
    ("", 0, (16, 2048, 16384), (8, 1024, 8192)),                      # skinny split-K (heuristic)
    ("a4w4_tile_64x128_splitk", 2, (64, 1024, 4096), (40, 512, 2048)),  # split tile + reduce
])
def test_no_alloc_matches_gemm_a4w4_asm(cuda, name, log2_split, big, small):
    for i, (m, n, k) in enumerate((big, small)):
        announce(f"no-alloc {name or 'heuristic'} call {i} {m}x{n}x{k}")
        _both(cuda, m, n, k, 70 + i, name, log2_split)


def test_no_alloc_rejects_oversized_partials(cuda):
    from aiter_amd._lib import call, lib

    cap = lib().gemm_a4w4_noalloc_scratch_bytes()
    assert cap == 32 << 20
    m, n, k = 64, 16384, 4096          # 16 slices x 64 x 16384 x 4 B = 64 MiB of partials
    announce(f"no-alloc oversized {m}x{n}x{k}")
    A, B, As, Bs, _ = _case(m, n, k, 90, cuda)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(RuntimeError, match="scratch"):
        call("gemm_a4w4_asm_noalloc", A, B, As, Bs, out, "a4w4_tile_64x128_splitk", None, 1.0, 0.0, 1, 4)


def test_no_alloc_reserves_nothing_and_captures(cuda):
    """The no-allocation entry never touches the library workspace: on a
    stream whose workspace was released it leaves the workspace at 0 bytes
    (gemm_a4w4_asm on another released stream reserves its split-K partials
    there, which shows the probe sees a reservation), and it captures in a
    HIP graph on that stream, where a workspace reservation would raise;
    every replay equals the eager output."""
    from aiter_amd._lib import call, lib

    m, n, k = 16, 2048, 16384     # skinny split-K (heuristic): partials needed
    announce(f"no-alloc workspace probe and graph capture {m}x{n}x{k}")
    A, B, As, Bs, ref = _case(m, n, k, 95, cuda)
    dev = cuda.index or 0
    pad = (m + 31) // 32 * 32

    s_lib = torch.cuda.Stream()
    with torch.cuda.stream(s_lib):
        out_lib = torch.empty((pad, n), dtype=torch.bfloat16, device=cuda)
        assert lib().aiter_amd_workspace_release(dev, s_lib.cuda_stream) == 0
        call("gemm_a4w4_asm", A, B, As, Bs, out_lib, None, None, 1.0, 0.0, 1, 0)
        s_lib.synchronize()
    assert lib().aiter_amd_workspace_bytes(dev, s_lib.cuda_stream) > 0

    s = torch.cuda.Stream()
    assert s.cuda_stream != s_lib.cuda_stream
    with torch.cuda.stream(s):
        eager = torch.full((pad, n), float("nan"), dtype=torch.bfloat16, device=cuda)
        assert lib().aiter_amd_workspace_release(dev, s.cuda_stream) == 0
        call("gemm_a4w4_asm_noalloc", A, B, As, Bs, eager, None, None, 1.0, 0.0, 1, 0)
        s.synchronize()
        assert lib().aiter_amd_workspace_bytes(dev, s.cuda_stream) == 0
        out = torch.full((pad, n), float("nan"), dtype=torch.bfloat16, device=cuda)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            call("gemm_a4w4_asm_noalloc", A, B, As, Bs, out, None, None, 1.0, 0.0, 1, 0)
        for i in range(3):
            out.fill_(float("nan"))
            g.replay()
            s.synchronize()
            assert torch.equal(out[:m], eager[:m]), f"replay {i} differs from the eager no-alloc output"
        assert lib().aiter_amd_workspace_bytes(dev, s.cuda_stream) == 0
    assert torch.equal(eager[:m], out_lib[:m])
    ok, msg = allclose_report(eager[:m].float().cpu().numpy(), ref)
    assert ok, msg
