"""Stream-K skinny bf16 kernels (row-major B through LDS, `*_lds_sk`): every
output element against the f32 matmul of the same bf16 operands (rtol = atol =
1e-2), in each regime of the unit split over the CUs:

* fewer units than CUs (one workgroup per unit, every block a fold of many);
* the decode shape N = 7168, K = 2048 (224 blocks on 256 CUs: blocks split
  over two ranges);
* ranges over several blocks (windows of two blocks, whole blocks stored
  directly between partial ones);
* a last 32-column block half past N;

each called twice in a row into a NaN-filled output (the first call's
arrival counters must be back at zero for the second to be right), and
captured in a HIP graph whose replays must equal the eager bytes (the fold
adds the ranges' partials in range order, whichever arrives last)."""
import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report, bf16_operand

pytestmark = pytest.mark.gpu

SK = {1: "a16w16_skinny_m16_n32_bplain_lds_sk", 2: "a16w16_skinny_m32_n32_bplain_lds_sk",
      4: "a16w16_skinny_m64_n32_bplain_lds_sk"}

# (M, N, K): units = ceil(N / 32) * K / 64 against 256 CUs
SHAPES = [(1, 32, 128), (16, 48, 256), (32, 7168, 2048), (1, 7168, 2048), (64, 7168, 2048),
          (9, 28672, 512), (32, 14336, 4096), (40, 2064, 1024), (3, 4096, 7168)]


def _dev(x, cuda):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda)


def _case(cuda, m, n, k, seed):
    a = bf16_operand(m, k, seed)
    b = bf16_operand(n, k, seed + 1)
    ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T))
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev(b.view(np.int16), cuda).view(torch.bfloat16)
    return at, bt, ref


def _name(m):
    return SK[1 if m <= 16 else (2 if m <= 32 else 4)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_stream_k_matches_reference(cuda, m, n, k):
    import aiter_amd

    name = _name(m)
    announce(f"stream-K {name} {m}x{n}x{k}")
    at, bt, ref = _case(cuda, m, n, k, 41 + m)
    out = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda)
    for call in range(2):
        out.fill_(float("nan"))
        aiter_amd.gemm_a16w16_asm(at, bt, out, kernelName=name, bpreshuffle=False)
        torch.cuda.synchronize()
        ok, msg = allclose_report(out.float().cpu().numpy(), ref)
        assert ok, f"call {call}: {msg}"


def test_stream_k_after_other_shapes(cuda):
    """Back-to-back calls of different shapes on one stream (the counters of
    one call's blocks are the next call's), then the first shape again."""
    import aiter_amd

    announce("stream-K back to back")
    cases = [(32, 7168, 2048), (16, 48, 256), (9, 28672, 512), (32, 7168, 2048)]
    data = [_case(cuda, m, n, k, 90 + i) for i, (m, n, k) in enumerate(cases)]
    outs = [torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=cuda) for (m, n, k) in cases]
    for (m, n, k), (at, bt, _), o in zip(cases, data, outs):
        aiter_amd.gemm_a16w16_asm(at, bt, o, kernelName=_name(m), bpreshuffle=False)
    torch.cuda.synchronize()
    for (m, n, k), (_, _, ref), o in zip(cases, data, outs):
        ok, msg = allclose_report(o.float().cpu().numpy(), ref)
        assert ok, f"{m}x{n}x{k}: {msg}"


def test_stream_k_bias(cuda):
    """The bias added by both stores (a whole block's and the fold's)."""
    import aiter_amd

    m, n, k = 32, 7168, 2048
    announce(f"stream-K bias {m}x{n}x{k}")
    a = bf16_operand(m, k, 7)
    b = bf16_operand(n, k, 8)
    bias = np.random.default_rng(9).standard_normal(n).astype(np.float32)
    c = O.bf16_bits_to_f32(a) @ O.bf16_bits_to_f32(b).T + bias
    ref = O.bf16_bits_to_f32(O.f32_to_bf16_bits(c))
    at = _dev(a.view(np.int16), cuda).view(torch.bfloat16)
    bt = _dev(b.view(np.int16), cuda).view(torch.bfloat16)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
    aiter_amd.gemm_a16w16_asm(at, bt, out, bias=_dev(bias, cuda), kernelName=_name(m), bpreshuffle=False)
    torch.cuda.synchronize()
    ok, msg = allclose_report(out.float().cpu().numpy(), ref)
    assert ok, msg


@pytest.mark.parametrize("m,n,k", [(32, 7168, 2048), (16, 48, 256), (9, 28672, 512)])
def test_stream_k_graph_replays(cuda, m, n, k):
    import aiter_amd

    name = _name(m)
    announce(f"stream-K graph {name} {m}x{n}x{k}")
    at, bt, _ = _case(cuda, m, n, k, 60 + m)
    out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(s):
        aiter_amd.gemm_a16w16_asm(at, bt, out, kernelName=name, bpreshuffle=False)
    torch.cuda.synchronize(cuda)
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        aiter_amd.gemm_a16w16_asm(at, bt, out, kernelName=name, bpreshuffle=False)
    junk = torch.randn(1 << 20, device=cuda)
    for rep in range(3):
        out.fill_(0)
        junk.mul_(1.0001).add_(0.5)
        torch.cuda.synchronize(cuda)
        g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {rep} differs"


def test_stream_k_refuses_batch(cuda):
    from aiter_amd._lib import kernel_table
    from aiter_amd.batched_gemm_op_bf16 import batched_gemm_bf16_tune

    announce("stream-K refuses a batch")
    kid = [r[0] for r in kernel_table() if r[1] == SK[1]][0]
    x = torch.randn((2, 16, 256), device=cuda).to(torch.bfloat16)
    w = torch.randn((2, 64, 256), device=cuda).to(torch.bfloat16)
    out = torch.empty((2, 16, 64), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(RuntimeError, match="stream-K"):
        batched_gemm_bf16_tune(x, w, out, kid)
