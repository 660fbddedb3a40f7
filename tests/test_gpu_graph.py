"""HIP graph capture of the entry points: each call is captured once, on a
stream whose library workspace an eager call has already sized, then the graph
is replayed several times with the program's own eager work and
synchronisations between replays; every replay must equal the eager result
(bit-exact; the end-to-end MoE path, whose stage 2 adds the slots with
packed-bf16 atomics in any order, within 8 bf16 ulps of the largest output:
a sum of bf16-rounded adds in another order moves by a few ulps of its
largest partial sum, which can exceed the result where terms cancel; a
missing or doubled contribution moves an element by the size of the
outputs)."""
import importlib

import numpy as np
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _replay_check(fn, cuda, exact=True):
    """fn() -> tensor (or tuple); eager on stream s, capture on s, replays."""
    s = torch.cuda.Stream(device=cuda)
    s.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(s):
        eager = fn()
        eager = tuple(t.clone() for t in eager) if isinstance(eager, tuple) else (eager.clone(),)
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = fn()
    out = out if isinstance(out, tuple) else (out,)
    junk = torch.randn(1 << 20, device=cuda)
    for rep in range(REPLAYS):
        for o in out:   # poison what the replay must rewrite
            if o.element_size() >= 2:
                o.fill_(0)
            else:
                o.view(torch.uint8).fill_(0xA5)
        junk.mul_(1.0001).add_(0.5)   # eager work between replays
        torch.cuda.synchronize(cuda)
        g.replay()
        torch.cuda.synchronize(cuda)
        for o, e in zip(out, eager):
            if exact:
                assert torch.equal(o.view(torch.uint8), e.view(torch.uint8)), f"replay {rep} differs"
            else:
                tol = 2.0 ** -5 * e.float().abs().max().item() + 1e-2
                err = (o.float() - e.float()).abs().max().item()
                assert err <= tol, f"replay {rep}: max difference {err} > {tol}"


def _mx(cuda, m, n, k, seed):
    import aiter_amd

    g = torch.Generator().manual_seed(seed)
    a = torch.randn((m, k), generator=g).to(torch.bfloat16).to(cuda)
    b = torch.randn((n, k), generator=g).to(torch.bfloat16).to(cuda)
    aq, as_ = aiter_amd.dynamic_mxfp4_quant(a, shuffle=True)
    bq, bs = aiter_amd.dynamic_mxfp4_quant(b, shuffle=True)
    return a, aq, as_, aiter_amd.shuffle_weight(bq), bs


@pytest.mark.parametrize("m,n,k,kname,l2", [(1, 7168, 2048, "", 0), (32, 1024, 4096, "a4w4_skinny_m32_splitk", 2),
                                           (300, 1024, 1024, "", 0), (1024, 1024, 512, "a4w4_tile_256x256_persist", 0),
                                           (64, 2048, 4096, "a4w4_tile_64x128_splitk", 2)])
def test_graph_gemm_a4w4(cuda, m, n, k, kname, l2):
    import aiter_amd

    announce(f"graph gemm_a4w4 {m}x{n}x{k} {kname or 'dispatch'} l2={l2}")
    _, aq, as_, bq, bs = _mx(cuda, m, n, k, 90)
    out = torch.empty(((m + 31) // 32 * 32, n), dtype=torch.bfloat16, device=cuda)

    def run():
        aiter_amd.gemm_a4w4_asm(aq, bq, as_, bs, out, kernelName=kname, log2_k_split=l2)
        return out[:m]   # rows past M are padding the kernel never writes

    _replay_check(run, cuda)


def test_graph_quant_and_lowp_outputs(cuda):
    import aiter_amd

    announce("graph dynamic_mxfp4_quant / gemm_a4w4o4 (fused epilogue) / gemm_a4w4o8")
    a, aq, as_, bq, bs = _mx(cuda, 4096, 4096, 256, 91)
    _replay_check(lambda: aiter_amd.dynamic_mxfp4_quant(a, shuffle=True), cuda)
    _replay_check(lambda: aiter_amd.gemm_a4w4o4(aq, bq, as_, bs), cuda)
    _replay_check(lambda: aiter_amd.gemm_a4w4o8(aq[:256], bq[:1024], as_[:256], bs[:1024]), cuda)


def test_graph_bf16_and_batched(cuda):
    import aiter_amd

    announce("graph gemm_a16w16 / batched_gemm_bf16")
    g = torch.Generator().manual_seed(92)
    x = torch.randn((32, 1024), generator=g).to(torch.bfloat16).to(cuda)
    w = torch.randn((2048, 1024), generator=g).to(torch.bfloat16).to(cuda)
    _replay_check(lambda: aiter_amd.gemm_a16w16(x, w), cuda)
    xb = torch.randn((4, 16, 512), generator=g).to(torch.bfloat16).to(cuda)
    wb = torch.randn((4, 256, 512), generator=g).to(torch.bfloat16).to(cuda)
    _replay_check(lambda: aiter_amd.batched_gemm_bf16_CK(xb, wb), cuda)


# model_dim 7168 at one token: stage 1 splits K, and the split that finishes a
# tile last sums it (tile counters that every replay must leave at zero)
@pytest.mark.parametrize("m,dim", [(1, 512), (300, 512), (1, 7168)])
def test_graph_fused_moe(cuda, m, dim):
    import aiter_amd

    announce(f"graph fused_moe m={m} dim={dim}")
    rng = np.random.default_rng(93 + m)
    e, topk, inter = 16, 4, 256
    ids = torch.from_numpy(np.stack([rng.choice(e, topk, replace=False) for _ in range(m)]).astype(np.int32)).to(cuda)
    wts = torch.from_numpy(rng.random((m, topk)).astype(np.float32)).to(cuda)

    def w_dev(rows, k):
        q = rng.integers(0, 256, (e * rows, k // 2), dtype=np.uint8)
        sc = rng.integers(119, 123, (e * rows, k // 32), dtype=np.uint8)
        return (torch.from_numpy(O.shuffle_weight(q).reshape(e, rows, k // 2)).to(cuda),
                torch.from_numpy(O.shuffle_scale(sc)).to(cuda))

    w1, s1 = w_dev(2 * inter, dim)
    w2, s2 = w_dev(dim, inter)
    x = torch.from_numpy(rng.standard_normal((m, dim)).astype(np.float32)).to(torch.bfloat16).to(cuda)
    _replay_check(lambda: aiter_amd.fused_moe(x, w1, w2, wts, ids, quant_type=aiter_amd.QuantType.per_1x32,
                                              w1_scale=s1, w2_scale=s2), cuda, exact=False)


@pytest.mark.parametrize("m", [1, 4])
def test_graph_moe_stage1_split_k(cuda, m):
    """Stage 1 at model_dim 7168 splits K (10 / 7 splits); the split that
    finishes a tile last sums it in split order, so every replay writes the
    eager call's bytes: the MXFP4 rows of every routed pair and the sorted
    scale rows below num_valid_ids[0]."""
    import aiter_amd
    from aiter_amd import dtypes

    FM = importlib.import_module("aiter_amd.fused_moe")
    announce(f"graph moe stage1 split-K m={m}")
    rng = np.random.default_rng(77 + m)
    e, topk, dim, inter, bs = 16, 9, 7168, 256, 32
    ids = torch.from_numpy(np.stack([rng.choice(e, topk, replace=False) for _ in range(m)]).astype(np.int32)).to(cuda)
    wts = torch.from_numpy(rng.random((m, topk)).astype(np.float32) + 0.05).to(cuda)
    q = rng.integers(0, 256, (e * 2 * inter, dim // 2), dtype=np.uint8)
    sc = rng.integers(119, 123, (e * 2 * inter, dim // 32), dtype=np.uint8)
    w1 = torch.from_numpy(O.shuffle_weight(q).reshape(e, 2 * inter, dim // 2)).to(cuda)
    w1s = torch.from_numpy(O.shuffle_scale(sc)).to(cuda)
    x = torch.from_numpy(rng.standard_normal((m, dim)).astype(np.float32)).to(torch.bfloat16).to(cuda)
    s, sw, se, nv, _ = FM.moe_sorting(ids, wts, e, dim, torch.bfloat16, bs, accumulate=False)
    a1, a1s = FM.fused_dynamic_mx_quant_moe_sort(x, s, nv, m, topk, bs, dtypes.fp4x2, sorted_weights=sw)
    torch.cuda.synchronize(cuda)
    rows = (int(nv[0].item()) + 31) // 32 * 32

    def run():
        q2, s2 = FM.ck_moe_stage1_fuse_quant(a1, w1, s, se, nv, m, topk, bs, w1s, a1s, None, sw, 0)
        return q2, s2[:rows]

    _replay_check(run, cuda)
