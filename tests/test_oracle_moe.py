"""Pins of the MoE oracle (oracle/moe_oracle.py) against facts its own
formulas do not restate: hand-worked known answers, invariants of the sort,
the closed-form scale index, torch's activation routines and float64
per-pair loops."""
import numpy as np
import pytest
import torch

from oracle import moe_oracle as MO
from oracle import mx_oracle as O


def _routing(m, e, topk, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.choice(e, topk, replace=False) for _ in range(m)]).astype(np.int32)
    w = rng.random((m, topk)).astype(np.float32) + 0.05
    return ids, w / w.sum(1, keepdims=True)


def test_sorting_known_answer():
    # 3 tokens, topk 2, 3 experts, block 2:
    #   token 0 -> experts (2, 0), token 1 -> (0, 1), token 2 -> (2, 1)
    ids = np.array([[2, 0], [0, 1], [2, 1]], dtype=np.int32)
    w = np.array([[0.1, 0.2], [0.3, 0.4], [0.5, 0.6]], dtype=np.float32)
    s, sw, se, nv = MO.moe_sorting_ref(ids, w, 3, 2)
    pad = (2 << 24) | 3
    # expert 0: (t0,s1), (t1,s0); expert 1: (t1,s1), (t2,s1); expert 2: (t0,s0), (t2,s0)
    want = [(1 << 24) | 0, 1, (1 << 24) | 1, (1 << 24) | 2, 0, 2]
    assert s[:6].tolist() == want
    assert (s[6:] == pad).all()
    np.testing.assert_array_equal(sw[:6], np.float32([0.2, 0.3, 0.4, 0.6, 0.1, 0.5]))
    assert se[:3].tolist() == [0, 1, 2] and (se[3:] == -1).all()
    assert nv.tolist() == [6, 3]
    # mask expert 1: expert 2 becomes local id 1; odd counts pad to 2
    s, sw, se, nv = MO.moe_sorting_ref(ids, w, 3, 2, expert_mask=np.array([1, 0, 1]))
    assert s[:4].tolist() == [(1 << 24) | 0, 1, 0, 2] and nv.tolist() == [4, 3]
    assert se[:2].tolist() == [0, 1]
    # num_local_tokens = 1: only token 0; expert 0 run of 1 padded to 2
    s, _, se, nv = MO.moe_sorting_ref(ids, w, 3, 2, num_local_tokens=1)
    assert s[:4].tolist() == [(1 << 24) | 0, pad, 0, pad] and se[:2].tolist() == [0, 2] and nv.tolist() == [4, 1]


@pytest.mark.parametrize("m,e,topk,bs", [(1, 257, 9, 32), (37, 16, 4, 32), (300, 64, 8, 64), (128, 8, 2, 128)])
def test_sorting_invariants(m, e, topk, bs):
    ids, w = _routing(m, e, topk, m + e)
    s, sw, se, nv = MO.moe_sorting_ref(ids, w, e, bs)
    total = int(nv[0])
    assert total % bs == 0 and nv[1] == m
    live = s[:total]
    tok, slot = live & 0xFFFFFF, live >> 24
    real = tok < m
    # every routed pair exactly once
    pairs = sorted(zip(tok[real].tolist(), slot[real].tolist()))
    assert pairs == sorted((t, k) for t in range(m) for k in range(topk))
    # each block holds one expert; entries of that expert in row-major order
    for b in range(total // bs):
        blk = live[b * bs:(b + 1) * bs]
        bt, bsl = blk & 0xFFFFFF, blk >> 24
        r = bt < m
        assert (ids[bt[r], bsl[r]] == se[b]).all()
        key = bt[r] * topk + bsl[r]
        assert (np.diff(key) > 0).all()
        # padding only at the end of an expert's run
        if not r.all():
            assert (~r[np.argmin(r):]).all()
    np.testing.assert_array_equal(sw[:total][real], w[tok[real], slot[real]])
    # experts appear in increasing order and blocks past the total are -1
    used = se[: total // bs]
    assert (np.diff(used) >= 0).all() and (se[total // bs:] == -1).all()


def test_source_rows_known_answer():
    ids = np.array([(1 << 24) | 2, 0, (3 << 24) | 5, (2 << 24) | 7], dtype=np.int32)
    rows, valid = MO.sorted_source_rows(ids, 3, 7, 4)
    assert valid.tolist() == [True, True, True, False]
    assert rows[:3].tolist() == [2 * 4 + 1, 0, 5 * 4 + 3]
    rows1, valid1 = MO.sorted_source_rows(ids, 4, 7, 1)
    assert rows1[:3].tolist() == [2, 0, 5] and valid1.tolist() == [True, True, True, False]


def test_sort_scale_matches_closed_form_index():
    ids, w = _routing(40, 12, 3, 5)
    s, _, _, nv = MO.moe_sorting_ref(ids, w, 12, 32)
    rng = np.random.default_rng(6)
    scale_rows = rng.integers(1, 255, (40 * 3, 10), dtype=np.uint8)   # K/32 = 10 -> padded to 16
    got = MO.sort_scale_ref(scale_rows, s, int(nv[0]), 40, 3)
    want = np.zeros_like(got)
    rows, valid = MO.sorted_source_rows(s, int(nv[0]), 40, 3)
    for x in range(len(s)):
        for y in range(16):
            b = scale_rows[rows[x], y] if (valid[x] and y < 10) else 0
            want.reshape(-1)[O.mx_scale_shuffle_idx(16, x, y)] = b
    np.testing.assert_array_equal(got, want)


def test_act_matches_torch():
    g = np.linspace(-12, 12, 2001, dtype=np.float32)
    t = torch.from_numpy(g)
    np.testing.assert_allclose(MO.act_ref(g, MO.SILU), torch.nn.functional.silu(t).numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(MO.act_ref(g, MO.GELU), torch.nn.functional.gelu(t).numpy(), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("doweight", [False, True])
def test_stages_match_pair_loop(doweight):
    rng = np.random.default_rng(7)
    m, e, topk, k, inter, d = 9, 5, 3, 64, 32, 48
    ids, w = _routing(m, e, topk, 8)
    a = rng.standard_normal((m, k)).astype(np.float32)
    w1 = rng.standard_normal((e, 2 * inter, k)).astype(np.float32)
    w2 = rng.standard_normal((e, d, inter)).astype(np.float32)
    h = MO.moe_stage1_ref(a, w1, ids, w, MO.SILU, doweight)
    y = MO.moe_stage2_ref(h, w2, ids, w, not doweight)
    hw = np.zeros((m, topk, inter))
    yw = np.zeros((m, d))
    for t in range(m):
        for s in range(topk):
            x = w1[ids[t, s]].astype(np.float64) @ a[t].astype(np.float64)
            if doweight:
                x = x * w[t, s]
            g, u = x[:inter], x[inter:]
            hw[t, s] = g / (1 + np.exp(-g)) * u
            o = w2[ids[t, s]].astype(np.float64) @ h[t, s].astype(np.float64)
            yw[t] += o * (1.0 if doweight else w[t, s])
    np.testing.assert_allclose(h, hw, rtol=1e-4, atol=1e-3)
    np.testing.assert_allclose(y, yw, rtol=1e-4, atol=1e-2)


def test_quant_sort_is_row_quant_plus_sort():
    rng = np.random.default_rng(9)
    ids, w = _routing(20, 6, 2, 10)
    s, sw, _, nv = MO.moe_sorting_ref(ids, w, 6, 32)
    x = rng.standard_normal((40, 64)).astype(np.float32)
    q, written, ss = MO.quant_sort_ref(x, s, int(nv[0]), 20)
    q0, s0 = O.quant_mxfp4(x, O.ROUND_UP, amax_floor=1e-10)
    assert written.all()
    np.testing.assert_array_equal(q, q0)
    np.testing.assert_array_equal(ss, MO.sort_scale_ref(s0, s, int(nv[0]), 20, 2))
