"""The product's torch layouts (aiter_amd/shuffle.py) byte for byte against
the oracle's index formulas (oracle/mx_oracle.py, pinned in test_oracle.py),
on the CPU: e2m1 / e4m3 bytes, bf16 (2-byte elements, 8-element chunks),
K padding, batched (expert) weights and the e8m0 scale swizzle."""
import numpy as np
import pytest
import torch

import aiter_amd
from oracle import mx_oracle as O


@pytest.mark.parametrize("n,kb", [(16, 32), (48, 96), (64, 256)])
def test_shuffle_weight_bytes(n, kb):
    w = np.random.default_rng(n + kb).integers(0, 256, (n, kb), dtype=np.uint8)
    got = aiter_amd.shuffle_weight(torch.from_numpy(w))
    assert got.dtype == torch.uint8 and tuple(got.shape) == (n, kb)
    assert getattr(got, "is_shuffled", False)
    np.testing.assert_array_equal(got.numpy(), O.shuffle_weight(w))


def test_shuffle_weight_fp4x2_and_fp8_dtypes_keep_their_dtype():
    w = np.random.default_rng(3).integers(0, 256, (32, 64), dtype=np.uint8)
    for dt in (aiter_amd.dtypes.fp4x2, aiter_amd.dtypes.fp8):
        t = torch.from_numpy(w).view(dt)
        got = aiter_amd.shuffle_weight(t)
        assert got.dtype == dt
        np.testing.assert_array_equal(got.view(torch.uint8).numpy(), O.shuffle_weight(w))


@pytest.mark.parametrize("n,k", [(16, 32), (32, 64), (48, 128)])
def test_shuffle_weight_bf16_bytes(n, k):
    bits = np.random.default_rng(n * k).integers(0, 2 ** 16, (n, k), dtype=np.uint16)
    t = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16)
    got = aiter_amd.shuffle_weight(t)
    assert got.dtype == torch.bfloat16
    np.testing.assert_array_equal(got.view(torch.int16).numpy().view(np.uint16), O.shuffle_weight(bits))


def test_shuffle_weight_batched_experts():
    """[E, N, K] weights shuffle expert by expert (the MoE weights)."""
    w = np.random.default_rng(4).integers(0, 256, (3, 32, 64), dtype=np.uint8)
    got = aiter_amd.shuffle_weight(torch.from_numpy(w)).numpy()
    for e in range(3):
        np.testing.assert_array_equal(got[e], O.shuffle_weight(w[e]))


def test_shuffle_weight_pad_k():
    """pad_k_to pads K with zero bytes to the next multiple, then shuffles;
    the original and padded K ride on the result."""
    w = np.random.default_rng(5).integers(0, 256, (16, 80), dtype=np.uint8)
    got = aiter_amd.shuffle_weight(torch.from_numpy(w), pad_k_to=64)
    assert tuple(got.shape) == (16, 128)
    assert got.aiter_original_k == 80 and got.aiter_padded_k == 128
    padded = np.zeros((16, 128), dtype=np.uint8)
    padded[:, :80] = w
    np.testing.assert_array_equal(got.numpy(), O.shuffle_weight(padded))
    same = aiter_amd.shuffle_weight(torch.from_numpy(padded), pad_k_to=64)
    np.testing.assert_array_equal(same.numpy(), got.numpy())
    with pytest.raises(ValueError):
        aiter_amd.shuffle_weight(torch.from_numpy(w), pad_k_to=-1)


def test_shuffle_weight_rejects_partial_blocks():
    with pytest.raises(AssertionError):
        aiter_amd.shuffle_weight(torch.zeros((24, 64), dtype=torch.uint8))
    with pytest.raises(AssertionError):
        aiter_amd.shuffle_weight(torch.zeros((16, 48), dtype=torch.uint8))


@pytest.mark.parametrize("rows,cols", [(1, 1), (33, 5), (256, 64), (300, 130)])
def test_shuffle_scale_bytes(rows, cols):
    s = np.random.default_rng(rows * cols).integers(0, 256, (rows, cols), dtype=np.uint8)
    got = aiter_amd.shuffle_scale(torch.from_numpy(s).view(aiter_amd.dtypes.fp8_e8m0))
    want = O.shuffle_scale(s, fill=0)
    assert tuple(got.shape) == want.shape
    np.testing.assert_array_equal(got.view(torch.uint8).numpy(), want)


def test_shuffle_scale_passes_f32_and_none():
    f = torch.ones((4, 4), dtype=torch.float32)
    assert aiter_amd.shuffle_scale(f) is f
    assert aiter_amd.shuffle_scale(None) is None
