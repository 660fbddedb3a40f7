"""Seeded MX inputs shared by the parity tests (CPU-side generation through
the oracle; only the product path under test runs on the GPU)."""
from __future__ import annotations

import numpy as np

from oracle import mx_oracle as O


def randn(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


def to_bf16_f32(x: np.ndarray) -> np.ndarray:
    """Round f32 to the nearest bf16 value (kept as f32)."""
    return O.bf16_bits_to_f32(O.f32_to_bf16_bits(x))


def mxfp4_operand(rows, k, seed, mode=O.EVEN):
    """randn -> per-1x32 MXFP4 (packed, plain scale, shuffled scale)."""
    x = randn((rows, k), seed)
    if mode == "triton":
        q, s = O.quant_mxfp4_triton_even(x)
    else:
        q, s = O.quant_mxfp4(x, mode)
    return q, s, O.shuffle_scale(s)


def mxfp8_operand(rows, k, seed):
    x = randn((rows, k), seed)
    q, s = O.quant_mxfp8(x, O.EVEN)
    return q, s, O.shuffle_scale(s)


def bf16_operand(rows, k, seed):
    return O.f32_to_bf16_bits(randn((rows, k), seed))


def allclose_report(got: np.ndarray, ref: np.ndarray, rtol=1e-2, atol=1e-2):
    """(ok, message): every element within atol + rtol*|ref| (the north-star
    bf16 tolerance against the f32-accumulated dequantised matmul)."""
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    err = np.abs(got - ref)
    lim = atol + rtol * np.abs(ref)
    bad = err > lim
    n_bad = int(bad.sum())
    if n_bad == 0 and np.all(np.isfinite(got)):
        return True, ""
    idx = np.argwhere(bad)[:5]
    return False, (f"{n_bad}/{bad.size} elements out of tolerance; max err {err.max():.4g}; "
                   f"first {[tuple(i) + (got[tuple(i)], ref[tuple(i)]) for i in idx]}")


def tile_samples(n: int, band: int, seed: int) -> np.ndarray:
    """One index in every band of `band` consecutive indices of range(n)
    (random offset inside the band): a grid of row samples x column samples
    then touches every output tile of `band` x `band` or larger."""
    rs = np.random.default_rng(seed)
    starts = np.arange(0, n, band)
    return np.array([s + rs.integers(0, min(band, n - s)) for s in starts], dtype=np.int64)
