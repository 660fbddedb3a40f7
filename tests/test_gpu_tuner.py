"""The tuner end to end on the GPU: one small shape per family is tuned in
this process (the worker that the driver runs per shape,
aiter/utility/base_tuner.py:1573-1595 writes the same per-shape rows), the
row is written to a temporary tuned CSV, the library's dispatch is pointed at
that CSV (``AITER_CONFIG_GEMM_A4W4`` / ``AITER_CONFIG_GEMM_BF16``) and must
pick the winner, and the winner's output is checked against the oracle."""
import pandas as pd
import pytest
import torch

from tests.conftest import announce
from tests.test_gpu_configs import _a4w4_on_the_fly, _randn_bf16
from tests.test_gpu_reference_csv import _bf16_check, _clear

pytestmark = pytest.mark.gpu


def test_tune_a4w4_shape_then_dispatch(cuda, tmp_path, monkeypatch):
    import aiter_amd
    from aiter_amd import tuner
    from aiter_amd._lib import kernel_names

    m, n, k = 48, 512, 1024
    path = tmp_path / "a4w4_tuned.csv"
    announce(f"tune a4w4 {m}x{n}x{k}")
    assert tuner.worker("a4w4", (m, n, k), str(path), 3, 0.05, False, 3.0) == 0
    df = pd.read_csv(path)
    assert len(df) == 1
    row = df.iloc[0]
    assert (int(row.M), int(row.N), int(row.K)) == (m, n, k)
    assert row.kernelName in kernel_names() and row.us > 0 and row.errRatio <= 0.05
    # a rerun of the same shape replaces its row (the winner may differ: timing)
    assert tuner.worker("a4w4", (m, n, k), str(path), 3, 0.05, False, 3.0) == 0
    df = pd.read_csv(path)
    assert len(df) == 1
    row = df.iloc[0]

    monkeypatch.setenv("AITER_CONFIG_GEMM_A4W4", str(path))
    _clear()
    try:
        cfg = aiter_amd.get_GEMM_config(m, n, k)
        assert cfg is not None and cfg["kernelName"] == row.kernelName
        announce(f"tuned a4w4 {m}x{n}x{k} {row.kernelName}")
        _a4w4_on_the_fly(m, n, k, 71, cuda, what=f"tuned {row.kernelName}")
    finally:
        _clear()


def test_tune_bf16_shape_then_dispatch(cuda, tmp_path, monkeypatch):
    import aiter_amd
    from aiter_amd import tuner
    from aiter_amd._lib import kernel_names

    m, n, k = 96, 512, 512
    path = tmp_path / "bf16_tuned.csv"
    announce(f"tune bf16 {m}x{n}x{k}")
    assert tuner.worker("a16w16", (m, n, k, False, "torch.bfloat16", False), str(path), 3, 0.05, False, 3.0) == 0
    df = pd.read_csv(path)
    assert len(df) == 1
    row = df.iloc[0]
    assert (int(row.M), int(row.N), int(row.K)) == (m, n, k) and row.libtype == "aiter_amd"
    assert row.kernelName in kernel_names()

    monkeypatch.setenv("AITER_CONFIG_GEMM_BF16", str(path))
    _clear()
    try:
        cfg = aiter_amd.get_GEMM_A16W16_config(m, n, k, False, "torch.bfloat16", "torch.bfloat16", False, False)
        assert cfg is not None and cfg["kernelName"] == row.kernelName
        announce(f"tuned bf16 {m}x{n}x{k} {row.kernelName}")
        x = _randn_bf16(m, k, 81, cuda)
        w = _randn_bf16(n, k, 82, cuda)
        out = aiter_amd.gemm_a16w16(x, w)
        torch.cuda.synchronize()
        _bf16_check(out, x, w, m, n, 83)
    finally:
        _clear()
