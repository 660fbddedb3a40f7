"""Tuned-CSV drop-in: rows of the reference's own tuned CSVs served by this
library, checked against the oracle.

* ``AITER_CONFIG_GEMM_A4W4`` points at tests/golden/reference_a4w4_rows.csv
  (rows of the reference's aiter/configs/a4w4_blockscale_tuned_gemm.csv: ASM
  tile names this library has and lacks, CK instance names routed through
  ``gemm_a4w4_blockscale`` as aiter/ops/gemm_op_a4w4.py:207-221 does, and one
  name of no kernel at all, which warns and takes the heuristic);
* reference opus kernel ids (csrc/opus_gemm/opus_gemm_common.py:238-513)
  through ``gemm_a16w16_opus(kernelId=...)`` and a tuned bf16 row with
  libtype ``opus`` / ``asm``.
"""
import logging
import os

import numpy as np
import pandas as pd
import pytest
import torch

from oracle import mx_oracle as O
from tests.conftest import announce
from tests.mx_inputs import allclose_report
from tests.test_gpu_configs import _a4w4_on_the_fly, _randn_bf16, _sample, _take_rows

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
ROWS = pd.read_csv(os.path.join(GOLDEN, "reference_a4w4_rows.csv"))


def _clear():
    from aiter_amd import config, gemm_op_a4w4, tuned_gemm

    config.get_gfx.cache_clear()
    config.get_cu_num.cache_clear()
    gemm_op_a4w4._a4w4_table.cache_clear()
    gemm_op_a4w4.get_GEMM_config.cache_clear()
    tuned_gemm._bf16_table.cache_clear()
    tuned_gemm.get_GEMM_A16W16_config.cache_clear()


@pytest.fixture
def reference_a4w4_csv(monkeypatch):
    monkeypatch.setenv("AITER_CONFIG_GEMM_A4W4", os.path.join(GOLDEN, "reference_a4w4_rows.csv"))
    monkeypatch.setenv("GPU_ARCHS", "gfx950")
    monkeypatch.setenv("CU_NUM", "256")
    _clear()
    yield
    _clear()


@pytest.mark.parametrize("m,n,k,name", [tuple(r) for r in ROWS[["M", "N", "K", "kernelName"]].values])
def test_gemm_a4w4_reference_rows(cuda, reference_a4w4_csv, caplog, m, n, k, name):
    import aiter_amd

    cfg = aiter_amd.get_GEMM_config(int(m), int(n), int(k))
    assert cfg is not None and cfg["kernelName"] == name
    announce(f"reference row {m}x{n}x{k} {name}")
    with caplog.at_level(logging.WARNING, logger="aiter_amd"):
        _a4w4_on_the_fly(int(m), int(n), int(k), 500 + int(m), cuda, what=f"{m}x{n}x{k} {name}")
    if name == "not_a_kernel_of_anyone":
        assert any("not a kernel of this library" in r.message for r in caplog.records)


def _bf16_check(out, x, w, m, n, seed, bias=None):
    rows = _sample(m, 16, seed)
    cols = _sample(n, 256, seed + 1)
    a_bits = _take_rows(x, rows).view(torch.int16).cpu().numpy().view(np.uint16)
    b_bits = _take_rows(w, cols).view(torch.int16).cpu().numpy().view(np.uint16)
    ref = O.bf16_bits_to_f32(O.gemm_a16w16_ref(a_bits, b_bits, None if bias is None else bias[cols]))
    got = out[torch.from_numpy(rows).to(out.device)][:, torch.from_numpy(cols).to(out.device)].float().cpu().numpy()
    ok, msg = allclose_report(got, ref)
    assert ok, msg


@pytest.mark.parametrize("kid,m,n,k", [(6401, 2048, 4096, 4096), (300, 1024, 2048, 1024), (1208, 1, 2048, 4096),
                                       (206, 48, 4096, 2048), (9, 512, 1024, 512), (5300, 256, 512, 2048)])
def test_opus_reference_kernel_ids(cuda, kid, m, n, k):
    import aiter_amd

    announce(f"opus kid {kid} {m}x{n}x{k}")
    x = _randn_bf16(m, k, kid, cuda)
    w = _randn_bf16(n, k, kid + 1, cuda)
    bias = torch.from_numpy(np.random.default_rng(kid).standard_normal(n).astype(np.float32))
    out = aiter_amd.gemm_a16w16_opus(x, w, bias.to(cuda), kernelId=kid, splitK=2 if 200 <= kid % 1000 < 300 else 0)
    torch.cuda.synchronize()
    assert out.shape == (m, n)
    _bf16_check(out, x, w, m, n, kid + 2, bias.numpy())


@pytest.mark.parametrize("entry,split,expect", [("opus", 5, 5), ("opus", 4, 4), ("opus", 1, 0), ("opus", 0, 0),
                                                ("asm", 5, 5), ("asm", 1, 0)])
def test_split_count_is_literal(cuda, entry, split, expect):
    """splitK of the opus API and of gemm_a16w16_asm is a literal split count
    (aiter/ops/opus/gemm_op_a16w16.py:488, csrc/py_itfs_cu/asm_gemm_a16w16.cu:113-114;
    <= 1 runs one pass).  Opus kid 200 (64x64) and the reference's 64x64 split-K ASM
    name are split-K tiles here too; the call reserves its f32 partials,
    splits * M * N * 4 bytes, in the stream's workspace, so the stream's
    workspace size after the call, released first, gives the split count it
    ran (torch hands out pooled streams, which earlier calls may have used)."""
    import aiter_amd
    from aiter_amd._lib import lib

    m, n, k = 64, 1024, 1280   # 20 K stages of 64: 5 and 4 splits divide them evenly
    announce(f"split count {entry} splitK={split}")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        x = _randn_bf16(m, k, 40 + split, cuda)
        w = _randn_bf16(n, k, 41 + split, cuda)
        assert lib().aiter_amd_workspace_release(cuda.index or 0, s.cuda_stream) == 0
        if entry == "opus":
            out = aiter_amd.gemm_a16w16_opus(x, w, kernelId=200, splitK=split)
        else:
            out = torch.empty((m, n), dtype=torch.bfloat16, device=cuda)
            aiter_amd.gemm_a16w16_asm(x, w, out, splitK=split,
                                      kernelName="_ZN5aiter39bf16gemm_fp32bf16_tn_64x64_splitk_cleanE")
        s.synchronize()
        held = lib().aiter_amd_workspace_bytes(cuda.index or 0, s.cuda_stream)
    assert held == expect * m * n * 4, f"workspace {held} B, expected {expect} splits of {m}x{n} f32"
    _bf16_check(out, x, w, m, n, 42 + split)


def test_opus_unknown_kernel_id_raises(cuda):
    import aiter_amd

    x = _randn_bf16(64, 512, 1, cuda)
    with pytest.raises(RuntimeError, match="unknown opus kernel id"):
        aiter_amd.gemm_a16w16_opus(x, x, kernelId=10300)


@pytest.mark.parametrize("libtype,solidx,name,split", [
    ("opus", 6401, "opus_gemm_mono_tile_512x128x256x64_2x4_16x16x32_0x0x0_nooob_4g_safe", 0),
    ("asm", 0, "_ZN5aiter24bf16gemm_bf16_tn_256x256E", 0),
    ("asm", 0, "_ZN5aiter39bf16gemm_fp32bf16_tn_64x64_splitk_cleanE", 2),
    ("torch", 0, "native", 0),
])
def test_tuned_bf16_reference_libtypes(cuda, monkeypatch, tmp_path, libtype, solidx, name, split):
    """A bf16 tuned row of each reference backend serves gemm_a16w16."""
    import aiter_amd

    m, n, k = 2048, 4096, 1024
    row = {"gfx": "gfx950", "cu_num": 256, "M": m, "N": n, "K": k, "bias": False, "dtype": "torch.bfloat16",
           "outdtype": "torch.bfloat16", "scaleAB": False, "bpreshuffle": False, "libtype": libtype,
           "solidx": solidx, "splitK": split, "us": 1.0, "kernelName": name, "err_ratio": 0.0, "tflops": 1.0,
           "bw": 1.0}
    p = tmp_path / "bf16.csv"
    pd.DataFrame([row]).to_csv(p, index=False)
    monkeypatch.setenv("AITER_CONFIG_GEMM_BF16", str(p))
    monkeypatch.setenv("GPU_ARCHS", "gfx950")
    monkeypatch.setenv("CU_NUM", "256")
    _clear()
    try:
        cfg = aiter_amd.get_GEMM_A16W16_config(m, n, k, False, "torch.bfloat16", "torch.bfloat16", False, False)
        assert cfg["libtype"] == libtype
        announce(f"tuned bf16 row libtype={libtype} {name}")
        x = _randn_bf16(m, k, 3, cuda)
        w = _randn_bf16(n, k, 4, cuda)
        out = aiter_amd.gemm_a16w16(x, w)
        torch.cuda.synchronize()
        _bf16_check(out, x, w, m, n, 5)
    finally:
        _clear()
