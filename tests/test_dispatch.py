"""Host-side dispatch: tuned-CSV merge and lookup (padded-M retries), the
shipped tables, and the tuner's CPU helpers.  No GPU compute."""
import os

import numpy as np
import pandas as pd
import pytest
import torch

import aiter_amd
from aiter_amd import config, gemm_op_a4w4, gemm_op_a8w4, tuned_gemm, tuner
from oracle import mx_oracle as O


def _clear():
    gemm_op_a4w4._a4w4_table.cache_clear()
    gemm_op_a4w4.get_GEMM_config.cache_clear()
    gemm_op_a8w4._a8w4_table.cache_clear()
    gemm_op_a8w4.get_GEMM_A8W4_config.cache_clear()
    tuned_gemm._bf16_table.cache_clear()
    tuned_gemm.get_GEMM_A16W16_config.cache_clear()


@pytest.fixture
def gfx950(monkeypatch):
    monkeypatch.setenv("GPU_ARCHS", "gfx950")
    monkeypatch.setenv("CU_NUM", "256")
    config.get_gfx.cache_clear()
    config.get_cu_num.cache_clear()
    _clear()
    yield
    config.get_gfx.cache_clear()
    config.get_cu_num.cache_clear()
    _clear()


def _row(m, n, k, name, kid=0, split=0):
    return {"gfx": "gfx950", "cu_num": 256, "M": m, "N": n, "K": k, "kernelId": kid, "splitK": split,
            "us": 1.0, "kernelName": name, "tflops": 1.0, "bw": 1.0, "errRatio": 0.0}


def test_merge_dedups_and_raises_on_conflict(tmp_path):
    a = tmp_path / "a.csv"
    b = tmp_path / "b.csv"
    pd.DataFrame([_row(32, 4096, 4096, "x"), _row(64, 4096, 4096, "y")]).to_csv(a, index=False)
    pd.DataFrame([_row(32, 4096, 4096, "x"), _row(128, 4096, 4096, "z")]).to_csv(b, index=False)
    df = config.merge_csvs([str(a), str(b)], config.A4W4_KEYS)
    assert len(df) == 3
    pd.DataFrame([_row(32, 4096, 4096, "other")]).to_csv(b, index=False)
    with pytest.raises(ValueError):
        config.merge_csvs([str(a), str(b)], config.A4W4_KEYS)


def test_a4w4_lookup_with_padded_m(tmp_path, monkeypatch, gfx950):
    p = tmp_path / "t.csv"
    # exact M, padded gl=0 (M=17 -> 32), padded gl=1 (M=3 -> 4)
    pd.DataFrame([_row(300, 7168, 2048, "exact"), _row(32, 7168, 2048, "pad0"),
                  _row(4, 8192, 1024, "pad1")]).to_csv(p, index=False)
    monkeypatch.setenv("AITER_CONFIG_GEMM_A4W4", str(p))
    _clear()
    assert aiter_amd.get_GEMM_config(300, 7168, 2048)["kernelName"] == "exact"
    assert aiter_amd.get_GEMM_config(17, 7168, 2048)["kernelName"] == "pad0"
    assert aiter_amd.get_GEMM_config(3, 8192, 1024)["kernelName"] == "pad1"
    assert aiter_amd.get_GEMM_config(5000, 7168, 2048) is None


def test_env_lists_merge_in_order(tmp_path, monkeypatch, gfx950):
    a = tmp_path / "a.csv"
    b = tmp_path / "b.csv"
    pd.DataFrame([_row(64, 4096, 4096, "from_a")]).to_csv(a, index=False)
    pd.DataFrame([_row(128, 4096, 4096, "from_b")]).to_csv(b, index=False)
    monkeypatch.setenv("AITER_CONFIG_GEMM_A4W4", f"{a}:{b}")
    _clear()
    assert aiter_amd.get_GEMM_config(64, 4096, 4096)["kernelName"] == "from_a"
    assert aiter_amd.get_GEMM_config(128, 4096, 4096)["kernelName"] == "from_b"


def test_other_arch_rows_are_ignored(tmp_path, monkeypatch, gfx950):
    p = tmp_path / "t.csv"
    r = _row(64, 4096, 4096, "wrong_arch")
    r["gfx"] = "gfx942"
    pd.DataFrame([r]).to_csv(p, index=False)
    monkeypatch.setenv("AITER_CONFIG_GEMM_A4W4", str(p))
    _clear()
    assert aiter_amd.get_GEMM_config(64, 4096, 4096) is None


def test_bf16_lookup_and_default(gfx950):
    cfg = aiter_amd.get_GEMM_A16W16_config(1, 4096, 4096, False, "torch.bfloat16", "torch.bfloat16", False, False)
    assert cfg["libtype"] == "aiter_amd" and cfg["solidx"] >= 0
    cfg = aiter_amd.get_GEMM_A16W16_config(3, 123, 4096, False, "torch.bfloat16", "torch.bfloat16", False, False)
    assert cfg["solidx"] == -1  # untuned shape -> the library heuristic


@pytest.mark.parametrize("fname,keys", [("a4w4_blockscale_tuned_gemm.csv", config.A4W4_KEYS),
                                        ("a8w4_tuned_gemm.csv", config.A4W4_KEYS),
                                        ("bf16_tuned_gemm.csv", config.BF16_KEYS)])
def test_shipped_tables_are_consistent(fname, keys):
    from aiter_amd._lib import LIB_PATH, kernel_table

    df = pd.read_csv(os.path.join(config.CONFIG_DIR, fname))
    assert len(df) > 0
    assert not df.duplicated(subset=keys).any()
    assert set(df["gfx"]) == {"gfx950"} and set(df["cu_num"]) == {256}
    err = "errRatio" if "errRatio" in df else "err_ratio"
    assert (df[err] <= 0.05).all()
    if os.path.exists(LIB_PATH):
        names = {r[1]: r[0] for r in kernel_table()}
        idcol = "kernelId" if "kernelId" in df else "solidx"
        for _, r in df.iterrows():
            assert names[r["kernelName"]] == r[idcol]


def test_shipped_a4w4_table_covers_the_benchmark_shapes():
    df = pd.read_csv(os.path.join(config.CONFIG_DIR, "a4w4_blockscale_tuned_gemm.csv"))
    have = set(zip(df.M, df.N, df.K))
    for s in tuner.sweep_shapes("a4w4"):
        assert s in have, s


def test_tuner_dequant_matches_oracle():
    rs = np.random.default_rng(0)
    q = rs.integers(0, 256, (8, 64), dtype=np.uint8)
    s = rs.integers(110, 140, (8, 4), dtype=np.uint8)
    got = tuner._dequant_fp4(torch.from_numpy(q), torch.from_numpy(s)).numpy()
    np.testing.assert_array_equal(got, O.dequant_mxfp4(q, s))
    q8 = O.e4m3_encode_rne(rs.standard_normal((8, 128)).astype(np.float32))
    s8 = rs.integers(110, 140, (8, 4), dtype=np.uint8)
    got8 = tuner._dequant_fp8(torch.from_numpy(q8), torch.from_numpy(s8)).numpy()
    np.testing.assert_array_equal(got8, O.dequant_mxfp8(q8, s8))


def test_tuner_err_ratio():
    ref = torch.zeros(100)
    out = ref.clone()
    out[:7] = 0.5
    assert tuner.err_ratio(out, ref) == pytest.approx(0.07)


def test_tuner_candidates_respect_shape():
    for kid, name, l2 in tuner.candidates("a4w4", 1):
        assert "256x" not in name and "128x" not in name
    big = tuner.candidates("a4w4", 4096)
    assert all("skinny" not in n for _, n, _ in big)
    assert any(n == "a4w4_tile_256x256" for _, n, _ in big)
