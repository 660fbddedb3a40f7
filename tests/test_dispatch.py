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


# ---------------------------------------------------------------- reference kernel names
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _lines(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return [l.strip() for l in f if l.strip()]


def _resolve(name, fam=0, m=4096, b_pre=1, out_f32=0):
    from aiter_amd._lib import lib

    return lib().aiter_amd_resolve_kernel_name(name.encode(), fam, 0, b_pre, out_f32, m)


def test_every_reference_a4w4_kernel_name_resolves():
    """All 43 kernel names of the reference's a4w4_blockscale_tuned_gemm.csv
    (ASM tiles and CK instances; list in tests/golden) resolve without error:
    to the tile of the same shape here, else to the heuristic (-1)."""
    from aiter_amd._lib import kernel_table

    table = {r[0]: r for r in kernel_table()}
    names = _lines("reference_a4w4_kernel_names.txt")
    assert len(names) == 43
    for nm in names:
        for m in (1, 32, 33, 4096):
            kid = _resolve(nm, m=m)
            assert kid >= -1, (nm, m)
            if m <= 32:
                assert kid == -1, (nm, m)   # small M: this library's skinny kernels via the heuristic
            if kid >= 0:
                row = table[kid]
                assert row[2] == "a4w4" and not row[3] and row[8], (nm, row)
    # tiles this library has map to them exactly, others to the heuristic
    assert table[_resolve("_ZN5aiter42f4gemm_bf16_per1x32Fp4_BpreShuffle_256x256E")][1] == "a4w4_tile_256x256"
    assert table[_resolve("_ZN5aiter41f4gemm_bf16_per1x32Fp4_BpreShuffle_64x128E")][1] == "a4w4_tile_64x128"
    assert _resolve("_ZN5aiter42f4gemm_bf16_per1x32Fp4_BpreShuffle_160x256E") == -1
    ck = "a4w4_blockscale_256x128x256x128_16x16_16x16_8x32x1_8x32x1_1x32x1x8_8_2x2_intrawave_v3"
    assert table[_resolve(ck)][1] == "a4w4_tile_128x256"
    assert _resolve("a4w4_blockscale_256x96x384x128_16x16_16x16_8x32x1_8x32x1_1x32x1x8_8_2x2_intrawave_v3") == -1
    # row-major B: the no-preshuffle reference kernel
    nm = "_ZN5aiter44f4gemm_bf16_per1x32Fp4_noBpreShuffle_256x256E"
    assert table[_resolve(nm, b_pre=0)][1] == "a4w4_tile_256x256_bplain"


def test_library_and_unknown_names():
    from aiter_amd._lib import kernel_table

    for row in kernel_table()[:20]:
        assert _resolve(row[1]) == row[0]
    for bad in ("not_a_kernel", "_ZN5aiter3fooE", "a4w4_blockscale_garbage", "_ZN5aiter_12x34"):
        assert _resolve(bad) == -2, bad


def test_reference_bf16_asm_names_resolve():
    from aiter_amd._lib import kernel_table

    table = {r[0]: r for r in kernel_table()}
    for nm in _lines("reference_bf16_asm_names.txt"):
        for m in (1, 64, 8192):
            kid = _resolve(nm, fam=2, m=m, b_pre=0)
            assert kid >= -1, (nm, m)
            if kid >= 0:
                assert table[kid][2] == "a16w16" and not table[kid][8]
    big = _resolve("_ZN5aiter24bf16gemm_bf16_tn_256x256E", fam=2, m=8192, b_pre=0)
    assert table[big][1] == "a16w16_tile_256x256_bplain"
    sk = _resolve("_ZN5aiter39bf16gemm_fp32bf16_tn_64x64_splitk_cleanE", fam=2, m=64, b_pre=0)
    assert table[sk][1] == "a16w16_tile_64x64_splitk_bplain"


def test_reference_opus_kids_resolve():
    """Every gfx950 opus kid in the reference's bf16 tuned CSVs decodes; 6401
    (mono tile 128x256, >4 GiB-safe) and 300 (persistent 256x256) land on the
    same tiles here; gfx942 ids (>= 10000) and removed ids are errors."""
    from aiter_amd._lib import kernel_table, lib

    table = {r[0]: r for r in kernel_table()}
    kids = [int(x) for x in _lines("reference_opus_kids.txt")]
    assert 6401 in kids and len(kids) == 35
    for kid in kids:
        for m in (1, 2048):
            r = lib().aiter_amd_resolve_opus_kid(kid, 0, m)
            assert r >= -1, kid
            if m == 1:
                assert r == -1
    assert table[lib().aiter_amd_resolve_opus_kid(6401, 0, 2048)][1] == "a16w16_tile_128x256_bplain"
    assert table[lib().aiter_amd_resolve_opus_kid(300, 0, 8192)][1] == "a16w16_tile_256x256_bplain"
    assert table[lib().aiter_amd_resolve_opus_kid(200, 1, 256)][1] == "a16w16_tile_64x64_splitk_bplain_f32"
    for bad in (3, 100, 1100, 10000, 10300, -5):
        assert lib().aiter_amd_resolve_opus_kid(bad, 0, 1024) == -2, bad


def test_reference_row_fixture_routes(gfx950, monkeypatch):
    """The reference-CSV fixture merges and its rows look up like any other."""
    p = os.path.join(GOLDEN, "reference_a4w4_rows.csv")
    monkeypatch.setenv("AITER_CONFIG_GEMM_A4W4", p)
    _clear()
    assert "_ZN" in aiter_amd.get_GEMM_config(1, 4096, 4096)["kernelName"]
    assert aiter_amd.get_GEMM_config(2048, 7168, 2048)["kernelName"].startswith("a4w4_blockscale_")
    assert aiter_amd.get_GEMM_config(96, 1024, 512)["kernelName"] == "not_a_kernel_of_anyone"
