"""bench.py's MoE stage timing calls the fused_moe module's own entry points
(not the package-level fused_moe function of the same name): the module it
binds must be that module, and every name it uses must resolve on it.  CPU
only: nothing is launched."""
import os
import re
import types


def test_bench_moe_stage_names_resolve():
    import bench

    fm = bench.fused_moe_module()
    assert isinstance(fm, types.ModuleType) and fm.__name__ == "aiter_amd.fused_moe"
    src = open(os.path.join(os.path.dirname(__file__), "..", "bench.py")).read()
    used = set(re.findall(r"\bFM\.([A-Za-z_]\w*)", src))
    assert used, "bench.py no longer times the MoE stages through FM"
    missing = sorted(n for n in used if not hasattr(fm, n))
    assert not missing, f"bench.py uses names the fused_moe module lacks: {missing}"


def test_bench_moe_reference_rows():
    """bench.py's per-model reference stage times and shapes equal the rows
    of the reference's tuned fused-MoE tables they cite (skipped where the
    reference tree is absent, as on the GPU box)."""
    import csv

    import pytest

    import bench

    base = "/root/reference/aiter/configs/model_configs"
    if not os.path.isdir(base):
        pytest.skip("reference tree not present")
    files = {"deepseek": "dsv3_fp4_tuned_fmoe.csv", "glm5": "glm5_fp4_tuned_fmoe.csv",
             "kimik2": "kimik2_fp4_tuned_fmoe.csv", "minimax_m25": "minimax_m25_fp4_tuned_fmoe.csv",
             "qwen3_5_397b": "qwen3_5_397b_fp4_tuned_fmoe.csv"}
    for model, fn in files.items():
        rows = list(csv.DictReader(open(os.path.join(base, fn))))
        e, topk, dim, inter = bench.MOE_MODELS[model]
        for tokens, (us1, us2) in bench.REF_MOE[model].items():
            r = next(r for r in rows if r["cu_num"] == "256" and int(r["token"]) == tokens)
            assert (int(r["expert"]), int(r["topk"]), int(r["model_dim"]), int(r["inter_dim"])) == (e, topk, dim, inter)
            assert abs(float(r["us1"]) - us1) < 1e-3 and abs(float(r["us2"]) - us2) < 1e-3, (model, tokens)
