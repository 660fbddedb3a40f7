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
