"""Build libaiter_amd.so (gfx950) in-tree with hipcc.

Usage: python -m aiter_amd.csrc.build   (or build() from Python)
The library lands next to the package (aiter_amd/libaiter_amd.so) so it
travels with the source tree.
"""
from __future__ import annotations

import os
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
ROOT = os.path.dirname(PKG)
SOURCES = ["gemm.hip", "gemm_reg_mx.hip", "gemm_reg_bf16.hip", "gemm_reg_bf16_f32.hip", "gemm_reg_split.hip",
           "gemm_reg_rest.hip", "gemm_reg_direct.hip", "gemm_reg_late.hip", "quant.hip", "fused_quant.hip", "moe_sorting.hip", "moe_gemm.hip", "calib.hip"]
LIB = os.path.join(PKG, "libaiter_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-munsafe-fp-atomics",
    # packed-FP32 VALU forms (v_pk_*_f32) stay off: some of their forms have given
    # wrong results on this hardware without any error
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + HERE,
    "-Wno-unused-command-line-argument",
]


# the compiler's per-kernel resource remarks (registers, spills, LDS)
USAGE_FLAG = "-Rpass-analysis=kernel-resource-usage"


def vgpr_spills(remarks: str) -> dict:
    """{kernel symbol: spilled VGPRs} for every kernel that spills, from the
    remarks of USAGE_FLAG."""
    out, fn = {}, None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            fn = m.group(1)
            continue
        m = re.search(r"VGPRs Spill: (\d+)", line)
        if m and fn and int(m.group(1)) > 0:
            out[fn] = int(m.group(1))
    return out


def _compile(src: str, out_dir: str, extra=()) -> tuple:
    obj = os.path.join(out_dir, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, USAGE_FLAG, *extra, "-c", os.path.join(HERE, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr[-6000:]}")
    return obj, vgpr_spills(r.stderr)


def build(verbose: bool = True) -> str:
    out_dir = os.path.join(PKG, "_build")
    os.makedirs(out_dir, exist_ok=True)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        res = list(ex.map(lambda s: _compile(s, out_dir), SOURCES))
    objs = [o for o, _ in res]
    spills = {k: v for _, sp in res for k, v in sp.items()}
    with open(os.path.join(out_dir, "vgpr_spills.txt"), "w") as f:
        for k, v in sorted(spills.items()):
            f.write(f"{v}\t{k}\n")
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
        if spills:
            print(f"note: {len(spills)} kernel(s) spill VGPRs (list in {out_dir}/vgpr_spills.txt)")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
