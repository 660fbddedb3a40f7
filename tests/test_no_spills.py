"""The large-M tile kernels keep their accumulators and operand rings in
registers: a VGPR spill there turns every stage into scratch traffic (one
body carrying two stage sequences once spilled ~400 VGPRs of the 256x256
persistent A4W4 tile and made it 1.5x slower with bit-identical results, which
no parity test can see).  Compiles the registry units of those kernels for
gfx950 (device code only) and reads the compiler's resource remarks."""
import os
import shutil
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor

import pytest

from aiter_amd.csrc import build

UNITS = ["gemm_reg_mx.hip", "gemm_reg_split.hip", "gemm_reg_bf16.hip"]


def _spills(src, out_dir):
    cmd = [build.HIPCC, *build.FLAGS, build.USAGE_FLAG, "--cuda-device-only", "-c",
           os.path.join(build.HERE, src), "-o", os.path.join(out_dir, src + ".o")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return build.vgpr_spills(r.stderr)


@pytest.mark.skipif(not os.path.exists(build.HIPCC) and shutil.which("hipcc") is None, reason="no hipcc")
def test_tile_kernels_do_not_spill():
    with tempfile.TemporaryDirectory() as d, ThreadPoolExecutor(len(UNITS)) as ex:
        res = dict(zip(UNITS, ex.map(lambda s: _spills(s, d), UNITS)))
    bad = {u: sp for u, sp in res.items() if sp}
    assert not bad, f"VGPR spills: {bad}"


def test_spill_remark_parser():
    text = ("x.h:1:1: remark: Function Name: _Zkern_a [-Rpass-analysis=kernel-resource-usage]\n"
            "x.h:1:1: remark:     VGPRs Spill: 0 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.h:1:1: remark: Function Name: _Zkern_b [-Rpass-analysis=kernel-resource-usage]\n"
            "x.h:1:1: remark:     SGPRs Spill: 7 [-Rpass-analysis=kernel-resource-usage]\n"
            "x.h:1:1: remark:     VGPRs Spill: 398 [-Rpass-analysis=kernel-resource-usage]\n")
    assert build.vgpr_spills(text) == {"_Zkern_b": 398}
