"""The tuner's driver on the CPU (no GPU): per-shape worker processes under a
watchdog, each row merged into the output as soon as its shape is done,
resume (shapes already tuned are skipped, --all retunes), and a crashing or
hanging worker costing only its own shape.  A stand-in worker script plays
the GPU worker's part (writes a row, crashes or hangs by shape)."""
import os
import subprocess
import sys
import textwrap

import pandas as pd
import pytest

from aiter_amd import tuner

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# The stand-in worker imports the package (and torch with it): a cold import on
# a loaded machine has taken more than 5 s, so the watchdog leaves room for it.
WATCHDOG_S = 20.0

FAKE = textwrap.dedent('''
    import sys, time
    from aiter_amd import tuner
    a = sys.argv[1:]
    out = a[a.index("-o") + 1]
    for spec in a[a.index("--worker") + 1].split(";"):
        m, n, k = tuner._parse_shape(a[a.index("--family") + 1], spec)
        if m == 2:
            sys.exit(3)                  # a worker that dies
        if m == 3:
            time.sleep(300)              # a worker that hangs
        tuner.write_row(out, "a4w4", {"gfx": "gfx950", "cu_num": 256, "M": m, "N": n, "K": k, "kernelId": 7,
                                      "splitK": 0, "us": 1.0 + m, "kernelName": "a4w4_skinny_m32", "tflops": 1.0,
                                      "bw": 1.0, "errRatio": 0.0})
''')


@pytest.fixture
def fake_worker(tmp_path, monkeypatch):
    p = tmp_path / "fake_worker.py"
    p.write_text(FAKE)
    monkeypatch.setenv("GPU_ARCHS", "gfx950")
    monkeypatch.setenv("CU_NUM", "256")
    monkeypatch.setenv("PYTHONPATH", os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    return [sys.executable, str(p)]


def test_driver_isolates_failures_and_resumes(tmp_path, fake_worker):
    out = str(tmp_path / "tuned.csv")
    shapes = [(1, 256, 512), (2, 256, 512), (3, 256, 512), (4, 256, 512)]
    res = tuner.drive("a4w4", shapes, out, 5, 0.05, False, timeout=WATCHDOG_S, worker_cmd=fake_worker)
    assert res["tuned"] == [(1, 256, 512), (4, 256, 512)]
    assert [s for s, _ in res["failed"]] == [(2, 256, 512), (3, 256, 512)]
    assert "exit 3" in res["failed"][0][1] and "no result within" in res["failed"][1][1]
    df = pd.read_csv(out)
    assert sorted(df.M.tolist()) == [1, 4]          # each shape's row landed when it finished
    # resume: finished shapes are skipped, failed ones are tried again
    res2 = tuner.drive("a4w4", shapes, out, 5, 0.05, False, timeout=WATCHDOG_S, worker_cmd=fake_worker)
    assert res2["skipped"] == [(1, 256, 512), (4, 256, 512)]
    assert len(res2["failed"]) == 2
    # --all retunes every shape; rows are replaced, not duplicated
    res3 = tuner.drive("a4w4", [(1, 256, 512)], out, 5, 0.05, True, timeout=WATCHDOG_S, worker_cmd=fake_worker)
    assert res3["tuned"] == [(1, 256, 512)]
    assert sorted(pd.read_csv(out).M.tolist()) == [1, 4]


def test_driver_batches_shapes(tmp_path, fake_worker):
    """Several shapes per worker: each finished shape keeps its row; a worker
    that dies fails the shapes of its batch without a row, and the next batch
    runs."""
    out = str(tmp_path / "tuned.csv")
    shapes = [(1, 256, 512), (2, 256, 512), (4, 256, 512), (5, 256, 512), (6, 256, 512)]
    res = tuner.drive("a4w4", shapes, out, 5, 0.05, False, timeout=WATCHDOG_S, worker_cmd=fake_worker, batch=2)
    assert res["tuned"] == [(1, 256, 512), (4, 256, 512), (5, 256, 512), (6, 256, 512)]
    assert [s for s, _ in res["failed"]] == [(2, 256, 512)]
    assert sorted(pd.read_csv(out).M.tolist()) == [1, 4, 5, 6]


def test_write_row_replaces_same_key(tmp_path):
    out = str(tmp_path / "t.csv")
    row = {"gfx": "gfx950", "cu_num": 256, "M": 8, "N": 64, "K": 256, "kernelId": 1, "splitK": 0, "us": 2.0,
           "kernelName": "x", "tflops": 1.0, "bw": 1.0, "errRatio": 0.0}
    tuner.write_row(out, "a4w4", row)
    tuner.write_row(out, "a4w4", dict(row, M=16))
    tuner.write_row(out, "a4w4", dict(row, us=1.5, kernelName="y"))
    df = pd.read_csv(out)
    assert len(df) == 2 and df[df.M == 8].kernelName.tolist() == ["y"]
    assert tuner.tuned_keys(out, "a4w4") == {("gfx950", 256, 8, 64, 256), ("gfx950", 256, 16, 64, 256)}


def test_bf16_keys_round_trip(tmp_path):
    out = str(tmp_path / "b.csv")
    s = (32, 4096, 4096, False, "torch.bfloat16", True)
    row = {"gfx": "gfx950", "cu_num": 256, "M": 32, "N": 4096, "K": 4096, "bias": False, "dtype": "torch.bfloat16",
           "outdtype": "torch.bfloat16", "scaleAB": False, "bpreshuffle": True, "libtype": "aiter_amd", "solidx": 3,
           "splitK": 0, "us": 1.0, "kernelName": "k", "err_ratio": 0.0, "tflops": 1.0, "bw": 1.0}
    tuner.write_row(out, "a16w16", row)
    assert tuner._shape_key("a16w16", "gfx950", 256, s) in tuner.tuned_keys(out, "a16w16")
    assert tuner._parse_shape("a16w16", tuner._shape_arg("a16w16", s)) == s


@pytest.mark.parametrize("compare,pct", [(False, 3.0), (True, -1e30), (True, 5.0)])
def test_worker_command_line_parses(tmp_path, compare, pct):
    """The worker command that the driver builds is accepted by the tuner's
    own argument parser (a negative threshold included); without a GPU the
    worker then stops with its own message, not a usage error."""
    from aiter_amd import tuner

    shape = (64, 512, 256, False, "torch.bfloat16", True)
    args = tuner.worker_args("a16w16", shape, str(tmp_path / "t.csv"), 5, 0.05, compare, pct)
    env = dict(os.environ, HIP_VISIBLE_DEVICES="-1", CUDA_VISIBLE_DEVICES="-1")
    r = subprocess.run([sys.executable, "-m", "aiter_amd.tuner"] + args, cwd=ROOT, env=env, capture_output=True,
                       text=True, timeout=300)
    assert "error: argument" not in r.stderr, r.stderr
    assert r.returncode == 2 and "the tuner needs a GPU" in r.stderr, (r.returncode, r.stderr)
    assert tuner._parse_shape("a16w16", args[args.index("--worker") + 1]) == shape
