"""Tuned-config CSV handling and chip identification.

Schema and lookup follow the reference:
* A4W4 rows ``gfx,cu_num,M,N,K,kernelId,splitK,us,kernelName,tflops,bw,errRatio``
  keyed ``(gfx, cu_num, M, N, K)`` (aiter/ops/gemm_op_a4w4.py:33-78).
* bf16 rows ``gfx,cu_num,M,N,K,bias,dtype,outdtype,scaleAB,bpreshuffle,libtype,
  solidx,splitK,us,kernelName,err_ratio,tflops,bw`` keyed on the first ten
  columns (aiter/tuned_gemm.py:207-300; aiter/configs/bf16_tuned_gemm.csv:1).
* ``AITER_CONFIG_GEMM_A4W4`` / ``AITER_CONFIG_GEMM_BF16``: colon-separated
  CSV lists merged in order; a key tuned twice with different kernels raises
  (aiter/jit/core.py:216-377).
"""
from __future__ import annotations

import functools
import os

import pandas as pd

_HERE = os.path.dirname(os.path.abspath(__file__))
CONFIG_DIR = os.path.join(_HERE, "configs")
DEFAULT_A4W4_CSV = os.path.join(CONFIG_DIR, "a4w4_blockscale_tuned_gemm.csv")
DEFAULT_BF16_CSV = os.path.join(CONFIG_DIR, "bf16_tuned_gemm.csv")
DEFAULT_A8W4_CSV = os.path.join(CONFIG_DIR, "a8w4_tuned_gemm.csv")

A4W4_KEYS = ["gfx", "cu_num", "M", "N", "K"]
BF16_KEYS = ["gfx", "cu_num", "M", "N", "K", "bias", "dtype", "outdtype", "scaleAB", "bpreshuffle"]
A4W4_COLUMNS = ["gfx", "cu_num", "M", "N", "K", "kernelId", "splitK", "us", "kernelName", "tflops", "bw",
                "errRatio"]
BF16_COLUMNS = ["gfx", "cu_num", "M", "N", "K", "bias", "dtype", "outdtype", "scaleAB", "bpreshuffle",
                "libtype", "solidx", "splitK", "us", "kernelName", "err_ratio", "tflops", "bw"]


@functools.lru_cache(maxsize=None)
def get_gfx() -> str:
    """gfx arch of device 0 (``GPU_ARCHS`` overrides, as
    aiter/jit/utils/chip_info.py:139-161)."""
    env = os.environ.get("GPU_ARCHS")
    if env:
        return env.split(";")[0]
    import torch

    if torch.cuda.is_available():
        return torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    return "gfx950"


@functools.lru_cache(maxsize=None)
def get_cu_num() -> int:
    env = os.environ.get("CU_NUM")
    if env:
        return int(env)
    import torch

    if torch.cuda.is_available():
        return torch.cuda.get_device_properties(0).multi_processor_count
    return 256


def config_files(env_name: str, default: str) -> list[str]:
    env = os.environ.get(env_name)
    files = [f for f in env.split(":") if f] if env else [default]
    return [f for f in files if os.path.exists(f)]


def merge_csvs(files: list[str], keys: list[str], result_cols=("kernelName",)) -> pd.DataFrame:
    """Concatenate tuned CSVs, drop exact duplicates, raise when one key maps
    to two different kernels (aiter/jit/core.py:216-377)."""
    frames = [pd.read_csv(f) for f in files]
    frames = [f for f in frames if len(f)]
    if not frames:
        return pd.DataFrame(columns=keys)
    df = pd.concat(frames, ignore_index=True)
    present = [k for k in keys if k in df.columns]
    sub = present + [c for c in result_cols if c in df.columns]
    df = df.drop_duplicates(subset=sub, keep="last")
    dup = df.duplicated(subset=present, keep=False)
    if dup.any():
        raise ValueError(f"conflicting tuned rows for keys {present}:\n{df[dup].head()}")
    return df


def load_tuned(env_name: str, default: str, keys: list[str]) -> dict:
    df = merge_csvs(config_files(env_name, default), keys)
    if not len(df):
        return {}
    present = [k for k in keys if k in df.columns]
    return df.set_index(present).to_dict("index")
