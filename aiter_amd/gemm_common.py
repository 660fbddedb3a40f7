"""Padded-M lookup bucketing (aiter/ops/gemm_op_common.py -> C getPaddedM,
csrc/py_itfs_cu/gemm_common.cu:12-41)."""
from __future__ import annotations

import functools

from ._lib import lib


@functools.lru_cache(maxsize=4096)
def get_padded_m(M: int, N: int, K: int, gl: int) -> int:
    return int(lib().getPaddedM(int(M), int(N), int(K), int(gl)))
