"""The C-ABI library (CPU side, no GPU compute): it loads, exports every symbol
declared in include/*.h with the ctypes signature the Python layer binds,
and its host-only entry points behave as the reference's."""
import ctypes
import glob
import os
import re
import subprocess

import pytest

from tests.conftest import ROOT

HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def _declared_functions():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b([A-Za-z_]\w*)\s*\(", text, flags=re.M):
            name = m.group(1)
            if name not in ("if", "while", "for", "sizeof"):
                names.append(name)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    from aiter_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libaiter_amd.so not built (run __graft_entry__.build())")
    return _lib.lib()


def test_header_declares_expected_entry_points():
    names = _declared_functions()
    for n in ("gemm_a4w4_asm", "gemm_a4w4_blockscale", "mxfp8_mxfp4_gemm_asm", "gemm_a16w16_asm",
              "opus_gemm", "opus_gemm_a16w16_tune", "dynamic_per_group_scaled_quant", "quant_mxfp4",
              "dynamic_mxfp4_quant", "dynamic_mxfp8_quant", "getPaddedM", "aiter_ctypes_abi_version",
              "aiter_get_last_error", "aiter_clear_last_error"):
        assert n in names, n


def test_library_exports_every_declared_symbol(lib):
    from aiter_amd import _lib

    exported = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                              text=True, check=True).stdout
    dyn = {line.split()[-1] for line in exported.splitlines() if " T " in line}
    for n in _declared_functions():
        assert n in dyn, f"{n} declared in include/ but not exported"
        assert hasattr(lib, n)
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in aiter_amd/_lib.py"


def test_no_unexpected_c_exports():
    """Every C (unmangled) export is declared in the header."""
    from aiter_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("library not built")
    exported = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                              text=True, check=True).stdout
    c_syms = {line.split()[-1] for line in exported.splitlines()
              if " T " in line and not line.split()[-1].startswith("_Z")}
    assert c_syms <= set(_declared_functions()), c_syms - set(_declared_functions())


def test_abi_version_and_error_channel(lib):
    assert lib.aiter_ctypes_abi_version() == 2
    lib.aiter_clear_last_error()
    # NULL tensors are rejected on the host, before any device call
    rc = lib.gemm_a4w4_asm(None, None, None, None, None, None, None, ctypes.c_float(1.0),
                           ctypes.c_float(0.0), 1, -1, None)
    assert rc == -1
    msg = lib.aiter_get_last_error()
    assert msg and b"null" in msg.lower()
    lib.aiter_clear_last_error()
    assert not lib.aiter_get_last_error()


def test_getpaddedm_matches_oracle(lib):
    """getPaddedM is host code: compare it with the oracle restatement of
    csrc/py_itfs_cu/gemm_common.cu:12-41 over a sweep."""
    from oracle.mx_oracle import get_padded_m

    for gl in (0, 1):
        for m in list(range(1, 300)) + [511, 512, 513, 1023, 4095, 4096, 4097, 8191, 8192, 8193, 20000]:
            for n, k in ((4096, 4096), (8192, 1024)):
                assert lib.getPaddedM(m, n, k, gl) == get_padded_m(m, n, k, gl), (m, n, k, gl)


def test_kernel_table_is_consistent(lib):
    from aiter_amd._lib import kernel_table

    tab = kernel_table()
    assert len(tab) == lib.aiter_amd_num_kernels() > 0
    assert [t[0] for t in tab] == list(range(len(tab)))
    names = [t[1] for t in tab]
    assert len(set(names)) == len(names)
    fams = {t[2] for t in tab}
    assert fams == {"a4w4", "a8w4", "a16w16"}
    for t in tab:
        assert t[4] in (16, 32, 64, 128, 256) and t[5] in (16, 32, 64, 128, 256), t
    buf = ctypes.create_string_buffer(8)
    assert lib.aiter_amd_kernel_info(len(tab), buf, 8) == -1
    assert lib.aiter_amd_kernel_info(-1, buf, 8) == -1
