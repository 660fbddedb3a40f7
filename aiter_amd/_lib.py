"""ctypes binding of libaiter_amd.so (the C ABI declared in include/aiter_amd.h).

Mirrors the reference's ctypes calling convention (aiter/jit/core.py:1252-1555,
aiter/utility/aiter_types.py:26-77): Tensor -> ``aiter_tensor_t*``,
Optional[Tensor] -> NULL, str -> ``char*``, bool -> int, float -> float, plus
the current torch stream appended last.  A non-zero status raises
``RuntimeError("<fn> failed: <message>")``.

The shared library is built in-tree by ``aiter_amd.csrc.build``.  There is
no fallback: if the library is missing or cannot be loaded, every op raises.
"""
from __future__ import annotations

import ctypes
import functools
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libaiter_amd.so")

# AiterDtype ids (include/aiter_amd.h; csrc/include/aiter_enum.h:40-56)
DT_FP8, DT_E8M0, DT_FP16, DT_BF16, DT_FP32 = 0, 1, 2, 3, 4
DT_I4X2, DT_FP4X2, DT_U32, DT_I32, DT_I16, DT_I8, DT_U8, DT_I64, DT_U64 = range(5, 14)

_TORCH_TO_DT = {
    torch.float16: DT_FP16,
    torch.bfloat16: DT_BF16,
    torch.float32: DT_FP32,
    torch.uint32: DT_U32,
    torch.int32: DT_I32,
    torch.int16: DT_I16,
    torch.int8: DT_I8,
    torch.uint8: DT_U8,
    torch.int64: DT_I64,
    torch.uint64: DT_U64,
    torch.float8_e4m3fn: DT_FP8,
}
if hasattr(torch, "float8_e8m0fnu"):
    _TORCH_TO_DT[torch.float8_e8m0fnu] = DT_E8M0
if hasattr(torch, "float4_e2m1fn_x2"):
    _TORCH_TO_DT[torch.float4_e2m1fn_x2] = DT_FP4X2


class AiterTensor(ctypes.Structure):
    """POD tensor descriptor (csrc/include/aiter_tensor.h:8-17)."""

    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("numel", ctypes.c_size_t),
        ("ndim", ctypes.c_int),
        ("shape", ctypes.c_int64 * 8),
        ("strides", ctypes.c_int64 * 8),
        ("dtype", ctypes.c_int),
        ("device_id", ctypes.c_int),
    ]


def to_aiter_tensor(t: torch.Tensor | None, dtype_override: int | None = None):
    if t is None:
        return None
    if t.dim() > 8:
        raise ValueError("aiter_tensor_t supports at most 8 dims")
    dt = dtype_override if dtype_override is not None else _TORCH_TO_DT.get(t.dtype)
    if dt is None:
        raise TypeError(f"unsupported dtype {t.dtype}")
    a = AiterTensor()
    a.ptr = t.data_ptr() if t.numel() > 0 else 0
    a.numel = t.numel()
    a.ndim = t.dim()
    for i, (s, st) in enumerate(zip(t.shape, t.stride())):
        a.shape[i] = s
        a.strides[i] = st
    a.dtype = dt
    a.device_id = t.device.index if t.is_cuda else -1
    return a


_lib = None
_lock = threading.Lock()

# (name, argtypes) of every exported entry point; the trailing void* is the stream.
_T = ctypes.POINTER(AiterTensor)
_S = ctypes.c_void_p
SIGNATURES = {
    "aiter_ctypes_abi_version": ([], ctypes.c_int),
    "aiter_get_last_error": ([], ctypes.c_char_p),
    "aiter_clear_last_error": ([], None),
    "getPaddedM": ([ctypes.c_int] * 4, ctypes.c_int),
    "gemm_a4w4_asm": ([_T, _T, _T, _T, _T, ctypes.c_char_p, _T, ctypes.c_float, ctypes.c_float,
                       ctypes.c_int, ctypes.c_int, _S], ctypes.c_int),
    "gemm_a4w4_blockscale": ([_T, _T, _T, _T, _T, ctypes.c_int, ctypes.c_int, _S], ctypes.c_int),
    "gemm_a4w4_asm_noalloc": ([_T, _T, _T, _T, _T, ctypes.c_char_p, _T, ctypes.c_float, ctypes.c_float,
                               ctypes.c_int, ctypes.c_int, _S], ctypes.c_int),
    "gemm_a4w4_noalloc_scratch_bytes": ([], ctypes.c_size_t),
    "mxfp8_mxfp4_gemm_asm": ([_T, _T, _T, _T, _T, ctypes.c_char_p, ctypes.c_int, _S], ctypes.c_int),
    "gemm_a16w16_asm": ([_T, _T, _T, _T, _T, ctypes.c_int, ctypes.c_char_p, ctypes.c_int, _S], ctypes.c_int),
    "opus_gemm": ([_T, _T, _T, _T, _S], ctypes.c_int),
    "opus_gemm_a16w16_tune": ([_T, _T, _T, _T, ctypes.c_int, ctypes.c_int, _S], ctypes.c_int),
    "dynamic_per_group_scaled_quant": ([_T, _T, _T, ctypes.c_int, ctypes.c_int, _T, ctypes.c_int, _S],
                                       ctypes.c_int),
    "quant_mxfp4": ([_T, _T, _T, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                     ctypes.c_int, _S], ctypes.c_int),
    "dynamic_mxfp4_quant": ([_T, _T, _T, ctypes.c_int, _S], ctypes.c_int),
    "dynamic_mxfp8_quant": ([_T, _T, _T, ctypes.c_int, _S], ctypes.c_int),
    "fused_rms_mx_quant": ([_T, _T, ctypes.c_float, _T, _T, ctypes.c_float, _T, _T, _T, _T, _T, _T, ctypes.c_int,
                            ctypes.c_int, _S], ctypes.c_int),
    "fused_gemm_afp4wfp4_mul_add": ([_T, _T, _T, _T, _T, ctypes.c_float, _T, ctypes.c_float, ctypes.c_int, _T,
                                     ctypes.c_int, ctypes.c_char_p, _S], ctypes.c_int),
    "fused_gemm_afp4wfp4_split_cat": ([_T] * 7 + [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_char_p, _S],
                                      ctypes.c_int),
    "fused_gemm_afp4wfp4_a16w16": ([_T] * 6 + [ctypes.c_char_p] + [_T] * 4 + [ctypes.c_char_p, ctypes.c_int, _S],
                                   ctypes.c_int),
    "moe_sorting_fwd": ([_T] * 7 + [ctypes.c_int, ctypes.c_int, _T, _T, ctypes.c_int, _S], ctypes.c_int),
    "moe_sorting_mx_quant": ([_T] * 10 + [ctypes.c_int, ctypes.c_int, _S], ctypes.c_int),
    "fused_dynamic_mx_quant_moe_sort_hip": ([_T] * 5 + [ctypes.c_int] * 3 + [_T, _S], ctypes.c_int),
    "mxfp4_moe_sort_hip": ([_T] * 4 + [ctypes.c_int] * 2 + [_S], ctypes.c_int),
    "ck_moe_stage1": ([_T] * 7 + [ctypes.c_int, ctypes.c_char_p, _T, _T, ctypes.c_int, _T] + [ctypes.c_int] * 4
                      + [ctypes.c_char_p, ctypes.c_int, _S], ctypes.c_int),
    "ck_moe_stage1_fuse_quant": ([_T] * 7 + [ctypes.c_int, ctypes.c_char_p, _T, _T, ctypes.c_int, _T, _T,
                                  ctypes.c_int, ctypes.c_int, _S], ctypes.c_int),
    "ck_moe_stage2": ([_T] * 7 + [ctypes.c_int, ctypes.c_char_p, _T, _T, ctypes.c_int, _T] + [ctypes.c_int] * 4
                      + [ctypes.c_char_p, ctypes.c_int, _S], ctypes.c_int),
    "moe_sum": ([_T, _T, _S], ctypes.c_int),
    "mxfp4_gemm_asm": ([_T] * 6 + [ctypes.c_char_p, ctypes.c_int, _S], ctypes.c_int),
    "batched_gemm_bf16": ([_T] * 4 + [ctypes.c_int, _S], ctypes.c_int),
    "batched_gemm_bf16_tune": ([_T] * 3 + [ctypes.c_int, ctypes.c_int, _S], ctypes.c_int),
    "aiter_amd_num_kernels": ([], ctypes.c_int),
    "aiter_amd_kernel_info": ([ctypes.c_int, ctypes.c_char_p, ctypes.c_int], ctypes.c_int),
    "aiter_amd_resolve_kernel_name": ([ctypes.c_char_p] + [ctypes.c_int] * 4 + [ctypes.c_int64], ctypes.c_int),
    "aiter_amd_resolve_opus_kid": ([ctypes.c_int, ctypes.c_int, ctypes.c_int64], ctypes.c_int),
    "gemm_workspace_reserve": ([ctypes.c_int, _S, ctypes.c_size_t], ctypes.c_int),
    "aiter_amd_workspace_bytes": ([ctypes.c_int, _S], ctypes.c_int64),
    "aiter_amd_workspace_release": ([ctypes.c_int, _S], ctypes.c_int),
    "hbm_stream_read": ([_T, _T, ctypes.c_int, _S], ctypes.c_int),
    "hbm_stream_read_cfg": ([_T, _T] + [ctypes.c_int] * 4 + [_S], ctypes.c_int),
}


def lib():
    """Load the in-tree library (raises if it is missing: there is no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"aiter_amd HIP library not built: {LIB_PATH} is missing "
                    "(run `python -m aiter_amd.csrc.build`)")
            l = ctypes.CDLL(LIB_PATH)
            for name, (argt, rest) in SIGNATURES.items():
                fn = getattr(l, name)
                fn.argtypes = argt
                fn.restype = rest
            if l.aiter_ctypes_abi_version() != 2:
                raise RuntimeError("aiter_amd ABI version mismatch")
            _lib = l
    return _lib


def _stream_handle(device: torch.device | None) -> int:
    if device is None or device.type != "cuda":
        return 0
    return torch.cuda.current_stream(device).cuda_stream


def call(name: str, *args, device: torch.device | None = None):
    """Call entry point ``name`` converting tensors, appending the stream."""
    l = lib()
    fn = getattr(l, name)
    keep = []
    conv = []
    for a in args:
        if isinstance(a, torch.Tensor):
            at = to_aiter_tensor(a)
            keep.append(at)
            conv.append(ctypes.byref(at))
        elif isinstance(a, AiterTensor):
            keep.append(a)
            conv.append(ctypes.byref(a))
        elif a is None:
            conv.append(None)
        elif isinstance(a, str):
            conv.append(a.encode())
        elif isinstance(a, bool):
            conv.append(int(a))
        else:
            conv.append(a)
    if device is None:
        for a in args:
            if isinstance(a, torch.Tensor):
                device = a.device
                break
    conv.append(_stream_handle(device))
    rc = fn(*conv)
    if rc != 0:
        msg = l.aiter_get_last_error()
        raise RuntimeError(f"{name} failed: {msg.decode() if msg else 'unknown error'}")


def kernel_table():
    """[(id, name, family, skinny, bm, bn, split, a_pre, b_pre, out_f32)] of the library."""
    l = lib()
    out = []
    buf = ctypes.create_string_buffer(256)
    for i in range(l.aiter_amd_num_kernels()):
        if l.aiter_amd_kernel_info(i, buf, 256) == 0:
            f = buf.value.decode().split(",")
            out.append((int(f[0]), f[1], f[2], bool(int(f[3])), int(f[4]), int(f[5]),
                        bool(int(f[6])), bool(int(f[7])), bool(int(f[8])), bool(int(f[9]))))
    return out


@functools.lru_cache(maxsize=1)
def kernel_names() -> frozenset:
    """Names of this library's kernel instances."""
    return frozenset(row[1] for row in kernel_table())
