"""ctypes binding of libpcamd_fp8.so (the C ABI declared in include/pcamd_fp8.h,
plus the test-only include/pcamd_fp8_selftest.h).

The library must have been built (``python -m practice_cuda_amd.build`` or
``__graft_entry__.build()``). There is no fallback: if it is missing every
entry point raises, so a GPU run can never silently use another path.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

from .build import LIB_PATH

_LOCK = threading.Lock()
_LIB = None

F32, BF16, F16, E4M3FN, E5M2 = 0, 1, 2, 3, 4
F64 = 5  # scale arithmetic of pcamd_quant_tensor only (torchao's tensorwise form)
QUANT_CACHED_OUTPUT = 1  # quantizer flag: outputs with cache-allocating stores
SCALE_BLOCK, SCALE_CHANNEL, SCALE_TENSOR = 0, 1, 2
ACT_NONE, ACT_GELU = 0, 1
# status codes (include/pcamd_fp8.h)
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_LAUNCH = 0, -1, -2, -3

_DTYPE_CODES = {
    torch.float32: F32,
    torch.bfloat16: BF16,
    torch.float16: F16,
    torch.float8_e4m3fn: E4M3FN,
    torch.float8_e5m2: E5M2,
}

EXPORTED_SYMBOLS = (
    "pcamd_abi_version",
    "pcamd_last_error",
    "pcamd_quant_block",
    "pcamd_quant_block_dual",
    "pcamd_quant_block_ex",
    "pcamd_quant_block_dual_ex",
    "pcamd_quant_channel",
    "pcamd_quant_tensor",
    "pcamd_bmm_scaled",
    "pcamd_bmm_scaled_mixed",
    "pcamd_bmm_quant_a",
    "pcamd_repack_fp8",
)
# test-only entry points (include/pcamd_fp8_selftest.h), exported by the same library
TEST_SYMBOLS = ("pcamd_selftest_fp8_convert", "pcamd_selftest_copy16", "pcamd_selftest_narrow16")

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_flt = ctypes.c_float


class ExtensionMissing(RuntimeError):
    pass


def _declare(lib: ctypes.CDLL) -> None:
    lib.pcamd_abi_version.restype = _int
    lib.pcamd_abi_version.argtypes = []
    lib.pcamd_last_error.restype = ctypes.c_char_p
    lib.pcamd_last_error.argtypes = []
    quant_head = [_ptr, _int, _i64, _i64, _i64, _i64, _i64, _i64, _ptr, _int, _i64, _i64, _i64]
    lib.pcamd_quant_block.restype = _int
    lib.pcamd_quant_block.argtypes = quant_head + [_ptr, _i64, _i64, _i64, _i64, _i64, _flt, _flt, _ptr]
    lib.pcamd_quant_block_dual.restype = _int
    lib.pcamd_quant_block_dual.argtypes = (
        [_ptr, _int, _i64, _i64, _i64, _i64, _i64, _i64] + [_ptr, _i64, _i64, _i64] * 2 + [_int]
        + [_ptr, _i64, _i64, _i64] * 2 + [_i64, _flt, _flt, _ptr])
    lib.pcamd_quant_block_ex.restype = _int
    lib.pcamd_quant_block_ex.argtypes = (quant_head + [_ptr, _i64, _i64, _i64, _i64, _i64, _flt, _flt, _int, _ptr])
    lib.pcamd_quant_block_dual_ex.restype = _int
    lib.pcamd_quant_block_dual_ex.argtypes = (
        [_ptr, _int, _i64, _i64, _i64, _i64, _i64, _i64] + [_ptr, _i64, _i64, _i64] * 2 + [_int]
        + [_ptr, _i64, _i64, _i64] * 2 + [_i64, _flt, _flt, _int, _ptr])
    lib.pcamd_quant_channel.restype = _int
    lib.pcamd_quant_channel.argtypes = quant_head + [_ptr, _i64, _i64, _int, _flt, _flt, _ptr]
    lib.pcamd_quant_tensor.restype = _int
    lib.pcamd_quant_tensor.argtypes = quant_head + [_ptr, _ptr, _flt, _flt, _int, _ptr]
    lib.pcamd_bmm_scaled.restype = _int
    lib.pcamd_bmm_scaled.argtypes = (
        [_ptr, _ptr, _int] + [_i64] * 4 + [_i64] * 6 + [_ptr, _int] + [_i64] * 3
        + [_ptr, _int] + [_i64] * 3 + [_ptr] + [_i64] * 3 + [_ptr] + [_i64] * 3
        + [_int, _int, _i64, _i64, _i64, _int, _ptr])
    lib.pcamd_bmm_scaled_mixed.restype = _int
    lib.pcamd_bmm_scaled_mixed.argtypes = (
        [_ptr, _int, _ptr, _int] + [_i64] * 4 + [_i64] * 6 + [_ptr, _int] + [_i64] * 3
        + [_ptr, _int] + [_i64] * 3 + [_ptr] + [_i64] * 3 + [_ptr] + [_i64] * 3
        + [_int, _int, _i64, _i64, _i64, _int, _ptr])
    lib.pcamd_bmm_quant_a.restype = _int
    lib.pcamd_bmm_quant_a.argtypes = (
        [_ptr, _int, _ptr, _int] + [_i64] * 4 + [_i64] * 6 + [_ptr, _int] + [_i64] * 3
        + [_ptr, _int] + [_i64] * 3 + [_ptr] + [_i64] * 3 + [_i64]
        + [_ptr] + [_i64] * 3 + [_ptr] + [_i64] * 3 + [_flt, _flt, _int, _ptr])
    lib.pcamd_repack_fp8.restype = _int
    lib.pcamd_repack_fp8.argtypes = [_ptr] + [_i64] * 6 + [_ptr] + [_i64] * 3 + [_ptr]
    lib.pcamd_selftest_fp8_convert.restype = _int
    lib.pcamd_selftest_fp8_convert.argtypes = [_int, _ptr, _ptr]
    lib.pcamd_selftest_copy16.restype = _int
    lib.pcamd_selftest_copy16.argtypes = [_ptr, _ptr, _i64, _ptr]
    lib.pcamd_selftest_narrow16.restype = _int
    lib.pcamd_selftest_narrow16.argtypes = [_ptr, _ptr, _i64, _ptr]


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it was not built."""
    global _LIB
    if _LIB is None:
        with _LOCK:
            if _LIB is None:
                if not os.path.exists(LIB_PATH):
                    raise ExtensionMissing(
                        f"HIP extension not built: {LIB_PATH} is missing; run "
                        "`python -m practice_cuda_amd.build` (or __graft_entry__.build())")
                handle = ctypes.CDLL(LIB_PATH)
                _declare(handle)
                _LIB = handle
    return _LIB


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dtype for the HIP path: {dtype}") from exc


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    """hipStream_t of torch's current stream on the tensor's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().pcamd_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what} failed with status {status}: {msg}")


def require_gpu_tensor(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor for the HIP path, got device {t.device}")
