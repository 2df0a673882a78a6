"""TEST INFRASTRUCTURE ONLY - CPU oracle for the FP8 hot path.

Restates the reference's arithmetic (xuOAO/practice_cuda) on the CPU so the
HIP kernels can be checked against it. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module; the product package never does.

* Quantizers: thin ctypes wrappers over ``fp8_oracle.c`` (built by
  ``oracle/Makefile`` into ``oracle/_build/liboracle.so``), which follows
  ``fp8_training/fp8_bench/kernels/quant/per_block.py:35-48``,
  ``kernels/quant/per_channel.py:136-267`` and
  ``impls/triton_per_tensor.py:40-44``.
* Dequantize: ``fp8_training/fp8_bench/registry.py:18-70`` restated in numpy.
* BMM reference: fp64 matmul of the dequantized operands, as the reference's
  accuracy oracle ``bench_bmm.py:414-419`` does in fp32, followed by the
  kernel epilogue order of ``kernels/bmm/per_block.py:108-137`` (scale, bias,
  activation ``kernels/bmm/activation.py:12-19``, cast).

Parity status of every function is listed in the module docstring of
``tests/test_oracle.py`` together with the check that pins it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_LIB = None

F32, BF16, F16, E4M3, E5M2 = 0, 1, 2, 3, 4
F64 = 5  # scale arithmetic only: torchao's tensorwise form
FP8_MAX = {E4M3: 448.0, E5M2: 57344.0}
_FMT_NAMES = {"e4m3": E4M3, "e4m3fn": E4M3, "e5m2": E5M2, E4M3: E4M3, E5M2: E5M2}
_DT_NAMES = {"f32": F32, "fp32": F32, "float32": F32, "bf16": BF16, "bfloat16": BF16,
             "f16": F16, "fp16": F16, "float16": F16}

_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.oracle_encode_e4m3fn.restype = ctypes.c_uint8
        L.oracle_encode_e4m3fn.argtypes = [ctypes.c_float]
        L.oracle_encode_e5m2.restype = ctypes.c_uint8
        L.oracle_encode_e5m2.argtypes = [ctypes.c_float]
        L.oracle_decode_fp8.restype = ctypes.c_float
        L.oracle_decode_fp8.argtypes = [ctypes.c_uint8, ctypes.c_int]
        L.oracle_encode_array.restype = None
        L.oracle_encode_array.argtypes = [_ptr, _ptr, _i64, ctypes.c_int]
        L.oracle_quant_block.restype = ctypes.c_int
        L.oracle_quant_block.argtypes = (
            [_ptr, ctypes.c_int] + [_i64] * 6 + [_ptr, ctypes.c_int] + [_i64] * 3
            + [_ptr] + [_i64] * 5 + [ctypes.c_float, ctypes.c_float, ctypes.c_int])
        L.oracle_quant_channel.restype = ctypes.c_int
        L.oracle_quant_channel.argtypes = (
            [_ptr, ctypes.c_int] + [_i64] * 6 + [_ptr, ctypes.c_int] + [_i64] * 3
            + [_ptr, _i64, _i64, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.c_int])
        L.oracle_quant_tensor.restype = ctypes.c_int
        L.oracle_quant_tensor.argtypes = (
            [_ptr, ctypes.c_int] + [_i64] * 6 + [_ptr, ctypes.c_int] + [_i64] * 3
            + [_ptr, _ptr, ctypes.c_float, ctypes.c_float, ctypes.c_int])
        L.oracle_round_dt.restype = ctypes.c_float
        L.oracle_round_dt.argtypes = [ctypes.c_float, ctypes.c_int]
        _LIB = L
    return _LIB


def fmt_code(fmt) -> int:
    if isinstance(fmt, str) or isinstance(fmt, int):
        return _FMT_NAMES[fmt]
    name = str(fmt)
    if "e5m2" in name:
        return E5M2
    if "e4m3" in name:
        return E4M3
    raise ValueError(f"unknown fp8 format {fmt!r}")


def as_bits(x, dtype: Optional[str] = None) -> tuple[np.ndarray, int]:
    """Return (numpy array holding the raw elements, dtype code).

    Accepts numpy arrays (float32 / float16, or uint16 bf16 bits with
    ``dtype="bf16"``) and CPU torch tensors (float32 / bfloat16 / float16).
    """
    try:
        import torch  # local: the oracle itself only needs numpy
        if isinstance(x, torch.Tensor):
            x = x.detach().cpu()
            if x.dtype == torch.bfloat16:
                return x.contiguous().view(torch.int16).numpy().view(np.uint16), BF16
            if x.dtype == torch.float16:
                return x.contiguous().numpy(), F16
            if x.dtype == torch.float32:
                return x.contiguous().numpy(), F32
            raise ValueError(f"unsupported oracle input dtype {x.dtype}")
    except ImportError:  # pragma: no cover
        pass
    x = np.ascontiguousarray(x)
    if dtype is not None:
        return x, _DT_NAMES[dtype]
    if x.dtype == np.float32:
        return x, F32
    if x.dtype == np.float16:
        return x, F16
    raise ValueError("pass dtype='bf16' for uint16 bf16 bit patterns")


def _dims(arr: np.ndarray):
    if arr.ndim == 2:
        b, (m, n) = 1, arr.shape
        sxb = 0
        sxm, sxn = (s // arr.itemsize for s in arr.strides)
    elif arr.ndim == 3:
        b, m, n = arr.shape
        sxb, sxm, sxn = (s // arr.itemsize for s in arr.strides)
    else:
        raise ValueError(f"expected 2D or 3D input, got {arr.shape}")
    return b, m, n, sxb, sxm, sxn


def encode(values: np.ndarray, fmt="e4m3") -> np.ndarray:
    """fp32 -> fp8 bytes (round to nearest even, no clamping)."""
    v = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty(v.shape, dtype=np.uint8)
    lib().oracle_encode_array(v.ctypes.data, out.ctypes.data, v.size, fmt_code(fmt))
    return out


_DECODE_CACHE: dict[int, np.ndarray] = {}


def decode_table(fmt="e4m3") -> np.ndarray:
    code = fmt_code(fmt)
    if code not in _DECODE_CACHE:
        L = lib()
        _DECODE_CACHE[code] = np.array(
            [L.oracle_decode_fp8(i, code) for i in range(256)], dtype=np.float32)
    return _DECODE_CACHE[code]


def decode(q: np.ndarray, fmt="e4m3") -> np.ndarray:
    return decode_table(fmt)[np.asarray(q, dtype=np.uint8)]


def quant_block(x, block_m: int, block_n: int, fmt="e4m3", eps: float = 1e-12,
                dtype: Optional[str] = None, threads: int = 1,
                fp8_max: Optional[float] = None):
    """Per-block quantization; returns (q uint8 [.., m, n], scale fp32).

    The scale has the reference's shape: [m_blocks, n_blocks] for 2D input
    (``impls/triton_per_block.py:96-100,138``) and [b, m_blocks, n_blocks]
    for 3D input. fp8_max defaults to the format's largest finite value.
    """
    arr, xd = as_bits(x, dtype)
    b, m, n, sxb, sxm, sxn = _dims(arr)
    code = fmt_code(fmt)
    mb, nb = -(-m // block_m), -(-n // block_n)
    q = np.empty((b, m, n), dtype=np.uint8)
    s = np.empty((b, mb, nb), dtype=np.float32)
    rc = lib().oracle_quant_block(
        arr.ctypes.data, xd, b, m, n, sxb, sxm, sxn, q.ctypes.data, code,
        m * n, n, 1, s.ctypes.data, mb * nb, nb, 1, block_m, block_n,
        FP8_MAX[code] if fp8_max is None else fp8_max, eps, threads)
    if rc != 0:
        raise ValueError("oracle_quant_block rejected its arguments")
    if arr.ndim == 2:
        return q[0], s[0]
    return q, s


def quant_channel(x, channel_axis: int = -1, fmt="e4m3", eps: float = 1e-12,
                  dtype: Optional[str] = None, threads: int = 1,
                  fp8_max: Optional[float] = None):
    """Per-channel quantization; scale [channels] (2D) or [b, channels]."""
    arr, xd = as_bits(x, dtype)
    b, m, n, sxb, sxm, sxn = _dims(arr)
    code = fmt_code(fmt)
    ch = m if channel_axis == -2 else n
    q = np.empty((b, m, n), dtype=np.uint8)
    s = np.empty((b, ch), dtype=np.float32)
    rc = lib().oracle_quant_channel(
        arr.ctypes.data, xd, b, m, n, sxb, sxm, sxn, q.ctypes.data, code,
        m * n, n, 1, s.ctypes.data, ch, 1, channel_axis,
        FP8_MAX[code] if fp8_max is None else fp8_max, eps, threads)
    if rc != 0:
        raise ValueError("oracle_quant_channel rejected its arguments")
    if arr.ndim == 2:
        return q[0], s[0]
    return q, s


def quant_tensor(x, fmt="e4m3", eps: float = 1e-12, dtype: Optional[str] = None,
                 scale_dt: Optional[int] = None, fp8_max: Optional[float] = None):
    """Per-tensor quantization; returns (q, dequant_scale, quant_scale).

    scale_dt (F32 / BF16 / F16) is the dtype of the scale arithmetic: F32 for
    impls/triton_per_tensor.py, the input's dtype for the legacy
    kernels/fp8_bmm/fp8_warper.py:21-25 (pass ``scale_dt="input"``). F64 is
    torchao's tensorwise scale (modules/float8/float8_utils.py:45-48):
    qs = fp32(fp8_max / max(fp64(amax), eps)), dequant = fp32 reciprocal.
    fp8_max defaults to the format's largest finite value (the legacy API's
    fp8_range argument can override it).
    """
    arr, xd = as_bits(x, dtype)
    b, m, n, sxb, sxm, sxn = _dims(arr)
    code = fmt_code(fmt)
    sdt = xd if scale_dt == "input" else (F32 if scale_dt is None else scale_dt)
    q = np.empty((b, m, n), dtype=np.uint8)
    ds = np.zeros(1, dtype=np.float32)
    qs = np.zeros(1, dtype=np.float32)
    lib().oracle_quant_tensor(arr.ctypes.data, xd, b, m, n, sxb, sxm, sxn,
                              q.ctypes.data, code, m * n, n, 1, ds.ctypes.data,
                              qs.ctypes.data, FP8_MAX[code] if fp8_max is None else fp8_max, eps, sdt)
    q = q[0] if arr.ndim == 2 else q
    return q, ds[0], qs[0]


def round_dt(v: float, dtype: int) -> float:
    """oracle_round_dt: RNE of an fp32 value to bf16 / fp16 (identity for F32)."""
    return float(lib().oracle_round_dt(ctypes.c_float(v), dtype))


# ---------------------------------------------------------------------------
# dequantize (registry.py:18-70) and the BMM reference
# ---------------------------------------------------------------------------

def dequant_block(q: np.ndarray, scale: np.ndarray, block_m: int, block_n: int,
                  fmt="e4m3") -> np.ndarray:
    """registry.py:38-69: expand block scales with arange//block and multiply."""
    v = decode(q, fmt).astype(np.float64)
    m, n = q.shape[-2:]
    rows = np.arange(m) // block_m
    cols = np.arange(n) // block_n
    s = np.asarray(scale, dtype=np.float32).astype(np.float64)
    s = np.take(np.take(s, rows, axis=-2), cols, axis=-1)
    return v * s


def dequant_channel(q: np.ndarray, scale: np.ndarray, channel_axis: int,
                    fmt="e4m3") -> np.ndarray:
    """registry.py:22-33: unsqueeze the per-channel scale and multiply."""
    v = decode(q, fmt).astype(np.float64)
    s = np.asarray(scale, dtype=np.float32).astype(np.float64)
    s = np.expand_dims(s, -1 if channel_axis == -2 else -2)
    return v * s


def dequant_tensor(q: np.ndarray, scale: float, fmt="e4m3") -> np.ndarray:
    return decode(q, fmt).astype(np.float64) * float(np.float32(scale))


def gelu_exact(x: np.ndarray) -> np.ndarray:
    """kernels/bmm/activation.py:12-19: 0.5 x (1 + erf(x / sqrt 2))."""
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x * 0.7071067811865475))


def bmm_reference(a_deq: np.ndarray, b_deq: np.ndarray, bias=None,
                  activation: str = "none") -> np.ndarray:
    """fp64 [B,M,K] @ [B,K,N] of dequantized operands, then bias, activation.

    bench_bmm.py:414-419 computes the kernel reference as
    ``torch.bmm(qa.dequantize(), qb.dequantize())`` (+ bias); the kernels
    apply the activation after the bias (kernels/bmm/per_block.py:113-137).
    """
    out = np.matmul(np.asarray(a_deq, np.float64), np.asarray(b_deq, np.float64))
    if bias is not None:
        out = out + np.asarray(bias, np.float64)
    if activation == "gelu":
        out = gelu_exact(out)
    return out


def max_abs_rel(actual: np.ndarray, expected: np.ndarray) -> float:
    """max |actual - expected| / max |expected| (0 when both are all zero)."""
    actual = np.asarray(actual, np.float64)
    expected = np.asarray(expected, np.float64)
    denom = float(np.max(np.abs(expected))) if expected.size else 0.0
    diff = float(np.max(np.abs(actual - expected))) if expected.size else 0.0
    if denom == 0.0:
        return diff
    return diff / denom
