"""Layout classification, validation and launch plumbing shared by the HIP impls.

Messages and conditions follow the reference wrappers
(fp8_training/fp8_bench/impls/triton_per_block.py:34-57, :153-229, :245-358;
impls/triton_per_channel.py:32-51, :222-268) so callers see the same
ValueErrors; only the kernel launch differs.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _lib
from ..registry import QuantResult

_INPUT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
_FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)
_OUT_DTYPES = (torch.bfloat16, torch.float16, torch.float32, torch.float8_e4m3fn, torch.float8_e5m2)


def matrix_layout(tensor: torch.Tensor, name: str) -> str:
    """'n-major' when the last dim is contiguous, 'k-major' when the second-last is."""
    if tensor.stride(-1) == 1:
        return "n-major"
    if tensor.stride(-2) == 1:
        return "k-major"
    raise ValueError(
        f"{name} must be contiguous along one matrix dimension; "
        f"shape={tuple(tensor.shape)}, strides={tensor.stride()}")


def a_layout(tensor: torch.Tensor) -> str:
    if tensor.stride(-1) == 1:
        return "k-major"
    if tensor.stride(-2) == 1:
        return "m-major"
    raise ValueError(
        "A must be contiguous along either K or M; "
        f"shape={tuple(tensor.shape)}, strides={tensor.stride()}")


def b_layout(tensor: torch.Tensor) -> str:
    if tensor.stride(-1) == 1:
        return "n-major"
    if tensor.stride(-2) == 1:
        return "k-major"
    raise ValueError(
        "B must be contiguous along either N or K; "
        f"shape={tuple(tensor.shape)}, strides={tensor.stride()}")


def is_power_of_two(value: int) -> bool:
    return value > 0 and (value & (value - 1)) == 0


def prepare_a_layout(value: QuantResult, layout: str) -> QuantResult:
    if layout not in ("k", "m"):
        raise ValueError(f"unknown A layout: {layout}")
    actual, expected = a_layout(value.tensor), f"{layout}-major"
    if actual != expected:
        raise ValueError(f"expected {expected} A, got {actual}")
    return value


def prepare_b_layout(value: QuantResult, layout: str) -> QuantResult:
    if layout not in ("n", "k"):
        raise ValueError(f"unknown B layout: {layout}")
    actual, expected = matrix_layout(value.tensor, "B"), f"{layout}-major"
    if actual != expected:
        raise ValueError(f"expected {expected} B, got {actual}")
    return value


def check_quant_input(x: torch.Tensor, fp8_dtype: torch.dtype, what: str) -> None:
    if x.ndim not in (2, 3):
        raise ValueError(f"{what} expects a 2D or 3D tensor, got {tuple(x.shape)}")
    if x.dtype not in _INPUT_DTYPES:
        raise ValueError(f"{what} input dtype must be float32, bfloat16 or float16, got {x.dtype}")
    if fp8_dtype not in _FP8_DTYPES:
        raise ValueError(f"{what} fp8_dtype must be float8_e4m3fn or float8_e5m2, got {fp8_dtype}")


def dims3(x: torch.Tensor, y: torch.Tensor):
    """(batch, m, n, x strides, y strides) with batch stride 0 for 2D tensors."""
    if x.ndim == 2:
        m, n = x.shape
        return 1, m, n, (0, x.stride(0), x.stride(1)), (0, y.stride(0), y.stride(1))
    b, m, n = x.shape
    return b, m, n, tuple(x.stride()), tuple(y.stride())


def repack_rows_major(x: torch.Tensor) -> torch.Tensor:
    """Contiguous copy of a 3-D fp8 view that is contiguous along dim -2: the
    transposing copy of the do_transpose_a / do_transpose_b variants
    (reference: `.contiguous()` of the strided view,
    fp8_training/fp8_bench/impls/triton_per_block.py:254-272), made on the GPU
    by pcamd_repack_fp8. Tensors off the GPU take torch's copy, and so do the
    views the kernel does not take: a single row or column (its other stride
    is arbitrary), columns that overlap the rows they step over (expanded
    views), and shapes past the kernel's grid (PCAMD_ERR_UNSUPPORTED: more
    than 65535 batches or 65535 x 128 rows)."""
    if not x.is_cuda or x.stride(-2) != 1 or x.element_size() != 1 or min(x.shape[-2:]) <= 1:
        return x.contiguous()
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    if y.numel() == 0:
        return y
    bsz, rows, cols = x.shape
    sxb = x.stride(0) if bsz > 1 else 0
    if x.stride(2) < rows or sxb < 0:
        return x.contiguous()
    rc = _lib.lib().pcamd_repack_fp8(
        _lib.ptr(x), bsz, rows, cols, sxb, x.stride(1), x.stride(2),
        _lib.ptr(y), y.stride(0), y.stride(1), y.stride(2), _lib.stream_of(y))
    if rc == _lib.ERR_UNSUPPORTED:
        return x.contiguous()
    _lib.check(rc, "pcamd_repack_fp8")
    return y


def prepare_operands(a: QuantResult, b: QuantResult, do_transpose_a: bool, do_transpose_b: bool,
                     activation: str, b_layout_fn=matrix_layout):
    """Shared BMM front end (reference impls/triton_per_block.py:245-292)."""
    if a.tensor.ndim != 3 or b.tensor.ndim != 3:
        raise ValueError("BMM expects 3D quantized tensors")
    if activation not in ("none", "gelu"):
        raise ValueError(f"activation must be 'none' or 'gelu', got {activation!r}")

    in_a = a_layout(a.tensor)
    if do_transpose_a:
        if in_a != "m-major":
            raise ValueError(
                f"do_transpose_a=True requires an M-major A input; strides={a.tensor.stride()}")
        a_tensor = repack_rows_major(a.tensor)
    else:
        a_tensor = a.tensor

    if b_layout_fn is matrix_layout:
        in_b = matrix_layout(b.tensor, "B")
    else:
        in_b = b_layout_fn(b.tensor)
    if do_transpose_b:
        if in_b != "n-major":
            raise ValueError(
                f"do_transpose_b=True requires an N-major B input; strides={b.tensor.stride()}")
        b_tensor = repack_rows_major(b.tensor.transpose(-1, -2)).transpose(-1, -2)
    else:
        b_tensor = b.tensor

    batch, m, k = a_tensor.shape
    b_batch, b_k, n = b_tensor.shape
    if batch != b_batch or k != b_k:
        raise ValueError(f"shape mismatch: A={tuple(a_tensor.shape)}, B={tuple(b_tensor.shape)}")
    if a_tensor.device != b_tensor.device:
        raise ValueError(
            f"A and B must be on the same device: A={a_tensor.device}, B={b_tensor.device}")
    if a_tensor.dtype != b_tensor.dtype:
        raise ValueError(
            f"A and B must have the same FP8 dtype: A={a_tensor.dtype}, B={b_tensor.dtype}")
    if a_tensor.dtype not in _FP8_DTYPES:
        raise ValueError(f"A and B must be FP8 tensors, got {a_tensor.dtype}")
    return a_tensor, b_tensor, batch, m, n, k


def prepare_out(out: Optional[torch.Tensor], out_dtype: torch.dtype, batch: int, m: int, n: int,
                device: torch.device) -> torch.Tensor:
    if out_dtype not in _OUT_DTYPES:
        raise ValueError(f"unsupported out_dtype for the HIP BMM: {out_dtype}")
    if out is None:
        return torch.empty((batch, m, n), device=device, dtype=out_dtype)
    if out.shape != (batch, m, n):
        raise ValueError(f"out must have shape {(batch, m, n)}, got {tuple(out.shape)}")
    if out.device != device:
        raise ValueError(f"out must be on {device}, got {out.device}")
    if out.dtype != out_dtype:
        raise ValueError(f"out must have dtype {out_dtype}, got {out.dtype}")
    if out.stride(-1) != 1:
        raise ValueError(
            f"out must be contiguous along N; shape={tuple(out.shape)}, strides={out.stride()}")
    return out


def check_bias(bias: Optional[torch.Tensor], batch: int, m: int, n: int, device: torch.device,
               require_n_contiguous: bool = True):
    if bias is None:
        return None, (0, 0, 0), 0
    if bias.shape != (batch, m, n):
        raise ValueError(f"bias must have shape {(batch, m, n)}, got {tuple(bias.shape)}")
    if bias.device != device:
        raise ValueError(f"bias must be on {device}, got {bias.device}")
    if require_n_contiguous and bias.stride(-1) != 1:
        raise ValueError(
            f"bias must be contiguous along N; shape={tuple(bias.shape)}, strides={bias.stride()}")
    if bias.dtype not in _INPUT_DTYPES:
        raise ValueError(f"bias dtype must be float32, bfloat16 or float16, got {bias.dtype}")
    return bias, tuple(bias.stride()), _lib.dtype_code(bias.dtype)


def launch_bmm(a_tensor, b_tensor, out, bias, bias_strides, bias_code, sa, sa_strides, sb,
               sb_strides, scale_mode, scales_are_quant, qbm, qbk, qbn, activation,
               batch, m, n, k) -> torch.Tensor:
    _lib.require_gpu_tensor(a_tensor, "A")
    L = _lib.lib()
    # one fp8 format for both operands (the registry wrappers' contract), or
    # one each (the training layer's e5m2 gradient times an e4m3 operand)
    fmt = ((_lib.dtype_code(a_tensor.dtype),) if a_tensor.dtype == b_tensor.dtype
           else (_lib.dtype_code(a_tensor.dtype), _lib.dtype_code(b_tensor.dtype)))
    entry = L.pcamd_bmm_scaled if len(fmt) == 1 else L.pcamd_bmm_scaled_mixed
    with torch.cuda.device(a_tensor.device):
        rc = entry(
            *((_lib.ptr(a_tensor), _lib.ptr(b_tensor), fmt[0]) if len(fmt) == 1
              else (_lib.ptr(a_tensor), fmt[0], _lib.ptr(b_tensor), fmt[1])),
            batch, m, n, k,
            *a_tensor.stride(), *b_tensor.stride(),
            _lib.ptr(out), _lib.dtype_code(out.dtype), *out.stride(),
            _lib.ptr(bias), bias_code, *bias_strides,
            _lib.ptr(sa), *sa_strides, _lib.ptr(sb), *sb_strides,
            scale_mode, int(scales_are_quant), qbm, qbk, qbn,
            _lib.ACT_GELU if activation == "gelu" else _lib.ACT_NONE,
            _lib.stream_of(a_tensor))
    _lib.check(rc, "pcamd_bmm_scaled" if len(fmt) == 1 else "pcamd_bmm_scaled_mixed")
    return out
