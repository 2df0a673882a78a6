"""Legacy tuple API of kernels/fp8_bmm (per-tensor quant + scalar-scaled BMM).

Drop-in for xuOAO/practice_cuda ``kernels/fp8_bmm/fp8_warper.py``:

* ``fp8_quant(x, quant_dtype, fp8_range, eps, is_test)`` replaces
  ``fp8_quant_triton`` (fp8_warper.py:9-77) and returns ``(q, reciprocal)``.
  The reference computes the scale with torch ops on 0-d tensors of x's dtype
  (fp8_warper.py:21-25):
  ``qs = reciprocal(max(|min|, |max|).clamp(eps)) * fp8_range`` and
  ``reciprocal = reciprocal(qs)``. For bf16 / fp16 inputs every step is
  therefore rounded to that dtype, and the returned reciprocal has x's
  dtype. Its kernel (kernel/fp8_quant_kernel.py:56-60) computes
  ``fp8(clamp(float(x) * qs, -fp8_range, fp8_range))``.
* ``fp8_bmm_quant(A, B, bias, *, quant_scale, out_dtype, is_test)`` replaces
  ``fp8_bmm_quant_triton`` (fp8_warper.py:79-129; kernel
  kernel/fp8_quant_bmm_kernel.py:31-132):
  ``C = ((A @ B) * quant_scale + bias).to(out_dtype)`` with fp32
  accumulation.

Both run entirely in libpcamd_fp8.so: the amax, the scale steps and the cast
in ``pcamd_quant_tensor`` (with ``scale_dtype`` = x's dtype), the GEMM in
``pcamd_bmm_scaled`` (tensor scale mode). The reference's names are kept as
aliases (``fp8_quant_triton``, ``fp8_bmm_quant_triton``) so callers can swap
the import; ``is_test`` (which picks a fixed Triton config there) is accepted
and ignored.
"""
from __future__ import annotations

from enum import Enum
from typing import NamedTuple, Optional, Union

import torch

from . import _lib
from .impls import _common as C
from .impls.hip_per_tensor import quant_tensor_raw


class _FormatHelper(NamedTuple):
    max_fwd: float
    max_bwd: float
    dtype_fwd: torch.dtype
    dtype_bwd: torch.dtype


class FP8Format(Enum):
    """Same members and values as kernels/fp8_bmm/fp8_utils.py:11-31."""

    E4M3 = _FormatHelper(448.0, 448.0, torch.float8_e4m3fn, torch.float8_e4m3fn)
    E5M2 = _FormatHelper(57344.0, 57344.0, torch.float8_e5m2, torch.float8_e5m2)
    HYBRID = _FormatHelper(448.0, 57344.0, torch.float8_e4m3fn, torch.float8_e5m2)


_SCALE_DTYPES = (torch.float32, torch.bfloat16, torch.float16)
_OUT_DTYPES = (torch.float32, torch.bfloat16, torch.float16, torch.float8_e4m3fn, torch.float8_e5m2)


def fp8_quant(
    x: torch.Tensor,
    quant_dtype: Union[torch.dtype, FP8Format] = FP8Format.E4M3.value.dtype_fwd,
    fp8_range: float = FP8Format.E4M3.value.max_fwd,
    eps: float = 1e-12,
    is_test: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-tensor fp8 quantization; returns ``(q, reciprocal_factor)``.

    ``q`` has x's shape and strides (``empty_like``); ``reciprocal_factor`` is
    a 0-d tensor of x's dtype holding ``1 / quant_factor``.
    """
    del is_test
    if isinstance(quant_dtype, FP8Format):
        quant_dtype = quant_dtype.value.dtype_fwd
    if x.dim() not in (2, 3):
        raise RuntimeError("dim must eq 2 or 3")
    if x.dtype not in _SCALE_DTYPES:
        raise ValueError(f"x must be float32, bfloat16 or float16, got {x.dtype}")
    if quant_dtype not in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise ValueError(f"quant_dtype must be float8_e4m3fn or float8_e5m2, got {quant_dtype}")
    q, dequant, _ = quant_tensor_raw(x, quant_dtype, eps, fp8_max=float(fp8_range), scale_dtype=x.dtype)
    # the scale steps were rounded to x's dtype on the GPU, so this cast is exact
    return q, dequant.to(x.dtype)


def fp8_bmm_quant(
    A: torch.Tensor,
    B: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    *,
    quant_scale: Union[torch.Tensor, float],
    out_dtype: torch.dtype = torch.float16,
    is_test: bool = False,
) -> torch.Tensor:
    """``C[b] = (A[b] @ B[b]) * quant_scale (+ bias[b])``, cast to out_dtype.

    A: fp8 [Bs, M, K]; B: fp8 [Bs, K, N] of the same fp8 dtype. bias: [Bs, M, N]
    or [M, N] (broadcast over the batch), float32 / bfloat16 / float16.
    quant_scale: a one-element tensor (any float dtype, read as fp32) or a
    Python number.
    """
    del is_test
    if A.dim() != 3 or B.dim() != 3:
        raise ValueError(f"A and B must be 3-D (B,M,K) and (B,K,N); got {tuple(A.shape)} and {tuple(B.shape)}")
    bs, m, k = A.shape
    if B.shape[0] != bs or B.shape[1] != k:
        raise ValueError(f"shape mismatch: A {tuple(A.shape)}, B {tuple(B.shape)}")
    n = B.shape[2]
    if A.dtype != B.dtype or A.dtype not in (torch.float8_e4m3fn, torch.float8_e5m2):
        raise ValueError(f"A and B must share an fp8 dtype, got {A.dtype} and {B.dtype}")
    if A.device != B.device:
        raise ValueError(f"A and B must be on the same device, got {A.device} and {B.device}")
    if out_dtype not in _OUT_DTYPES:
        raise ValueError(f"unsupported out_dtype {out_dtype}")
    _lib.require_gpu_tensor(A, "A")
    # the kernels read A along K or M and B along N or K; other strides
    # (which the reference's block pointers accept) are packed first
    if A.stride(2) != 1 and A.stride(1) != 1:
        A = A.contiguous()
    if B.stride(2) != 1 and B.stride(1) != 1:
        B = B.contiguous()
    if not torch.is_tensor(quant_scale):
        quant_scale = torch.tensor(float(quant_scale), device=A.device, dtype=torch.float32)
    if quant_scale.numel() != 1:
        raise ValueError(f"quant_scale must hold one value, got shape {tuple(quant_scale.shape)}")
    if quant_scale.device != A.device:
        raise ValueError(f"quant_scale must be on {A.device}, got {quant_scale.device}")
    # kernel/fp8_quant_bmm_kernel.py:115 loads the scale in its own dtype and
    # multiplies the fp32 accumulator: widening to fp32 is exact
    scale = quant_scale.reshape(1).to(torch.float32)
    if bias is not None:
        if bias.dim() == 2:
            if tuple(bias.shape) != (m, n):
                raise ValueError(f"2-D bias must have shape {(m, n)}, got {tuple(bias.shape)}")
            bias = bias.unsqueeze(0).expand(bs, m, n)  # batch stride 0: no copy
        bias, bias_strides, bias_code = C.check_bias(bias, bs, m, n, A.device, require_n_contiguous=False)
    else:
        bias_strides, bias_code = (0, 0, 0), 0
    out = torch.empty((bs, m, n), dtype=out_dtype, device=A.device)
    return C.launch_bmm(A, B, out, bias, bias_strides, bias_code, scale, (0, 0, 0), None, (0, 0, 0),
                        _lib.SCALE_TENSOR, False, 1, 128, 1, "none", bs, m, n, k)


# the reference's names, for an import swap
fp8_quant_triton = fp8_quant
fp8_bmm_quant_triton = fp8_bmm_quant

__all__ = ["FP8Format", "fp8_quant", "fp8_bmm_quant", "fp8_quant_triton", "fp8_bmm_quant_triton"]
