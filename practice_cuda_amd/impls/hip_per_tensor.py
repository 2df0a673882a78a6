"""Per-tensor FP8 quantizer and scalar-scaled BMM.

Drop-in for fp8_training/fp8_bench/impls/triton_per_tensor.py of
xuOAO/practice_cuda (``triton_per_tensor_quant`` :28-95,
``triton_per_tensor_bmm`` :140-306, registrations :321-398). The amax, the
scale and the cast all run on the GPU in csrc/quant.hip (the reference
computes the amax and scale with torch reductions before its kernel).
"""
from __future__ import annotations

from functools import partial
from typing import Optional

import torch

from .. import _lib
from ..registry import QuantResult, register_bmm, register_quant
from . import _common as C


def quant_tensor_raw(x: torch.Tensor, fp8_dtype: torch.dtype, eps: float, *,
                     fp8_max: float | None = None, scale_dtype: torch.dtype = torch.float32):
    """Launch the per-tensor kernels; returns (fp8 tensor, dequant scale, quant scale).

    scale_dtype is the dtype the scalar scale steps are rounded to (fp32 for
    the fp8_bench path; the input's dtype for the legacy fp8_warper API), or
    torch.float64 for torchao's tensorwise scale (reference
    modules/float8/float8_utils.py:45-48: qs = fp32(fp8_max / max(fp64(amax),
    eps)), dequant = its fp32 reciprocal), which the reference's training
    layer quantizes with. fp8_max defaults to the fp8 format's largest finite
    value.
    """
    output = torch.empty_like(x, dtype=fp8_dtype, memory_format=torch.preserve_format)
    batch, m, n, xs, ys = C.dims3(x, output)
    scales = torch.empty(2, device=x.device, dtype=torch.float32)
    L = _lib.lib()
    _lib.require_gpu_tensor(x, "x")
    with torch.cuda.device(x.device):
        rc = L.pcamd_quant_tensor(
            _lib.ptr(x), _lib.dtype_code(x.dtype), batch, m, n, *xs,
            _lib.ptr(output), _lib.dtype_code(fp8_dtype), *ys,
            _lib.ptr(scales[0:1]), _lib.ptr(scales[1:2]),
            float(torch.finfo(fp8_dtype).max if fp8_max is None else fp8_max), float(eps),
            _lib.F64 if scale_dtype == torch.float64 else _lib.dtype_code(scale_dtype), _lib.stream_of(x))
    _lib.check(rc, "pcamd_quant_tensor")
    return output, scales[0], scales[1]


def hip_per_tensor_quant(
    x: torch.Tensor,
    *,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    eps: float = 1e-12,
    profile: bool = False,
) -> QuantResult:
    del profile
    if x.ndim not in (2, 3):
        raise ValueError(f"per-tensor quant expects a 2D or 3D tensor, got shape={tuple(x.shape)}")
    C.check_quant_input(x, fp8_dtype, "per-tensor quant")
    _lib.require_gpu_tensor(x, "x")
    output, dequant_scale, _ = quant_tensor_raw(x, fp8_dtype, eps)
    return QuantResult(
        tensor=output,
        dequant_scale=dequant_scale,
        impl="hip_per_tensor",
        granularity="tensor",
        meta={"logical_shape": tuple(x.shape), "fp8_dtype": str(fp8_dtype)},
    )


def hip_per_tensor_bmm(
    a: QuantResult,
    b: QuantResult,
    *,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    do_transpose_a: bool = False,
    do_transpose_b: bool = False,
    dequant_scale: Optional[torch.Tensor] = None,
    profile: bool = False,
    use_tma: bool = False,
    activation: str = "none",
) -> torch.Tensor:
    """Scalar-scaled FP8 BMM: (A @ B) * dequant_scale (default sa * sb)."""
    del profile, use_tma
    a_tensor, b_tensor, batch, m, n, k = C.prepare_operands(
        a, b, do_transpose_a, do_transpose_b, activation, b_layout_fn=C.b_layout)
    out = C.prepare_out(out, out_dtype, batch, m, n, a_tensor.device)
    bias, bias_strides, bias_code = C.check_bias(bias, batch, m, n, a_tensor.device,
                                                 require_n_contiguous=False)
    if dequant_scale is None:
        dequant_scale = a.dequant_scale * b.dequant_scale
    if dequant_scale.numel() != 1:
        raise ValueError(
            "per-tensor BMM expects one combined dequant scale, "
            f"got shape={tuple(dequant_scale.shape)}")
    if dequant_scale.dtype != torch.float32:
        raise ValueError(f"dequant_scale must be float32, got {dequant_scale.dtype}")
    if dequant_scale.device != a_tensor.device:
        raise ValueError(
            "dequant_scale must be on the same device as A and B: "
            f"scale={dequant_scale.device}, tensors={a_tensor.device}")
    return C.launch_bmm(
        a_tensor, b_tensor, out, bias, bias_strides, bias_code,
        dequant_scale, (0, 0, 0), None, (0, 0, 0),
        _lib.SCALE_TENSOR, False, 1, 128, 1, activation, batch, m, n, k)


def _combined(a: QuantResult, b: QuantResult) -> dict:
    return {"dequant_scale": a.dequant_scale * b.dequant_scale}


register_quant(
    "hip_per_tensor",
    hip_per_tensor_quant,
    "Per-tensor scale quantization; supports E4M3 and E5M2.",
)
_PT = {"quant_impl": "hip_per_tensor", "prepare_call_kwargs": _combined}
register_bmm(
    "hip_per_tensor_a_k_b_n", partial(hip_per_tensor_bmm, do_transpose_b=False),
    layout="n", prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="FP8 BMM with contiguous [B,K,N] right operand.", **_PT)
register_bmm(
    "hip_per_tensor_a_k_b_k", partial(hip_per_tensor_bmm, do_transpose_b=False),
    layout="k", prepare_b=lambda v: C.prepare_b_layout(v, "k"),
    description="FP8 BMM with a prepacked K-major [B,K,N] right operand.", **_PT)
register_bmm(
    "hip_per_tensor_a_k_b_n_transpose", partial(hip_per_tensor_bmm, do_transpose_b=True),
    layout="n", prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="N-major FP8 BMM with explicit N-to-K packing inside the call.", **_PT)
register_bmm(
    "hip_per_tensor_a_m_b_n",
    partial(hip_per_tensor_bmm, do_transpose_a=False, do_transpose_b=False),
    a_layout="m", layout="n",
    prepare_a=lambda v: C.prepare_a_layout(v, "m"), prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="FP8 BMM with direct M-major A and N-major B operands.", **_PT)
register_bmm(
    "hip_per_tensor_a_m_transpose_b_n_transpose",
    partial(hip_per_tensor_bmm, do_transpose_a=True, do_transpose_b=True),
    a_layout="m", layout="n",
    prepare_a=lambda v: C.prepare_a_layout(v, "m"), prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="M-major A and N-major B with both operands packed inside the BMM call.", **_PT)
