"""Per-channel FP8 quantizer and channel-scaled BMM.

Drop-in for fp8_training/fp8_bench/impls/triton_per_channel.py of
xuOAO/practice_cuda: ``hip_per_channel_quant`` mirrors
``triton_per_channel_quant`` (:90-219) and ``hip_per_channel_bmm`` mirrors
``triton_per_channel_bmm`` (:271-427).

Both the ``one_pass`` and the default ("two_pass") modes run the same HIP
kernels: rows up to 8192 elements are held in registers and read from HBM
once; longer reductions and column (channel_axis=-1) reductions take a
second pass over the data. ``one_pass=True`` keeps the reference's limit and
error (reduction size 1..4096) and its metadata so callers see the same
contract.
"""
from __future__ import annotations

from functools import partial
from typing import Optional

import torch

from .. import _lib
from ..registry import QuantResult, register_bmm, register_quant
from . import _common as C


def hip_per_channel_quant(
    x: torch.Tensor,
    *,
    channel_axis: int = -1,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    eps: float = 1e-12,
    profile: bool = False,
    one_pass: bool = False,
) -> QuantResult:
    """channel_axis=-2: one scale per row; channel_axis=-1: one per column."""
    del profile
    if x.ndim not in (2, 3):
        raise ValueError(f"per-channel quant expects a 2D or 3D tensor, got {tuple(x.shape)}")
    if channel_axis not in (-1, -2):
        raise ValueError(f"channel_axis must be -1 or -2, got {channel_axis}")
    C.matrix_layout(x, "quant input")
    C.check_quant_input(x, fp8_dtype, "per-channel quant")
    m, n = x.shape[-2:]
    reduction = n if channel_axis == -2 else m
    if one_pass:
        if reduction == 0:
            raise ValueError("one-pass per-channel quant requires a non-empty reduction")
        if reduction > 4096:
            raise ValueError(
                f"one-pass per-channel quant supports reduction sizes up to 4096, got {reduction}")
    _lib.require_gpu_tensor(x, "x")

    output = torch.empty_like(x, dtype=fp8_dtype, memory_format=torch.preserve_format)
    C.matrix_layout(output, "quant output")
    batch, m, n, xs, ys = C.dims3(x, output)
    channels = m if channel_axis == -2 else n
    scale_storage = torch.empty((batch, channels), device=x.device, dtype=torch.float32)

    L = _lib.lib()
    with torch.cuda.device(x.device):
        rc = L.pcamd_quant_channel(
            _lib.ptr(x), _lib.dtype_code(x.dtype), batch, m, n, *xs,
            _lib.ptr(output), _lib.dtype_code(fp8_dtype), *ys,
            _lib.ptr(scale_storage), *scale_storage.stride(), channel_axis,
            float(torch.finfo(fp8_dtype).max), float(eps), _lib.stream_of(x))
    _lib.check(rc, "pcamd_quant_channel")

    dequant_scale = scale_storage.squeeze(0) if x.ndim == 2 else scale_storage
    return QuantResult(
        tensor=output,
        dequant_scale=dequant_scale,
        impl="hip_per_channel_one_pass" if one_pass else "hip_per_channel",
        granularity="channel",
        meta={
            "logical_shape": tuple(x.shape),
            "fp8_dtype": str(fp8_dtype),
            "channel_axis": channel_axis,
            "quant_strategy": "one_pass" if one_pass else "two_pass",
        },
    )


def _validate_scale(value: QuantResult, *, expected_shape, expected_axis: int, operand: str) -> None:
    scale = value.dequant_scale
    if scale.shape != expected_shape:
        raise ValueError(
            f"{operand} dequant scale must have shape {expected_shape}, got {tuple(scale.shape)}")
    if scale.dtype != torch.float32:
        raise ValueError(f"{operand} dequant scale must be float32, got {scale.dtype}")
    if scale.device != value.tensor.device:
        raise ValueError(f"{operand} dequant scale must be on {value.tensor.device}, got {scale.device}")
    if value.meta.get("channel_axis") != expected_axis:
        raise ValueError(
            f"{operand} must be quantized with channel_axis={expected_axis}, "
            f"got {value.meta.get('channel_axis')}")


def hip_per_channel_bmm(
    a: QuantResult,
    b: QuantResult,
    *,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    do_transpose_a: bool = False,
    do_transpose_b: bool = False,
    profile: bool = False,
    use_tma: bool = False,
    activation: str = "none",
) -> torch.Tensor:
    """Channel-scaled FP8 BMM: (A @ B) * sa[b, m] * sb[b, n]."""
    del profile, use_tma
    a_tensor, b_tensor, batch, m, n, k = C.prepare_operands(
        a, b, do_transpose_a, do_transpose_b, activation)
    _validate_scale(a, expected_shape=(batch, m), expected_axis=-2, operand="A")
    _validate_scale(b, expected_shape=(batch, n), expected_axis=-1, operand="B")
    out = C.prepare_out(out, out_dtype, batch, m, n, a_tensor.device)
    # the reference's per-channel wrapper accepts any bias strides (:362-373)
    bias, bias_strides, bias_code = C.check_bias(bias, batch, m, n, a_tensor.device,
                                                 require_n_contiguous=False)
    sa, sb = a.dequant_scale, b.dequant_scale
    return C.launch_bmm(
        a_tensor, b_tensor, out, bias, bias_strides, bias_code,
        sa, (sa.stride(0), sa.stride(1), 0), sb, (sb.stride(0), sb.stride(1), 0),
        _lib.SCALE_CHANNEL, False, 1, 128, 1, activation, batch, m, n, k)


def hip_torch_compile_role_quant(
    x: torch.Tensor,
    *,
    channel_axis: int = -1,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    eps: float = 1e-12,
    profile: bool = False,
) -> QuantResult:
    """The reference's ``torch_compile_per_channel`` entry
    (fp8_training/fp8_bench/impls/triton_per_channel.py:54-87, math at
    kernels/quant/per_channel.py:9-29), served by the HIP per-channel kernel:
    the same arguments, the same two checks before anything runs (rank,
    channel_axis), and the result fields that entry returns (impl name,
    ``quant_strategy: "torch_compile"``). Scales are the per-channel ones,
    ds = max(amax, eps) / fp8_max; the quant scale is the true quotient
    fp8_max / s, as in the Triton kernels (the compiled form evaluates it as
    reciprocal(s) * fp8_max, which can differ in its last bit)."""
    del profile
    if x.ndim not in (2, 3):
        raise ValueError(f"per-channel quant expects a 2D or 3D tensor, got {tuple(x.shape)}")
    if channel_axis not in (-1, -2):
        raise ValueError(f"channel_axis must be -1 or -2, got {channel_axis}")
    q = hip_per_channel_quant(x, channel_axis=channel_axis, fp8_dtype=fp8_dtype, eps=eps)
    q.impl = "torch_compile_per_channel"
    q.meta["quant_strategy"] = "torch_compile"
    return q


register_quant(
    "torch_compile_per_channel",
    hip_torch_compile_role_quant,
    "The reference's torch.compile per-channel entry, run by the HIP per-channel kernel; "
    "E4M3 and E5M2.",
)
register_quant(
    "hip_per_channel_one_pass",
    partial(hip_per_channel_quant, one_pass=True),
    "One-pass HIP per-channel quantization for reductions up to 4096.",
)
register_quant(
    "hip_per_channel",
    hip_per_channel_quant,
    "Per-channel scale quantization; supports E4M3 and E5M2.",
)

_CH = {"quant_impl": "hip_per_channel", "quant_a_kwargs": {"channel_axis": -2},
       "quant_b_kwargs": {"channel_axis": -1}}
register_bmm(
    "hip_per_channel_a_k_b_n", partial(hip_per_channel_bmm, do_transpose_b=False),
    layout="n", prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="Per-channel FP8 BMM with an N-major [B,K,N] right operand.", **_CH)
register_bmm(
    "hip_per_channel_a_k_b_k", partial(hip_per_channel_bmm, do_transpose_b=False),
    layout="k", prepare_b=lambda v: C.prepare_b_layout(v, "k"),
    description="Per-channel FP8 BMM with a prepacked K-major right operand.", **_CH)
register_bmm(
    "hip_per_channel_a_k_b_n_transpose", partial(hip_per_channel_bmm, do_transpose_b=True),
    layout="n", prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="N-major per-channel FP8 BMM with packing inside the call.", **_CH)
register_bmm(
    "hip_per_channel_a_m_b_n",
    partial(hip_per_channel_bmm, do_transpose_a=False, do_transpose_b=False),
    a_layout="m", layout="n",
    prepare_a=lambda v: C.prepare_a_layout(v, "m"), prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="Per-channel FP8 BMM with direct M-major A and N-major B operands.", **_CH)
register_bmm(
    "hip_per_channel_a_m_transpose_b_n_transpose",
    partial(hip_per_channel_bmm, do_transpose_a=True, do_transpose_b=True),
    a_layout="m", layout="n",
    prepare_a=lambda v: C.prepare_a_layout(v, "m"), prepare_b=lambda v: C.prepare_b_layout(v, "n"),
    description="M-major A and N-major B with both operands packed inside the BMM call.", **_CH)
