"""FP8 batched linear layers for training on the HIP kernels.

Counterpart of xuOAO/practice_cuda ``fp8_training/fp8_bench/modules/
bmm_linear.py`` (``BMMLinear`` :453-508, ``Float8BMMLinear`` :511-657,
``_Float8BMMLinearFunction`` :326-451, custom op ``fp8_bench::bmm_linear_tma``
:121-227, ``convert_to_float8_bmm_training`` :660-673) for the block-scaled
recipe the reference leaves unfinished (``modules/per_block.py:13-67``):

* forward  ``Y = X W^T (+ bias)``: X quantized 1x128 along K, W 128x128;
* dgrad    ``dX = dY W``: dY quantized 1x128 along N, W reused from forward;
* wgrad    ``dW = dY^T X``: dY and X quantized 128x1 (blocks of 128 along
  M, the reduction dimension of this GEMM) from their high-precision values,
  each in the same pass as its 1x128 quantization (``pcamd_quant_block_dual``:
  one read of X in forward, one of dY in backward; the 128x1 results are
  stored transposed, which makes both wgrad operands K-major; the 128x1 fp8
  X is what forward saves);
* dbias    ``dY.sum(1)``.

Every GEMM is ``pcamd::block_scaled_bmm``, a ``torch.library`` custom op over
``pcamd_bmm_scaled`` (block mode: each 128-wide K block's partial sum is
multiplied by sa * sb, kernels/bmm/per_block.py:99-111), so the layer also
traces under ``torch.compile``. Quantization is the 1x128 / 128x128 / 128x1
``pcamd_quant_block`` kernel. A per-tensor variant (``granularity="tensor"``)
uses the per-tensor quantizer with torchao's tensorwise scale, the form the
reference layer quantizes with (modules/float8/float8_utils.py:45-48:
qs = fp32(fp8_max / max(fp64(amax), 1e-12)), bytes fp8(clamp(x * qs)),
float8_training_tensor.py:153-154), and the scalar-scaled GEMM.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch
import torch.nn as nn

from . import _lib
from .impls import _common as C
from .impls.hip_per_block import hip_per_block_quant, hip_per_block_quant_dual
from .impls.hip_per_tensor import quant_tensor_raw

_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)


# ---------------------------------------------------------------------------
# custom ops
# ---------------------------------------------------------------------------
@torch.library.custom_op("pcamd::block_scaled_bmm", mutates_args=())
def block_scaled_bmm(
    a: torch.Tensor,
    sa: torch.Tensor,
    b: torch.Tensor,
    sb: torch.Tensor,
    bias: Optional[torch.Tensor],
    qbm: int,
    qbk: int,
    qbn: int,
    out_dtype: torch.dtype,
) -> torch.Tensor:
    """``C[b] = sum_kq (A[b, :, kq] @ B[b, kq, :]) * sa[b, m/qbm, kq] * sb[b, kq, n/qbn] (+ bias)``.

    a: fp8 [B, M, K] contiguous along K or M; b: fp8 [B, K, N] contiguous
    along N or K (each e4m3fn or e5m2, the same or not: the recipe's e5m2
    gradient times an e4m3fn weight or activation); sa: fp32
    [B, ceil(M/qbm), ceil(K/qbk)]; sb: fp32
    [B, ceil(K/qbk), ceil(N/qbn)] (any strides); bias: [B, N] (broadcast over
    M) or None. qbk must be a multiple of 128; a last, partial K block is
    scaled like the others (its quantization covered the same columns).
    """
    batch, m, k = a.shape
    n = b.shape[2]
    if b.shape[0] != batch or b.shape[1] != k:
        raise ValueError(f"incompatible BMM shapes: A={tuple(a.shape)}, B={tuple(b.shape)}")
    if a.dtype not in _FP8 or b.dtype not in _FP8:
        raise ValueError(f"A and B must be fp8 (e4m3fn or e5m2), got {a.dtype} and {b.dtype}")
    if qbk <= 0 or qbk % 128:
        raise ValueError(f"quant block K ({qbk}) must be a positive multiple of 128")
    want_a = (batch, -(-m // qbm), -(-k // qbk))
    want_b = (batch, -(-k // qbk), -(-n // qbn))
    if tuple(sa.shape) != want_a or tuple(sb.shape) != want_b:
        raise ValueError(f"scale shapes must be {want_a} and {want_b}, got {tuple(sa.shape)} and {tuple(sb.shape)}")
    if sa.dtype != torch.float32 or sb.dtype != torch.float32:
        raise ValueError("block scales must be float32")
    C.a_layout(a)
    C.b_layout(b)
    out = torch.empty((batch, m, n), dtype=out_dtype, device=a.device)
    bias_strides, bias_code = (0, 0, 0), 0
    if bias is not None:
        if tuple(bias.shape) != (batch, n):
            raise ValueError(f"bias must have shape {(batch, n)}, got {tuple(bias.shape)}")
        bias = bias.unsqueeze(1).expand(batch, m, n)  # stride 0 along M
        bias, bias_strides, bias_code = C.check_bias(bias, batch, m, n, a.device, require_n_contiguous=False)
    return C.launch_bmm(a, b, out, bias, bias_strides, bias_code, sa, tuple(sa.stride()), sb, tuple(sb.stride()),
                        _lib.SCALE_BLOCK, False, qbm, qbk, qbn, "none", batch, m, n, k)


@block_scaled_bmm.register_fake
def _(a, sa, b, sb, bias, qbm, qbk, qbn, out_dtype):
    return a.new_empty((a.shape[0], a.shape[1], b.shape[2]), dtype=out_dtype)


@torch.library.custom_op("pcamd::tensor_scaled_bmm", mutates_args=())
def tensor_scaled_bmm(a: torch.Tensor, b: torch.Tensor, scale: torch.Tensor, bias: Optional[torch.Tensor],
                      out_dtype: torch.dtype) -> torch.Tensor:
    """``C[b] = (A[b] @ B[b]) * scale (+ bias[b] over M)``; scale: fp32, one element."""
    batch, m, k = a.shape
    n = b.shape[2]
    if b.shape[0] != batch or b.shape[1] != k:
        raise ValueError(f"incompatible BMM shapes: A={tuple(a.shape)}, B={tuple(b.shape)}")
    C.a_layout(a)
    C.b_layout(b)
    out = torch.empty((batch, m, n), dtype=out_dtype, device=a.device)
    bias_strides, bias_code = (0, 0, 0), 0
    if bias is not None:
        bias = bias.unsqueeze(1).expand(batch, m, n)
        bias, bias_strides, bias_code = C.check_bias(bias, batch, m, n, a.device, require_n_contiguous=False)
    return C.launch_bmm(a, b, out, bias, bias_strides, bias_code, scale.reshape(1), (0, 0, 0), None, (0, 0, 0),
                        _lib.SCALE_TENSOR, False, 1, 128, 1, "none", batch, m, n, k)


@tensor_scaled_bmm.register_fake
def _(a, b, scale, bias, out_dtype):
    return a.new_empty((a.shape[0], a.shape[1], b.shape[2]), dtype=out_dtype)


@torch.library.custom_op("pcamd::quant_block", mutates_args=())
def quant_block(x: torch.Tensor, block_m: int, block_n: int, fp8_dtype: torch.dtype,
                eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(fp8 [B,M,N], fp32 dequant scales [B, ceil(M/block_m), ceil(N/block_n)]),
    written with cache-allocating stores: the layer's GEMM reads them next."""
    q = hip_per_block_quant(x, block_m=block_m, block_n=block_n, fp8_dtype=fp8_dtype, eps=eps,
                            cache_outputs=True)
    return q.tensor, q.dequant_scale


@quant_block.register_fake
def _(x, block_m, block_n, fp8_dtype, eps):
    b, m, n = x.shape
    return (torch.empty_like(x, dtype=fp8_dtype),
            x.new_empty((b, -(-m // block_m), -(-n // block_n)), dtype=torch.float32))


@torch.library.custom_op("pcamd::quant_block_dual", mutates_args=())
def quant_block_dual(x: torch.Tensor, block: int, fp8_dtype: torch.dtype,
                     eps: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """``quant_block(x, 1, block)`` and ``quant_block(x, block, 1)`` from one read
    of x: (fp8 1 x block, its scales [B, M, ceil(N/block)], fp8 block x 1 stored
    transposed (a [B, N, M] buffer with rows padded to 16 bytes, seen as
    [B, M, N]: the K-major operand of a GEMM reducing over M), its scales
    [B, ceil(M/block), N]); cache-allocating stores, as for quant_block."""
    r, c = hip_per_block_quant_dual(x, block=block, fp8_dtype=fp8_dtype, eps=eps, col_transposed=True,
                                    cache_outputs=True)
    return r.tensor, r.dequant_scale, c.tensor, c.dequant_scale


@quant_block_dual.register_fake
def _(x, block, fp8_dtype, eps):
    b, m, n = x.shape
    return (torch.empty_like(x, dtype=fp8_dtype), x.new_empty((b, m, -(-n // block)), dtype=torch.float32),
            x.new_empty((b, n, -(-m // 16) * 16), dtype=fp8_dtype)[..., :m].transpose(-1, -2),
            x.new_empty((b, -(-m // block), n), dtype=torch.float32))


@torch.library.custom_op("pcamd::quant_tensor", mutates_args=())
def quant_tensor(x: torch.Tensor, fp8_dtype: torch.dtype, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(fp8 tensor like x, fp32 dequant scale of shape [1]) with torchao's
    tensorwise scale (the division in fp64, rounded once to fp32)."""
    q, dequant, _ = quant_tensor_raw(x, fp8_dtype, eps, scale_dtype=torch.float64)
    return q, dequant.reshape(1).clone()


@quant_tensor.register_fake
def _(x, fp8_dtype, eps):
    return torch.empty_like(x, dtype=fp8_dtype), x.new_empty((1,), dtype=torch.float32)


# ---------------------------------------------------------------------------
# config and autograd
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class Float8BlockBMMLinearConfig:
    """Recipe of :class:`Float8BMMLinear`.

    granularity "block": 1x128 activations / gradients, 128x128 weights, 128x1
    re-quantization for wgrad (quant block 128). "tensor": one scale per
    tensor. fp8_dtype is the format of the input and the weight;
    grad_fp8_dtype that of the gradient dY (None: fp8_dtype, the block
    recipe's e4m3fn everywhere; torch.float8_e5m2: torchao's default for
    grad_output, which the reference layer keeps,
    fp8_training/fp8_bench/modules/bmm_linear.py:43-46 - dgrad and wgrad then
    multiply e5m2 by e4m3fn). eps is the amax floor of the quantizers.
    """

    granularity: str = "block"
    fp8_dtype: torch.dtype = torch.float8_e4m3fn
    block: int = 128
    eps: float = 1e-12
    grad_fp8_dtype: Optional[torch.dtype] = None

    def __post_init__(self) -> None:
        if self.granularity not in ("block", "tensor"):
            raise ValueError(f"granularity must be 'block' or 'tensor', got {self.granularity!r}")
        if self.fp8_dtype not in _FP8:
            raise ValueError(f"fp8_dtype must be float8_e4m3fn or float8_e5m2, got {self.fp8_dtype}")
        if self.grad_fp8_dtype is not None and self.grad_fp8_dtype not in _FP8:
            raise ValueError("grad_fp8_dtype must be float8_e4m3fn, float8_e5m2 or None, "
                             f"got {self.grad_fp8_dtype}")
        if self.block != 128:
            raise ValueError("the block recipe uses 128-wide quant blocks")


def _block_gemm(qa, sa, qb, sb, bias, qbm, qbn, out_dtype, block):
    return torch.ops.pcamd.block_scaled_bmm(qa, sa, qb, sb, bias, qbm, block, qbn, out_dtype)


class _Float8BlockBMMLinearFunction(torch.autograd.Function):
    """Y = X W^T (+ bias) with FP8 GEMMs for forward, dgrad and wgrad."""

    @staticmethod
    def forward(ctx, input: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor],
                config: Float8BlockBMMLinearConfig) -> torch.Tensor:
        f8, eps, blk = config.fp8_dtype, config.eps, config.block
        ctx.config = config
        ctx.has_bias = bias is not None
        bias_k = None if bias is None else bias.to(input.dtype)
        if config.granularity == "tensor":
            qx, sx = torch.ops.pcamd.quant_tensor(input, f8, eps)
            qw, sw = torch.ops.pcamd.quant_tensor(weight, f8, eps)
            ctx.save_for_backward(qx, sx, qw, sw)
            return torch.ops.pcamd.tensor_scaled_bmm(qx, qw.transpose(-2, -1), sx * sw, bias_k, input.dtype)
        if ctx.needs_input_grad[1]:
            # wgrad needs X quantized in 128-row blocks too: both from one read
            qx, sx, qxm, sxm = torch.ops.pcamd.quant_block_dual(input, blk, f8, eps)
        else:
            qx, sx = torch.ops.pcamd.quant_block(input, 1, blk, f8, eps)  # [B,M,K], [B,M,K/128]
            qxm = sxm = None
        qw, sw = torch.ops.pcamd.quant_block(weight, blk, blk, f8, eps)   # [B,N,K], [B,N/128,K/128]
        ctx.save_for_backward(qxm, sxm, qw, sw)
        # B = W^T: [B,K,N] contiguous along K; its scales [B,K/128,N/128]
        return _block_gemm(qx, sx, qw.transpose(-2, -1), sw.transpose(-2, -1), bias_k, 1, blk, input.dtype, blk)

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        config = ctx.config
        eps, blk = config.eps, config.block
        f8 = config.grad_fp8_dtype or config.fp8_dtype  # dY's format
        dy = grad_output.contiguous()
        grad_input = grad_weight = grad_bias = None
        if config.granularity == "tensor":
            qx, sx, qw, sw = ctx.saved_tensors
            qdy, sdy = torch.ops.pcamd.quant_tensor(dy, f8, eps)
            if ctx.needs_input_grad[0]:
                grad_input = torch.ops.pcamd.tensor_scaled_bmm(qdy, qw, sdy * sw, None, dy.dtype)
            if ctx.needs_input_grad[1]:
                grad_weight = torch.ops.pcamd.tensor_scaled_bmm(qdy.transpose(-2, -1), qx, sdy * sx, None, dy.dtype)
        else:
            qxm, sxm, qw, sw = ctx.saved_tensors
            need_dx, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
            if need_dx and need_dw:
                # dY quantized 1x128 along N (dgrad) and in 128-row blocks (wgrad) from one read
                qdy, sdy, qdt, sdt = torch.ops.pcamd.quant_block_dual(dy, blk, f8, eps)
            elif need_dx:
                qdy, sdy = torch.ops.pcamd.quant_block(dy, 1, blk, f8, eps)      # [B,M,N], [B,M,N/128]
            elif need_dw:
                qdt, sdt = torch.ops.pcamd.quant_block(dy, blk, 1, f8, eps)      # [B,M,N], [B,M/128,N]
            if need_dx:
                # dX = dY W: A = dY [B,M,N] 1x128 along N; B = W [B,N,K] (N = reduction)
                grad_input = _block_gemm(qdy, sdy, qw, sw, None, 1, blk, dy.dtype, blk)
            if need_dw:
                # dW = dY^T X: dY and X (quantized in forward) in 128-row blocks along M; from
                # quant_block_dual both are stored transposed, so A = dY^T and B = X are K-major
                grad_weight = _block_gemm(qdt.transpose(-2, -1), sdt.transpose(-2, -1), qxm, sxm, None,
                                          1, 1, dy.dtype, blk)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            grad_bias = dy.sum(dim=1)
        return grad_input, grad_weight, grad_bias, None


# ---------------------------------------------------------------------------
# modules
# ---------------------------------------------------------------------------
def _check_dims(batch_size: int, in_features: int, out_features: int) -> None:
    if batch_size <= 0 or in_features <= 0 or out_features <= 0:
        raise ValueError("batch_size, in_features and out_features must be positive")


class BMMLinear(nn.Module):
    """High-precision batched dense layer (the conversion baseline).

    ``input`` [batch, M, in_features]; ``weight`` [batch, out_features,
    in_features]; ``bias`` [batch, out_features].
    """

    def __init__(self, batch_size: int, in_features: int, out_features: int, bias: bool = True, *,
                 device=None, dtype=None) -> None:
        super().__init__()
        _check_dims(batch_size, in_features, out_features)
        self.batch_size, self.in_features, self.out_features = batch_size, in_features, out_features
        kw = {"device": device, "dtype": dtype}
        self.weight = nn.Parameter(torch.empty((batch_size, out_features, in_features), **kw))
        if bias:
            self.bias = nn.Parameter(torch.empty((batch_size, out_features), **kw))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        # nn.Linear's fan-in bound, without counting the batch dimension
        bound = 1 / math.sqrt(self.in_features)
        nn.init.uniform_(self.weight, -bound, bound)
        if self.bias is not None:
            nn.init.uniform_(self.bias, -bound, bound)

    def _check_input(self, input: torch.Tensor) -> None:
        if input.ndim != 3:
            raise ValueError(f"{type(self).__name__} expects [B,M,K], got {tuple(input.shape)}")
        if input.shape[0] != self.batch_size or input.shape[2] != self.in_features:
            raise ValueError(
                f"input shape mismatch: expected [{self.batch_size}, M, {self.in_features}], "
                f"got {tuple(input.shape)}")

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        self._check_input(input)
        out = torch.bmm(input, self.weight.transpose(-2, -1).contiguous())
        if self.bias is not None:
            out = out + self.bias.unsqueeze(1)
        return out

    def extra_repr(self) -> str:
        return (f"batch_size={self.batch_size}, in_features={self.in_features}, "
                f"out_features={self.out_features}, bias={self.bias is not None}")


class Float8BMMLinear(BMMLinear):
    """Batched dense layer whose three GEMMs run in FP8 on the HIP kernels."""

    def __init__(self, batch_size: int, in_features: int, out_features: int, bias: bool = True, *,
                 config: Optional[Float8BlockBMMLinearConfig] = None, device=None, dtype=None) -> None:
        super().__init__(batch_size, in_features, out_features, bias, device=device, dtype=dtype)
        self.config = config or Float8BlockBMMLinearConfig()

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        self._check_input(input)
        if torch.is_autocast_enabled():
            input = input.to(torch.get_autocast_gpu_dtype())
        return _Float8BlockBMMLinearFunction.apply(input, self.weight, self.bias, self.config)

    def extra_repr(self) -> str:
        return (super().extra_repr() + f", granularity={self.config.granularity}, "
                f"fp8_dtype={self.config.fp8_dtype}, grad_fp8_dtype={self.config.grad_fp8_dtype}")

    @classmethod
    def from_float(cls, module: BMMLinear,
                   config: Optional[Float8BlockBMMLinearConfig] = None) -> "Float8BMMLinear":
        """Wrap an existing :class:`BMMLinear`, sharing its parameters."""
        if not isinstance(module, BMMLinear):
            raise TypeError(f"expected BMMLinear, got {type(module)}")
        with torch.device("meta"):
            converted = cls(module.batch_size, module.in_features, module.out_features, bias=False,
                            config=config)
        converted.weight = module.weight
        converted.bias = module.bias
        return converted


def convert_to_float8_bmm_training(module: nn.Module,
                                   config: Optional[Float8BlockBMMLinearConfig] = None) -> nn.Module:
    """Recursively replace every :class:`BMMLinear` with :class:`Float8BMMLinear`."""
    if isinstance(module, BMMLinear) and not isinstance(module, Float8BMMLinear):
        return Float8BMMLinear.from_float(module, config)
    for name, child in list(module.named_children()):
        converted = convert_to_float8_bmm_training(child, config)
        if converted is not child:
            module.register_module(name, converted)
    return module


__all__ = ["BMMLinear", "Float8BMMLinear", "Float8BlockBMMLinearConfig", "convert_to_float8_bmm_training",
           "block_scaled_bmm", "tensor_scaled_bmm", "quant_block", "quant_block_dual", "quant_tensor"]
