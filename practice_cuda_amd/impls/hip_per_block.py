"""Per-block (1 x 128, 128 x 128, any power-of-two) FP8 quantizer and BMM.

Drop-in for fp8_training/fp8_bench/impls/triton_per_block.py of
xuOAO/practice_cuda: ``hip_per_block_quant`` mirrors ``triton_per_block_quant``
(:60-150) and ``hip_per_block_bmm`` mirrors ``triton_per_block_bmm``
(:232-420), with the same arguments, output layouts, metadata and
ValueErrors; the work runs in the gfx950 kernels of csrc/quant.hip and
csrc/bmm.hip through the C ABI. ``profile`` and ``use_tma`` are accepted for
signature compatibility; there is no autotuner to bypass and no TMA unit.
"""
from __future__ import annotations

from functools import partial
from typing import Optional

import torch

from .. import _lib
from ..registry import QuantResult, register_bmm, register_quant
from . import _common as C

_DEFAULT_QUANT_BLOCK_M = 128
_DEFAULT_QUANT_BLOCK_K = 128
_DEFAULT_QUANT_BLOCK_N = 128


def hip_per_block_quant(
    x: torch.Tensor,
    *,
    block_m: int = _DEFAULT_QUANT_BLOCK_M,
    block_n: int = _DEFAULT_QUANT_BLOCK_N,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    eps: float = 1e-12,
    profile: bool = False,
    cache_outputs: bool = False,
) -> QuantResult:
    """One fp32 dequant scale per block_m x block_n tile of the last two dims.

    cache_outputs: write the fp8 tensor and scales with cache-allocating
    stores (PCAMD_QUANT_CACHED_OUTPUT) for a GEMM that reads them next; the
    default non-temporal stores are faster for a quantization on its own.
    Same bytes either way."""
    del profile
    if x.ndim not in (2, 3):
        raise ValueError(f"per-block quant expects a 2D or 3D tensor, got {tuple(x.shape)}")
    if not C.is_power_of_two(block_m) or not C.is_power_of_two(block_n):
        raise ValueError(
            "per-block quant currently requires power-of-two block sizes; "
            f"got block_m={block_m}, block_n={block_n}")
    C.check_quant_input(x, fp8_dtype, "per-block quant")
    _lib.require_gpu_tensor(x, "x")

    output = torch.empty_like(x, dtype=fp8_dtype, memory_format=torch.preserve_format)
    batch, m, n, xs, ys = C.dims3(x, output)
    m_blocks = -(-m // block_m)
    n_blocks = -(-n // block_n)
    scale_storage = torch.empty((batch, m_blocks, n_blocks), device=x.device, dtype=torch.float32)

    L = _lib.lib()
    with torch.cuda.device(x.device):
        rc = L.pcamd_quant_block_ex(
            _lib.ptr(x), _lib.dtype_code(x.dtype), batch, m, n, *xs,
            _lib.ptr(output), _lib.dtype_code(fp8_dtype), *ys,
            _lib.ptr(scale_storage), *scale_storage.stride(),
            block_m, block_n, float(torch.finfo(fp8_dtype).max), float(eps),
            _lib.QUANT_CACHED_OUTPUT if cache_outputs else 0, _lib.stream_of(x))
    _lib.check(rc, "pcamd_quant_block")

    dequant_scale = scale_storage.squeeze(0) if x.ndim == 2 else scale_storage
    return QuantResult(
        tensor=output,
        dequant_scale=dequant_scale,
        impl="hip_per_block",
        granularity="block",
        meta={
            "logical_shape": tuple(x.shape),
            "fp8_dtype": str(fp8_dtype),
            "block_m": block_m,
            "block_n": block_n,
        },
    )


def hip_per_block_quant_dual(
    x: torch.Tensor,
    *,
    block: int = 128,
    fp8_dtype: torch.dtype = torch.float8_e4m3fn,
    eps: float = 1e-12,
    col_transposed: bool = False,
    cache_outputs: bool = False,
) -> tuple[QuantResult, QuantResult]:
    """``(hip_per_block_quant(x, block_m=1, block_n=block), hip_per_block_quant(x,
    block_m=block, block_n=1))`` from one read of x.

    The block-scaled training recipe needs both quantizations of the
    activations and of the output gradient: 1 x block groups along the last
    dim for the forward / dgrad GEMMs, block x 1 groups along the rows for
    wgrad. The results are bit-identical to the two separate calls.
    col_transposed: the block x 1 result is stored transposed (a [.., N, M]
    buffer seen as [.., M, N]), so a GEMM that reduces over M reads it
    K-major; its rows are padded to a multiple of 16 bytes (row pitch
    ceil(M / 16) * 16), which the kernel's 16-byte transposed stores need.
    cache_outputs: as for hip_per_block_quant.
    """
    if x.ndim not in (2, 3):
        raise ValueError(f"per-block quant expects a 2D or 3D tensor, got {tuple(x.shape)}")
    if not C.is_power_of_two(block):
        raise ValueError(f"per-block quant currently requires power-of-two block sizes; got block={block}")
    C.check_quant_input(x, fp8_dtype, "per-block quant")
    _lib.require_gpu_tensor(x, "x")

    out_row = torch.empty_like(x, dtype=fp8_dtype, memory_format=torch.preserve_format)
    if col_transposed:
        pitch = -(-x.shape[-2] // 16) * 16
        out_col = torch.empty(*x.shape[:-2], x.shape[-1], pitch, dtype=fp8_dtype,
                              device=x.device)[..., :x.shape[-2]].transpose(-1, -2)
    else:
        out_col = torch.empty_strided(out_row.shape, out_row.stride(), dtype=fp8_dtype, device=x.device)
    batch, m, n, xs, ys = C.dims3(x, out_row)
    yc = (0, *out_col.stride()) if out_col.ndim == 2 else tuple(out_col.stride())
    s_row = torch.empty((batch, m, -(-n // block)), device=x.device, dtype=torch.float32)
    s_col = torch.empty((batch, -(-m // block), n), device=x.device, dtype=torch.float32)

    L = _lib.lib()
    with torch.cuda.device(x.device):
        rc = L.pcamd_quant_block_dual_ex(
            _lib.ptr(x), _lib.dtype_code(x.dtype), batch, m, n, *xs,
            _lib.ptr(out_row), *ys, _lib.ptr(out_col), *yc, _lib.dtype_code(fp8_dtype),
            _lib.ptr(s_row), *s_row.stride(), _lib.ptr(s_col), *s_col.stride(),
            block, float(torch.finfo(fp8_dtype).max), float(eps),
            _lib.QUANT_CACHED_OUTPUT if cache_outputs else 0, _lib.stream_of(x))
    _lib.check(rc, "pcamd_quant_block_dual")

    def result(q, s, bm, bn):
        return QuantResult(
            tensor=q,
            dequant_scale=s.squeeze(0) if x.ndim == 2 else s,
            impl="hip_per_block",
            granularity="block",
            meta={"logical_shape": tuple(x.shape), "fp8_dtype": str(fp8_dtype), "block_m": bm, "block_n": bn},
        )

    return result(out_row, s_row, 1, block), result(out_col, s_col, block, 1)


def _validate_scale(value: QuantResult, *, expected_shape, expected_block_m, expected_block_n,
                    operand: str) -> None:
    scale = value.dequant_scale
    if value.granularity != "block":
        raise ValueError(f"{operand} must use block granularity, got {value.granularity!r}")
    if tuple(scale.shape) != expected_shape:
        raise ValueError(
            f"{operand} dequant scale must have shape {expected_shape}, got {tuple(scale.shape)}")
    if scale.dtype != torch.float32:
        raise ValueError(f"{operand} dequant scale must be float32, got {scale.dtype}")
    if scale.device != value.tensor.device:
        raise ValueError(f"{operand} dequant scale must be on {value.tensor.device}, got {scale.device}")
    if value.meta.get("block_m") != expected_block_m or value.meta.get("block_n") != expected_block_n:
        raise ValueError(
            f"{operand} must be quantized with block_m={expected_block_m} "
            f"and block_n={expected_block_n}, "
            f"got block_m={value.meta.get('block_m')} and block_n={value.meta.get('block_n')}")


def _block_shape(value: QuantResult, operand: str) -> tuple[int, int]:
    if value.granularity != "block":
        raise ValueError(f"{operand} must use block granularity, got {value.granularity!r}")
    bm, bn = value.meta.get("block_m"), value.meta.get("block_n")
    if not isinstance(bm, int) or not isinstance(bn, int) or bm <= 0 or bn <= 0:
        raise ValueError(f"{operand} has invalid per-block metadata: block_m={bm}, block_n={bn}")
    return bm, bn


def hip_per_block_bmm(
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
    """Block-scaled FP8 BMM: per quant-K block, acc += (A_blk @ B_blk) * (sa * sb)."""
    del profile, use_tma
    a_tensor, b_tensor, batch, m, n, k = C.prepare_operands(
        a, b, do_transpose_a, do_transpose_b, activation)

    qbm, qbk = _block_shape(a, "A")
    b_qbk, qbn = _block_shape(b, "B")
    if qbk != b_qbk:
        raise ValueError(f"A and B must use the same K quant block: A={qbk}, B={b_qbk}")
    if qbk < 128 or qbk % 128 != 0:
        raise ValueError(
            "the current per-block BMM configs require quant_block_k >= 128 "
            f"and divisible by 128, got {qbk}")
    mb, kb, nb = -(-m // qbm), -(-k // qbk), -(-n // qbn)
    _validate_scale(a, expected_shape=(batch, mb, kb), expected_block_m=qbm, expected_block_n=qbk,
                    operand="A")
    _validate_scale(b, expected_shape=(batch, kb, nb), expected_block_m=qbk, expected_block_n=qbn,
                    operand="B")

    out = C.prepare_out(out, out_dtype, batch, m, n, a_tensor.device)
    bias, bias_strides, bias_code = C.check_bias(bias, batch, m, n, a_tensor.device)
    return C.launch_bmm(
        a_tensor, b_tensor, out, bias, bias_strides, bias_code,
        a.dequant_scale, a.dequant_scale.stride(), b.dequant_scale, b.dequant_scale.stride(),
        _lib.SCALE_BLOCK, False, qbm, qbk, qbn, activation, batch, m, n, k)




# widest product hip_per_block_bmm_quant_a sends to the fused kernel by default
FUSED_MAX_N = 256


def fused_streams(n: int, k: int, qbn: int) -> bool:
    """Whether pcamd_bmm_quant_a runs its streaming kernel for this product
    (one workgroup holds all N columns and reads A once): the envelope of
    bmm_fused_stream_ok, for any bias, activation and output type. Outside it
    the call runs the tiled fused kernel, which quantizes A once per
    256-column tile and is slower than quantizing first at every measured
    shape."""
    return 0 < n <= FUSED_MAX_N and n % 16 == 0 and k >= 256 and k % 256 == 0 and qbn >= 128


def hip_per_block_bmm_quant_a(
    x: torch.Tensor,
    b: QuantResult,
    *,
    eps: float = 1e-12,
    out_dtype: torch.dtype = torch.bfloat16,
    bias: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
    activation: str = "none",
    return_quant: bool = False,
    always_fused: bool = False,
):
    """``hip_per_block_bmm(hip_per_block_quant(x, block_m=1, block_n=128), b)``
    with the activation quantization inside the GEMM's K loop.

    x: bf16 or fp16 [B, M, K] (or [M, K] with a 3D b of batch 1), quantized in
    1 x 128 groups along K into b's fp8 dtype; b: a block-scaled QuantResult
    with quant-K block 128. The product equals the unfused path's bit for
    bit: the A bytes and scales are those hip_per_block_quant produces. With
    return_quant=True the quantized A comes back too, as (out, QuantResult).

    This is the intent of the reference's fused quant + BMM kernel
    (kernels/fp8_bmm/kernel/fp8_quant_bmm_fused_kernel.py:30-146, unfinished
    there), on the per-block recipe. Layouts the fused kernel does not cover
    (an M-major or unaligned x, K not a multiple of 128) take the two-kernel
    path: hip_per_block_quant, then hip_per_block_bmm. Unless always_fused is
    set, so do the products outside the streaming kernel's envelope (N up to
    FUSED_MAX_N and a multiple of 16, K a multiple of 256, B's quant-N blocks
    >= 128; bias, activation and output type are free): there the fused call
    runs a tiled kernel that quantizes each A row block once per 256-column
    tile of C, and the two-kernel path is faster (MI355X, A [32768, 4096],
    N 128: 134.7 vs 125.2 us; M 16384, N 512: 133 vs 93 us)."""
    if x.ndim not in (2, 3):
        raise ValueError(f"fused quant BMM expects a 2D or 3D activation, got {tuple(x.shape)}")
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"fused quant BMM expects a bfloat16 or float16 activation, got {x.dtype}")
    if activation not in ("none", "gelu"):
        raise ValueError(f"activation must be 'none' or 'gelu', got {activation!r}")
    x3 = x if x.ndim == 3 else x[None]
    if b.tensor.ndim != 3:
        raise ValueError("BMM expects a 3D quantized right operand")
    b_qbk, qbn = _block_shape(b, "B")
    if b_qbk != 128:
        raise ValueError(f"the fused activation quantization uses quant-K blocks of 128; B has {b_qbk}")
    fp8_dtype = b.tensor.dtype
    in_b = C.matrix_layout(b.tensor, "B")
    batch, m, k = x3.shape
    b_batch, b_k, n = b.tensor.shape
    if batch != b_batch or k != b_k:
        raise ValueError(f"shape mismatch: A={tuple(x3.shape)}, B={tuple(b.tensor.shape)}")
    if x3.device != b.tensor.device:
        raise ValueError(f"A and B must be on the same device: A={x3.device}, B={b.tensor.device}")
    _validate_scale(b, expected_shape=(batch, -(-k // 128), -(-n // qbn)), expected_block_m=128,
                    expected_block_n=qbn, operand="B")
    _lib.require_gpu_tensor(x3, "x")
    out = C.prepare_out(out, out_dtype, batch, m, n, x3.device)
    bias, bias_strides, bias_code = C.check_bias(bias, batch, m, n, x3.device)
    qa = sa = None
    if return_quant:
        qa = torch.empty((batch, m, k), device=x3.device, dtype=fp8_dtype)
        sa = torch.empty((batch, m, -(-k // 128)), device=x3.device, dtype=torch.float32)
    L = _lib.lib()
    rc = _lib.ERR_UNSUPPORTED
    fused = always_fused or fused_streams(n, k, qbn)
    if in_b in ("n-major", "k-major") and x3.stride(-1) == 1 and fused:
        with torch.cuda.device(x3.device):
            rc = L.pcamd_bmm_quant_a(
                _lib.ptr(x3), _lib.dtype_code(x3.dtype), _lib.ptr(b.tensor), _lib.dtype_code(fp8_dtype),
                batch, m, n, k, *x3.stride(), *b.tensor.stride(),
                _lib.ptr(out), _lib.dtype_code(out.dtype), *out.stride(),
                _lib.ptr(bias), bias_code, *bias_strides,
                _lib.ptr(b.dequant_scale), *b.dequant_scale.stride(), qbn,
                _lib.ptr(qa), *(qa.stride() if qa is not None else (0, 0, 0)),
                _lib.ptr(sa), *(sa.stride() if sa is not None else (0, 0, 0)),
                float(torch.finfo(fp8_dtype).max), float(eps),
                _lib.ACT_GELU if activation == "gelu" else _lib.ACT_NONE, _lib.stream_of(x3))
    if rc == _lib.ERR_UNSUPPORTED:
        qres = hip_per_block_quant(x3, block_m=1, block_n=128, fp8_dtype=fp8_dtype, eps=eps)
        hip_per_block_bmm(qres, b, out_dtype=out_dtype, bias=bias, out=out, activation=activation)
        if return_quant:
            qa, sa = qres.tensor, qres.dequant_scale
    else:
        _lib.check(rc, "pcamd_bmm_quant_a")
    if x.ndim == 2:
        out = out.squeeze(0)
    if not return_quant:
        return out
    quant = QuantResult(
        tensor=qa if x.ndim == 3 else qa.squeeze(0),
        dequant_scale=sa if x.ndim == 3 else sa.squeeze(0),
        impl="hip_per_block",
        granularity="block",
        meta={"logical_shape": tuple(x.shape), "fp8_dtype": str(fp8_dtype), "block_m": 1, "block_n": 128},
    )
    return out, quant


def _register_block_scheme(quant_impl: str, *, quant_block_m: int, quant_block_k: int,
                           quant_block_n: int, description: str) -> None:
    """Register the quantizer and its five BMM layout variants
    (reference impls/triton_per_block.py:436-521)."""
    register_quant(
        quant_impl,
        partial(hip_per_block_quant, block_m=quant_block_m, block_n=quant_block_k),
        description,
    )
    common = {
        "quant_impl": quant_impl,
        "quant_a_kwargs": {"block_m": quant_block_m, "block_n": quant_block_k},
        "quant_b_kwargs": {"block_m": quant_block_k, "block_n": quant_block_n},
    }
    register_bmm(
        f"{quant_impl}_a_k_b_n", partial(hip_per_block_bmm, do_transpose_b=False),
        layout="n", prepare_b=lambda v: C.prepare_b_layout(v, "n"),
        description="Per-block FP8 BMM with an N-major [B,K,N] right operand.", **common)
    register_bmm(
        f"{quant_impl}_a_k_b_k", partial(hip_per_block_bmm, do_transpose_b=False),
        layout="k", prepare_b=lambda v: C.prepare_b_layout(v, "k"),
        description="Per-block FP8 BMM with a prepacked K-major right operand.", **common)
    register_bmm(
        f"{quant_impl}_a_k_b_n_transpose", partial(hip_per_block_bmm, do_transpose_b=True),
        layout="n", prepare_b=lambda v: C.prepare_b_layout(v, "n"),
        description="N-major per-block FP8 BMM with packing inside the call.", **common)
    register_bmm(
        f"{quant_impl}_a_m_b_n",
        partial(hip_per_block_bmm, do_transpose_a=False, do_transpose_b=False),
        a_layout="m", layout="n",
        prepare_a=lambda v: C.prepare_a_layout(v, "m"), prepare_b=lambda v: C.prepare_b_layout(v, "n"),
        description="Per-block FP8 BMM with direct M-major A and N-major B operands.", **common)
    register_bmm(
        f"{quant_impl}_a_m_transpose_b_n_transpose",
        partial(hip_per_block_bmm, do_transpose_a=True, do_transpose_b=True),
        a_layout="m", layout="n",
        prepare_a=lambda v: C.prepare_a_layout(v, "m"), prepare_b=lambda v: C.prepare_b_layout(v, "n"),
        description="M-major A and N-major B packed inside the per-block BMM call.", **common)


_register_block_scheme(
    "hip_per_block_1d", quant_block_m=1, quant_block_k=_DEFAULT_QUANT_BLOCK_K, quant_block_n=1,
    description="1D K-block scale quantization; defaults to 1x128 blocks.")
_register_block_scheme(
    "hip_per_block_2d", quant_block_m=_DEFAULT_QUANT_BLOCK_M, quant_block_k=_DEFAULT_QUANT_BLOCK_K,
    quant_block_n=_DEFAULT_QUANT_BLOCK_N,
    description="2D block scale quantization; defaults to 128x128 blocks.")
