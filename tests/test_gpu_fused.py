"""GPU parity of the BMM with the activation quantization fused into its K loop
(pcamd_bmm_quant_a / hip_per_block_bmm_quant_a).

The quantized A the kernel writes out must be the 1 x 128 quantizer's bytes
and scales bit for bit (hip_per_block_quant, itself bit-exact against the
oracle), so the fused product is the unfused product of the same operands:
both are checked against the oracle's fp64 product of the dequantized
operands at the BMM bar (max-abs-rel 1e-2), and against each other at fp32
rounding level. Layouts outside the fused kernel (M-major or unaligned A, K
not a multiple of 128) take the two-kernel path and must give the same
results. Reference intent: kernels/fp8_bmm/kernel/fp8_quant_bmm_fused_kernel.py:30-146.
"""
from __future__ import annotations

import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd.impls.hip_per_block import (hip_per_block_bmm, hip_per_block_bmm_quant_a,
                                                   hip_per_block_quant)

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _rand(shape, seed, scale=1.0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    x[..., ::37] *= 40.0  # outliers so groups differ in scale
    return x.to(dtype)


def _b_operand(bsz, k, n, seed, dev, qbn=128, k_major=False, fmt=torch.float8_e4m3fn):
    w = _rand((bsz, k, n), seed, 0.05).to(dev)
    if k_major:
        w = w.transpose(-1, -2).contiguous().transpose(-1, -2)
    return hip_per_block_quant(w, block_m=128, block_n=qbn, fp8_dtype=fmt)


CASES = [
    # (batch, m, n, k, x dtype, fp8 format, qbn, B K-major)
    (2, 256, 384, 512, torch.bfloat16, torch.float8_e4m3fn, 128, False),
    (1, 200, 256, 256, torch.bfloat16, torch.float8_e4m3fn, 128, True),     # ragged M
    (3, 128, 512, 128, torch.float16, torch.float8_e4m3fn, 128, False),     # one K step
    (2, 384, 256, 384, torch.bfloat16, torch.float8_e5m2, 128, False),
    (1, 136, 264, 640, torch.float16, torch.float8_e4m3fn, 32, True),       # ragged M and N, 128x32 B blocks
    (2, 128, 256, 256, torch.bfloat16, torch.float8_e4m3fn, 1, False),      # 128x1 B blocks
    # narrow products (N <= 256, K % 256 == 0, qbn >= 128): the streaming kernel
    (2, 300, 256, 1024, torch.bfloat16, torch.float8_e4m3fn, 128, True),    # ragged M, 8 K steps
    (1, 128, 128, 512, torch.float16, torch.float8_e4m3fn, 128, False),     # N 128, N-major B
    (2, 512, 192, 768, torch.bfloat16, torch.float8_e5m2, 256, False),      # N 192 (partial stage), 256-wide B blocks
    (1, 1000, 64, 256, torch.bfloat16, torch.float8_e4m3fn, 128, True),     # N 64, two K steps
    (1, 2048, 256, 4096, torch.bfloat16, torch.float8_e4m3fn, 128, False),  # 32 K steps
    # N <= 128 with K % 512 == 0: two K blocks per pipeline step
    (2, 300, 128, 2048, torch.bfloat16, torch.float8_e4m3fn, 128, True),    # ragged M, 8 steps
    (1, 520, 96, 1536, torch.float16, torch.float8_e5m2, 128, False),       # N 96, 6 steps, N-major
    (1, 256, 128, 768, torch.bfloat16, torch.float8_e4m3fn, 128, False),    # K % 512 != 0: one block per step
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}x{c[3]}-{str(c[4])[6:]}-"
                         f"{str(c[5])[12:]}-qbn{c[6]}-{'bk' if c[7] else 'bn'}")
def test_fused_matches_quantizer_and_unfused(dev, case):
    bsz, m, n, k, xdt, fmt, qbn, b_k = case
    print(f"fused quant bmm {case}", flush=True)
    x = _rand((bsz, m, k), 1, dtype=xdt).to(dev)
    qb = _b_operand(bsz, k, n, 2, dev, qbn=qbn, k_major=b_k, fmt=fmt)
    out, qa = hip_per_block_bmm_quant_a(x, qb, return_quant=True, always_fused=True)
    torch.cuda.synchronize()
    ref_q = hip_per_block_quant(x, block_m=1, block_n=128, fp8_dtype=fmt)
    # the A the kernel quantized is the quantizer's, bit for bit
    assert qa.tensor.dtype == fmt
    assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))
    assert torch.equal(qa.dequant_scale.view(torch.int32), ref_q.dequant_scale.view(torch.int32))
    # and so is the product: unfused path on the same operands, and the oracle
    unfused = hip_per_block_bmm(ref_q, qb)
    torch.cuda.synchronize()
    scale = unfused.float().abs().max().item()
    assert (out.float() - unfused.float()).abs().max().item() <= 1e-6 * scale + 1e-30
    ref = O.bmm_reference(ref_q.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= TOL
    # without the write-out the product is the same
    out2 = hip_per_block_bmm_quant_a(x, qb, always_fused=True)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("n", [256, 512])
def test_fused_clamped_instantiation(dev, n):
    # eps = 1e-40 makes fp8_max / eps overflow, so the kernels keep the clamp
    # before the cast (N 256: the streaming kernel; N 512: the tiled one)
    print(f"fused quant bmm clamp n={n}", flush=True)
    x = _rand((1, 256, 512), 13).to(dev)
    qb = _b_operand(1, 512, n, 14, dev)
    out, qa = hip_per_block_bmm_quant_a(x, qb, eps=1e-40, return_quant=True, always_fused=True)
    ref_q = hip_per_block_quant(x, block_m=1, block_n=128, eps=1e-40)
    unfused = hip_per_block_bmm(ref_q, qb)
    torch.cuda.synchronize()
    assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))
    assert torch.equal(qa.dequant_scale.view(torch.int32), ref_q.dequant_scale.view(torch.int32))
    assert (out.float() - unfused.float()).abs().max().item() <= 1e-6 * unfused.float().abs().max().item()


@pytest.mark.parametrize("n,k", [(192, 256), (128, 512), (512, 256)])  # streaming (one / two K blocks), tiled
@pytest.mark.parametrize("activation", ["none", "gelu"])
@pytest.mark.parametrize("out_dtype,bias_dtype", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.float32),
                                                  (torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                                                  (torch.float16, torch.bfloat16)])
def test_fused_bias_activation_out_dtype(dev, n, k, activation, out_dtype, bias_dtype):
    print(f"fused epilogue n={n} k={k} {activation} out={out_dtype} bias={bias_dtype}", flush=True)
    x = _rand((2, 160, k), 3).to(dev)
    qb = _b_operand(2, k, n, 4, dev)
    bias = _rand((2, 160, n), 5).to(bias_dtype).to(dev)
    out = hip_per_block_bmm_quant_a(x, qb, bias=bias, activation=activation, out_dtype=out_dtype)
    forced = hip_per_block_bmm_quant_a(x, qb, bias=bias, activation=activation, out_dtype=out_dtype,
                                       always_fused=True)
    qa = hip_per_block_quant(x, block_m=1, block_n=128)
    ref = hip_per_block_bmm(qa, qb, bias=bias, activation=activation, out_dtype=out_dtype)
    torch.cuda.synchronize()
    assert out.dtype == out_dtype and forced.dtype == out_dtype
    # fp32 results to rounding; 16-bit ones to one unit in the last place
    tol = 1e-6 if out_dtype == torch.float32 else 8e-3
    for r in (out, forced):
        assert (r.float() - ref.float()).abs().max().item() <= tol * ref.float().abs().max().item()


@pytest.mark.parametrize("bias_layout", ["broadcast", "row_stride_2_mod_4", "odd_offset"])
def test_fused_bias_layouts(dev, bias_layout):
    """A 16-bit bias broadcast over batch and rows (strides 0) takes the
    packed 8-byte epilogue; one whose rows are not 8-byte aligned takes the
    per-element one. Both give the unfused product's results."""
    print(f"fused bias layout {bias_layout}", flush=True)
    n, k = 192, 256
    x = _rand((2, 96, k), 21).to(dev)
    qb = _b_operand(2, k, n, 22, dev)
    if bias_layout == "broadcast":
        bias = _rand((n,), 23).to(torch.bfloat16).to(dev).expand(2, 96, n)
    elif bias_layout == "row_stride_2_mod_4":
        bias = _rand((2, 96, n + 2), 23).to(torch.bfloat16).to(dev)[..., :n]
    else:
        bias = _rand((2 * 96 * n + 1,), 23).to(torch.bfloat16).to(dev)[1:].view(2, 96, n)
    out = hip_per_block_bmm_quant_a(x, qb, bias=bias, activation="gelu", always_fused=True)
    qa = hip_per_block_quant(x, block_m=1, block_n=128)
    ref = hip_per_block_bmm(qa, qb, bias=bias, activation="gelu")
    torch.cuda.synchronize()
    assert (out.float() - ref.float()).abs().max().item() <= 8e-3 * ref.float().abs().max().item()


@pytest.mark.parametrize("act", ["none", "gelu"])
def test_fused_out_rows_not_8_byte_aligned(dev, act):
    """An `out` whose row pitch (N + 2 elements) leaves rows off 8-byte
    alignment takes the per-element epilogue; the columns past N are never
    written."""
    print(f"fused unaligned out rows {act}", flush=True)
    n, k = 128, 512
    x = _rand((2, 200, k), 31).to(dev)
    qb = _b_operand(2, k, n, 32, dev)
    bias = _rand((2, 200, n), 33).to(dev) if act == "gelu" else None
    buf = torch.full((2, 200, n + 2), 7.0, device=dev, dtype=torch.bfloat16)
    out = buf[..., :n]
    r = hip_per_block_bmm_quant_a(x, qb, out=out, bias=bias, activation=act, always_fused=True)
    qa = hip_per_block_quant(x, block_m=1, block_n=128)
    ref = hip_per_block_bmm(qa, qb, bias=bias, activation=act)
    torch.cuda.synchronize()
    assert r.data_ptr() == out.data_ptr()
    assert (out.float() - ref.float()).abs().max().item() <= 8e-3 * ref.float().abs().max().item()
    assert torch.all(buf[..., n:] == 7.0)


@pytest.mark.parametrize("layout", ["m_major", "unaligned_k"])
def test_fused_falls_back_outside_envelope(dev, layout):
    """An M-major activation, or K not a multiple of 128, takes the quantizer +
    BMM path: same results, same returned quantization."""
    if layout == "m_major":
        x = _rand((1, 128, 256), 6).to(dev).transpose(-1, -2).contiguous().transpose(-1, -2)
        k = 256
    else:
        k = 200
        x = _rand((1, 128, k), 6).to(dev)
    qb = _b_operand(1, k, 256, 7, dev)
    out, qa = hip_per_block_bmm_quant_a(x, qb, return_quant=True)
    ref_q = hip_per_block_quant(x, block_m=1, block_n=128)
    ref = hip_per_block_bmm(ref_q, qb)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))


def test_wide_products_take_two_kernel_path(dev):
    # above FUSED_MAX_N columns the default call quantizes, then multiplies:
    # the unfused results exactly, and the same quantization returned
    x = _rand((1, 256, 512), 15).to(dev)
    qb = _b_operand(1, 512, 512, 16, dev)
    out, qa = hip_per_block_bmm_quant_a(x, qb, return_quant=True)
    ref_q = hip_per_block_quant(x, block_m=1, block_n=128)
    ref = hip_per_block_bmm(ref_q, qb)
    fused = hip_per_block_bmm_quant_a(x, qb, always_fused=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))
    assert (fused.float() - ref.float()).abs().max().item() <= 1e-6 * ref.float().abs().max().item()


@pytest.mark.parametrize("k,n,qbn,extra", [(384, 128, 128, {}), (512, 128, 32, {}),
                                           (384, 128, 128, {"activation": "gelu"}),
                                           (512, 120, 128, {}), (384, 256, 128, {"out_dtype": torch.float32})])
def test_narrow_products_outside_the_stream_envelope_take_two_kernels(dev, k, n, qbn, extra):
    # N <= 256 but K % 256 != 0, quant-N blocks < 128 or N % 16 != 0: by
    # default the unfused results exactly
    print(f"fused default path k={k} n={n} qbn={qbn} {extra}", flush=True)
    x = _rand((1, 200, k), 17).to(dev)
    qb = _b_operand(1, k, n, 18, dev, qbn=qbn)
    out, qa = hip_per_block_bmm_quant_a(x, qb, return_quant=True, **extra)
    ref_q = hip_per_block_quant(x, block_m=1, block_n=128)
    ref = hip_per_block_bmm(ref_q, qb, **extra)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))


def test_fused_2d_activation(dev):
    x = _rand((256, 384), 8).to(dev)
    qb = _b_operand(1, 384, 256, 9, dev)
    out = hip_per_block_bmm_quant_a(x, qb, always_fused=True)
    ref = hip_per_block_bmm(hip_per_block_quant(x[None], block_m=1, block_n=128), qb)[0]
    torch.cuda.synchronize()
    assert out.shape == (256, 256)
    assert (out.float() - ref.float()).abs().max().item() <= 1e-6 * ref.float().abs().max().item()


def test_fused_config4_shape(dev):
    """BASELINE config 4 with the bf16 activations quantized inside the BMM:
    A [128, 2048, 128] 1x128, B [128, 128, 512] 128x128; every batch within
    the bar of an fp32 bmm of the dequantized operands."""
    g = torch.Generator().manual_seed(0)
    ah = torch.randn(128, 2048, 128, generator=g).bfloat16().to(dev)
    bh = torch.randn(128, 128, 512, generator=g).bfloat16().to(dev)
    qb = hip_per_block_quant(bh, block_m=128, block_n=128)
    print("fused config4", flush=True)
    out, qa = hip_per_block_bmm_quant_a(ah, qb, return_quant=True, always_fused=True)
    ref_q = hip_per_block_quant(ah, block_m=1, block_n=128)
    assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))
    ref = torch.bmm(ref_q.dequantize().contiguous(), qb.dequantize().contiguous())
    err = (out.float() - ref).abs().amax(dim=(1, 2)) / ref.abs().amax(dim=(1, 2))
    assert err.max().item() <= TOL


def test_fused_rejects_bad_arguments(dev):
    x = _rand((1, 128, 256), 10).to(dev)
    qb = _b_operand(1, 256, 128, 11, dev)
    with pytest.raises(ValueError, match="bfloat16 or float16"):
        hip_per_block_bmm_quant_a(x.float(), qb)
    with pytest.raises(ValueError, match="shape mismatch"):
        hip_per_block_bmm_quant_a(x[..., :128], qb)
    qb256 = hip_per_block_quant(_rand((1, 256, 128), 12).to(dev), block_m=256, block_n=128)
    with pytest.raises(ValueError, match="quant-K blocks of 128"):
        hip_per_block_bmm_quant_a(x, qb256)
