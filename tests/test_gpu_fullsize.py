"""Full-size BMM parity at the north_star bar.

The BASELINE config-4 and config-5 products are checked at their real shapes
against an fp32 GEMM of the dequantized operands computed on the GPU
(QuantResult.dequantize(), then torch.matmul / torch.bmm on contiguous fp32
operands: the reference's kernel_reference, fp8_training/fp8_bench/
bench_bmm.py:414-419). The bar is max|out - ref| / max|ref| <= 1e-2, applied
per 128 x 128 output tile (config 5) or per batch (config 4), so a wrong scale
on one tile, a bad batch offset or a broken half-tile tail cannot hide behind
the global maximum.

The scales_are_quant epilogue (acc / (sa * sb), the reference's
SCALES_ARE_QUANT path in kernels/bmm/per_channel.py:94-98 and
kernels/bmm/per_tensor.py:196-204) is checked in channel and tensor mode on
each of the three kernels that carry it: the single-K-step kernel (K = 128),
the wide kernel (K >= 256) and the general kernel (unaligned shapes).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd import _lib
from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm, hip_per_block_quant
from practice_cuda_amd.registry import QuantResult

pytestmark = pytest.mark.gpu
TOL = 1e-2
M5, K5, N5 = 8192, 4096, 14336


def _tile_err(out: torch.Tensor, ref: torch.Tensor, tile: int = 128) -> float:
    """Largest per-tile max|out - ref| / max|ref| over tile x tile blocks."""
    m, n = ref.shape[-2:]
    assert m % tile == 0 and n % tile == 0
    d = (out.float() - ref).abs().reshape(m // tile, tile, n // tile, tile).amax(dim=(1, 3))
    r = ref.abs().reshape(m // tile, tile, n // tile, tile).amax(dim=(1, 3))
    return (d / r).max().item()


def _transposed(q: QuantResult) -> QuantResult:
    """Logical transpose of the last two dims (a strided view) with its scales."""
    return QuantResult(q.tensor.transpose(-1, -2), q.dequant_scale.transpose(-1, -2), q.impl, "block",
                       {**q.meta, "block_m": q.meta["block_n"], "block_n": q.meta["block_m"]})


@pytest.fixture(scope="module")
def config5(dev, config5_host):
    """BASELINE config 5 operands: X ~ N(0,1), W ~ N(0,0.02), dY ~ N(0,1e-3),
    drawn from the CPU generator with seed 0 (the tensors bench.py times)."""
    x, w, dy = config5_host
    assert x.shape == (M5, K5) and w.shape == (N5, K5) and dy.shape == (M5, N5)
    return x[None].to(dev), w[None].to(dev), dy[None].to(dev)


def test_config5_forward_full(dev, config5):
    """fwd: X (1x128) times W^T (128x128), a_k_b_k."""
    x, w, _ = config5
    print("config5 fwd a_k_b_k", flush=True)
    qx = hip_per_block_quant(x, block_m=1, block_n=128)
    qw = hip_per_block_quant(w, block_m=128, block_n=128)
    out = hip_per_block_bmm(qx, _transposed(qw))
    ref = torch.matmul(qx.dequantize()[0], qw.dequantize()[0].t().contiguous())
    err = _tile_err(out[0], ref)
    assert err <= TOL, err


def test_config5_dgrad_full(dev, config5):
    """dgrad: dY (1x128) times W (128x128), a_k_b_n."""
    _, w, dy = config5
    print("config5 dgrad a_k_b_n", flush=True)
    qdy = hip_per_block_quant(dy, block_m=1, block_n=128)
    qw = hip_per_block_quant(w, block_m=128, block_n=128)
    out = hip_per_block_bmm(qdy, qw)
    ref = torch.matmul(qdy.dequantize()[0], qw.dequantize()[0])
    err = _tile_err(out[0], ref)
    assert err <= TOL, err


@pytest.mark.parametrize("k_major", [False, True], ids=["a_m_b_n", "layer_k_major"])
def test_config5_wgrad_full(dev, config5, k_major):
    """wgrad: dY^T times X, both re-quantized 128x1 along M. a_m_b_n is the
    reference's layout (strided views); the training layer stores the 128x1
    operands transposed, so its wgrad runs on K-major operands. 896 output
    tiles on 256 CUs: the last wave runs as half tiles."""
    x, _, dy = config5
    print(f"config5 wgrad k_major={k_major}", flush=True)
    qdy_m = hip_per_block_quant(dy, block_m=128, block_n=1)   # scales [1, M/128, N]
    qx_m = hip_per_block_quant(x, block_m=128, block_n=1)     # scales [1, M/128, K]
    a = _transposed(qdy_m)                                     # [1, N, M], M-major
    b = qx_m                                                   # [1, M, K], K-major rows
    if k_major:
        a = QuantResult(a.tensor.contiguous(), a.dequant_scale, a.impl, "block", dict(a.meta))
        b = QuantResult(b.tensor.transpose(-1, -2).contiguous().transpose(-1, -2), b.dequant_scale, b.impl,
                        "block", dict(b.meta))
        assert a.tensor.stride(-1) == 1 and b.tensor.stride(-2) == 1
    out = hip_per_block_bmm(a, b)
    ref = torch.matmul(qdy_m.dequantize()[0].t().contiguous(), qx_m.dequantize()[0])
    err = _tile_err(out[0], ref)
    assert err <= TOL, err


def test_config4_all_batches(dev):
    """BASELINE config 4 (A [128,2048,128] 1x128, B [128,128,512] 128x128),
    every one of the 128 batches against an fp32 bmm of the dequantized
    operands."""
    g = torch.Generator().manual_seed(0)
    ah = torch.randn(128, 2048, 128, generator=g).bfloat16().to(dev)
    bh = torch.randn(128, 128, 512, generator=g).bfloat16().to(dev)
    qa = hip_per_block_quant(ah, block_m=1, block_n=128)
    qb = hip_per_block_quant(bh, block_m=128, block_n=128)
    print("config4 all batches", flush=True)
    out = hip_per_block_bmm(qa, qb)
    ref = torch.bmm(qa.dequantize().contiguous(), qb.dequantize().contiguous())
    err = ((out.float() - ref).abs().amax(dim=(1, 2)) / ref.abs().amax(dim=(1, 2)))
    assert err.shape == (128,)
    assert err.max().item() <= TOL, (err.argmax().item(), err.max().item())


# ---------------------------------------------------------------------------
# scales_are_quant: the epilogue multiplies by 1 / (sa * sb)
# ---------------------------------------------------------------------------
def _fp8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * 2.0).to(torch.float8_e4m3fn)


def _quant_scales(shape, seed):
    # quant scales as a quantizer would produce them (fp8_max / amax), spread
    # over two decades so a wrongly oriented or un-inverted scale shows
    g = torch.Generator().manual_seed(seed)
    return torch.exp(torch.empty(*shape).uniform_(np.log(1.0), np.log(100.0), generator=g)).float()


def _bmm_abi(a, b, c, sa, sb, mode, saq):
    rc = _lib.lib().pcamd_bmm_scaled(
        _lib.ptr(a), _lib.ptr(b), _lib.E4M3FN, a.shape[0], a.shape[1], b.shape[2], a.shape[2],
        *a.stride(), *b.stride(), _lib.ptr(c), _lib.dtype_code(c.dtype), *c.stride(), None, 0, 0, 0, 0,
        _lib.ptr(sa), *(sa.stride() + (0,) * (3 - sa.dim())), _lib.ptr(sb),
        *(sb.stride() + (0,) * (3 - sb.dim())), mode, saq, 1, 128, 1, _lib.ACT_NONE, _lib.stream_of(c))
    _lib.check(rc, "pcamd_bmm_scaled")
    torch.cuda.synchronize()


# (batch, m, n, k): K = 128 takes the single-step kernel, K = 512 the wide
# kernel, the odd shape the general kernel
KERNEL_SHAPES = {"single_k128": (2, 256, 384, 128), "wide_k512": (2, 512, 512, 512),
                 "general_unaligned": (2, 33, 47, 200)}


@pytest.mark.parametrize("out", ["f32", "bf16"])
@pytest.mark.parametrize("mode", ["channel", "tensor"])
@pytest.mark.parametrize("kernel", sorted(KERNEL_SHAPES))
def test_scales_are_quant(dev, kernel, mode, out):
    """fp32 output goes through the per-element epilogue, bf16 output (aligned
    shapes) through the LDS-staged one of the single-step and wide kernels."""
    bsz, m, n, k = KERNEL_SHAPES[kernel]
    print(f"scales_are_quant {kernel} {mode} {out}", flush=True)
    odt = torch.float32 if out == "f32" else torch.bfloat16
    tol = 1e-4 if out == "f32" else 1e-2  # fp32: accumulation order and the scale rounding; bf16: its rounding
    a, b = _fp8((bsz, m, k), 1), _fp8((bsz, k, n), 2)
    if mode == "channel":
        qsa, qsb = _quant_scales((bsz, m), 3), _quant_scales((bsz, n), 4)
        code = _lib.SCALE_CHANNEL
        factor = 1.0 / (qsa.double()[:, :, None] * qsb.double()[:, None, :])
    else:
        qsa, qsb = _quant_scales((1,), 3), _quant_scales((1,), 4)
        code = _lib.SCALE_TENSOR
        factor = 1.0 / (qsa.double()[0] * qsb.double()[0])
    prod = np.matmul(O.decode(a.view(torch.uint8).numpy()).astype(np.float64),
                     O.decode(b.view(torch.uint8).numpy()).astype(np.float64))
    ref = prod * factor.numpy()
    ad, bd = a.to(dev), b.to(dev)
    c = torch.empty(bsz, m, n, dtype=odt, device=dev)
    _bmm_abi(ad, bd, c, qsa.to(dev), qsb.to(dev), code, 1)
    err = O.max_abs_rel(c.float().cpu().numpy(), ref)
    assert err <= tol, err
    # the same product through dequant scales (scales_are_quant = 0)
    c0 = torch.empty_like(c)
    if mode == "channel":
        _bmm_abi(ad, bd, c0, (1.0 / qsa).to(dev), (1.0 / qsb).to(dev), code, 0)
    else:
        _bmm_abi(ad, bd, c0, (1.0 / (qsa * qsb)).to(dev), qsb.to(dev), code, 0)
    assert O.max_abs_rel(c0.float().cpu().numpy(), ref) <= tol


@pytest.mark.parametrize("n", [64, 192, 256])
def test_fused_quant_bmm_bench_shape(dev, n):
    """The fused activation-quant BMM at the shape bench.py --fused times
    (bf16 A [32768, 4096], e4m3fn B [4096, N] with 128x128 scales), with the
    quantized A written out: those bytes and scales are the 1x128 quantizer's
    bit for bit, the product equals quantize-then-multiply to fp32 rounding,
    and every 64x64 output tile is within the bar of an fp32 GEMM of the
    dequantized operands."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm_quant_a
    g = torch.Generator().manual_seed(n)
    x = torch.randn(1, 32768, 4096, generator=g).bfloat16().to(dev)
    qb = hip_per_block_quant((torch.randn(1, 4096, n, generator=g) * 0.02).bfloat16().to(dev),
                             block_m=128, block_n=128)
    print(f"fused quant bmm full size n={n}", flush=True)
    out, qa = hip_per_block_bmm_quant_a(x, qb, return_quant=True)
    ref_q = hip_per_block_quant(x, block_m=1, block_n=128)
    unfused = hip_per_block_bmm(ref_q, qb)
    torch.cuda.synchronize()
    assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))
    assert torch.equal(qa.dequant_scale.view(torch.int32), ref_q.dequant_scale.view(torch.int32))
    scale = unfused.float().abs().max().item()
    assert (out.float() - unfused.float()).abs().max().item() <= 1e-6 * scale
    ref = torch.matmul(ref_q.dequantize()[0], qb.dequantize()[0].contiguous())
    err = _tile_err(out[0], ref, tile=64)
    assert err <= TOL, err
