"""GPU parity of the scaled FP8 BMM when K is not a multiple of 128.

The wide kernel takes K > 128 with K % 4 == 0: its last K step holds fewer
than 128 valid k, and the fragment words past them are zeroed in both
operands (a K-major row's tail holds the next row's bytes). The reference's
Triton kernels mask the same tail with `offs_k < K`
(xuOAO/practice_cuda kernels/bmm/per_block.py:82-107,
kernels/fp8_bmm/kernel/fp8_quant_bmm_kernel.py:87-132). 12 of the 31 shapes
the reference publishes timings for (fp8_training/fp8_bench/cases.py:25-41,
kernels/fp8_bmm/bench/fp8_quant_bmm_best*.json) have K = 160, 960 or 1600.

Checks, within max|out - ref| / max|ref| <= 1e-2 of the fp64 (small) or fp32
(GPU, per 128 x 128 tile) product of the dequantized operands:
- every scale scheme (1x128 / 128x128 block, channel, tensor) on the
  K-major and MN-major layouts at K = 160, 960, 1600;
- MN-major operands with K % 16 != 0 (K = 260, 300: a partial word boundary
  of 4 bytes inside the last step);
- more tiles than CUs, so the last wave runs as half tiles with the masked
  step;
- the legacy per-tensor API with fp16 output and an fp16 [B, M, N] bias (the
  reference sweep's signature, find_fp8_bmm_best.py:34-53) on published
  shapes, B N-major and K-major;
- NaN codes in the padding of K-major rows stored with a padded pitch (the
  bytes the last K step reads past K) leave the output bit-identical to the
  unpadded product.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd import get_bmm, get_quant
from practice_cuda_amd.fp8_bmm import fp8_bmm_quant

pytestmark = pytest.mark.gpu
TOL = 1e-2
SCHEMES = ("hip_per_block_1d", "hip_per_block_2d", "hip_per_channel", "hip_per_tensor")


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).bfloat16()


def _mn_major(t: torch.Tensor) -> torch.Tensor:
    return t.transpose(-1, -2).contiguous().transpose(-1, -2)


def _run(name, a, b, dev):
    impl = get_bmm(name)
    quant = get_quant(impl.quant_impl)
    a_in = _mn_major(a) if impl.a_layout == "m" else a
    b_in = _mn_major(b) if impl.layout == "k" else b
    qa = impl.prepare_a(quant.fn(a_in.to(dev), **impl.quant_a_kwargs))
    qb = impl.prepare_b(quant.fn(b_in.to(dev), **impl.quant_b_kwargs))
    out = impl.fn(qa, qb, **impl.prepare_call_kwargs(qa, qb))
    torch.cuda.synchronize()
    return out, qa, qb


@pytest.mark.parametrize("k", [160, 960, 1600])
@pytest.mark.parametrize("layout", ["a_k_b_k", "a_k_b_n", "a_m_b_n"])
@pytest.mark.parametrize("scheme", SCHEMES)
def test_ragged_k_matches_oracle(dev, scheme, layout, k):
    shape = (2, 256, 384, k)
    print(f"ragged K {scheme}_{layout} {shape}", flush=True)
    bsz, m, n, _ = shape
    out, qa, qb = _run(f"{scheme}_{layout}", _rand((bsz, m, k), k + 1), _rand((bsz, k, n), k + 2), dev)
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    err = O.max_abs_rel(out.float().cpu().numpy(), ref)
    assert err <= TOL, f"max_abs_rel {err}"


@pytest.mark.parametrize("k", [260, 300])
@pytest.mark.parametrize("scheme", SCHEMES)
def test_ragged_k_mn_major_word_boundary(dev, scheme, k):
    """Both operands MN-major (rows of 16-byte aligned k-rows for any K): the
    last step's valid k end inside a 16-byte chunk of the fragment."""
    shape = (2, 200, 320, k)
    print(f"ragged K mn-major {scheme} {shape}", flush=True)
    bsz, m, n, _ = shape
    out, qa, qb = _run(f"{scheme}_a_m_b_n", _rand((bsz, m, k), 7), _rand((bsz, k, n), 8), dev)
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    err = O.max_abs_rel(out.float().cpu().numpy(), ref)
    assert err <= TOL, f"max_abs_rel {err}"


def _tile_err(out: torch.Tensor, ref: torch.Tensor, tile: int = 128) -> float:
    m, n = ref.shape[-2:]
    d = (out.float() - ref).abs().reshape(-1, m // tile, tile, n // tile, tile).amax(dim=(2, 4))
    r = ref.abs().reshape(-1, m // tile, tile, n // tile, tile).amax(dim=(2, 4))
    return (d / r).max().item()


@pytest.mark.parametrize("scheme,layout", [("hip_per_tensor", "a_k_b_n"), ("hip_per_block_2d", "a_k_b_k"),
                                           ("hip_per_channel", "a_m_b_n")])
def test_ragged_k_half_tile_tail(dev, scheme, layout):
    """More 256 x 256 tiles than CUs with a short last wave: the tail runs as
    half tiles, also with the masked last K step."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    tiles_n = 8
    tiles_m = (cus + 16) // tiles_n + 1          # cus + a small tail of whole tiles
    m, n, k = tiles_m * 256, tiles_n * 256, 960
    print(f"ragged K half tiles {scheme}_{layout} m={m} n={n} k={k} cus={cus}", flush=True)
    out, qa, qb = _run(f"{scheme}_{layout}", _rand((1, m, k), 21), _rand((1, k, n), 22), dev)
    ref = torch.matmul(qa.dequantize()[0].float(), qb.dequantize()[0].float().contiguous())
    err = _tile_err(out[0], ref)
    assert err <= TOL, f"per-tile max_abs_rel {err}"


def _fp8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * 0.5).to(torch.float8_e4m3fn)


# (B, M, N, K) of the reference's published sweep with K % 128 != 0, and one
# aligned neighbour
PUBLISHED = [(16, 512, 1280, 160), (16, 2048, 1280, 960), (32, 512, 960, 1600), (16, 512, 960, 1280)]


@pytest.mark.parametrize("b_k_major", [False, True], ids=["b_n", "b_k"])
@pytest.mark.parametrize("shape", PUBLISHED)
def test_legacy_fp16_bias_published_shapes(dev, shape, b_k_major):
    """fp8_bmm_quant(A, B, bias, quant_scale=s, out_dtype=fp16) with an fp16
    [B, M, N] bias: C = (A @ B) * s + bias, rounded once to fp16."""
    bsz, m, n, k = shape
    print(f"legacy fp16+bias {shape} b_k_major={b_k_major}", flush=True)
    a, b = _fp8((bsz, m, k), 31), _fp8((bsz, k, n), 32)
    g = torch.Generator().manual_seed(33)
    bias = torch.randn(bsz, m, n, generator=g).half()
    bd = b.to(dev)
    if b_k_major:
        bd = bd.transpose(1, 2).contiguous().transpose(1, 2)  # stored [B, N, K]
    out = fp8_bmm_quant(a.to(dev), bd, bias.to(dev), quant_scale=0.75, out_dtype=torch.float16)
    assert out.dtype == torch.float16 and out.shape == (bsz, m, n)
    ref = torch.matmul(a.to(dev).float(), b.to(dev).float()) * 0.75 + bias.to(dev).float()
    assert torch.isfinite(out).all()
    err = ((out.float() - ref).abs().amax() / ref.abs().amax()).item()
    assert err <= TOL, err


@pytest.mark.parametrize("layout", ["a_k_b_k", "a_k_b_n"])
def test_ragged_k_tail_bytes_are_masked(dev, layout):
    """K-major rows stored with a padded pitch (1024 bytes for K = 960): the
    last K step reads each row's 64 padding bytes, which hold NaN codes
    (0x7F) here. The masked words never reach the MFMA, so the output equals
    the product of the same values stored unpadded, bit for bit."""
    bsz, m, n, k, pitch = 2, 256, 256, 960, 1024
    print(f"ragged K NaN padding {layout}", flush=True)
    a, b = _fp8((bsz, m, k), 41), _fp8((bsz, k, n), 42)
    ad, bd = a.to(dev), b.to(dev)
    if layout == "a_k_b_k":
        bd = bd.transpose(1, 2).contiguous().transpose(1, 2)  # stored [B, N, K]
    s = torch.tensor(1.0, device=dev)
    clean = fp8_bmm_quant(ad, bd, quant_scale=s, out_dtype=torch.float32)
    a_pad = torch.full((bsz, m, pitch), 0x7F, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    a_pad[:, :, :k] = ad
    ap = a_pad[:, :, :k]
    assert ap.stride() == (m * pitch, pitch, 1)
    bp = bd
    if layout == "a_k_b_k":
        b_pad = torch.full((bsz, n, pitch), 0x7F, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
        b_pad[:, :, :k] = bd.transpose(1, 2)
        bp = b_pad[:, :, :k].transpose(1, 2)
    dirty = fp8_bmm_quant(ap, bp, quant_scale=s, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.isfinite(dirty).all()
    assert torch.equal(clean, dirty)
    ref = np.matmul(a.float().numpy().astype(np.float64), b.float().numpy().astype(np.float64))
    assert O.max_abs_rel(clean.cpu().numpy(), ref) <= TOL
