"""GPU parity of the legacy tuple API (practice_cuda_amd.fp8_bmm).

Mirrors kernels/fp8_bmm/test/fp8_quant_test.py and fp8_quant_bmm_test.py of
the reference with the same shapes and invariants, and checks results
against the CPU oracle:
* fp8_quant: fp8 bytes and the reciprocal bit-exact against
  oracle.quant_tensor(scale_dt="input") (the fp8_warper.py:21-25 scale steps
  in x's dtype, then fp32 multiply / clamp / RNE cast) for float32, bfloat16
  and float16 inputs, E4M3 and E5M2;
* fp8_bmm_quant: within max-abs-relative 1e-2 of the fp64 product of the
  fp8 inputs times quant_scale plus bias; fp8 outputs within one e4m3 step
  (the fp32 sum order can flip a rounding, fp8_quant_bmm_test.py:154-160).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd.fp8_bmm import FP8Format, fp8_bmm_quant, fp8_quant, fp8_quant_triton

pytestmark = pytest.mark.gpu

SHAPES = [(128, 256), (17, 33), (32, 2048, 960), (80, 2048, 640), (14, 2048, 8192)]


def _randn(shape, seed, dtype=torch.float32, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _check_quant(x_cpu, dev, fmt="e4m3", quant_dtype=torch.float8_e4m3fn, fp8_range=448.0):
    q, recip = fp8_quant(x_cpu.to(dev), quant_dtype=quant_dtype, fp8_range=fp8_range)
    torch.cuda.synchronize()
    q_ref, ds_ref, _ = O.quant_tensor(x_cpu, fmt, scale_dt="input", fp8_max=fp8_range)
    assert q.dtype == quant_dtype and q.shape == x_cpu.shape
    assert recip.dtype == x_cpu.dtype and recip.dim() == 0
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.float32(recip.float().item()) == np.float32(ds_ref)
    return q, recip


@pytest.mark.parametrize("shape", SHAPES)
def test_quant_matches_oracle_fp32(dev, shape):
    print(f"legacy quant fp32 {shape}", flush=True)
    _check_quant(_randn(shape, 1), dev)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(128, 256), (17, 33), (32, 2048, 960)])
def test_quant_matches_oracle_half_dtypes(dev, dtype, shape):
    _check_quant(_randn(shape, 2, dtype, 3.0), dev)


def test_quant_e5m2_format_enum(dev):
    x = _randn((64, 128), 3)
    q, _ = fp8_quant(x.to(dev), quant_dtype=FP8Format.E5M2, fp8_range=FP8Format.E5M2.value.max_fwd)
    q_ref, _, _ = O.quant_tensor(x, "e5m2", scale_dt="input", fp8_max=57344.0)
    assert q.dtype == torch.float8_e5m2
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)


@pytest.mark.parametrize("dtype,quant_dtype,fmt,fp8_range", [
    (torch.bfloat16, torch.float8_e4m3fn, "e4m3", 240.0),
    (torch.float16, torch.float8_e4m3fn, "e4m3", 100.0),
    (torch.float32, torch.float8_e4m3fn, "e4m3", float(np.nextafter(np.float32(248.0), np.float32(0.0)))),
    (torch.bfloat16, torch.float8_e5m2, "e5m2", 36864.0),
])
def test_quant_fp8_range_argument(dev, dtype, quant_dtype, fmt, fp8_range):
    """A caller-chosen fp8_range (fp8_warper.py:12) below the format maximum:
    the clamping kernel and the scale arithmetic in the input's dtype, bit for
    bit against the oracle."""
    print(f"legacy fp8_range={fp8_range} {dtype} {fmt}", flush=True)
    _check_quant(_randn((3, 100, 300), 9, dtype, 2.0), dev, fmt, quant_dtype, fp8_range)


def test_quant_reference_name_alias(dev):
    assert fp8_quant_triton is fp8_quant
    x = _randn((32, 64), 4)
    q1, r1 = fp8_quant_triton(x.to(dev), is_test=True)
    q2, r2 = fp8_quant(x.to(dev))
    assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(r1, r2)


def test_quant_outliers_saturate_and_range(dev):
    x = _randn((64, 64), 5)
    x[0, 0], x[1, 1] = 1e6, -1e6
    q, _ = _check_quant(x, dev)
    f = q.float().cpu()
    assert f.abs().max().item() <= 448.0
    assert f[0, 0].item() == 448.0 and f[1, 1].item() == -448.0
    big = _randn((3, 50, 70), 6, scale=1000.0)
    q, _ = _check_quant(big, dev)
    assert q.float().abs().max().item() <= 448.0


def test_fp16_all_zero_edge(dev):
    # eps rounds to 0 in fp16: quant factor inf, reciprocal 0 as in the
    # reference (kernels/fp8_bmm/fp8_warper.py:21-25); the elements are 0 * inf = NaN before
    # the clamp, which here gives -448 (the reference leaves NaN to tl.clamp)
    q, recip = fp8_quant(torch.zeros(4, 64, dtype=torch.float16, device=dev))
    torch.cuda.synchronize()
    assert recip.item() == 0.0
    assert torch.equal(q.view(torch.uint8).unique().cpu(), torch.tensor([0xFE], dtype=torch.uint8))
    assert torch.all((q.float() * recip.float()) == 0)


def test_quant_zeros_and_roundtrip(dev):
    q, recip = _check_quant(torch.zeros(32, 64), dev)
    assert q.float().abs().max().item() == 0.0 and torch.isfinite(recip).item()
    x = _randn((4, 64, 128), 7)
    q, recip = fp8_quant(x.to(dev))
    x_hat = q.float() * recip.float()
    assert torch.allclose(x_hat.cpu(), x, rtol=1e-1, atol=0.1 * x.abs().max().item() / 16)


def test_quant_determinism_and_bad_rank(dev):
    x = _randn((64, 128), 8).to(dev)
    a, _ = fp8_quant(x)
    b, _ = fp8_quant(x)
    assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    with pytest.raises(RuntimeError, match="dim must eq 2 or 3"):
        fp8_quant(torch.zeros(4, device=dev))


# --------------------------------------------------------------------------- BMM
BMM_SHAPES = [(1, 128, 128, 128), (2, 64, 64, 64), (3, 33, 47, 65), (4, 256, 512, 256)]


def _fp8(shape, seed, dtype=torch.float8_e4m3fn):
    return (_randn(shape, seed) * 0.5).to(dtype)


def _ref(a, b, scale, bias=None):
    out = np.matmul(a.float().numpy().astype(np.float64), b.float().numpy().astype(np.float64)) * scale
    if bias is not None:
        out = out + bias.double().numpy()
    return out


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("shape", BMM_SHAPES)
def test_bmm_matches_reference(dev, shape, out_dtype):
    bs, m, k, n = shape
    a, b = _fp8((bs, m, k), 10), _fp8((bs, k, n), 11)
    scale = torch.tensor(0.75, device=dev)
    out = fp8_bmm_quant(a.to(dev), b.to(dev), quant_scale=scale, out_dtype=out_dtype)
    assert out.dtype == out_dtype and out.shape == (bs, m, n)
    assert O.max_abs_rel(out.float().cpu().numpy(), _ref(a, b, 0.75)) <= 1e-2


@pytest.mark.parametrize("shape", BMM_SHAPES)
def test_bmm_fp8_output(dev, shape):
    bs, m, k, n = shape
    a, b = _fp8((bs, m, k), 12), _fp8((bs, k, n), 13)
    out = fp8_bmm_quant(a.to(dev), b.to(dev), quant_scale=1.0, out_dtype=torch.float8_e4m3fn)
    ref = torch.from_numpy(np.clip(_ref(a, b, 1.0), -448, 448)).float().to(torch.float8_e4m3fn).float()
    got = out.float().cpu()
    assert torch.allclose(got, ref, rtol=2e-1, atol=1e-1)


@pytest.mark.parametrize("shape", BMM_SHAPES)
def test_bmm_bias_3d_and_2d(dev, shape):
    bs, m, k, n = shape
    a, b = _fp8((bs, m, k), 14), _fp8((bs, k, n), 15)
    bias3 = _randn((bs, m, n), 16)
    out = fp8_bmm_quant(a.to(dev), b.to(dev), bias3.to(dev), quant_scale=1.0, out_dtype=torch.bfloat16)
    assert O.max_abs_rel(out.float().cpu().numpy(), _ref(a, b, 1.0, bias3)) <= 1e-2
    bias2 = _randn((m, n), 17)
    out = fp8_bmm_quant(a.to(dev), b.to(dev), bias2.to(dev), quant_scale=1.0, out_dtype=torch.bfloat16)
    assert O.max_abs_rel(out.float().cpu().numpy(), _ref(a, b, 1.0, bias2)) <= 1e-2


def test_bmm_scale_applied_and_saturation(dev):
    a, b = _fp8((1, 64, 64), 18), _fp8((1, 64, 64), 19)
    s1 = fp8_bmm_quant(a.to(dev), b.to(dev), quant_scale=1.0, out_dtype=torch.float32)
    s2 = fp8_bmm_quant(a.to(dev), b.to(dev), quant_scale=2.0, out_dtype=torch.float32)
    nz = s1.abs() > 1e-3
    assert torch.allclose(s2[nz] / s1[nz], torch.full_like(s1[nz], 2.0), rtol=1e-2, atol=1e-2)
    a, b = _fp8((1, 64, 128), 20), _fp8((1, 128, 64), 21)
    out = fp8_bmm_quant(a.to(dev), b.to(dev), quant_scale=100.0, out_dtype=torch.float8_e4m3fn)
    assert out.float().abs().max().item() <= 448.0


def test_bmm_quant_scale_from_legacy_quant(dev):
    """The usual chain: quantize both operands, pass recip_a * recip_b (bf16)."""
    xa, xb = _randn((2, 96, 256), 22, torch.bfloat16), _randn((2, 256, 80), 23, torch.bfloat16)
    qa, ra = fp8_quant(xa.to(dev))
    qb, rb = fp8_quant(xb.to(dev))
    scale = ra * rb  # bf16 0-d, as the reference callers form it
    out = fp8_bmm_quant(qa, qb, quant_scale=scale, out_dtype=torch.bfloat16)
    ref = _ref(qa.cpu(), qb.cpu(), float(scale.float().item()))
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= 1e-2


def test_bmm_zeros_batch_independence_determinism(dev):
    z = torch.zeros(2, 32, 64, dtype=torch.float8_e4m3fn, device=dev)
    zb = torch.zeros(2, 64, 32, dtype=torch.float8_e4m3fn, device=dev)
    out = fp8_bmm_quant(z, zb, quant_scale=1.0, out_dtype=torch.float32)
    assert not torch.isnan(out).any() and out.abs().max().item() == 0.0
    a, b = _fp8((2, 32, 32), 24).to(dev), _fp8((2, 32, 32), 25).to(dev)
    full = fp8_bmm_quant(a, b, quant_scale=1.0, out_dtype=torch.float32)
    for i in range(2):
        one = fp8_bmm_quant(a[i:i + 1], b[i:i + 1], quant_scale=1.0, out_dtype=torch.float32)
        assert torch.allclose(full[i], one[0], rtol=1e-3, atol=1e-3)
    o1 = fp8_bmm_quant(a, b, quant_scale=1.0, out_dtype=torch.bfloat16)
    o2 = fp8_bmm_quant(a, b, quant_scale=1.0, out_dtype=torch.bfloat16)
    assert torch.equal(o1, o2)


def test_bmm_strided_operands(dev):
    """Transposed-storage operands (A M-major, B K-major) and a generic stride."""
    a, b = _fp8((2, 96, 128), 26), _fp8((2, 128, 160), 27)
    a_m = a.transpose(-1, -2).contiguous().transpose(-1, -2).to(dev)
    b_k = b.transpose(-1, -2).contiguous().transpose(-1, -2).to(dev)
    out = fp8_bmm_quant(a_m, b_k, quant_scale=1.0, out_dtype=torch.bfloat16)
    assert O.max_abs_rel(out.float().cpu().numpy(), _ref(a, b, 1.0)) <= 1e-2
    wide = _fp8((2, 96, 256), 28)
    a_s = wide.to(dev)[:, :, ::2]  # neither K nor M contiguous
    out = fp8_bmm_quant(a_s, b.to(dev), quant_scale=1.0, out_dtype=torch.bfloat16)
    assert O.max_abs_rel(out.float().cpu().numpy(), _ref(wide[:, :, ::2], b, 1.0)) <= 1e-2
