"""Pins of the oracle's legacy per-tensor scale arithmetic (CPU only).

kernels/fp8_bmm/fp8_warper.py:21-25 computes the per-tensor quant factor with
torch ops on 0-d tensors of the input's dtype, so for bf16 / fp16 inputs each
step rounds to that dtype. The oracle restates that with an explicit RNE
rounding (oracle_round_dt). These tests pin it against torch's own CPU
arithmetic (torch is a library here, not the reference):
* oracle_round_dt against torch's float32 -> bf16 / fp16 casts over ranges
  that include subnormals, ties and overflow;
* the full scale pipeline (aminmax, clamp(eps), fp8_range / t, reciprocal) of
  fp8_warper.py evaluated by torch eagerly in the input's dtype, and the
  kernel's fp32 multiply + clamp + cast (kernel/fp8_quant_kernel.py:56-60).
A mistake such as rounding in fp32 instead of bf16, dropping the eps clamp or
computing fp8_range / s as a true division changes these scales.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O


def _sample_f32(seed: int, n: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    bits = rng.integers(0, 1 << 32, size=n, dtype=np.uint64).astype(np.uint32)
    v = bits.view(np.float32)
    v = v[np.isfinite(v)]
    # plus values around the fp16 subnormal / overflow edges and bf16 ties
    edges = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 6.1035156e-05, 5.9604645e-08,
                      2.9802322e-08, 2.98023259e-08, 1e-12, 448.0, 1.00390625, 1.01171875, 3.0e38],
                     dtype=np.float32)
    return np.concatenate([v, edges, -edges])


@pytest.mark.parametrize("dt,torch_dt", [(O.BF16, torch.bfloat16), (O.F16, torch.float16)])
def test_round_dt_matches_torch_cast(dt, torch_dt):
    vals = _sample_f32(7, 20000)
    ours = np.array([O.round_dt(float(v), dt) for v in vals], dtype=np.float32)
    ref = torch.from_numpy(vals).to(torch_dt).float().numpy()
    assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))


def _legacy_torch(x: torch.Tensor, fp8_dtype, fp8_range: float, eps: float = 1e-12):
    """fp8_warper.py:21-25 in torch eager ops (x's dtype), then the kernel's
    fp32 multiply / clamp / cast (kernel/fp8_quant_kernel.py:56-60)."""
    x_min, x_max = x.aminmax()
    x_max_abs = torch.maximum(x_min.abs(), x_max.abs()).clamp(min=eps)
    quant_factor = fp8_range / x_max_abs
    reciprocal = quant_factor.reciprocal()
    q = torch.clamp(x.float() * quant_factor.float(), -fp8_range, fp8_range).to(fp8_dtype)
    return q, reciprocal


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape,scale", [((17, 33), 1.0), ((3, 40, 64), 37.0), ((64, 64), 1e-3), ((8, 8), 3e4)])
def test_legacy_scale_pipeline_matches_torch(dtype, shape, scale):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(*shape, generator=g) * scale).to(dtype)
    q_ref, recip_ref = _legacy_torch(x, torch.float8_e4m3fn, 448.0)
    q, ds, qs = O.quant_tensor(x, "e4m3", scale_dt="input")
    assert np.array_equal(q, q_ref.view(torch.uint8).numpy())
    assert np.float32(ds) == np.float32(recip_ref.float().item())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_legacy_e5m2_and_zero_input(dtype):
    x = (torch.randn(32, 48, generator=torch.Generator().manual_seed(3)) * 5).to(dtype)
    q_ref, recip_ref = _legacy_torch(x, torch.float8_e5m2, 57344.0)
    q, ds, _ = O.quant_tensor(x, "e5m2", scale_dt="input", fp8_max=57344.0)
    assert np.array_equal(q, q_ref.view(torch.uint8).numpy())
    assert np.float32(ds) == np.float32(recip_ref.float().item())
    z = torch.zeros(16, 16, dtype=dtype)
    q_ref, recip_ref = _legacy_torch(z, torch.float8_e4m3fn, 448.0)
    q, ds, _ = O.quant_tensor(z, "e4m3", scale_dt="input")
    assert not q.any() and np.float32(ds) == np.float32(recip_ref.float().item())


def test_fp32_scale_dt_is_the_fp8_bench_form():
    """scale_dt=F32 keeps the reciprocal-multiply form of triton_per_tensor.py:40-44."""
    x = torch.randn(50, 70, generator=torch.Generator().manual_seed(11))
    _, ds32, qs32 = O.quant_tensor(x, "e4m3")
    _, ds_in, qs_in = O.quant_tensor(x, "e4m3", scale_dt="input")
    amax = np.float32(x.abs().max().item())
    qs = np.float32(np.float32(1.0) / amax) * np.float32(448.0)
    assert qs32 == qs and ds32 == np.float32(np.float32(1.0) / qs)
    assert (ds32, qs32) == (ds_in, qs_in)
