"""CPU checks of the FP8 training layer API (practice_cuda_amd.modules).

Mirrors the module-level contract of fp8_training/fp8_bench/modules/
bmm_linear.py: constructor validation, the high-precision BMMLinear
baseline, recursive conversion sharing parameters (from_float), input shape
errors raised before any launch, and the fake (meta) implementations that let
the custom ops trace under torch.compile.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn
from torch._subclasses.fake_tensor import FakeTensorMode

from practice_cuda_amd.modules import (BMMLinear, Float8BlockBMMLinearConfig, Float8BMMLinear,
                                       convert_to_float8_bmm_training)


def test_config_validation():
    with pytest.raises(ValueError, match="granularity"):
        Float8BlockBMMLinearConfig(granularity="axis")
    with pytest.raises(ValueError, match="fp8_dtype"):
        Float8BlockBMMLinearConfig(fp8_dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="128"):
        Float8BlockBMMLinearConfig(block=64)
    with pytest.raises(ValueError, match="grad_fp8_dtype"):
        Float8BlockBMMLinearConfig(grad_fp8_dtype=torch.float16)
    assert Float8BlockBMMLinearConfig(grad_fp8_dtype=torch.float8_e5m2).grad_fp8_dtype == torch.float8_e5m2


def test_bmm_linear_baseline_and_errors():
    torch.manual_seed(0)
    layer = BMMLinear(2, 16, 24)
    x = torch.randn(2, 5, 16)
    ref = torch.bmm(x, layer.weight.transpose(-2, -1)) + layer.bias.unsqueeze(1)
    assert torch.allclose(layer(x), ref, atol=1e-6)
    bound = 1 / 16 ** 0.5
    assert layer.weight.abs().max() <= bound and layer.bias.abs().max() <= bound
    with pytest.raises(ValueError, match="positive"):
        BMMLinear(0, 16, 24)
    with pytest.raises(ValueError, match=r"expects \[B,M,K\]"):
        layer(torch.randn(5, 16))
    with pytest.raises(ValueError, match="shape mismatch"):
        layer(torch.randn(2, 5, 17))
    assert "bias=True" in layer.extra_repr()


def test_convert_replaces_nested_and_shares_parameters():
    model = nn.Sequential(BMMLinear(2, 8, 8), nn.ReLU(), nn.Sequential(BMMLinear(2, 8, 4, bias=False)))
    w0, w1 = model[0].weight, model[2][0].weight
    convert_to_float8_bmm_training(model, Float8BlockBMMLinearConfig(granularity="tensor"))
    assert isinstance(model[0], Float8BMMLinear) and isinstance(model[2][0], Float8BMMLinear)
    assert model[0].weight is w0 and model[2][0].weight is w1 and model[2][0].bias is None
    assert model[0].config.granularity == "tensor"
    assert "granularity=tensor" in model[0].extra_repr()
    # already converted modules are left alone
    assert convert_to_float8_bmm_training(model[0]) is model[0]
    with pytest.raises(TypeError):
        Float8BMMLinear.from_float(nn.Linear(2, 2))


def test_float8_layer_checks_input_before_launch():
    layer = Float8BMMLinear(1, 128, 128)
    with pytest.raises(ValueError, match="shape mismatch"):
        layer(torch.randn(1, 4, 64))


def test_fake_impls_give_shapes():
    with FakeTensorMode():
        a = torch.empty(2, 64, 256, dtype=torch.float8_e4m3fn)
        b = torch.empty(2, 256, 96, dtype=torch.float8_e4m3fn)
        sa = torch.empty(2, 64, 2)
        sb = torch.empty(2, 2, 1)
        out = torch.ops.pcamd.block_scaled_bmm(a, sa, b, sb, None, 1, 128, 128, torch.bfloat16)
        assert out.shape == (2, 64, 96) and out.dtype == torch.bfloat16
        x = torch.empty(3, 200, 300, dtype=torch.bfloat16)
        q, s = torch.ops.pcamd.quant_block(x, 128, 128, torch.float8_e4m3fn, 1e-12)
        assert q.shape == x.shape and q.dtype == torch.float8_e4m3fn and s.shape == (3, 2, 3)
        q, s = torch.ops.pcamd.quant_tensor(x, torch.float8_e5m2, 1e-12)
        assert q.dtype == torch.float8_e5m2 and s.shape == (1,)
        out = torch.ops.pcamd.tensor_scaled_bmm(a, b, torch.empty(1), None, torch.float32)
        assert out.shape == (2, 64, 96) and out.dtype == torch.float32
