"""GPU parity of the FP8 training layer (practice_cuda_amd.modules).

The block recipe is checked GEMM by GEMM against the oracle: X 1x128, W
128x128, dY 1x128 and the 128x1 re-quantizations of dY and X are computed on
the CPU by oracle.quant_block, dequantized, and multiplied in float64;
forward, dgrad and wgrad must each be within max-abs-relative 1e-2 (the BMM
bar). dbias is dY summed over M. The per-tensor recipe is checked the same
way with oracle.quant_tensor in torchao's tensorwise form (scale arithmetic
in fp64, the reference layer's), and its quantization op byte for byte. The
layer also runs under torch.compile
(aot_eager) with the same results, and at the config-5 shape its outputs stay
within the fp8 quantization error of an fp32 GEMM of the unquantized values.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd.modules import Float8BlockBMMLinearConfig, Float8BMMLinear

pytestmark = pytest.mark.gpu


def _deq_block(x: torch.Tensor, bm: int, bn: int) -> np.ndarray:
    q, s = O.quant_block(x.cpu(), bm, bn)
    return O.dequant_block(q, s, bm, bn)


def _deq_tensor(x: torch.Tensor) -> np.ndarray:
    q, ds, _ = O.quant_tensor(x.cpu(), scale_dt=O.F64)
    return O.decode(q).astype(np.float64) * np.float64(ds)


def _run(layer, x, dy, dev):
    xg = x.to(dev).requires_grad_(True)
    y = layer(xg)
    y.backward(dy.to(dev))
    torch.cuda.synchronize()
    return y.detach(), xg.grad, layer.weight.grad, None if layer.bias is None else layer.bias.grad


def _layer(b, k, n, dev, config, bias=True, seed=0):
    torch.manual_seed(seed)
    layer = Float8BMMLinear(b, k, n, bias=bias, config=config, device=dev, dtype=torch.bfloat16)
    return layer


@pytest.mark.parametrize("shape", [(2, 256, 384, 512), (1, 384, 256, 128), (3, 128, 128, 256),
                                   (2, 200, 256, 384), (1, 130, 200, 256)])
def test_block_recipe_gemms_match_oracle(dev, shape):
    # M, K and N are each some GEMM's reduction; the last two shapes have ragged
    # M (wgrad's: the dual quantizer's transposed 128x1 output then takes the
    # two-quantizer path) and ragged K (partial last quant-K blocks)
    b, m, k, n = shape
    print(f"block recipe {shape}", flush=True)
    layer = _layer(b, k, n, dev, Float8BlockBMMLinearConfig())
    g = torch.Generator().manual_seed(1)
    x = torch.randn(b, m, k, generator=g).bfloat16()
    dy = (torch.randn(b, m, n, generator=g) * 1e-3).bfloat16()
    y, dx, dw, db = _run(layer, x, dy, dev)
    w = layer.weight.detach().cpu()
    bias = layer.bias.detach().cpu().double().numpy()
    y_ref = np.matmul(_deq_block(x, 1, 128), np.swapaxes(_deq_block(w, 128, 128), -1, -2)) + bias[:, None, :]
    dx_ref = np.matmul(_deq_block(dy, 1, 128), _deq_block(w, 128, 128))
    dw_ref = np.matmul(np.swapaxes(_deq_block(dy, 128, 1), -1, -2), _deq_block(x, 128, 1))
    assert O.max_abs_rel(y.float().cpu().numpy(), y_ref) <= 1e-2
    assert O.max_abs_rel(dx.float().cpu().numpy(), dx_ref) <= 1e-2
    assert O.max_abs_rel(dw.float().cpu().numpy(), dw_ref) <= 1e-2
    assert O.max_abs_rel(db.float().cpu().numpy(), dy.double().sum(1).numpy()) <= 1e-2
    assert y.dtype == dx.dtype == dw.dtype == torch.bfloat16


@pytest.mark.parametrize("shape", [(2, 256, 384, 512), (1, 130, 200, 256), (1, 512, 640, 960)])
def test_block_recipe_e5m2_grads_match_oracle(dev, shape):
    """grad_fp8_dtype = e5m2 (torchao's grad_output format, kept by the
    reference layer, fp8_training/fp8_bench/modules/bmm_linear.py:43-46):
    dgrad multiplies e5m2 dY (1x128) by e4m3 W (128x128) and wgrad e5m2 dY
    (128x1) by e4m3 X (128x1), each against the fp64 product of the oracle's
    quantizations in those formats; the forward stays e4m3 x e4m3."""
    b, m, k, n = shape
    print(f"block recipe e5m2 grads {shape}", flush=True)
    cfg = Float8BlockBMMLinearConfig(grad_fp8_dtype=torch.float8_e5m2)
    layer = _layer(b, k, n, dev, cfg)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(b, m, k, generator=g).bfloat16()
    dy = (torch.randn(b, m, n, generator=g) * 1e-3).bfloat16()
    y, dx, dw, _ = _run(layer, x, dy, dev)
    w = layer.weight.detach().cpu()

    def deq(t, bm, bn, fmt):
        q, sc = O.quant_block(t.cpu(), bm, bn, fmt=fmt)
        return O.dequant_block(q, sc, bm, bn, fmt=fmt)

    y_ref = np.matmul(deq(x, 1, 128, "e4m3"), np.swapaxes(deq(w, 128, 128, "e4m3"), -1, -2))
    y_ref = y_ref + layer.bias.detach().cpu().double().numpy()[:, None, :]
    dx_ref = np.matmul(deq(dy, 1, 128, "e5m2"), deq(w, 128, 128, "e4m3"))
    dw_ref = np.matmul(np.swapaxes(deq(dy, 128, 1, "e5m2"), -1, -2), deq(x, 128, 1, "e4m3"))
    assert O.max_abs_rel(y.float().cpu().numpy(), y_ref) <= 1e-2
    assert O.max_abs_rel(dx.float().cpu().numpy(), dx_ref) <= 1e-2
    assert O.max_abs_rel(dw.float().cpu().numpy(), dw_ref) <= 1e-2
    # and the e5m2 gradient is not the e4m3 one: the formats differ in the products
    dx4 = np.matmul(deq(dy, 1, 128, "e4m3"), deq(w, 128, 128, "e4m3"))
    assert not np.array_equal(dx_ref, dx4)


def test_tensor_recipe_e5m2_grads_match_oracle(dev):
    b, m, k, n = 2, 96, 160, 200
    cfg = Float8BlockBMMLinearConfig(granularity="tensor", grad_fp8_dtype=torch.float8_e5m2)
    layer = _layer(b, k, n, dev, cfg, bias=False)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(b, m, k, generator=g).bfloat16()
    dy = torch.randn(b, m, n, generator=g).bfloat16()
    y, dx, dw, _ = _run(layer, x, dy, dev)
    w = layer.weight.detach().cpu()

    def deq(t, fmt):
        q, ds, _ = O.quant_tensor(t.cpu(), fmt, scale_dt=O.F64)
        return O.decode(q, fmt).astype(np.float64) * np.float64(ds)

    assert O.max_abs_rel(dx.float().cpu().numpy(), np.matmul(deq(dy, "e5m2"), deq(w, "e4m3"))) <= 1e-2
    assert O.max_abs_rel(dw.float().cpu().numpy(),
                         np.matmul(np.swapaxes(deq(dy, "e5m2"), -1, -2), deq(x, "e4m3"))) <= 1e-2


@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_tensor_recipe_quantization_is_torchao_form(dev, fmt):
    # the layer's per-tensor op writes the bytes and scale of torchao's form
    # (the reference layer's), not the fp32 reciprocal-multiply form: the
    # planted amax is one where the two scales differ
    x = (torch.randn(2, 96, 160, generator=torch.Generator().manual_seed(8)) * 0.05).bfloat16()
    x[0, 3, 4] = 0.5234375
    q, ds = torch.ops.pcamd.quant_tensor(x.to(dev), fmt, 1e-12)
    torch.cuda.synchronize()
    name = "e4m3" if fmt == torch.float8_e4m3fn else "e5m2"
    q_ref, ds_ref, qs_ref = O.quant_tensor(x, name, scale_dt=O.F64)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.float32(ds.item()) == np.float32(ds_ref)
    assert np.float32(O.quant_tensor(x, name)[2]) != np.float32(qs_ref)


def test_tensor_recipe_gemms_match_oracle(dev):
    b, m, k, n = 2, 96, 160, 200
    layer = _layer(b, k, n, dev, Float8BlockBMMLinearConfig(granularity="tensor"), bias=False)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(b, m, k, generator=g).bfloat16()
    dy = torch.randn(b, m, n, generator=g).bfloat16()
    y, dx, dw, _ = _run(layer, x, dy, dev)
    w = layer.weight.detach().cpu()
    assert O.max_abs_rel(y.float().cpu().numpy(), np.matmul(_deq_tensor(x), np.swapaxes(_deq_tensor(w), -1, -2))) <= 1e-2
    assert O.max_abs_rel(dx.float().cpu().numpy(), np.matmul(_deq_tensor(dy), _deq_tensor(w))) <= 1e-2
    assert O.max_abs_rel(dw.float().cpu().numpy(),
                         np.matmul(np.swapaxes(_deq_tensor(dy), -1, -2), _deq_tensor(x))) <= 1e-2


def test_only_requested_grads(dev):
    layer = _layer(1, 256, 128, dev, Float8BlockBMMLinearConfig(), bias=False)
    layer.weight.requires_grad_(False)
    x = torch.randn(1, 128, 256, device=dev, dtype=torch.bfloat16, requires_grad=True)
    layer(x).sum().backward()
    assert x.grad is not None and layer.weight.grad is None


def test_compiled_matches_eager(dev):
    layer = _layer(1, 256, 256, dev, Float8BlockBMMLinearConfig())
    x = torch.randn(1, 256, 256, device=dev, dtype=torch.bfloat16)
    dy = torch.randn(1, 256, 256, device=dev, dtype=torch.bfloat16) * 1e-3
    y0, dx0, dw0, db0 = _run(layer, x, dy, dev)
    layer.weight.grad = None
    layer.bias.grad = None
    compiled = torch.compile(layer, backend="aot_eager", fullgraph=True)
    y1, dx1, dw1, db1 = _run(compiled, x, dy, dev)
    assert torch.equal(y0, y1) and torch.equal(dx0, dx1) and torch.equal(dw0, dw1) and torch.equal(db0, db1)


def test_config5_shape_within_fp8_error(dev):
    """M=8192, K=4096, N=14336: forward, dgrad and wgrad vs fp32 GEMMs of the
    unquantized bf16 values (relative Frobenius error of a few % is the fp8
    e4m3 quantization error; a wrong scale or layout gives O(1))."""
    print("config-5 shape layer", flush=True)
    m, k, n = 8192, 4096, 14336
    torch.manual_seed(0)
    layer = Float8BMMLinear(1, k, n, bias=False, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        layer.weight.normal_(0.0, 0.02)
    x = torch.randn(1, m, k, device=dev, dtype=torch.bfloat16)
    dy = torch.randn(1, m, n, device=dev, dtype=torch.bfloat16) * 1e-3
    y, dx, dw, _ = _run(layer, x, dy, dev)
    w = layer.weight.detach().float()

    def rel(a, b):
        return ((a.float() - b).norm() / b.norm()).item()

    assert rel(y, torch.matmul(x.float(), w.transpose(-1, -2).contiguous())) < 0.05
    assert rel(dx, torch.matmul(dy.float(), w)) < 0.05
    assert rel(dw, torch.matmul(dy.float().transpose(-1, -2).contiguous(), x.float())) < 0.05
