"""CPU tests of the drop-in Python boundary: registry API, QuantResult layout
contract and the wrappers' validation errors (all raised before any launch).

Mirrors the contract of fp8_training/fp8_bench/registry.py and
impls/triton_per_{block,channel,tensor}.py of xuOAO/practice_cuda.
"""
from __future__ import annotations

import pytest
import torch

import practice_cuda_amd as P
from practice_cuda_amd import registry as R
from practice_cuda_amd.impls import _common as C
from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm, hip_per_block_quant
from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_bmm, hip_per_channel_quant
from practice_cuda_amd.impls.hip_per_tensor import hip_per_tensor_bmm

FP8 = torch.float8_e4m3fn


def test_builtin_names():
    R.load_builtin_impls()
    for name in ("hip_per_block_1d", "hip_per_block_2d", "hip_per_channel",
                 "hip_per_channel_one_pass", "hip_per_tensor", "torch_compile_per_channel"):
        assert name in R.QUANT_IMPLS
    layouts = ("a_k_b_k", "a_k_b_n", "a_k_b_n_transpose", "a_m_b_n", "a_m_transpose_b_n_transpose")
    names = R.bmm_impl_names()
    assert names[:5] == [f"hip_per_block_1d_{l}" for l in layouts]
    for scheme in ("hip_per_block_1d", "hip_per_block_2d", "hip_per_channel", "hip_per_tensor"):
        for l in layouts:
            assert f"{scheme}_{l}" in names


def test_registered_quant_kwargs():
    # the 1d scheme quantizes A as 1x128 and B as 128x1 (reference :455-462)
    b1 = R.get_bmm("hip_per_block_1d_a_k_b_n")
    assert b1.quant_a_kwargs == {"block_m": 1, "block_n": 128}
    assert b1.quant_b_kwargs == {"block_m": 128, "block_n": 1}
    b2 = R.get_bmm("hip_per_block_2d_a_m_b_n")
    assert (b2.a_layout, b2.layout) == ("m", "n")
    assert b2.quant_b_kwargs == {"block_m": 128, "block_n": 128}
    ch = R.get_bmm("hip_per_channel_a_k_b_k")
    assert ch.quant_a_kwargs == {"channel_axis": -2} and ch.quant_b_kwargs == {"channel_axis": -1}
    assert R.get_quant("hip_per_block_1d").fn.keywords == {"block_m": 1, "block_n": 128}


def test_duplicate_and_unknown_names():
    with pytest.raises(ValueError, match="duplicate quant implementation"):
        R.register_quant("hip_per_channel", lambda x: x)
    with pytest.raises(ValueError, match="duplicate BMM implementation"):
        R.register_bmm("hip_per_channel_a_k_b_n", lambda a, b: a, quant_impl="x", layout="n",
                       prepare_b=lambda v: v)
    with pytest.raises(ValueError, match="a_layout must be"):
        R.register_bmm("new_bmm_x", lambda a, b: a, quant_impl="x", layout="n",
                       prepare_b=lambda v: v, a_layout="q")
    with pytest.raises(ValueError, match="layout must be"):
        R.register_bmm("new_bmm_y", lambda a, b: a, quant_impl="x", layout="m",
                       prepare_b=lambda v: v)
    with pytest.raises(KeyError, match="choices="):
        R.get_quant("nope")
    with pytest.raises(KeyError, match="choices="):
        R.get_bmm("nope")


def test_public_aliases():
    assert P.per_block_quant is hip_per_block_quant
    assert P.per_channel_bmm is hip_per_channel_bmm


def test_dequantize_contract():
    q = torch.tensor([[1.0, 2.0, 3.0, 4.0], [5.0, 6.0, 7.0, 8.0]]).to(FP8)
    s = torch.tensor([[2.0, 3.0]])
    r = R.QuantResult(q, s, "t", "block", {"block_m": 2, "block_n": 2})
    assert torch.equal(r.dequantize(), torch.tensor([[2.0, 4.0, 9.0, 12.0], [10.0, 12.0, 21.0, 24.0]]))
    r = R.QuantResult(q, torch.tensor([1.0, 10.0]), "t", "channel", {"channel_axis": -2})
    assert torch.equal(r.dequantize()[1], torch.tensor([50.0, 60.0, 70.0, 80.0]))
    r = R.QuantResult(q, torch.tensor([1.0, 2.0, 3.0, 4.0]), "t", "channel", {"channel_axis": -1})
    assert torch.equal(r.dequantize()[0], torch.tensor([1.0, 4.0, 9.0, 16.0]))
    r = R.QuantResult(q, torch.tensor(0.5), "t", "tensor")
    assert torch.equal(r.dequantize()[0], torch.tensor([0.5, 1.0, 1.5, 2.0]))
    with pytest.raises(ValueError, match="must have shape"):
        R.QuantResult(q, torch.ones(2, 2), "t", "block", {"block_m": 2, "block_n": 2}).dequantize()
    with pytest.raises(ValueError, match="one fewer dimension"):
        R.QuantResult(q, torch.ones(2, 1), "t", "channel", {"channel_axis": -2}).dequantize()
    with pytest.raises(ValueError, match="unknown quantization granularity"):
        R.QuantResult(q, torch.ones(1), "t", "row").dequantize()


def test_layout_helpers():
    x = torch.zeros(2, 8, 16)
    assert C.matrix_layout(x, "B") == "n-major" and C.a_layout(x) == "k-major"
    xt = x.transpose(-1, -2).contiguous().transpose(-1, -2)
    assert C.matrix_layout(xt, "B") == "k-major" and C.a_layout(xt) == "m-major"
    with pytest.raises(ValueError, match="contiguous along"):
        C.a_layout(torch.zeros(4, 8, 16)[:, ::2, ::2])


def test_quant_validation_errors():
    x = torch.zeros(4, 256)
    with pytest.raises(ValueError, match="2D or 3D"):
        hip_per_block_quant(torch.zeros(256))
    with pytest.raises(ValueError, match="power-of-two block sizes"):
        hip_per_block_quant(x, block_m=3, block_n=128)
    with pytest.raises(ValueError, match="channel_axis must be -1 or -2"):
        hip_per_channel_quant(x, channel_axis=0)
    with pytest.raises(ValueError, match="up to 4096"):
        hip_per_channel_quant(torch.zeros(4, 5000), channel_axis=-2, one_pass=True)
    with pytest.raises(ValueError, match="non-empty reduction"):
        hip_per_channel_quant(torch.zeros(4, 0), channel_axis=-2, one_pass=True)
    with pytest.raises(ValueError, match="input dtype"):
        hip_per_block_quant(torch.zeros(4, 256, dtype=torch.float64))
    with pytest.raises(ValueError, match="GPU tensor"):
        hip_per_block_quant(x)


def _qr(shape, gran, meta, scale_shape, strides_from=None):
    t = torch.zeros(shape).to(FP8)
    if strides_from == "t":
        t = t.transpose(-1, -2).contiguous().transpose(-1, -2)
    return R.QuantResult(t, torch.ones(scale_shape), "t", gran, meta)


def test_bmm_validation_errors():
    blk = lambda bm, bn: {"block_m": bm, "block_n": bn}
    a = _qr((2, 64, 256), "block", blk(1, 128), (2, 64, 2))
    b = _qr((2, 256, 96), "block", blk(128, 128), (2, 2, 1))
    with pytest.raises(ValueError, match="3D quantized tensors"):
        hip_per_block_bmm(_qr((64, 256), "block", blk(1, 128), (64, 2)), b)
    with pytest.raises(ValueError, match="activation must be"):
        hip_per_block_bmm(a, b, activation="relu")
    with pytest.raises(ValueError, match="shape mismatch"):
        hip_per_block_bmm(a, _qr((2, 128, 96), "block", blk(128, 128), (2, 1, 1)))
    with pytest.raises(ValueError, match="same K quant block"):
        hip_per_block_bmm(a, _qr((2, 256, 96), "block", blk(256, 128), (2, 1, 1)))
    with pytest.raises(ValueError, match="quant_block_k >= 128"):
        hip_per_block_bmm(_qr((2, 64, 256), "block", blk(1, 64), (2, 64, 4)),
                          _qr((2, 256, 96), "block", blk(64, 128), (2, 4, 1)))
    with pytest.raises(ValueError, match="A dequant scale must have shape"):
        hip_per_block_bmm(_qr((2, 64, 256), "block", blk(1, 128), (2, 64, 3)), b)
    with pytest.raises(ValueError, match="do_transpose_a=True requires an M-major"):
        hip_per_block_bmm(a, b, do_transpose_a=True)
    with pytest.raises(ValueError, match="out must have shape"):
        hip_per_block_bmm(a, b, out=torch.empty(2, 64, 95, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="out must have dtype"):
        hip_per_block_bmm(a, b, out=torch.empty(2, 64, 96, dtype=torch.float16))
    with pytest.raises(ValueError, match="bias must have shape"):
        hip_per_block_bmm(a, b, bias=torch.zeros(2, 64, 95))
    with pytest.raises(ValueError, match="GPU tensor"):
        hip_per_block_bmm(a, b)
    # the registry wrappers keep the reference's one-format rule
    # (impls/triton_per_block.py:288-290); mixed formats are the training
    # layer's (pcamd::block_scaled_bmm over pcamd_bmm_scaled_mixed)
    b5 = R.QuantResult(b.tensor.to(torch.float8_e5m2), b.dequant_scale, "t", "block", blk(128, 128))
    with pytest.raises(ValueError, match="same FP8 dtype"):
        hip_per_block_bmm(a, b5)
    ca = _qr((2, 64, 256), "channel", {"channel_axis": -2}, (2, 64))
    cb = _qr((2, 256, 96), "channel", {"channel_axis": -2}, (2, 96))
    with pytest.raises(ValueError, match="channel_axis=-1"):
        hip_per_channel_bmm(ca, cb)
    ta = _qr((2, 64, 256), "tensor", {}, ())
    tb = _qr((2, 256, 96), "tensor", {}, ())
    with pytest.raises(ValueError, match="one combined dequant scale"):
        hip_per_tensor_bmm(ta, tb, dequant_scale=torch.ones(2))


def test_torch_compile_role_checks_before_launch():
    # impls/triton_per_channel.py:63-68: rank, then channel_axis, both ValueError
    fn = R.get_quant("torch_compile_per_channel").fn
    with pytest.raises(ValueError, match="2D or 3D"):
        fn(torch.zeros(4, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="channel_axis must be -1 or -2"):
        fn(torch.zeros(4, 4, dtype=torch.bfloat16), channel_axis=0)
