"""GPU parity of the HIP scaled FP8 BMM against the CPU oracle.

The oracle is the fp64 product of the dequantized operands (the reference's
kernel_reference, bench_bmm.py:414-419) followed by bias and activation;
the bar is max|out - ref| / max|ref| <= 1e-2 (north_star). Cases: every
scaling scheme x the five registered layouts, unaligned shapes from the
reference tests, bias / GELU / output dtypes, the BASELINE config-4 shape,
multi-block quant-K, and the invariants of kernels/fp8_bmm/test/
fp8_quant_bmm_test.py (zeros, linearity, batch independence, determinism).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd import get_bmm, get_quant
from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm, hip_per_block_quant
from practice_cuda_amd.impls.hip_per_tensor import hip_per_tensor_bmm
from practice_cuda_amd.registry import QuantResult

pytestmark = pytest.mark.gpu
TOL = 1e-2
LAYOUTS = ("a_k_b_k", "a_k_b_n", "a_k_b_n_transpose", "a_m_b_n", "a_m_transpose_b_n_transpose")
SCHEMES = ("hip_per_block_1d", "hip_per_block_2d", "hip_per_channel", "hip_per_tensor")


def materialize(t: torch.Tensor, layout: str) -> torch.Tensor:
    """Same logical tensor, the other dim contiguous (bench_bmm.py:280-288)."""
    if layout in ("m", "k_of_b"):
        return t.transpose(-1, -2).contiguous().transpose(-1, -2)
    return t


def run_registered(name, a, b, dev, bias=None, activation="none", out_dtype=torch.bfloat16):
    impl = get_bmm(name)
    quant = get_quant(impl.quant_impl)
    a_in = materialize(a, "m") if impl.a_layout == "m" else a
    b_in = materialize(b, "k_of_b") if impl.layout == "k" else b
    qa = impl.prepare_a(quant.fn(a_in.to(dev), **impl.quant_a_kwargs))
    qb = impl.prepare_b(quant.fn(b_in.to(dev), **impl.quant_b_kwargs))
    kw = impl.prepare_call_kwargs(qa, qb)
    out = impl.fn(qa, qb, bias=None if bias is None else bias.to(dev), activation=activation,
                  out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(),
                          qb.dequantize().double().cpu().numpy(),
                          None if bias is None else bias.double().numpy(), activation)
    return out, ref


def rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).bfloat16()


SHAPES = [(2, 128, 128, 128), (3, 33, 47, 65), (3, 129, 131, 127), (2, 256, 384, 512), (1, 64, 96, 1024),
          (2, 272, 528, 384)]


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("shape", SHAPES)
def test_bmm_matches_oracle(dev, scheme, layout, shape):
    b_, m, n, k = shape
    print(f"bmm {scheme}_{layout} {shape}", flush=True)
    out, ref = run_registered(f"{scheme}_{layout}", rand((b_, m, k), 1), rand((b_, k, n), 2), dev)
    assert out.shape == (b_, m, n) and out.dtype == torch.bfloat16
    err = O.max_abs_rel(out.float().cpu().numpy(), ref)
    assert err <= TOL, f"max_abs_rel {err}"


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("activation", ["none", "gelu"])
def test_bmm_bias_activation_dtypes(dev, out_dtype, activation):
    bias = rand((2, 96, 80), 3)
    out, ref = run_registered("hip_per_block_2d_a_k_b_n", rand((2, 96, 256), 4), rand((2, 256, 80), 5),
                              dev, bias=bias, activation=activation, out_dtype=out_dtype)
    assert out.dtype == out_dtype
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_bmm_staged_gelu_matches_direct_epilogue(dev, scheme, out_dtype):
    """A 16-bit bias with 8-byte aligned rows and GELU go through the staged
    (LDS) epilogue; the same bias one element off alignment goes through the
    per-element one. Same accumulators, same order of operations: with block
    scales (applied in the K loop) the outputs are identical; with channel /
    tensor scales the inlined path may contract scale and bias into one fma,
    so they agree to one 16-bit unit. Partial tiles (M = 300, N = 136)."""
    print(f"bmm staged gelu {scheme} {out_dtype}", flush=True)
    impl = get_bmm(f"{scheme}_a_k_b_n")
    quant = get_quant(impl.quant_impl)
    qa = impl.prepare_a(quant.fn(rand((2, 300, 384), 12).to(dev), **impl.quant_a_kwargs))
    qb = impl.prepare_b(quant.fn(rand((2, 384, 136), 13).to(dev), **impl.quant_b_kwargs))
    kw = impl.prepare_call_kwargs(qa, qb)
    bias = rand((2, 300, 136), 14).to(dev)
    shifted = torch.empty(bias.numel() + 1, device=dev, dtype=bias.dtype)[1:].view_as(bias)
    shifted.copy_(bias)
    staged = impl.fn(qa, qb, bias=bias, activation="gelu", out_dtype=out_dtype, **kw)
    direct = impl.fn(qa, qb, bias=shifted, activation="gelu", out_dtype=out_dtype, **kw)
    no_bias = impl.fn(qa, qb, activation="gelu", out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    if "per_block" in scheme:
        assert torch.equal(staged, direct)
    else:
        assert (staged.float() - direct.float()).abs().max().item() <= 8e-3 * direct.float().abs().max().item()
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy(),
                          bias.double().cpu().numpy(), "gelu")
    assert O.max_abs_rel(staged.float().cpu().numpy(), ref) <= TOL
    ref0 = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy(),
                           None, "gelu")
    assert O.max_abs_rel(no_bias.float().cpu().numpy(), ref0) <= TOL


def test_bmm_fp8_output_saturates(dev):
    # reference fp8_quant_bmm_test.py:227-237: fp8 output saturates at +-448
    a = (rand((1, 64, 128), 6).float() * 4).bfloat16()
    qa = hip_per_block_quant(a.to(dev), block_m=1, block_n=128)
    qb = hip_per_block_quant(rand((1, 128, 64), 7).to(dev), block_m=128, block_n=128)
    out = hip_per_block_bmm(qa, qb, out_dtype=torch.float8_e4m3fn)
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    v = out.float().cpu().numpy()
    assert np.isfinite(v).all() and np.abs(v).max() <= 448.0
    close = np.abs(ref) < 400
    assert np.allclose(v[close], ref[close], rtol=0.2, atol=0.1)


def test_bmm_multi_block_quant_k(dev):
    # quant_block_k = 256: two 128-wide MFMA steps accumulate before each rescale
    a, b = rand((2, 100, 512), 8), rand((2, 512, 200), 9)
    qa = hip_per_block_quant(a.to(dev), block_m=1, block_n=256)
    qb = hip_per_block_quant(b.to(dev), block_m=256, block_n=128)
    out = hip_per_block_bmm(qa, qb)
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("qbn", [1, 8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("b_layout", ["n", "k"])
def test_bmm_b_block_widths(dev, qbn, b_layout):
    # B quant blocks of every width class of the 256x256-tile kernel: one scale
    # per column (< 16), per 16-column sub-tile (16..64), per wave (>= 128);
    # K = 640 gives five K steps, shapes span several output tiles
    print(f"bmm b-block width {qbn} layout {b_layout}", flush=True)
    a, b = rand((2, 300, 640), 10), rand((2, 640, 520), 11)
    qa = hip_per_block_quant(a.to(dev), block_m=1, block_n=128)
    b_in = materialize(b, "k_of_b") if b_layout == "k" else b
    qb = hip_per_block_quant(b_in.to(dev), block_m=128, block_n=qbn)
    out = hip_per_block_bmm(qa, qb)
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("shape", [(3, 1280, 384, 4608), (1, 2816, 256, 6144)])
@pytest.mark.parametrize("scheme,layout,qbn", [
    ("hip_per_block_1d", "a_k_b_k", None),   # per-column B scales
    ("hip_per_block_2d", "a_k_b_n", None),   # one B scale per 128 columns
    ("hip_per_block_1d", "a_m_b_n", None),   # both operands MN-major
    ("direct", "a_k_b_n", 16),               # one B scale per 16 columns
    ("hip_per_tensor", "a_k_b_k", None),
    ("hip_per_channel", "a_k_b_k", None),
])
def test_bmm_more_tiles_than_cus(dev, shape, scheme, layout, qbn):
    # 3 x 5 x 18 = 270 and 11 x 24 = 264 output tiles of 256 x 256: more than
    # MI355X's 256 CUs, so the last 14 / 8 tiles run as half tiles (28 / 16
    # workgroups: both ways of pairing halves). The first shape also has three
    # batches and an odd number (3) of 128-deep K steps.
    b_, m, k, n = shape
    print(f"bmm more tiles than CUs {shape} {scheme} {layout} qbn={qbn}", flush=True)
    a, b = rand((b_, m, k), 12), rand((b_, k, n), 13)
    if scheme == "direct":
        qa = hip_per_block_quant(a.to(dev), block_m=1, block_n=128)
        qb = hip_per_block_quant(b.to(dev), block_m=128, block_n=qbn)
        out = hip_per_block_bmm(qa, qb)
        torch.cuda.synchronize()
        ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    else:
        out, ref = run_registered(f"{scheme}_{layout}", a, b, dev)
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("shape", [(2, 200, 128, 300), (2, 260, 640, 520), (3, 1280, 384, 4608)])
@pytest.mark.parametrize("b_layout", ["n", "k"])
def test_bmm_e5m2(dev, shape, b_layout):
    # e5m2 x e5m2 (the reference requires one fp8 dtype for both operands):
    # the single-step kernel (K = 128), the 256 x 256 kernel, and a grid whose
    # last tiles run as half tiles
    b_, m, k, n = shape
    print(f"bmm e5m2 {shape} b_layout {b_layout}", flush=True)
    a, b = rand((b_, m, k), 14), rand((b_, k, n), 15)
    qa = hip_per_block_quant(a.to(dev), block_m=1, block_n=128, fp8_dtype=torch.float8_e5m2)
    b_in = materialize(b, "k_of_b") if b_layout == "k" else b
    qb = hip_per_block_quant(b_in.to(dev), block_m=128, block_n=128, fp8_dtype=torch.float8_e5m2)
    assert qa.tensor.dtype == torch.float8_e5m2 and qb.tensor.dtype == torch.float8_e5m2
    out = hip_per_block_bmm(qa, qb)
    torch.cuda.synchronize()
    ref = O.bmm_reference(qa.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy())
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= TOL


def test_bmm_golden(dev):
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "bmm_golden.npz"))
    qa = QuantResult(torch.from_numpy(d["qa"]).view(torch.float8_e4m3fn).to(dev),
                     torch.from_numpy(d["sa"]).to(dev), "golden", "block", {"block_m": 1, "block_n": 128})
    qb = QuantResult(torch.from_numpy(d["qb"]).view(torch.float8_e4m3fn).to(dev),
                     torch.from_numpy(d["sb"]).to(dev), "golden", "block", {"block_m": 128, "block_n": 128})
    bias = torch.from_numpy(d["bias"].view(np.int16)).view(torch.bfloat16).to(dev)
    out = hip_per_block_bmm(qa, qb, bias=bias, out_dtype=torch.float32)
    assert O.max_abs_rel(out.cpu().numpy(), d["expected"]) <= TOL


def test_config4_shape(dev):
    """A [128,2048,128] 1x128, B [128,128,512] 128x128, bf16 out."""
    g = torch.Generator().manual_seed(0)
    ah = torch.randn(128, 2048, 128, generator=g).bfloat16()
    bh = torch.randn(128, 128, 512, generator=g).bfloat16()
    qa = hip_per_block_quant(ah.to(dev), block_m=1, block_n=128)
    qb = hip_per_block_quant(bh.to(dev), block_m=128, block_n=128)
    out = hip_per_block_bmm(qa, qb)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    da, db = qa.dequantize().double().cpu(), qb.dequantize().double().cpu()
    for bi in (0, 37, 127):
        ref = O.bmm_reference(da[bi:bi + 1].numpy(), db[bi:bi + 1].numpy())
        assert O.max_abs_rel(out[bi:bi + 1].float().cpu().numpy(), ref) <= TOL


def test_fixed_tile_microbench_points(dev):
    """fp8_training/microbench/profile_fixed_b_n.py:235-283: one 64x64x128 fp8
    tile times 0.5, bf16 output, assert_close(2e-2) for a_k_b_k / a_k_b_n / a_m_b_n."""
    torch.manual_seed(0)
    a = (torch.randn(64, 128) * 0.25).to(torch.float8_e4m3fn)
    b = (torch.randn(128, 64) * 0.25).to(torch.float8_e4m3fn)
    ref = ((a.float() @ b.float()) * 0.5).bfloat16().float()
    scale = torch.tensor(0.5, device=dev)
    for a_m, b_k in ((False, True), (False, False), (True, False)):
        at = a.to(dev)[None]
        bt = b.to(dev)[None]
        if a_m:
            at = at.transpose(-1, -2).contiguous().transpose(-1, -2)
        if b_k:
            bt = bt.transpose(-1, -2).contiguous().transpose(-1, -2)
        qa = QuantResult(at, scale, "t", "tensor")
        qb = QuantResult(bt, torch.tensor(1.0, device=dev), "t", "tensor")
        out = hip_per_tensor_bmm(qa, qb, dequant_scale=scale)
        torch.testing.assert_close(out[0].float().cpu(), ref, rtol=2e-2, atol=2e-2)


def _fp8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * 0.5).to(torch.float8_e4m3fn)


def _tensor_bmm(a, b, s, dev, out_dtype=torch.float32):
    qa = QuantResult(a.to(dev), torch.tensor(1.0, device=dev), "t", "tensor")
    qb = QuantResult(b.to(dev), torch.tensor(1.0, device=dev), "t", "tensor")
    return hip_per_tensor_bmm(qa, qb, dequant_scale=torch.tensor(s, device=dev), out_dtype=out_dtype)


def test_zeros(dev):
    a = torch.zeros(2, 32, 64).to(torch.float8_e4m3fn)
    b = torch.zeros(2, 64, 32).to(torch.float8_e4m3fn)
    out = _tensor_bmm(a, b, 1.0, dev)
    assert not torch.isnan(out).any() and out.abs().max().item() == 0.0


def test_scale_linearity(dev):
    a, b = _fp8((1, 64, 64), 1), _fp8((1, 64, 64), 2)
    o1 = _tensor_bmm(a, b, 1.0, dev)
    o2 = _tensor_bmm(a, b, 2.0, dev)
    assert torch.equal(o2, o1 * 2)  # power-of-two scaling is exact in fp32


def test_batch_independence(dev):
    a, b = _fp8((2, 32, 32), 3), _fp8((2, 32, 32), 4)
    out = _tensor_bmm(a, b, 1.0, dev)
    for i in range(2):
        single = _tensor_bmm(a[i:i + 1], b[i:i + 1], 1.0, dev)
        assert torch.allclose(out[i], single[0], rtol=1e-3, atol=1e-3)


def test_exact_small_integers(dev):
    # fp8 inputs with small integer values: every product and partial sum is
    # exact in fp32, so the fp32 output must equal the integer matmul exactly
    g = torch.Generator().manual_seed(5)
    a = torch.randint(-4, 5, (2, 48, 256), generator=g).float()
    b = torch.randint(-4, 5, (2, 256, 40), generator=g).float()
    out = _tensor_bmm(a.to(torch.float8_e4m3fn), b.to(torch.float8_e4m3fn), 1.0, dev)
    assert torch.equal(out.cpu(), torch.bmm(a, b))


def test_determinism(dev):
    a, b = _fp8((2, 64, 64), 5), _fp8((2, 64, 64), 6)
    assert torch.equal(_tensor_bmm(a, b, 1.0, dev, torch.bfloat16), _tensor_bmm(a, b, 1.0, dev, torch.bfloat16))


@pytest.mark.parametrize("layout", ["a_k_b_k", "a_k_b_n"])
def test_channel_bmm_config5_shape(dev, layout):
    """Channel-scaled BMM (one scale per row of A, one per column of B) at the
    config-5 forward shape M=8192, K=4096, N=14336, against an fp32 GEMM of
    the dequantized operands computed on the GPU (contiguous operands)."""
    from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_quant
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 8192, 4096, generator=g).bfloat16().to(dev)
    w = (torch.randn(1, 14336, 4096, generator=g) * 0.02).bfloat16().to(dev)
    bmm = get_bmm(f"hip_per_channel_{layout}")
    qa = hip_per_channel_quant(x, channel_axis=-2)                      # one scale per row of A
    if layout == "a_k_b_k":                                              # B = W^T, K-major
        qw = hip_per_channel_quant(w, channel_axis=-2)                  # one scale per row of W
        qb = QuantResult(qw.tensor.transpose(-1, -2), qw.dequant_scale, qw.impl, "channel",
                         {**qw.meta, "channel_axis": -1})
    else:                                                                # B = W^T materialized N-major
        qb = hip_per_channel_quant(w.transpose(-1, -2).contiguous(), channel_axis=-1)
    print(f"channel bmm config5 {layout}", flush=True)
    out = bmm.fn(qa, qb)
    da = qa.tensor.float() * qa.dequant_scale[..., :, None]
    db = qb.tensor.float() * qb.dequant_scale[..., None, :]
    ref = torch.matmul(da.contiguous(), db.contiguous())
    err = ((out.float() - ref).abs().max() / ref.abs().max()).item()
    assert err <= TOL, err
