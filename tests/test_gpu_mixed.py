"""GPU parity of the scaled FP8 BMM with one e5m2 and one e4m3fn operand
(pcamd_bmm_scaled_mixed).

The reference training layer multiplies torchao's e5m2 grad_output by e4m3fn
weights and inputs in dgrad and wgrad (fp8_training/fp8_bench/modules/
bmm_linear.py:43-46, :402-410, :441-446, through fp8_bench::bmm_linear_tma,
:121-227, which has no same-dtype rule). Each operand's format goes to the
MFMA as its own code. Checked here, within max|out - ref| / max|ref| <= 1e-2
of the fp64 product of the dequantized operands, for both pairs, block /
channel / tensor scales, K-major and MN-major operands, and shapes that take
the wide kernel (aligned and ragged K), the general kernel (unaligned) and
K = 128 (which the same-format path gives the single-step kernel; mixed
formats take the general one). The mixed result must also differ from the
same call with B's bytes read as A's format, so a dropped format code fails.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd import _lib
from practice_cuda_amd import modules  # noqa: F401  (registers pcamd::block_scaled_bmm)
from practice_cuda_amd.impls import _common as C
from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant
from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_quant
from practice_cuda_amd.impls.hip_per_tensor import quant_tensor_raw

pytestmark = pytest.mark.gpu
TOL = 1e-2
E4, E5 = torch.float8_e4m3fn, torch.float8_e5m2
FMT = {E4: "e4m3", E5: "e5m2"}


def _rand(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).bfloat16()


def _mn(t):
    return t.transpose(-1, -2).contiguous().transpose(-1, -2)


def _gemm(scheme, a, b, fa, fb, dev):
    """Quantize A in fa and B in fb with the scheme, multiply, and return
    (out, dequantized A, dequantized B) as float64 numpy."""
    bsz, m, k = a.shape
    n = b.shape[2]
    out = torch.empty(bsz, m, n, dtype=torch.float32, device=dev)
    if scheme == "block":
        qa = hip_per_block_quant(a, block_m=1, block_n=128, fp8_dtype=fa)
        qb = hip_per_block_quant(b, block_m=128, block_n=128, fp8_dtype=fb)
        out = torch.ops.pcamd.block_scaled_bmm(qa.tensor, qa.dequant_scale, qb.tensor, qb.dequant_scale, None,
                                               1, 128, 128, torch.float32)
        da = O.dequant_block(qa.tensor.view(torch.uint8).cpu().numpy(), qa.dequant_scale.cpu().numpy(), 1, 128,
                             FMT[fa])
        db = O.dequant_block(qb.tensor.view(torch.uint8).cpu().numpy(), qb.dequant_scale.cpu().numpy(), 128, 128,
                             FMT[fb])
    elif scheme == "channel":
        qa = hip_per_channel_quant(a, channel_axis=-2, fp8_dtype=fa)
        qb = hip_per_channel_quant(b, channel_axis=-1, fp8_dtype=fb)
        sa, sb = qa.dequant_scale, qb.dequant_scale
        C.launch_bmm(qa.tensor, qb.tensor, out, None, (0, 0, 0), 0, sa, (sa.stride(0), sa.stride(1), 0), sb,
                     (sb.stride(0), sb.stride(1), 0), _lib.SCALE_CHANNEL, False, 1, 128, 1, "none", bsz, m, n, k)
        da = O.decode(qa.tensor.view(torch.uint8).cpu().numpy(), FMT[fa]) * sa.cpu().double().numpy()[:, :, None]
        db = O.decode(qb.tensor.view(torch.uint8).cpu().numpy(), FMT[fb]) * sb.cpu().double().numpy()[:, None, :]
    else:
        qa, sa, _ = quant_tensor_raw(a, fa, 1e-12)
        qb, sb, _ = quant_tensor_raw(b, fb, 1e-12)
        s = (sa * sb).reshape(1).float()
        C.launch_bmm(qa, qb, out, None, (0, 0, 0), 0, s, (0, 0, 0), None, (0, 0, 0), _lib.SCALE_TENSOR, False,
                     1, 128, 1, "none", bsz, m, n, k)
        da = O.decode(qa.view(torch.uint8).cpu().numpy(), FMT[fa]) * float(sa.item())
        db = O.decode(qb.view(torch.uint8).cpu().numpy(), FMT[fb]) * float(sb.item())
    torch.cuda.synchronize()
    return out, np.asarray(da, np.float64), np.asarray(db, np.float64)


SHAPES = [(2, 256, 384, 512),   # wide kernel
          (2, 256, 384, 960),   # wide kernel, masked last K step
          (3, 129, 131, 127),   # general kernel (unaligned)
          (2, 256, 512, 128)]   # one K step: the general kernel for mixed formats


@pytest.mark.parametrize("pair", [(E5, E4), (E4, E5)], ids=["a_e5m2_b_e4m3", "a_e4m3_b_e5m2"])
@pytest.mark.parametrize("layout", ["a_k_b_n", "a_k_b_k", "a_m_b_n"])
@pytest.mark.parametrize("scheme", ["block", "channel", "tensor"])
@pytest.mark.parametrize("shape", SHAPES)
def test_mixed_formats_match_oracle(dev, shape, scheme, layout, pair):
    fa, fb = pair
    bsz, m, n, k = shape
    print(f"mixed {FMT[fa]} x {FMT[fb]} {scheme} {layout} {shape}", flush=True)
    a, b = _rand((bsz, m, k), 51).to(dev), _rand((bsz, k, n), 52).to(dev)
    if layout == "a_m_b_n":
        a = _mn(a)
    if layout == "a_k_b_k":
        b = _mn(b)
    out, da, db = _gemm(scheme, a, b, fa, fb, dev)
    ref = np.matmul(da, db)
    err = O.max_abs_rel(out.cpu().numpy(), ref)
    assert err <= TOL, f"max_abs_rel {err}"


def test_format_codes_are_per_operand(dev):
    """The same bytes read with B as e4m3 instead of e5m2 give another
    product: the kernel honours B's own format code."""
    a = _rand((1, 256, 512), 61).to(dev)
    b = _rand((1, 512, 256), 62).to(dev)
    qa = hip_per_block_quant(a, block_m=1, block_n=128, fp8_dtype=E5)
    qb = hip_per_block_quant(b, block_m=128, block_n=128, fp8_dtype=E4)
    mixed = torch.ops.pcamd.block_scaled_bmm(qa.tensor, qa.dequant_scale, qb.tensor, qb.dequant_scale, None,
                                             1, 128, 128, torch.float32)
    same = torch.ops.pcamd.block_scaled_bmm(qa.tensor, qa.dequant_scale, qb.tensor.view(torch.uint8).view(E5),
                                            qb.dequant_scale, None, 1, 128, 128, torch.float32)
    torch.cuda.synchronize()
    da = O.dequant_block(qa.tensor.view(torch.uint8).cpu().numpy(), qa.dequant_scale.cpu().numpy(), 1, 128, "e5m2")
    db = O.dequant_block(qb.tensor.view(torch.uint8).cpu().numpy(), qb.dequant_scale.cpu().numpy(), 128, 128, "e4m3")
    assert O.max_abs_rel(mixed.cpu().numpy(), np.matmul(da, db)) <= TOL
    # (e4m3 bytes read as e5m2 include inf / NaN codes: the error is large or NaN)
    assert not O.max_abs_rel(same.cpu().numpy(), np.matmul(da, db)) <= TOL
