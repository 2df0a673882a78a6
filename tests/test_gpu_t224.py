"""GPU parity of the wide kernel's transposed launch on 256 x 224 tiles.

When 256 x 256 tiles leave a short last wave and the A operand has one block
scale per row (qbm = 1: the wgrad recipe, dY^T and X both quantized 128 x 1),
the launcher computes C^T = B^T A^T on 256 x 224 tiles (whole waves) and the
epilogue writes C through a transposing LDS stage. Checked per 128 x 128
output tile against the fp32 product of the dequantized operands (the
reference's kernel_reference, fp8_training/fp8_bench/bench_bmm.py:414-419),
within max-abs-relative 1e-2: M a multiple of 224 and ragged, both operand
layouts of the wgrad product (the reference's a_m_b_n and the training
layer's K-major operands), e4m3 and an e5m2 gradient, fp16 output.
"""
from __future__ import annotations

import pytest
import torch

from practice_cuda_amd import modules  # noqa: F401  (registers pcamd::block_scaled_bmm)
from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _tile_err(out: torch.Tensor, ref: torch.Tensor, tile: int = 128) -> float:
    m, n = ref.shape[-2:]
    pm, pn = -(-m // tile) * tile, -(-n // tile) * tile
    d = torch.zeros(pm, pn, device=ref.device)
    r = torch.zeros(pm, pn, device=ref.device)
    d[:m, :n] = (out.float() - ref).abs()
    r[:m, :n] = ref.abs()
    d = d.reshape(pm // tile, tile, pn // tile, tile).amax(dim=(1, 3))
    r = r.reshape(pm // tile, tile, pn // tile, tile).amax(dim=(1, 3))
    return (d / r.clamp_min(1e-30)).max().item()


def _shape(dev, ragged):
    """(M, N, K) whose 256 x 256 tiling leaves a short last wave that the
    224-column transposed tiling fills (cost model of bmm_wide.h), for this
    device's CU count."""
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    n = 4096                                   # 16 tile columns
    for m224 in range(2, 400):
        m = 224 * m224 - (20 if ragged else 0)
        t1 = -(-m // 256) * 16
        if t1 <= cus:
            continue
        tail = t1 % cus
        now = t1 // cus + (0 if tail == 0 else 0.85 if 2 * tail <= cus else 1.0)
        alt = -(-(16 * -(-m // 224)) // cus) * (224 / 256)
        if alt < 0.95 * now:
            return m, n, 512
    pytest.skip("no shape found for this CU count")


@pytest.mark.parametrize("ragged", [False, True], ids=["m_aligned", "m_ragged"])
@pytest.mark.parametrize("k_major", [False, True], ids=["a_m_b_n", "k_major"])
@pytest.mark.parametrize("fa,out_dtype", [(torch.float8_e4m3fn, torch.bfloat16), (torch.float8_e5m2, torch.float16)],
                         ids=["e4m3_bf16", "e5m2_f16"])
def test_transposed_224_tiles(dev, ragged, k_major, fa, out_dtype):
    m, n, k = _shape(dev, ragged)
    print(f"t224 m={m} n={n} k={k} k_major={k_major} {fa} -> {out_dtype}", flush=True)
    g = torch.Generator().manual_seed(m + k_major)
    dy = (torch.randn(1, k, m, generator=g) * 1e-3).bfloat16().to(dev)   # [tokens, out features]
    x = torch.randn(1, k, n, generator=g).bfloat16().to(dev)             # [tokens, in features]
    qdy = hip_per_block_quant(dy, block_m=128, block_n=1, fp8_dtype=fa)                # scales [1, k/128, m]
    qx = hip_per_block_quant(x, block_m=128, block_n=1, fp8_dtype=torch.float8_e4m3fn)  # scales [1, k/128, n]
    a, sa = qdy.tensor.transpose(-1, -2), qdy.dequant_scale.transpose(-1, -2)  # A = dY^T [m, k], M-major
    b, sb = qx.tensor, qx.dequant_scale                                         # B = X [k, n], N-major
    if k_major:
        a = a.contiguous()
        b = b.transpose(-1, -2).contiguous().transpose(-1, -2)
    out = torch.ops.pcamd.block_scaled_bmm(a, sa, b, sb, None, 1, 128, 1, out_dtype)
    ref = torch.matmul(qdy.dequantize()[0].t().contiguous(), qx.dequantize()[0])
    torch.cuda.synchronize()
    assert out.shape == (1, m, n) and out.dtype == out_dtype
    err = _tile_err(out[0], ref)
    assert err <= TOL, f"per-tile max_abs_rel {err}"
