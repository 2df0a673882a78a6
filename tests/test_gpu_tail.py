"""GPU parity of the wide kernel's tail tiles (bmm_wide.hip).

When the last wave of 256 x 256 tiles would fill at most half the CUs, those
tiles run in a second launch as 256 x 128 halves, two workgroups per tile, so
that the partial wave still occupies every CU. Shapes here are sized from the
device's CU count so that the tile count is CUs + a small tail, and cover:
- even and odd numbers of K steps;
- K-major and MN-major operands, and one scale per column of B (128 x 1
  quantization, the wgrad recipe);
- a batch whose tail tiles lie in the second batch;
- a ragged M, whose partial tile row is in the tail;
- bf16, fp16 and fp32 C, bias and GELU.
Each result is compared with an fp32 GEMM of the dequantized operands (the
reference's kernel_reference, fp8_training/fp8_bench/bench_bmm.py:414-419)
at max-abs-rel <= 1e-2 per 128 x 128 output tile, so one wrong tile or half
fails; repeated calls must give the same bits.
"""
from __future__ import annotations

import pytest
import torch

from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm, hip_per_block_quant
from practice_cuda_amd.registry import QuantResult

pytestmark = pytest.mark.gpu
TOL = 1e-2
TILE = 256


def _cus(dev) -> int:
    return torch.cuda.get_device_properties(dev).multi_processor_count


def _tile_err(out: torch.Tensor, ref: torch.Tensor, tile: int = 128) -> float:
    """Largest per-tile max|out - ref| / max|ref| over tile x tile blocks
    (the last row / column of tiles may be partial)."""
    m, n = ref.shape[-2:]
    pm, pn = -(-m // tile) * tile, -(-n // tile) * tile
    d = torch.zeros(pm, pn, device=ref.device)
    r = torch.zeros(pm, pn, device=ref.device)
    d[:m, :n] = (out.float() - ref).abs()
    r[:m, :n] = ref.abs()
    d = d.reshape(pm // tile, tile, pn // tile, tile).amax(dim=(1, 3))
    r = r.reshape(pm // tile, tile, pn // tile, tile).amax(dim=(1, 3))
    keep = r > 0
    return (d[keep] / r[keep]).max().item()


def _transposed(q: QuantResult) -> QuantResult:
    return QuantResult(q.tensor.transpose(-1, -2), q.dequant_scale.transpose(-1, -2), q.impl, "block",
                       {**q.meta, "block_m": q.meta["block_n"], "block_n": q.meta["block_m"]})


def _shape_m(cus: int, tail: int, n: int, batch: int = 1) -> int:
    """M (a multiple of 256) such that batch * (M / 256) * (n / 256) = cus + tail."""
    total = cus + tail
    tiles_n = n // TILE
    assert total % (batch * tiles_n) == 0
    return total // (batch * tiles_n) * TILE


def _check(out, ref, name):
    for b in range(out.shape[0]):
        err = _tile_err(out[b], ref[b])
        assert err <= TOL, (name, b, err)


@pytest.mark.parametrize("k", [512, 640, 1024])
@pytest.mark.parametrize("layout", ["a_k_b_k", "a_k_b_n"])
def test_tail_row_and_tile_scales(dev, k, layout):
    """A 1 x 128, B 128 x 128: the forward (a_k_b_k) and dgrad (a_k_b_n) recipes."""
    cus = _cus(dev)
    n = 4096
    m = _shape_m(cus, cus // 8, n)
    print(f"tail {layout} m={m} n={n} k={k} cus={cus}", flush=True)
    g = torch.Generator(device=dev).manual_seed(k + len(layout))
    a = torch.randn(1, m, k, generator=g, device=dev).bfloat16()
    qa = hip_per_block_quant(a, block_m=1, block_n=128)
    if layout == "a_k_b_k":
        w = (torch.randn(1, n, k, generator=g, device=dev) * 0.02).bfloat16()
        qb = _transposed(hip_per_block_quant(w, block_m=128, block_n=128))
    else:
        w = (torch.randn(1, k, n, generator=g, device=dev) * 0.02).bfloat16()
        qb = hip_per_block_quant(w, block_m=128, block_n=128)
    out = hip_per_block_bmm(qa, qb)
    ref = torch.matmul(qa.dequantize(), qb.dequantize().contiguous())
    _check(out, ref, layout)
    for _ in range(2):
        assert torch.equal(hip_per_block_bmm(qa, qb).view(torch.int16), out.view(torch.int16))


@pytest.mark.parametrize("kmajor", [False, True])
def test_tail_column_scales_wgrad(dev, kmajor):
    """dW = dY^T X with dY and X quantized 128 x 1 along the reduction (one
    scale per column of B): on the reference's a_m_b_n layout and on K-major
    copies of the operands."""
    cus = _cus(dev)
    n_in = 4096
    n_out = _shape_m(cus, cus // 4, n_in)
    t = 1024
    print(f"tail wgrad kmajor={kmajor} m={n_out} n={n_in} k={t}", flush=True)
    g = torch.Generator(device=dev).manual_seed(5 + kmajor)
    dy = (torch.randn(1, t, n_out, generator=g, device=dev) * 1e-3).bfloat16()
    x = torch.randn(1, t, n_in, generator=g, device=dev).bfloat16()
    qdy = hip_per_block_quant(dy, block_m=128, block_n=1)
    qx = hip_per_block_quant(x, block_m=128, block_n=1)
    a = _transposed(qdy)                        # [1, n_out, t], M-major
    b = qx                                      # [1, t, n_in], N-major
    if kmajor:
        a = QuantResult(a.tensor.contiguous(), a.dequant_scale, a.impl, "block", dict(a.meta))
        b = QuantResult(b.tensor.transpose(-1, -2).contiguous().transpose(-1, -2), b.dequant_scale, b.impl,
                        "block", dict(b.meta))
    out = hip_per_block_bmm(a, b)
    ref = torch.matmul(a.dequantize().contiguous(), b.dequantize().contiguous())
    _check(out, ref, "wgrad")


def test_tail_batched_and_ragged(dev):
    """Two batches (the tail tiles lie in the second) and, separately, an M
    that is not a multiple of 256 (the partial tile row is in the tail)."""
    cus = _cus(dev)
    n, k = 4096, 768
    m = _shape_m(cus, cus // 8, n, batch=2)
    g = torch.Generator(device=dev).manual_seed(11)
    for bsz, mm in ((2, m), (1, _shape_m(cus, cus // 8, n) - 100)):
        print(f"tail batch={bsz} m={mm}", flush=True)
        a = torch.randn(bsz, mm, k, generator=g, device=dev).bfloat16()
        w = (torch.randn(bsz, k, n, generator=g, device=dev) * 0.02).bfloat16()
        qa = hip_per_block_quant(a, block_m=1, block_n=128)
        qb = hip_per_block_quant(w, block_m=128, block_n=128)
        out = hip_per_block_bmm(qa, qb)
        ref = torch.matmul(qa.dequantize(), qb.dequantize())
        _check(out, ref, f"batch {bsz}")


@pytest.mark.parametrize("out_dtype,bias,act", [(torch.float32, False, "none"), (torch.float16, True, "gelu"),
                                                (torch.bfloat16, True, "none")])
def test_tail_out_dtypes_bias_gelu(dev, out_dtype, bias, act):
    """The half tiles' epilogue: C dtype, bias, GELU."""
    cus = _cus(dev)
    n, k = 4096, 512
    m = _shape_m(cus, cus // 8, n)
    print(f"tail out={out_dtype} bias={bias} act={act}", flush=True)
    g = torch.Generator(device=dev).manual_seed(3)
    a = torch.randn(1, m, k, generator=g, device=dev).bfloat16()
    w = (torch.randn(1, k, n, generator=g, device=dev) * 0.05).bfloat16()
    qa = hip_per_block_quant(a, block_m=1, block_n=128)
    qb = hip_per_block_quant(w, block_m=128, block_n=128)
    bias_t = (torch.randn(1, m, n, generator=g, device=dev) * 0.5).to(out_dtype) if bias else None
    out = hip_per_block_bmm(qa, qb, out_dtype=out_dtype, bias=bias_t, activation=act)
    ref = torch.matmul(qa.dequantize(), qb.dequantize())
    if bias:
        ref = ref + bias_t.float()
    if act == "gelu":
        ref = torch.nn.functional.gelu(ref)
    assert out.dtype == out_dtype
    _check(out, ref, str(out_dtype))
