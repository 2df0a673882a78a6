"""GPU tests of the quantizers' output store policy (pcamd_quant_block_ex /
pcamd_quant_block_dual_ex with PCAMD_QUANT_CACHED_OUTPUT, the training
layer's quantization ops): cache-allocating stores write the same fp8 bytes
and scales as the default non-temporal ones on every kernel path, and the
oracle's bytes."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant, hip_per_block_quant_dual

from test_gpu_quant import assert_same, make_input, qbits, sbits

pytestmark = pytest.mark.gpu


def _same(a, b, label):
    torch.cuda.synchronize()
    assert np.array_equal(qbits(a.tensor), qbits(b.tensor)), f"{label}: fp8 bytes differ"
    assert np.array_equal(sbits(a.dequant_scale), sbits(b.dequant_scale)), f"{label}: scales differ"


BLOCK_PATHS = [
    # (shape, dtype, block_m, block_n, slice_cols)   kernel path
    ((256, 1024), "bf16", 1, 128, None),             # row groups, flat
    ((64, 640), "bf16", 1, 128, 384),                # row groups, row-indexed (padded rows)
    ((4096, 7168), "bf16", 128, 128, None),          # 128 x 128, eight blocks per workgroup (config 3)
    ((4096, 4096), "f16", 128, 128, None),           # 128 x 128, four blocks per workgroup
    ((256, 384), "bf16", 128, 128, None),            # 128 x 128, one block per workgroup
    ((512, 384), "bf16", 128, 1, None),              # column groups
    ((33, 70), "f32", 4, 32, None),                  # generic
]


@pytest.mark.parametrize("shape,dtype,bm,bn,cols", BLOCK_PATHS)
def test_cached_outputs_same_bytes(dev, shape, dtype, bm, bn, cols):
    print(f"cached outputs: block {shape} {dtype} {bm}x{bn} cols={cols}", flush=True)
    x = make_input(shape, dtype, seed=sum(shape) + bm, scale=0.5, outliers=0.002).to(dev)
    if cols is not None:
        x = x[:, :cols]
    plain = hip_per_block_quant(x, block_m=bm, block_n=bn)
    cached = hip_per_block_quant(x, block_m=bm, block_n=bn, cache_outputs=True)
    _same(plain, cached, f"{shape} {bm}x{bn}")
    q_ref, s_ref = O.quant_block(x.cpu().contiguous(), bm, bn)
    assert_same(cached, q_ref, s_ref, f"cached {shape} {bm}x{bn}")


@pytest.mark.parametrize("shape,block,col_t", [((256, 512), 128, True), ((256, 512), 128, False),
                                               ((2, 333, 264), 128, True), ((128, 256), 64, False)])
def test_cached_outputs_dual_same_bytes(dev, shape, block, col_t):
    # (2, 333, 264): ragged blocks with the transposed column output; block 64:
    # the two-quantizer fallback
    print(f"cached outputs: dual {shape} block={block} col_t={col_t}", flush=True)
    x = make_input(shape, "bf16", seed=sum(shape), scale=0.5, outliers=0.002).to(dev)
    r0, c0 = hip_per_block_quant_dual(x, block=block, col_transposed=col_t)
    r1, c1 = hip_per_block_quant_dual(x, block=block, col_transposed=col_t, cache_outputs=True)
    _same(r0, r1, f"dual rows {shape}")
    _same(c0, c1, f"dual columns {shape}")


def test_layer_quant_ops_match_registry_quantizer(dev):
    # the training layer's custom ops write with cached stores: same bytes as
    # the registry's quantizer
    print("cached outputs: layer custom ops", flush=True)
    from practice_cuda_amd import modules  # noqa: F401  (registers the ops)
    x = make_input((1, 1024, 2048), "bf16", seed=3).to(dev)
    q, s = torch.ops.pcamd.quant_block(x, 128, 128, torch.float8_e4m3fn, 1e-12)
    ref = hip_per_block_quant(x, block_m=128, block_n=128)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.uint8), ref.tensor.view(torch.uint8))
    assert torch.equal(s.view(torch.int32), ref.dequant_scale.view(torch.int32))
    qr, sr, qc, sc = torch.ops.pcamd.quant_block_dual(x, 128, torch.float8_e4m3fn, 1e-12)
    r, c = hip_per_block_quant_dual(x, block=128, col_transposed=True)
    torch.cuda.synchronize()
    assert torch.equal(qr.view(torch.uint8), r.tensor.view(torch.uint8))
    assert torch.equal(qc.contiguous().view(torch.uint8), c.tensor.contiguous().view(torch.uint8))
    assert torch.equal(sr.view(torch.int32), r.dequant_scale.view(torch.int32))
    assert torch.equal(sc.view(torch.int32), c.dequant_scale.view(torch.int32))
