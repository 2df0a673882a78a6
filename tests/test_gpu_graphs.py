"""HIP graph capture of the C-ABI launches: every entry point launches only
kernels on the caller's stream (no allocation, no memset, no host sync), so a
captured graph replays them. Each replay is checked bit for bit against the
eager result, with the outputs overwritten by eager work between replays."""
from __future__ import annotations

import pytest
import torch

from practice_cuda_amd.impls.hip_per_block import (hip_per_block_bmm, hip_per_block_bmm_quant_a,
                                                   hip_per_block_quant, hip_per_block_quant_dual)
from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_quant
from practice_cuda_amd.impls.hip_per_tensor import hip_per_tensor_quant

pytestmark = pytest.mark.gpu


def _tensors(res):
    """The output tensors of a quantizer / BMM call, flattened to a list."""
    if isinstance(res, torch.Tensor):
        return [res]
    if isinstance(res, (tuple, list)):
        return [t for r in res for t in _tensors(r)]
    return [res.tensor, res.dequant_scale]


def _raw(t: torch.Tensor) -> torch.Tensor:
    """The tensor's bytes as a uint8 view of the same storage (0-d scales included)."""
    return (t if t.dim() > 0 else t.reshape(1)).view(torch.uint8)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return _raw(t).contiguous().clone()


def _replay_matches_eager(dev, fns):
    eager = {k: [_bits(t) for t in _tensors(f())] for k, f in fns.items()}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up launches off the capture stream
        for f in fns.values():
            f()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = {k: _tensors(f()) for k, f in fns.items()}
    for rep in range(3):
        for ts in outs.values():  # eager work between replays: clobber every output
            for t in ts:
                _raw(t).fill_(0xA5)
        torch.cuda.synchronize()
        print(f"replay {rep}", flush=True)
        graph.replay()
        torch.cuda.synchronize()
        for k, ts in outs.items():
            for i, t in enumerate(ts):
                assert torch.equal(_bits(t), eager[k][i]), f"replay {rep}: {k} output {i} differs"


def test_quantizers_replay(dev):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn(512, 1024, generator=g) * 3).bfloat16().to(dev)
    x3 = torch.randn(2, 256, 7168, generator=g).bfloat16().to(dev)
    fns = {
        "1x128": lambda: hip_per_block_quant(x, block_m=1, block_n=128),
        "128x128": lambda: hip_per_block_quant(x, block_m=128, block_n=128),
        "128x1": lambda: hip_per_block_quant(x, block_m=128, block_n=1),
        "dual": lambda: hip_per_block_quant_dual(x, block=128),
        "dual transposed": lambda: hip_per_block_quant_dual(x, block=128, col_transposed=True),
        "channel rows": lambda: hip_per_channel_quant(x3, channel_axis=-2),
        "channel cols": lambda: hip_per_channel_quant(x, channel_axis=-1),
        "tensor": lambda: hip_per_tensor_quant(x),
        "generic 2x64": lambda: hip_per_block_quant(x.t(), block_m=2, block_n=64),
    }
    _replay_matches_eager(dev, fns)


def test_bmm_replay(dev):
    g = torch.Generator().manual_seed(8)
    ah = torch.randn(2, 512, 512, generator=g).bfloat16().to(dev)
    bh = torch.randn(2, 512, 384, generator=g).bfloat16().to(dev)
    qa = hip_per_block_quant(ah, block_m=1, block_n=128)
    qb = hip_per_block_quant(bh, block_m=128, block_n=128)
    a1 = torch.randn(4, 256, 128, generator=g).bfloat16().to(dev)  # K = 128: single-step kernel
    b1 = torch.randn(4, 128, 256, generator=g).bfloat16().to(dev)
    qa1 = hip_per_block_quant(a1, block_m=1, block_n=128)
    qb1 = hip_per_block_quant(b1, block_m=128, block_n=128)
    a2 = torch.randn(1, 33, 256, generator=g).bfloat16().to(dev)  # ragged M / N: general kernel
    b2 = torch.randn(1, 256, 47, generator=g).bfloat16().to(dev)
    qa2 = hip_per_block_quant(a2, block_m=1, block_n=128)
    qb2 = hip_per_block_quant(b2, block_m=128, block_n=128)
    b3 = torch.randn(2, 512, 128, generator=g).bfloat16().to(dev)  # N = 128: fused streaming kernel
    b4 = torch.randn(2, 512, 256, generator=g).bfloat16().to(dev)  # N = 256
    qb3 = hip_per_block_quant(b3, block_m=128, block_n=128)
    qb4 = hip_per_block_quant(b4, block_m=128, block_n=128)
    b5 = torch.randn(2, 512, 192, generator=g).bfloat16().to(dev)  # N = 192: 12 sub-tiles, two K blocks per step
    b6 = torch.randn(2, 512, 64, generator=g).bfloat16().to(dev)   # N = 64: 4 sub-tiles
    qb5 = hip_per_block_quant(b5, block_m=128, block_n=128)
    qb6 = hip_per_block_quant(b6, block_m=128, block_n=128)
    bias5 = torch.randn(2, 512, 192, generator=g).bfloat16().to(dev)
    bias_w = torch.randn(2, 512, 384, generator=g).bfloat16().to(dev)
    fns = {
        "wide": lambda: hip_per_block_bmm(qa, qb),
        "single": lambda: hip_per_block_bmm(qa1, qb1),
        "general": lambda: hip_per_block_bmm(qa2, qb2),
        "fused_stream_n128": lambda: hip_per_block_bmm_quant_a(ah, qb3, return_quant=True),
        "fused_stream_n256": lambda: hip_per_block_bmm_quant_a(ah, qb4),
        "fused_tiled": lambda: hip_per_block_bmm_quant_a(ah, qb, always_fused=True),
        # epilogues: 16-bit bias + GELU (8-byte loads and stores), fp32 output
        # (per-element), and the wide GEMM's LDS-staged bias + GELU
        "fused_stream_n192_bias_gelu": lambda: hip_per_block_bmm_quant_a(ah, qb5, bias=bias5, activation="gelu"),
        "fused_stream_n64_f32": lambda: hip_per_block_bmm_quant_a(ah, qb6, out_dtype=torch.float32),
        "wide_bias_gelu": lambda: hip_per_block_bmm(qa, qb, bias=bias_w, activation="gelu"),
    }
    _replay_matches_eager(dev, fns)
