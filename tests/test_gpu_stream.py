"""GPU parity of the streaming K = 128 BMM (bmm_stream.hip).

The dispatch sends a block-scaled product with K = 128, N = 512, A K-major,
B N-major, 1 x 128 A scales and contiguous column-block B scales to the
persistent streaming kernel; the same product with the B scales given as a
strided view goes to the single-K-step tile kernel. Both compute
bf16(P * (sa * sb)) with the same fp32 MFMA product, so their outputs must be
bit-identical; each is also checked per batch against an fp32 bmm of the
dequantized operands at the north_star bar (max-abs-rel <= 1e-2,
fp8_training/fp8_bench/bench_bmm.py:414-419).

Shapes cover one unit, a partial last unit, fewer units than CUs with a
partial one among them, more units than CUs (each
workgroup walks several units and crosses batch boundaries, reloading B),
ragged M on top of that, four B block widths and both fp8 formats.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from practice_cuda_amd import _lib

pytestmark = pytest.mark.gpu
TOL = 1e-2
K, N = 128, 512

FMTS = {"e4m3": (torch.float8_e4m3fn, _lib.E4M3FN), "e5m2": (torch.float8_e5m2, _lib.E5M2)}


def _operands(bsz, m, qbn, fmt, seed, dev):
    g = torch.Generator().manual_seed(seed)
    dt, _ = FMTS[fmt]
    a = (torch.randn(bsz, m, K, generator=g) * 2.0).to(dt).to(dev)
    b = (torch.randn(bsz, K, N, generator=g) * 2.0).to(dt).to(dev)
    # dequant scales over two decades, as quantizers produce them; the row
    # scales of a batch start on a 16-byte boundary (the streaming kernel
    # copies them 16 bytes per lane)
    m_pad = (m + 3) // 4 * 4
    sa = torch.exp(torch.empty(bsz, m_pad, 1).uniform_(np.log(0.01), np.log(1.0), generator=g)).float().to(dev)
    sa = sa[:, :m]
    sb = torch.exp(torch.empty(bsz, 1, N // qbn).uniform_(np.log(0.01), np.log(1.0), generator=g)).float().to(dev)
    return a, b, sa, sb


def _bmm(a, b, sa, sb, qbn, fmt):
    bsz, m, _ = a.shape
    c = torch.empty(bsz, m, N, dtype=torch.bfloat16, device=a.device)
    rc = _lib.lib().pcamd_bmm_scaled(
        _lib.ptr(a), _lib.ptr(b), FMTS[fmt][1], bsz, m, N, K, *a.stride(), *b.stride(), _lib.ptr(c), _lib.BF16,
        *c.stride(), None, 0, 0, 0, 0, _lib.ptr(sa), *sa.stride(), _lib.ptr(sb), *sb.stride(), _lib.SCALE_BLOCK, 0,
        1, 128, qbn, _lib.ACT_NONE, _lib.stream_of(c))
    _lib.check(rc, "pcamd_bmm_scaled")
    torch.cuda.synchronize()
    return c


CASES = [
    # (batch, M, qbn, fmt)
    (1, 128, 128, "e4m3"),      # one unit
    (3, 200, 128, "e4m3"),      # partial last unit per batch
    (2, 2048, 16, "e4m3"),      # one B scale per 16-column sub-tile
    (2, 384, 64, "e5m2"),
    (1, 77, 512, "e4m3"),       # a single partial unit, one B scale for all columns
    (1, 600, 128, "e4m3"),      # 5 units (one workgroup each), the last partial
    (3, 25600, 128, "e4m3"),    # 600 units: ranges of 2-3 units crossing batch boundaries
    (2, 38477, 128, "e4m3"),    # the same with a partial unit at the end of each batch
    (128, 2048, 128, "e4m3"),
]


@pytest.mark.parametrize("bsz,m,qbn,fmt", CASES)
def test_stream_matches_tile_kernel_and_fp32(dev, bsz, m, qbn, fmt):
    print(f"stream bmm batch={bsz} m={m} qbn={qbn} {fmt}", flush=True)
    a, b, sa, sb = _operands(bsz, m, qbn, fmt, 7 + m + bsz, dev)
    out = _bmm(a, b, sa, sb, qbn, fmt)
    # the same B scales as a strided view: the tile kernel computes this one
    sb_wide = torch.zeros(bsz, 1, 2 * (N // qbn), device=dev)
    sb_wide[..., ::2] = sb
    sb_strided = sb_wide[..., ::2]
    assert sb_strided.stride(-1) == 2 and torch.equal(sb_strided, sb)
    out_tile = _bmm(a, b, sa, sb_strided, qbn, fmt)
    assert torch.equal(out.view(torch.int16), out_tile.view(torch.int16))
    sb_cols = sb.repeat_interleave(qbn, dim=-1)                       # [B, 1, N]
    ref = torch.bmm((a.float() * sa).contiguous(), (b.float() * sb_cols).contiguous())
    err = (out.float() - ref).abs().amax(dim=(1, 2)) / ref.abs().amax(dim=(1, 2))
    assert err.max().item() <= TOL, (err.argmax().item(), err.max().item())


def test_stream_repeat_launches_identical(dev):
    """Back-to-back launches on the same buffers (the loop's waits are
    hand-written): every launch must give the same bits."""
    a, b, sa, sb = _operands(3, 25600, 128, "e4m3", 11, dev)
    first = _bmm(a, b, sa, sb, 128, "e4m3")
    for _ in range(3):
        assert torch.equal(_bmm(a, b, sa, sb, 128, "e4m3").view(torch.int16), first.view(torch.int16))
