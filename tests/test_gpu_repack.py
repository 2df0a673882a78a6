"""GPU parity of the fp8 repack (pcamd_repack_fp8, csrc/repack.hip).

The BMM wrappers' transpose variants copy an M-major A or an N-major B into
K-major order before the GEMM; the reference does it with `.contiguous()` on
the strided view (fp8_training/fp8_bench/impls/triton_per_block.py:254-272).
The repack moves the same bytes, so its output must equal torch's copy bit
for bit: whole 128 x 128 tiles, ragged edges (rows and columns not multiples
of 16 or 128), batches with padded batch strides, views that are not 16-byte
aligned (the byte path), both fp8 formats, and the operand preparation of
the transpose variants through the registry.
"""
from __future__ import annotations

import pytest
import torch

from practice_cuda_amd.impls._common import repack_rows_major

pytestmark = pytest.mark.gpu


def _rows_major(dev, bsz, rows, cols, dtype, seed, pad_rows=0, pad_batch=0, offset=0):
    """A [bsz, rows, cols] fp8 view contiguous along rows (stride(-2) == 1),
    over storage with padded column pitch / batch pitch and a byte offset."""
    g = torch.Generator(device=dev).manual_seed(seed)
    pitch = rows + pad_rows
    bpitch = cols * pitch + pad_batch
    raw = torch.randint(0, 256, (offset + bsz * bpitch,), generator=g, device=dev, dtype=torch.uint8)
    return raw.view(dtype).as_strided((bsz, rows, cols), (bpitch, 1, pitch), offset)


CASES = [
    # (bsz, rows, cols, pad_rows, pad_batch, offset)
    (1, 8192, 4096, 0, 0, 0),        # config-5 X: whole tiles
    (1, 4096, 14336, 0, 0, 0),
    (3, 200, 333, 0, 0, 0),          # ragged both ways
    (2, 77, 130, 3, 5, 0),           # not multiples of 16, padded pitches (byte path)
    (2, 256, 256, 16, 32, 0),        # padded but 16-byte aligned pitches
    (1, 512, 640, 0, 0, 1),          # unaligned base (byte path)
    (1, 1000, 2, 0, 0, 0),           # narrow: fewer columns than one 16-byte store,
    (2, 333, 7, 0, 0, 0),            #   rows not multiples of 16 (per-byte masked stores)
    (1, 77, 15, 5, 0, 0),
    (3, 130, 9, 16, 8, 0),
]


@pytest.mark.parametrize("fmt", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("bsz,rows,cols,pad_rows,pad_batch,offset", CASES)
def test_repack_equals_torch_copy(dev, fmt, bsz, rows, cols, pad_rows, pad_batch, offset):
    print(f"repack {bsz}x{rows}x{cols} pads {pad_rows},{pad_batch} offset {offset} {fmt}", flush=True)
    x = _rows_major(dev, bsz, rows, cols, fmt, rows + cols, pad_rows, pad_batch, offset)
    assert x.stride(-2) == 1
    y = repack_rows_major(x)
    ref = x.contiguous()
    assert y.is_contiguous() and y.shape == x.shape and y.dtype == fmt
    assert torch.equal(y.view(torch.uint8), ref.view(torch.uint8))


def test_transpose_variants_use_repacked_operands(dev):
    """The registry's transpose variants give the same result as the plain
    layouts on the same values (their operands are repacked copies)."""
    from practice_cuda_amd import get_bmm, get_quant
    g = torch.Generator().manual_seed(9)
    a = torch.randn(2, 384, 512, generator=g).bfloat16().to(dev)
    b = torch.randn(2, 512, 640, generator=g).bfloat16().to(dev)
    plain = get_bmm("hip_per_block_2d_a_k_b_n")
    trans = get_bmm("hip_per_block_2d_a_k_b_n_transpose")
    quant = get_quant(plain.quant_impl)
    qa = quant.fn(a, block_m=1, block_n=128)
    qb = quant.fn(b, **plain.quant_b_kwargs)
    ref = plain.fn(qa, qb)
    out = trans.fn(qa, qb)
    # B N-major repacked to K-major: same math on the same values; the K-major
    # and N-major kernels read the operands through different fragment paths
    # but accumulate the same products in the same order
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_repack_in_hip_graph(dev):
    """Captured once, replayed three times with eager work between the
    replays: every replay's output equals torch's copy of the current input."""
    x = _rows_major(dev, 2, 640, 384, torch.float8_e4m3fn, 5, pad_rows=16)
    s = torch.cuda.Stream(device=dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        repack_rows_major(x)  # warm-up outside the capture
    torch.cuda.current_stream(dev).wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = repack_rows_major(x)
    for it in range(3):
        x.view(torch.uint8).copy_(torch.randint(0, 256, x.shape, device=dev, dtype=torch.uint8))  # new values
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.uint8), x.contiguous().view(torch.uint8)), it


@pytest.mark.parametrize("case", ["one_column", "expanded_columns", "batch_past_grid"])
def test_repack_fallback_to_torch_copy(dev, case):
    """Views the kernel does not take go to torch's copy and still come back
    contiguous and equal to it: a single column (its column stride is
    arbitrary), columns that overlap the rows (an expanded view, column
    stride 0) and more batches than the kernel's grid covers (the C entry
    point returns PCAMD_ERR_UNSUPPORTED without launching)."""
    from practice_cuda_amd import _lib
    fmt = torch.float8_e4m3fn
    print(f"repack fallback {case}", flush=True)
    if case == "one_column":
        x = _rows_major(dev, 1, 1000, 1, fmt, 3)
    elif case == "expanded_columns":
        x = _rows_major(dev, 2, 300, 1, fmt, 4).expand(2, 300, 40)
        assert x.stride(-1) == 0
    else:
        x = _rows_major(dev, 70000, 2, 16, fmt, 5)
        y = torch.empty(x.shape, dtype=fmt, device=dev)
        rc = _lib.lib().pcamd_repack_fp8(_lib.ptr(x), 70000, 2, 16, x.stride(0), 1, x.stride(2), _lib.ptr(y),
                                         *y.stride(), _lib.stream_of(y))
        assert rc == _lib.ERR_UNSUPPORTED
    assert x.stride(-2) == 1
    y = repack_rows_major(x)
    assert y.is_contiguous() and y.shape == x.shape
    assert torch.equal(y.view(torch.uint8), x.contiguous().view(torch.uint8))
