"""The C ABI from several host threads at once, each on its own stream.

The reference's autograd backward may run on a worker thread, and its
wrappers launch on torch's current stream of the calling thread
(fp8_training/fp8_bench/modules/bmm_linear.py:135-137). The library keeps
its error text per thread and its device-attribute caches atomic, and takes
the stream as an argument; these tests run quantizers and BMMs from four
threads concurrently (four default-priority streams) and require every
result to equal, bit for bit, the same call made alone on the default
stream, and each thread's error text to stay its own.
"""
from __future__ import annotations

import threading

import pytest
import torch

from practice_cuda_amd import _lib
from practice_cuda_amd.impls.hip_per_block import (hip_per_block_bmm, hip_per_block_bmm_quant_a, hip_per_block_quant,
                                                   hip_per_block_quant_dual)
from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_quant
from practice_cuda_amd.registry import QuantResult

pytestmark = pytest.mark.gpu
THREADS = 4
ITERS = 6


def _inputs(dev, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(384, 1024, generator=g).bfloat16().to(dev)
    w = (torch.randn(512, 1024, generator=g) * 0.02).bfloat16().to(dev)
    a4 = torch.randn(4, 256, 128, generator=g).bfloat16().to(dev)
    b4 = torch.randn(4, 128, 512, generator=g).bfloat16().to(dev)
    return x, w, a4, b4


def _run(x, w, a4, b4):
    """Quantizers (row groups, per-row channel, 128x128 tiles, the dual
    kernel), the wide BMM (K = 1024), the streaming BMM (K = 128, N = 512)
    and the fused activation-quant BMM (N = 128, K = 1024: its streaming
    kernel)."""
    qx = hip_per_block_quant(x[None], block_m=1, block_n=128)
    qw = hip_per_block_quant(w[None], block_m=128, block_n=128)
    qc = hip_per_channel_quant(x, channel_axis=-2)
    r_row, r_col = hip_per_block_quant_dual(x, block=128, col_transposed=True)
    wt = QuantResult(qw.tensor.transpose(-1, -2), qw.dequant_scale.transpose(-1, -2), qw.impl, "block",
                     {"block_m": 128, "block_n": 128})
    y = hip_per_block_bmm(qx, wt)
    qa4 = hip_per_block_quant(a4, block_m=1, block_n=128)
    qb4 = hip_per_block_quant(b4, block_m=128, block_n=128)
    y4 = hip_per_block_bmm(qa4, qb4)
    qw128 = hip_per_block_quant(w[None, :128], block_m=128, block_n=128)
    wt128 = QuantResult(qw128.tensor.transpose(-1, -2), qw128.dequant_scale.transpose(-1, -2), qw128.impl,
                        "block", {"block_m": 128, "block_n": 128})
    y5, qa5 = hip_per_block_bmm_quant_a(x[None], wt128, return_quant=True)
    return [qx.tensor, qx.dequant_scale, qw.tensor, qw.dequant_scale, qc.tensor, qc.dequant_scale,
            r_row.tensor, r_row.dequant_scale, r_col.tensor.contiguous(), r_col.dequant_scale, y, y4,
            y5, qa5.tensor, qa5.dequant_scale]


def _bits(t):
    t = t.contiguous()
    return t.view(torch.uint8) if t.element_size() == 1 else t.view(torch.int16 if t.element_size() == 2
                                                                    else torch.int32)


def test_threads_on_separate_streams_match_serial(dev):
    print(f"concurrency: {THREADS} threads x {ITERS} iterations", flush=True)
    inputs = [_inputs(dev, 100 + i) for i in range(THREADS)]
    expected = [[_bits(t).clone() for t in _run(*inp)] for inp in inputs]
    torch.cuda.synchronize()
    results = [None] * THREADS
    errors = []
    start = threading.Barrier(THREADS)

    def worker(i):
        try:
            s = torch.cuda.Stream(device=dev)  # default priority
            start.wait()
            with torch.cuda.stream(s):
                out = None
                for _ in range(ITERS):
                    out = _run(*inputs[i])
                results[i] = [_bits(t) for t in out]
            s.synchronize()
        except Exception as exc:  # surfaced below, with the thread's index
            errors.append((i, repr(exc)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    for i in range(THREADS):
        for j, (got, want) in enumerate(zip(results[i], expected[i])):
            assert torch.equal(got, want), f"thread {i}, output {j} differs from the serial call"


def test_error_text_is_per_thread(dev):
    """An invalid call fails in its own thread with its own message; a valid
    call in another thread, at the same time, leaves no error text there."""
    x = torch.randn(64, 256, device=dev).bfloat16()
    y = torch.empty(64, 256, device=dev, dtype=torch.float8_e4m3fn)
    s = torch.empty(64, 2, device=dev)
    L = _lib.lib()
    seen = {}
    start = threading.Barrier(2)

    def call(block_n, key):
        start.wait()
        rc = L.pcamd_quant_block(_lib.ptr(x), _lib.BF16, 1, 64, 256, 0, 256, 1, _lib.ptr(y), _lib.E4M3FN,
                                 0, 256, 1, _lib.ptr(s), 0, s.stride(0), 1, 1, block_n, 448.0, 1e-12,
                                 _lib.stream_of(x))
        seen[key] = (rc, L.pcamd_last_error().decode())

    bad = threading.Thread(target=call, args=(100, "bad"))     # block_n not a power of two
    good = threading.Thread(target=call, args=(128, "good"))
    bad.start(), good.start()
    bad.join(timeout=60), good.join(timeout=60)
    torch.cuda.synchronize()
    assert seen["bad"][0] != 0 and "powers of two" in seen["bad"][1], seen["bad"]
    assert seen["good"] == (0, ""), seen["good"]
