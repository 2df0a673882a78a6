"""Bit-exact parity of the training layer's quantization launches at the full
BASELINE config-5 size (M = 8192 tokens, K = 4096, N = 14336), on the inputs
bench.py times (BASELINE's CPU generator, seed 0).

The layer (practice_cuda_amd/modules.py) quantizes, per step:
- X [8192, 4096] and dY [8192, 14336] with ``pcamd::quant_block_dual``: 1 x 128
  along the last dim (forward / dgrad operand) and 128 x 1 along M (wgrad
  operand) from one read, the 128 x 1 result stored transposed;
- W [14336, 4096] 128 x 128 with ``pcamd::quant_block``.

Each launch is checked here, fp8 bytes and fp32 scale bit patterns, against
the oracle's restatement of the reference quantizer
(xuOAO/practice_cuda fp8_training/fp8_bench/kernels/quant/per_block.py:35-48):
the layer's own op, and the dual entry point with the plain (row-major)
128 x 1 layout too.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd import modules  # noqa: F401  (registers the pcamd:: ops)
from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant_dual

pytestmark = pytest.mark.gpu
E4M3 = torch.float8_e4m3fn


def _bytes(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).cpu().numpy()


def _scale_bits(t: torch.Tensor) -> np.ndarray:
    return t.float().cpu().numpy().astype(np.float32).reshape(-1).view(np.uint32)


def _check(q: torch.Tensor, s: torch.Tensor, q_ref: np.ndarray, s_ref: np.ndarray, label: str) -> None:
    qb = _bytes(q).reshape(q_ref.shape)
    if not np.array_equal(qb, q_ref):
        bad = np.argwhere(qb != q_ref)
        i = tuple(bad[0])
        raise AssertionError(f"{label}: {len(bad)} fp8 bytes differ, first at {i}: gpu {qb[i]:#x} "
                             f"oracle {q_ref[i]:#x}")
    sg, sr = _scale_bits(s), np.asarray(s_ref, np.float32).reshape(-1).view(np.uint32)
    assert sg.shape == sr.shape, (label, sg.shape, sr.shape)
    if not np.array_equal(sg, sr):
        bad = np.nonzero(sg != sr)[0]
        raise AssertionError(f"{label}: {len(bad)} scales differ, first at {bad[0]}: gpu {sg[bad[0]]:#x} "
                             f"oracle {sr[bad[0]]:#x}")


@pytest.mark.parametrize("which", ["x", "dy"])
def test_layer_dual_quant_full_size(dev, config5_host, which):
    """The layer's dual launch on X / dY: 1 x 128 and the transposed 128 x 1."""
    x_h, _, dy_h = config5_host
    t = x_h if which == "x" else dy_h
    print(f"config5 dual quant {which} {tuple(t.shape)}", flush=True)
    q_row, s_row, q_col, s_col = torch.ops.pcamd.quant_block_dual(t[None].to(dev), 128, E4M3, 1e-12)
    torch.cuda.synchronize()
    # the 128 x 1 operand is a transposed view of a [1, N, M] buffer (rows padded to 16 bytes)
    assert q_col.shape == (1, *t.shape) and q_col.stride(-2) == 1
    q1, s1 = O.quant_block(t, 1, 128, threads=16)
    _check(q_row[0], s_row[0], q1, s1, f"{which} 1x128")
    del q1, s1
    q2, s2 = O.quant_block(t, 128, 1, threads=16)
    _check(q_col[0], s_col[0], q2, s2, f"{which} 128x1 (transposed buffer)")


def test_dual_quant_plain_layout_full_size(dev, config5_host):
    """dY's dual launch with the 128 x 1 result in the input's own layout."""
    _, _, dy_h = config5_host
    print("config5 dual quant dy, plain 128x1 layout", flush=True)
    r_row, r_col = hip_per_block_quant_dual(dy_h.to(dev), block=128, col_transposed=False)
    q2, s2 = O.quant_block(dy_h, 128, 1, threads=16)
    _check(r_col.tensor, r_col.dequant_scale, q2, s2, "dy 128x1 (plain)")
    del q2, s2
    q1, s1 = O.quant_block(dy_h, 1, 128, threads=16)
    _check(r_row.tensor, r_row.dequant_scale, q1, s1, "dy 1x128 (plain launch)")


def test_layer_weight_quant_full_size(dev, config5_host):
    """The layer's 128 x 128 launch on W [14336, 4096]."""
    _, w_h, _ = config5_host
    print("config5 weight quant 128x128", flush=True)
    q, s = torch.ops.pcamd.quant_block(w_h[None].to(dev), 128, 128, E4M3, 1e-12)
    assert s.shape == (1, 14336 // 128, 4096 // 128)
    q_ref, s_ref = O.quant_block(w_h, 128, 128, threads=16)
    _check(q[0], s[0], q_ref, s_ref, "W 128x128")
