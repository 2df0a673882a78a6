"""Generate the committed golden vectors in tests/golden/.

The reference (xuOAO/practice_cuda) ships no golden data, and its tests draw
inputs from the CUDA RNG, which cannot be reproduced on a CPU. These
fixtures are therefore produced by an independent eager-PyTorch CPU
restatement of the reference kernels' arithmetic: torch's own fp8 cast
(round to nearest even), true fp32 division written as torch.div for the
Triton kernels, and the reference's literal `python_float / tensor` for the
per-tensor wrapper. The C oracle (oracle/fp8_oracle.c) and the HIP kernels
are both checked against them.

Formulas followed (reference paths):
  per-block   fp8_training/fp8_bench/kernels/quant/per_block.py:35-48
  per-channel fp8_training/fp8_bench/kernels/quant/per_channel.py:136-267
  per-tensor  fp8_training/fp8_bench/impls/triton_per_tensor.py:40-44
  block BMM   fp8_training/fp8_bench/kernels/bmm/per_block.py:99-137

    python tests/golden/make_golden.py      # rewrites quant_golden.npz etc.
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
FP8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _raw(x: torch.Tensor) -> np.ndarray:
    if x.dtype in (torch.bfloat16, torch.float16):
        return x.contiguous().view(torch.int16).numpy().view(np.uint16)
    return x.contiguous().numpy()


def _bits(q: torch.Tensor) -> np.ndarray:
    return q.contiguous().view(torch.uint8).numpy()


def block_quant(x, bm, bn, fmt, eps=1e-12):
    fp8 = FP8[fmt]
    fmax = torch.finfo(fp8).max
    xf = x.float()
    squeeze = xf.ndim == 2
    if squeeze:
        xf = xf.unsqueeze(0)
    b, m, n = xf.shape
    mb, nb = -(-m // bm), -(-n // bn)
    pad = torch.zeros(b, mb * bm, nb * bn)  # masked loads read 0.0 (per_block.py:40)
    pad[:, :m, :n] = xf
    amax = pad.reshape(b, mb, bm, nb, bn).abs().amax(dim=(2, 4))
    safe = torch.maximum(amax, torch.tensor(eps, dtype=torch.float32))
    qs = torch.div(torch.tensor(fmax, dtype=torch.float32), safe)  # fp8_max / safe
    ds = torch.div(torch.tensor(1.0, dtype=torch.float32), qs)     # 1.0 / qs
    qs_full = qs.repeat_interleave(bm, 1).repeat_interleave(bn, 2)[:, :m, :n]
    y = torch.clamp(xf * qs_full, -fmax, fmax).to(fp8)
    if squeeze:
        return y[0], ds[0]
    return y, ds


def channel_quant(x, axis, fmt, eps=1e-12):
    fp8 = FP8[fmt]
    fmax = torch.finfo(fp8).max
    xf = x.float()
    red = -1 if axis == -2 else -2
    amax = xf.abs().amax(dim=red)
    safe = torch.maximum(amax, torch.tensor(eps, dtype=torch.float32))
    qs = torch.div(torch.tensor(fmax, dtype=torch.float32), safe)
    ds = torch.div(safe, torch.tensor(fmax, dtype=torch.float32))
    y = torch.clamp(xf * qs.unsqueeze(red), -fmax, fmax).to(fp8)
    return y, ds


def tensor_quant(x, fmt, eps=1e-12):
    fp8 = FP8[fmt]
    fmax = torch.finfo(fp8).max
    x_min, x_max = x.aminmax()
    max_abs = torch.maximum(x_min.abs(), x_max.abs()).float().clamp(min=eps)
    qs = fmax / max_abs            # literal reference expression (triton_per_tensor.py:43)
    ds = qs.reciprocal()
    y = torch.clamp(x.float() * qs, -fmax, fmax).to(fp8)
    return y, ds


def _inputs():
    g = torch.Generator().manual_seed(1234)

    def randn(*shape, scale=1.0):
        return torch.randn(*shape, generator=g) * scale

    cases = []
    # 1x128 groups, bf16, with outliers, a zero group, -0.0 and sub-fp8-subnormal values
    x = randn(2, 5, 384)
    x[torch.rand(2, 5, 384, generator=g) < 0.01] *= 50.0
    x[0, 1, 128:256] = 0.0
    x[0, 1, 130] = -0.0
    x[1, 2, 0:128] = randn(128) * 1e-4
    x[1, 2, 5] = 1.0
    cases.append(("block_1x128_bf16", x.bfloat16(), dict(kind="block", bm=1, bn=128, fmt="e4m3")))
    # 128x128 with per-block magnitudes and ragged edge blocks
    w = randn(200, 300, scale=0.02)
    mult = torch.exp(torch.empty(2, 3).uniform_(np.log(0.1), np.log(10.0), generator=g))
    w = w * mult.repeat_interleave(128, 0).repeat_interleave(128, 1)[:200, :300]
    cases.append(("block_128x128_bf16", w.bfloat16(), dict(kind="block", bm=128, bn=128, fmt="e4m3")))
    # 128x1 column groups (wgrad operand layout)
    cases.append(("block_128x1_bf16", randn(256, 40).bfloat16(), dict(kind="block", bm=128, bn=1, fmt="e4m3")))
    # generic block shape, fp32 input, ragged
    cases.append(("block_4x32_f32", randn(37, 70, scale=3.0), dict(kind="block", bm=4, bn=32, fmt="e4m3")))
    # e5m2 from fp16
    cases.append(("block_1x128_f16_e5m2", randn(3, 256).half(), dict(kind="block", bm=1, bn=128, fmt="e5m2")))
    # per-channel rows / columns
    cases.append(("channel_rows_bf16", randn(2, 33, 200, scale=0.02).bfloat16(),
                  dict(kind="channel", axis=-2, fmt="e4m3")))
    cases.append(("channel_cols_f32", randn(50, 70), dict(kind="channel", axis=-1, fmt="e4m3")))
    cases.append(("channel_rows_bf16_e5m2", randn(40, 96).bfloat16(), dict(kind="channel", axis=-2, fmt="e5m2")))
    # per-tensor
    cases.append(("tensor_bf16", randn(3, 17, 33).bfloat16(), dict(kind="tensor", fmt="e4m3")))
    cases.append(("tensor_f32", randn(64, 64, scale=7.0), dict(kind="tensor", fmt="e4m3")))
    return cases


def make_quant_golden():
    arrays, meta = {}, {}
    for name, x, p in _inputs():
        if p["kind"] == "block":
            y, s = block_quant(x, p["bm"], p["bn"], p["fmt"])
        elif p["kind"] == "channel":
            y, s = channel_quant(x, p["axis"], p["fmt"])
        else:
            y, s = tensor_quant(x, p["fmt"])
        dt = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[x.dtype]
        arrays[f"{name}__x"] = _raw(x)
        arrays[f"{name}__q"] = _bits(y)
        arrays[f"{name}__scale"] = s.numpy().astype(np.float32).reshape(-1 if s.ndim == 0 else s.shape)
        meta[name] = dict(p, dtype=dt, shape=list(x.shape))
    np.savez_compressed(os.path.join(HERE, "quant_golden.npz"), **arrays)
    with open(os.path.join(HERE, "quant_golden.json"), "w") as fh:
        json.dump(meta, fh, indent=1, sort_keys=True)


def make_bmm_golden():
    """Block-scaled BMM (1x128 A, 128x128 B, K = 256 -> two quant-K blocks)
    plus bias: expected fp32 output of the fp64 product of dequantized
    operands (bench_bmm.py:414-419 computes this reference in fp32)."""
    g = torch.Generator().manual_seed(99)
    a = torch.randn(2, 33, 256, generator=g).bfloat16()
    b = torch.randn(2, 256, 40, generator=g).bfloat16()
    bias = torch.randn(2, 33, 40, generator=g).bfloat16()
    qa, sa = block_quant(a, 1, 128, "e4m3")
    qb, sb = block_quant(b, 128, 128, "e4m3")
    da = qa.double() * sa.double().repeat_interleave(128, 2)[:, :, :256]
    db = qb.double() * sb.double().repeat_interleave(128, 1).repeat_interleave(128, 2)[:, :256, :40]
    ref = torch.bmm(da, db) + bias.double()
    np.savez_compressed(
        os.path.join(HERE, "bmm_golden.npz"),
        a=_raw(a), b=_raw(b), bias=_raw(bias), qa=_bits(qa), sa=sa.numpy(), qb=_bits(qb),
        sb=sb.numpy(), expected=ref.numpy().astype(np.float32))


if __name__ == "__main__":
    make_quant_golden()
    make_bmm_golden()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith((".npz", ".json"))))
