"""Seeded random shapes through every quantizer entry point, bit-exact against
the oracle: ragged and aligned sizes, batches, all three input dtypes, both
fp8 formats, power-of-two blocks, both channel axes, per-tensor, and the dual
quantizer with either 128x1 layout; then the registered BMMs and the fused
activation-quant BMM at the BMM bar. Each case prints its parameters first."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant, hip_per_block_quant_dual
from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_quant
from practice_cuda_amd.impls.hip_per_tensor import hip_per_tensor_quant

pytestmark = pytest.mark.gpu
FMT = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _bits(t):
    return t.contiguous().view(torch.uint8).cpu().numpy()


def _sbits(t):
    return t.detach().float().cpu().numpy().astype(np.float32).reshape(-1).view(np.uint32)


def _same(res, q_ref, s_ref, label):
    assert np.array_equal(_bits(res.tensor), q_ref), f"{label}: fp8 bytes differ"
    assert np.array_equal(_sbits(res.dequant_scale), np.asarray(s_ref, np.float32).reshape(-1).view(np.uint32)), \
        f"{label}: scales differ"


def _case(i):
    rng = np.random.default_rng(1000 + i)
    batch = int(rng.choice([1, 1, 2, 3]))
    m = int(rng.choice([1, 7, 64, 128, 130, 256, 300, 384, 513]))
    n = int(rng.choice([8, 24, 128, 136, 256, 520, 1024, 7168, 70]))
    dtype = str(rng.choice(["bf16", "bf16", "f16", "f32"]))
    fmt = str(rng.choice(["e4m3", "e4m3", "e5m2"]))
    op = str(rng.choice(["block", "block", "channel", "tensor", "dual"]))
    bm = int(rng.choice([1, 1, 16, 128, 2, 64]))
    bn = int(rng.choice([128, 128, 1, 64, 8, 256]))
    axis = int(rng.choice([-1, -2]))
    col_t = bool(rng.integers(0, 2))
    return dict(batch=batch, m=m, n=n, dtype=dtype, fmt=fmt, op=op, bm=bm, bn=bn, axis=axis, col_t=col_t)


@pytest.mark.parametrize("i", range(48))
def test_random_quantizer_case(dev, i):
    c = _case(i)
    print(f"fuzz {i}: {c}", flush=True)
    g = torch.Generator().manual_seed(i)
    shape = (c["batch"], c["m"], c["n"]) if c["batch"] > 1 else (c["m"], c["n"])
    x = torch.randn(*shape, generator=g) * float(np.exp(np.random.default_rng(i).uniform(-6, 3)))
    x.view(-1)[:: max(1, x.numel() // 7)] *= 40.0          # a few outliers
    x = x.to(DT[c["dtype"]])
    xd, f8 = x.to(dev), FMT[c["fmt"]]
    if c["op"] == "block":
        r = hip_per_block_quant(xd, block_m=c["bm"], block_n=c["bn"], fp8_dtype=f8)
        q, s = O.quant_block(x, c["bm"], c["bn"], c["fmt"], threads=4)
        _same(r, q, s, f"block {c['bm']}x{c['bn']}")
    elif c["op"] == "channel":
        r = hip_per_channel_quant(xd, channel_axis=c["axis"], fp8_dtype=f8)
        q, s = O.quant_channel(x, c["axis"], c["fmt"], threads=4)
        _same(r, q, s, f"channel {c['axis']}")
    elif c["op"] == "tensor":
        r = hip_per_tensor_quant(xd, fp8_dtype=f8)
        q, ds, _ = O.quant_tensor(x, c["fmt"])
        assert np.array_equal(_bits(r.tensor), q), "tensor: fp8 bytes differ"
        assert np.array_equal(_sbits(r.dequant_scale), np.asarray([ds], np.float32).view(np.uint32))
    else:
        r_row, r_col = hip_per_block_quant_dual(xd, block=128, fp8_dtype=f8, col_transposed=c["col_t"])
        q1, s1 = O.quant_block(x, 1, 128, c["fmt"], threads=4)
        q2, s2 = O.quant_block(x, 128, 1, c["fmt"], threads=4)
        _same(r_row, q1, s1, "dual 1x128")
        _same(r_col, q2, s2, "dual 128x1")


def _bmm_case(i):
    from test_gpu_bmm import LAYOUTS, SCHEMES
    rng = np.random.default_rng(5000 + i)
    c = dict(scheme=str(rng.choice(SCHEMES)), layout=str(rng.choice(LAYOUTS)), b=int(rng.choice([1, 2])),
             m=int(rng.choice([1, 33, 128, 200, 256, 384, 520, 640])),
             n=int(rng.choice([16, 47, 128, 256, 300, 512, 640])),
             k=int(rng.choice([128, 256, 384, 512, 65, 200])))
    if c["layout"].startswith("a_m") and c["m"] == 1:
        # a single row is contiguous along K as well: the reference's layout check
        # (fp8_bench/impls/triton_per_block.py:45-53) reads it as k-major and rejects it here
        c["m"] = 2
    return c


@pytest.mark.parametrize("i", range(24))
def test_random_bmm_case(dev, i):
    """Seeded random shapes, schemes and layouts through the registered BMMs,
    within max-abs-rel 1e-2 of the fp64 product of the dequantized operands."""
    from test_gpu_bmm import TOL, rand, run_registered
    c = _bmm_case(i)
    print(f"bmm fuzz {i}: {c}", flush=True)
    out, ref = run_registered(f"{c['scheme']}_{c['layout']}", rand((c["b"], c["m"], c["k"]), 100 + i),
                              rand((c["b"], c["k"], c["n"]), 200 + i), dev)
    assert out.shape == (c["b"], c["m"], c["n"])
    err = O.max_abs_rel(out.float().cpu().numpy(), ref)
    assert err <= TOL, f"max_abs_rel {err}"


def _fused_case(i):
    rng = np.random.default_rng(3000 + i)
    return {
        "b": int(rng.choice([1, 1, 2, 3])),
        "m": int(rng.choice([1, 17, 128, 129, 300, 1000])),
        "n": int(rng.choice([16, 48, 64, 96, 128, 144, 192, 240, 256, 272, 384])),
        "k": int(rng.choice([128, 256, 384, 512, 768, 1024, 1536, 2048])),
        "dtype": str(rng.choice(["bf16", "f16"])),
        "fmt": str(rng.choice(["e4m3", "e5m2"])),
        "qbn": int(rng.choice([128, 128, 256, 32, 1])),
        "b_k": bool(rng.integers(2)),
        "wq": bool(rng.integers(2)),
        "always": bool(rng.integers(2)),
        # drawn last, so the draws above (and the cases they give) are unchanged
        "epi": str(rng.choice(["none", "none", "bias_gelu", "bias_f32", "out_f32_gelu"])),
    }


@pytest.mark.parametrize("i", range(24))
def test_random_fused_quant_bmm_case(dev, i):
    """Seeded random shapes through hip_per_block_bmm_quant_a, in and around
    the streaming kernel's envelope (N <= 256, K % 256 == 0, quant-N blocks
    >= 128): the quantized A is the 1 x 128 quantizer's bit for bit, the
    product equals quantize-then-multiply to fp32 rounding and is within
    max-abs-rel 1e-2 of the fp64 product of the dequantized operands. The
    epilogue draw adds a bf16 bias with GELU, an fp32 bias, or GELU into an
    fp32 output; a 16-bit output with an epilogue is held to one unit in the
    last place of quantize-then-multiply."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_bmm, hip_per_block_bmm_quant_a
    c = _fused_case(i)
    print(f"fused quant bmm fuzz {i}: {c}", flush=True)
    g = torch.Generator().manual_seed(4000 + i)
    x = (torch.randn(c["b"], c["m"], c["k"], generator=g) * 2).to(DT[c["dtype"]]).to(dev)
    w = torch.randn(c["b"], c["k"], c["n"], generator=g) * 0.05
    if c["b_k"]:
        w = w.transpose(-1, -2).contiguous().transpose(-1, -2)
    qb = hip_per_block_quant(w.bfloat16().to(dev), block_m=128, block_n=c["qbn"], fp8_dtype=FMT[c["fmt"]])
    bias = None
    if c["epi"] in ("bias_gelu", "bias_f32"):
        bias = torch.randn(c["b"], c["m"], c["n"], generator=g).to(
            torch.bfloat16 if c["epi"] == "bias_gelu" else torch.float32).to(dev)
    epi = {"bias": bias, "activation": "gelu" if c["epi"] in ("bias_gelu", "out_f32_gelu") else "none",
           "out_dtype": torch.float32 if c["epi"] == "out_f32_gelu" else torch.bfloat16}
    res = hip_per_block_bmm_quant_a(x, qb, return_quant=c["wq"], always_fused=c["always"], **epi)
    out, qa = res if c["wq"] else (res, None)
    ref_q = hip_per_block_quant(x, block_m=1, block_n=128, fp8_dtype=FMT[c["fmt"]])
    unfused = hip_per_block_bmm(ref_q, qb, **epi)
    torch.cuda.synchronize()
    if qa is not None:
        assert torch.equal(qa.tensor.view(torch.uint8), ref_q.tensor.view(torch.uint8))
        assert torch.equal(qa.dequant_scale.view(torch.int32), ref_q.dequant_scale.view(torch.int32))
    assert out.dtype == epi["out_dtype"]
    scale = unfused.float().abs().max().item()
    tol = 8e-3 if c["epi"] in ("bias_gelu", "bias_f32") else 1e-6
    assert (out.float() - unfused.float()).abs().max().item() <= tol * scale + 1e-30
    ref = O.bmm_reference(ref_q.dequantize().double().cpu().numpy(), qb.dequantize().double().cpu().numpy(),
                          None if bias is None else bias.double().cpu().numpy(), epi["activation"])
    assert O.max_abs_rel(out.float().cpu().numpy(), ref) <= 1e-2
