"""Pin the CPU oracle (oracle/) before trusting it as the parity checker.

Parity status of each oracle function and the check that pins it:

  encode e4m3fn / e5m2  PINNED  exhaustive against torch's CPU cast over every
                                fp32 bit pattern with |x| <= fp8 max, both signs
  decode_fp8            PINNED  all 256 codes against torch's fp8 -> fp32 cast,
                                and encode(decode(c)) == c
  quant_block           PINNED  golden vectors from an independent torch-eager
                                restatement; closed forms (zero block, power-of-two
                                amax); the reference tests' known answers
                                (outliers -> +-448, range); brute-force block
                                indexing on tiny ragged / strided / 3D inputs
  quant_channel         PINNED  golden vectors; closed form ds = s / fp8_max that
                                differs from the block formula on chosen amaxes
  quant_tensor          PINNED  golden vectors; reciprocal-multiply scale
                                (torch `float / tensor`) distinguished from true
                                division on chosen amaxes; amax/448 within 1e-5
                                (reference fp8_quant_test.py:94-103)
  dequant_* / bmm_ref   PINNED  against registry.QuantResult.dequantize (torch)
                                and a float64 triple-loop on tiny shapes, and
                                the BMM golden vector
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
F32 = np.float32


def f32(v):
    return np.float32(v)


# ---------------------------------------------------------------------------
# encoder / decoder
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("fmt,tdt,maxbits", [("e4m3", torch.float8_e4m3fn, 0x43E00000),
                                             ("e5m2", torch.float8_e5m2, 0x47600000)])
def test_encode_exhaustive_vs_torch(fmt, tdt, maxbits):
    step = 1 << 24
    for lo in range(0, maxbits + 1, step):
        u = np.arange(lo, min(lo + step, maxbits + 1), dtype=np.uint32)
        f = u.view(np.float32)
        for sign in (F32(1.0), F32(-1.0)):
            v = f * sign
            ours = O.encode(v, fmt)
            ref = torch.from_numpy(v).to(tdt).view(torch.uint8).numpy()
            bad = np.nonzero(ours != ref)[0]
            assert bad.size == 0, f"{fmt}: {v[bad[0]]!r} -> {ours[bad[0]]:#x}, torch {ref[bad[0]]:#x}"


@pytest.mark.parametrize("fmt,tdt", [("e4m3", torch.float8_e4m3fn), ("e5m2", torch.float8_e5m2)])
def test_decode_all_codes(fmt, tdt):
    codes = np.arange(256, dtype=np.uint8)
    ours = O.decode(codes, fmt)
    ref = torch.from_numpy(codes).view(tdt).float().numpy()
    finite = np.isfinite(ref)
    assert np.array_equal(ours[finite], ref[finite])
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    back = O.encode(ours[finite], fmt)
    assert np.array_equal(back, codes[finite])


def test_encode_known_answers():
    # largest finite, smallest normal / subnormal, ties to even, signed zero
    vals = np.array([448.0, -448.0, 2.0**-6, 2.0**-9, 1.5 * 2.0**-9, 2.5 * 2.0**-9,
                     0.0, -0.0, 1.0625, 1.1875], dtype=np.float32)
    assert list(O.encode(vals, "e4m3")) == [0x7E, 0xFE, 0x08, 0x01, 0x02, 0x02, 0x00, 0x80,
                                            0x38, 0x3A]
    assert list(O.encode(np.array([57344.0, 2.0**-14, 2.0**-16], np.float32), "e5m2")) == [
        0x7B, 0x04, 0x01]


# ---------------------------------------------------------------------------
# golden vectors (independent torch-eager restatement, tests/golden/make_golden.py)
# ---------------------------------------------------------------------------
def _golden_cases():
    with open(os.path.join(GOLDEN, "quant_golden.json")) as fh:
        return json.load(fh)


def golden_input(data, name, meta):
    x = data[f"{name}__x"]
    if meta["dtype"] == "bf16":
        return torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    if meta["dtype"] == "f16":
        return torch.from_numpy(x.view(np.float16))
    return torch.from_numpy(x)


def oracle_quant(x, meta):
    if meta["kind"] == "block":
        return O.quant_block(x, meta["bm"], meta["bn"], meta["fmt"])
    if meta["kind"] == "channel":
        return O.quant_channel(x, meta["axis"], meta["fmt"])
    q, ds, _ = O.quant_tensor(x, meta["fmt"])
    return q, np.float32(ds)


@pytest.mark.parametrize("name", sorted(_golden_cases()))
def test_oracle_matches_golden(name):
    meta = _golden_cases()[name]
    data = np.load(os.path.join(GOLDEN, "quant_golden.npz"))
    q, s = oracle_quant(golden_input(data, name, meta), meta)
    assert np.array_equal(q, data[f"{name}__q"])
    assert np.array_equal(np.asarray(s, np.float32).reshape(-1).view(np.uint32),
                          data[f"{name}__scale"].reshape(-1).view(np.uint32))


# ---------------------------------------------------------------------------
# closed forms and the reference tests' known answers
# ---------------------------------------------------------------------------
def test_zero_block_scale_and_signed_zero():
    x = np.zeros((2, 256), np.float32)
    x[1, 3] = -0.0
    q, s = O.quant_block(x, 1, 128)
    expect = f32(1.0) / (f32(448.0) / f32(1e-12))
    assert np.all(s.view(np.uint32) == np.float32(expect).view(np.uint32))
    assert q[1, 3] == 0x80 and np.count_nonzero(q) == 1
    qc, sc = O.quant_channel(x, -2)
    assert np.all(sc == f32(1e-12) / f32(448.0))


def test_power_of_two_amax():
    x = np.full((1, 128), 0.5, np.float32)
    x[0, 7] = -2.0
    q, s = O.quant_block(x, 1, 128)
    assert s[0, 0] == f32(1.0) / f32(224.0)          # qs = 448 / 2 = 224 exactly
    assert O.decode(q, "e4m3")[0, 7] == -448.0
    assert O.decode(q, "e4m3")[0, 0] == 112.0


def test_outliers_saturate_to_fp8_max():
    # reference kernels/fp8_bmm/test/fp8_quant_test.py:134-145
    g = np.random.default_rng(0)
    x = g.standard_normal((64, 64)).astype(np.float32)
    x[0, 0], x[1, 1] = 1e6, -1e6
    q, _, _ = O.quant_tensor(x)
    assert q[0, 0] == 0x7E and q[1, 1] == 0xFE
    qb, _ = O.quant_block(x, 1, 32)
    assert qb[0, 0] == 0x7E and qb[1, 1] == 0xFE


@pytest.mark.parametrize("fmt,fmax", [("e4m3", 448.0), ("e5m2", 57344.0)])
def test_output_range(fmt, fmax):
    # reference fp8_quant_test.py:126-131 (inputs x1000)
    x = np.random.default_rng(1).standard_normal((3, 50, 70)).astype(np.float32) * 1000
    for q in (O.quant_block(x, 1, 128, fmt)[0], O.quant_channel(x, -1, fmt)[0],
              O.quant_tensor(x, fmt)[0]):
        v = O.decode(q, fmt)
        assert np.all(np.isfinite(v)) and np.abs(v).max() <= fmax


def test_reduced_fp8_max_clamps_before_rounding():
    """With fp8_max F just below the 240/256 rounding midpoint (248), an amax
    s whose product fl(s * fl(F / s)) lands above F must encode as 240 (clamp
    to F, then round) and not as 256 (round the unclamped product)."""
    F = np.nextafter(f32(248.0), f32(0.0))
    s = _find_amax(lambda v: v * (F / v) > F)
    x = np.zeros((2, 128), np.float32)
    x[0, 0], x[1, 5] = s, -s
    prod = s * (F / s)
    assert O.encode(np.array([prod], np.float32))[0] == 0x78       # 256 unclamped
    for q in (O.quant_block(x, 1, 128, fp8_max=float(F))[0],
              O.quant_channel(x, -2, fp8_max=float(F))[0]):
        assert q[0, 0] == 0x77 and q[1, 5] == 0xF7                  # +-240
    # F = 100 is the 96/104 midpoint and ties to 96: after the clamp every
    # code decodes to at most 96, and the amax element reaches it
    xr = np.random.default_rng(5).standard_normal((40, 300)).astype(np.float32)
    for q in (O.quant_block(xr, 1, 128, fp8_max=100.0)[0], O.quant_block(xr, 128, 128, fp8_max=100.0)[0],
              O.quant_channel(xr, -1, fp8_max=100.0)[0]):
        v = np.abs(O.decode(q))
        assert v.max() == 96.0


def test_reciprocal_factor_closed_form():
    # reference fp8_quant_test.py:94-103: dequant scale == amax / 448 (rtol 1e-5)
    x = np.random.default_rng(2).standard_normal((32, 2048)).astype(np.float32)
    _, ds, _ = O.quant_tensor(x)
    assert np.isclose(ds, np.abs(x).max() / 448.0, rtol=1e-5, atol=1e-7)


def _find_amax(pred, start=1.0):
    """Smallest float32 >= start (walking ulps) satisfying pred(s)."""
    s = f32(start)
    for _ in range(100000):
        if pred(s):
            return s
        s = np.nextafter(s, f32(np.inf))
    raise AssertionError("no witness found")


def test_scale_formulas_distinguish_block_channel_tensor():
    fmax = f32(448.0)
    # an amax where 1/(448/s) != s/448 separates the block and channel formulas
    s1 = _find_amax(lambda s: f32(1.0) / (fmax / s) != s / fmax)
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = s1
    _, sb = O.quant_block(x, 1, 128)
    _, sc = O.quant_channel(x, -2)
    assert sb[0, 0] == f32(1.0) / (fmax / s1) and sc[0] == s1 / fmax and sb[0, 0] != sc[0]
    # an amax where (1/s)*448 != 448/s separates the per-tensor wrapper
    s2 = _find_amax(lambda s: (f32(1.0) / s) * fmax != fmax / s)
    x[0, 0] = s2
    _, ds, qs = O.quant_tensor(x)
    assert qs == (f32(1.0) / s2) * fmax and qs != fmax / s2
    assert ds == f32(1.0) / qs


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
def test_torchao_tensorwise_form(fmt):
    """scale_dt F64: torchao's amax_to_scale + cast (the reference layer's
    modules/float8/float8_utils.py:45-48, :134-137 and
    float8_training_tensor.py:153-154) evaluated by torch's own CPU ops: the
    fp64 division, its rounding to fp32 and torch's fp8 cast. The amax is one
    where fp32(448 / fp64(amax)) differs from the fp32 form (1 / amax) * 448,
    so dropping the fp64 step fails; a tiny tensor takes the eps floor."""
    f8 = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}[fmt]
    fmax = torch.finfo(f8).max
    g = torch.Generator().manual_seed(11)
    for amax_v in (0.5234375, 3.0e-13, 0.0):
        x = (torch.rand(3, 40, 72, generator=g) * 2 - 1) * 0.5
        if amax_v < 1e-3:
            x = x * amax_v
        x = x.bfloat16()
        x[1, 7, 5] = -amax_v
        amax = x.abs().max()
        s = (fmax / torch.clamp(amax.to(torch.float64), min=1e-12)).to(torch.float32)
        q_ref = (x.to(torch.float32) * s).clamp(-fmax, fmax).to(f8).view(torch.uint8).numpy()
        q, ds, qs = O.quant_tensor(x, fmt, scale_dt=O.F64)
        assert np.float32(qs) == np.float32(s.item()), amax_v
        assert np.float32(ds) == np.float32(s.reciprocal().item())
        assert np.array_equal(q, q_ref)
        if amax_v == 0.5234375:
            _, _, qs32 = O.quant_tensor(x, fmt)
            assert qs32 != qs


def test_block_structure_brute_force():
    """Tiny ragged / 3-D / strided inputs: per-block amax found by a Python
    loop over the block's elements, scale by the closed form, bytes by the
    (separately pinned) encoder."""
    g = np.random.default_rng(3)
    base = g.standard_normal((2, 9, 21)).astype(np.float32) * g.uniform(0.1, 10, (2, 9, 21)).astype(np.float32)
    for x in (base, base.transpose(0, 2, 1)):  # second one is strided (m-major)
        for bm, bn in ((1, 8), (4, 4), (8, 16), (2, 1)):
            q, s = O.quant_block(x, bm, bn)
            b, m, n = x.shape
            for bi in range(b):
                for i in range(-(-m // bm)):
                    for j in range(-(-n // bn)):
                        blk = x[bi, i * bm:(i + 1) * bm, j * bn:(j + 1) * bn]
                        qs = f32(448.0) / max(f32(np.abs(blk).max()), f32(1e-12))
                        assert s[bi, i, j] == f32(1.0) / qs
                        v = np.clip(blk * qs, -448, 448).astype(np.float32)
                        assert np.array_equal(q[bi, i * bm:(i + 1) * bm, j * bn:(j + 1) * bn],
                                              O.encode(v))


def test_channel_axes_brute_force():
    x = np.random.default_rng(4).standard_normal((2, 7, 11)).astype(np.float32)
    for axis, red in ((-2, 2), (-1, 1)):
        q, s = O.quant_channel(x, axis)
        amax = np.abs(x).max(axis=red)
        assert np.array_equal(s, amax / f32(448.0))
        qs = f32(448.0) / amax
        v = np.clip(x * np.expand_dims(qs, red), -448, 448).astype(np.float32)
        assert np.array_equal(q, O.encode(v))


# ---------------------------------------------------------------------------
# dequantize and BMM reference
# ---------------------------------------------------------------------------
def test_dequant_matches_registry():
    from practice_cuda_amd.registry import QuantResult

    x = np.random.default_rng(5).standard_normal((2, 130, 260)).astype(np.float32)
    q, s = O.quant_block(x, 128, 128)
    qt = torch.from_numpy(q).view(torch.float8_e4m3fn)
    r = QuantResult(qt, torch.from_numpy(s), "oracle", "block", {"block_m": 128, "block_n": 128})
    # fp8 x fp32 is exact in fp64, so the fp32 product is the fp64 one rounded
    assert np.array_equal(r.dequantize().numpy(), O.dequant_block(q, s, 128, 128).astype(np.float32))
    q, s = O.quant_channel(x, -1)
    r = QuantResult(torch.from_numpy(q).view(torch.float8_e4m3fn), torch.from_numpy(s), "oracle",
                    "channel", {"channel_axis": -1})
    assert np.array_equal(r.dequantize().numpy(), O.dequant_channel(q, s, -1).astype(np.float32))


def test_bmm_reference_triple_loop():
    g = np.random.default_rng(6)
    a = g.standard_normal((2, 3, 5))
    b = g.standard_normal((2, 5, 4))
    bias = g.standard_normal((2, 3, 4))
    out = O.bmm_reference(a, b, bias, activation="gelu")
    from math import erf, sqrt
    for bi in range(2):
        for i in range(3):
            for j in range(4):
                acc = sum(a[bi, i, kk] * b[bi, kk, j] for kk in range(5)) + bias[bi, i, j]
                assert out[bi, i, j] == pytest.approx(0.5 * acc * (1 + erf(acc / sqrt(2))), rel=1e-12)


def test_bmm_golden():
    d = np.load(os.path.join(GOLDEN, "bmm_golden.npz"))
    a = torch.from_numpy(d["a"].view(np.int16)).view(torch.bfloat16)
    b = torch.from_numpy(d["b"].view(np.int16)).view(torch.bfloat16)
    qa, sa = O.quant_block(a, 1, 128)
    qb, sb = O.quant_block(b, 128, 128)
    assert np.array_equal(qa, d["qa"]) and np.array_equal(qb, d["qb"])
    bias = torch.from_numpy(d["bias"].view(np.int16)).view(torch.bfloat16).float().numpy()
    ref = O.bmm_reference(O.dequant_block(qa, sa, 1, 128), O.dequant_block(qb, sb, 128, 128), bias)
    assert O.max_abs_rel(ref, d["expected"]) < 1e-6


def test_eps_zero_tiny_amax_saturates():
    """eps = 0 and a group whose amax is below fp8_max / FLT_MAX: the quant
    scale fp8_max / amax overflows to inf, every x * qs is +-inf and the clamp
    of the reference (kernels/quant/per_block.py:46-48) maps it to +-fp8_max;
    the block dequant scale 1 / qs is 0 and the channel one amax / fp8_max
    (per_channel.py:159-161) a subnormal."""
    x = np.full((2, 128), 1.5e-38, np.float32)
    x[:, 1::2] *= -1.0
    assert not np.isfinite(f32(448.0) / f32(1.5e-38))
    for fmt, pos, neg in (("e4m3", 0x7E, 0xFE), ("e5m2", 0x7B, 0xFB)):
        q, s = O.quant_block(x, 1, 128, fmt=fmt, eps=0.0)
        assert np.all(q[:, 0::2] == pos) and np.all(q[:, 1::2] == neg), fmt
        assert np.all(s == 0.0)
        q, s = O.quant_channel(x, -2, fmt=fmt, eps=0.0)
        assert np.all(q[:, 0::2] == pos) and np.all(q[:, 1::2] == neg), fmt
        fmax = 448.0 if fmt == "e4m3" else 57344.0
        assert np.all(s == f32(1.5e-38) / f32(fmax)) and 0.0 < s[0] < np.finfo(np.float32).tiny
    # a group of ordinary values beside it keeps finite, exact scales
    q, s = O.quant_block(np.array([[1.0] * 128], np.float32), 1, 128, eps=0.0)
    assert s[0, 0] == f32(1.0) / (f32(448.0) / f32(1.0)) and q[0, 0] == 0x7E
