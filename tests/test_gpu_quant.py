"""GPU parity of the HIP quantizers against the CPU oracle: fp8 bytes and fp32
scale bit patterns must be identical (the north_star's bit-exact bar).

Covers every kernel path of csrc/quant.hip (row groups, tiles, column groups,
register-resident rows, column strips, generic strided, per-tensor), the
BASELINE full-size configs 1-3, the golden vectors, and the edge cases of the
reference tests (zeros, outliers, ragged shapes, 3D batches, e5m2).
"""
from __future__ import annotations

import ctypes
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O
from practice_cuda_amd import _lib
from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant
from practice_cuda_amd.impls.hip_per_channel import hip_per_channel_quant
from practice_cuda_amd.impls.hip_per_tensor import hip_per_tensor_quant, quant_tensor_raw

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
FMT = {"e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}
DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def qbits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).cpu().numpy()


def sbits(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float32).reshape(-1).view(np.uint32)


def assert_same(res, q_ref, s_ref, label=""):
    q = qbits(res.tensor)
    if not np.array_equal(q, q_ref):
        bad = np.argwhere(q != q_ref)
        i = tuple(bad[0])
        raise AssertionError(f"{label}: {len(bad)} fp8 bytes differ, first at {i}: "
                             f"gpu {q[i]:#x} oracle {q_ref[i]:#x}")
    sr = np.asarray(s_ref, np.float32).reshape(-1).view(np.uint32)
    sg = sbits(res.dequant_scale)
    if not np.array_equal(sg, sr):
        bad = np.nonzero(sg != sr)[0]
        raise AssertionError(f"{label}: {len(bad)} scales differ, first at {bad[0]}: "
                             f"gpu {sg[bad[0]]:#x} oracle {sr[bad[0]]:#x}")


def make_input(shape, dtype, seed, scale=1.0, outliers=0.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    if outliers:
        m = torch.rand(*shape, generator=g) < outliers
        x[m] *= 50.0
    return x.to(DT[dtype])


# ---------------------------------------------------------------------------
# hardware fp8 conversion == integer restatement over every in-range fp32
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, 8192 * 4096 * 2])
def test_copy16_selftest(dev, nbytes):
    # the plain copy that bench.py --mem-ceiling times as the 1:1 ceiling
    x = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
    y = torch.zeros_like(x)
    _lib.check(_lib.lib().pcamd_selftest_copy16(_lib.ptr(x), _lib.ptr(y), nbytes, _lib.stream_of(x)), "copy16")
    torch.cuda.synchronize()
    assert torch.equal(x, y)


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, 4096 * 7168 * 2])
def test_narrow16_selftest(dev, nbytes):
    # the 2:1 narrowing that bench.py --mem-ceiling times as the quantizers'
    # ceiling: y is the high byte of every 16-bit element of x
    x = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=dev)
    y = torch.zeros(nbytes // 2 + 8, dtype=torch.uint8, device=dev)
    _lib.check(_lib.lib().pcamd_selftest_narrow16(_lib.ptr(x), _lib.ptr(y), nbytes, _lib.stream_of(x)), "narrow16")
    torch.cuda.synchronize()
    assert torch.equal(y[:nbytes // 2], x[1::2])
    assert not y[nbytes // 2:].any()  # nothing written past in_bytes / 2


@pytest.mark.parametrize("fmt", [_lib.E4M3FN, _lib.E5M2])
def test_hw_convert_selftest(dev, fmt):
    res = torch.zeros(4, dtype=torch.int32, device=dev)
    print(f"selftest fmt={fmt}", flush=True)
    _lib.check(_lib.lib().pcamd_selftest_fp8_convert(fmt, _lib.ptr(res), _lib.stream_of(res)),
               "selftest")
    torch.cuda.synchronize()
    r = res.cpu().numpy().view(np.uint32)
    assert r[2] > 0x40000000, "self-test did not cover the range"
    assert r[0] == 0, f"{r[0]} mismatches, first pattern {r[1]:#010x}"


# ---------------------------------------------------------------------------
# golden vectors
# ---------------------------------------------------------------------------
def _golden():
    with open(os.path.join(GOLDEN, "quant_golden.json")) as fh:
        return json.load(fh)


@pytest.mark.parametrize("name", sorted(_golden()))
def test_golden_vectors(dev, name):
    meta = _golden()[name]
    d = np.load(os.path.join(GOLDEN, "quant_golden.npz"))
    raw = d[f"{name}__x"]
    if meta["dtype"] == "bf16":
        x = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16)
    elif meta["dtype"] == "f16":
        x = torch.from_numpy(raw.view(np.float16))
    else:
        x = torch.from_numpy(raw)
    x = x.to(dev)
    fp8 = FMT[meta["fmt"]]
    print(f"golden {name}", flush=True)
    if meta["kind"] == "block":
        r = hip_per_block_quant(x, block_m=meta["bm"], block_n=meta["bn"], fp8_dtype=fp8)
    elif meta["kind"] == "channel":
        r = hip_per_channel_quant(x, channel_axis=meta["axis"], fp8_dtype=fp8)
    else:
        r = hip_per_tensor_quant(x, fp8_dtype=fp8)
    assert_same(r, d[f"{name}__q"], d[f"{name}__scale"], name)


# ---------------------------------------------------------------------------
# per-block: every kernel path
# ---------------------------------------------------------------------------
BLOCK_CASES = [
    # (shape, dtype, block_m, block_n, fmt)     path
    ((2, 5, 384), "bf16", 1, 128, "e4m3"),      # rows, 1x128
    ((37, 264), "f32", 1, 128, "e4m3"),         # rows, ragged last group, fp32 input
    ((3, 100, 520), "f16", 1, 64, "e4m3"),      # rows, 1x64
    ((7, 1032), "bf16", 1, 8, "e4m3"),          # rows, 1x8 (one lane per group)
    ((5, 2048), "bf16", 1, 512, "e5m2"),        # rows, 1x512 (whole wave per group)
    ((9, 9000), "bf16", 1, 128, "e4m3"),        # rows, two segments per row
    ((256, 384), "bf16", 128, 128, "e4m3"),     # tile
    # the 1024-thread tile kernel is taken for grids of one workgroup per CU
    # (256 CUs: 154-256 workgroups of 128 rows x 512 H columns)
    ((4096, 4096), "bf16", 128, 128, "e4m3"),     # tile, four blocks per workgroup (256 workgroups)
    ((2, 2048, 4096), "bf16", 128, 128, "e4m3"),  # tile, four blocks per workgroup, batch
    ((2, 2048, 7168), "f16", 128, 128, "e5m2"),   # tile, eight blocks per workgroup, batch, fp16
    ((2, 300, 264), "bf16", 128, 128, "e4m3"),  # tile, ragged blocks
    ((64, 256), "bf16", 64, 64, "e5m2"),        # tile, 64x64
    ((128, 512), "f32", 128, 256, "e4m3"),      # tile, 128x256, fp32
    ((1000, 136), "bf16", 128, 1, "e4m3"),      # column groups, ragged
    ((2, 512, 264), "f16", 256, 1, "e4m3"),     # column groups, 256x1
    ((96, 64), "bf16", 16, 1, "e4m3"),          # column groups, 16x1
    ((3, 192, 520), "f32", 64, 1, "e5m2"),      # column groups, 64x1, fp32, ragged strip
    ((200, 300), "bf16", 128, 128, "e4m3"),     # generic (n % 8 != 0)
    ((33, 70), "f32", 4, 32, "e4m3"),           # generic
    ((2, 64, 256), "bf16", 2, 128, "e4m3"),     # generic (2x128)
    ((40, 256), "bf16", 1, 1024, "e4m3"),       # generic (group wider than a wave)
    ((50, 64), "bf16", 8, 1, "e4m3"),           # generic (8x1)
    ((3, 17, 33), "f16", 1, 1, "e5m2"),         # generic (1x1)
]


@pytest.mark.parametrize("shape,dtype,bm,bn,fmt", BLOCK_CASES)
def test_block_quant_matches_oracle(dev, shape, dtype, bm, bn, fmt):
    x = make_input(shape, dtype, seed=hash((shape, bm, bn)) & 0xFFFF, scale=0.5, outliers=0.002)
    print(f"block {shape} {dtype} {bm}x{bn} {fmt}", flush=True)
    r = hip_per_block_quant(x.to(dev), block_m=bm, block_n=bn, fp8_dtype=FMT[fmt])
    q_ref, s_ref = O.quant_block(x, bm, bn, fmt, threads=8)
    assert r.dequant_scale.shape == s_ref.shape
    assert r.tensor.dtype == FMT[fmt] and r.tensor.shape == x.shape
    assert_same(r, q_ref, s_ref, f"{shape} {bm}x{bn}")


def test_block_quant_strided_input(dev):
    # an M-major (transposed) input goes through the generic strided kernel and
    # keeps its layout in the output (preserve_format)
    base = make_input((300, 200), "bf16", seed=5).to(dev)
    x = base.t()
    r = hip_per_block_quant(x, block_m=1, block_n=128)
    assert r.tensor.stride() == x.stride()
    q_ref, s_ref = O.quant_block(x.cpu(), 1, 128)
    assert_same(r, q_ref, s_ref, "transposed")


def test_wide_tiles_padded_rows(dev):
    # the eight-block 128 x 128 kernel on rows of a wider 3-D tensor (row pitch
    # 7296 elements in, 7168 out): input and output strides differ
    base = make_input((2, 2048, 7296), "bf16", seed=12, scale=0.5, outliers=0.002).to(dev)
    x = base[:, :, :7168]
    print("eight-block tiles, row pitch 7296", flush=True)
    r = hip_per_block_quant(x, block_m=128, block_n=128)
    q_ref, s_ref = O.quant_block(x.cpu().contiguous(), 128, 128)
    assert_same(r, q_ref, s_ref, "eight-block tiles, padded rows")


@pytest.mark.parametrize("bm,bn", [(1, 128), (1, 64), (128, 128), (128, 1), (32, 1)])
def test_block_quant_padded_rows(dev, bm, bn):
    # rows contiguous but with a row pitch wider than the row (a column slice of
    # a wider 3-D tensor): the row-indexed kernels, not the flat one
    base = make_input((2, 256, 640), "bf16", seed=11).to(dev)
    x = base[:, :, :384]
    print(f"padded rows {bm}x{bn}", flush=True)
    r = hip_per_block_quant(x, block_m=bm, block_n=bn)
    q_ref, s_ref = O.quant_block(x.cpu().contiguous(), bm, bn)
    assert_same(r, q_ref, s_ref, f"padded {bm}x{bn}")


def test_block_quant_zeros_and_outliers(dev):
    x = torch.zeros(4, 384, device=dev, dtype=torch.bfloat16)
    x[1, 5] = -0.0
    r = hip_per_block_quant(x, block_m=1, block_n=128)
    q = qbits(r.tensor)
    assert q[1, 5] == 0x80 and np.count_nonzero(q) == 1
    assert torch.isfinite(r.dequant_scale).all()
    y = make_input((64, 64), "f32", seed=6)
    y[0, 0], y[1, 1] = 1e6, -1e6
    r = hip_per_block_quant(y.to(dev), block_m=64, block_n=64)
    q = qbits(r.tensor)
    assert q[0, 0] == 0x7E and q[1, 1] == 0xFE


def test_config1_full_size(dev):
    """bf16 [4096, 7168], N(0,1) with 0.1% outliers x50, 1x128."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4096, 7168, generator=g)
    m = torch.rand(4096, 7168, generator=g) < 0.001
    x[m] *= 50
    x = x.bfloat16()
    r = hip_per_block_quant(x.to(dev), block_m=1, block_n=128)
    q_ref, s_ref = O.quant_block(x, 1, 128, threads=8)
    assert r.dequant_scale.shape == (4096, 56)
    assert_same(r, q_ref, s_ref, "config1")


def test_column_groups_full_size(dev):
    """128x1 groups (the wgrad operand quantization) over the config-1 input
    shape: bf16 [4096, 7168], N(0,1) with 0.1% outliers x50."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(4096, 7168, generator=g)
    m = torch.rand(4096, 7168, generator=g) < 0.001
    x[m] *= 50
    x = x.bfloat16()
    r = hip_per_block_quant(x.to(dev), block_m=128, block_n=1)
    q_ref, s_ref = O.quant_block(x, 128, 1, threads=8)
    assert r.dequant_scale.shape == (32, 7168)
    assert_same(r, q_ref, s_ref, "128x1 full size")


def test_config3_full_size(dev):
    """bf16 [4096, 7168] N(0,0.02) x log-uniform block
    multipliers in [0.1, 10], 128x128 blocks."""
    g = torch.Generator().manual_seed(0)
    w = torch.randn(4096, 7168, generator=g) * 0.02
    mult = torch.exp(torch.empty(32, 56).uniform_(np.log(0.1), np.log(10.0), generator=g))
    w = (w * mult.repeat_interleave(128, 0).repeat_interleave(128, 1)).bfloat16()
    r = hip_per_block_quant(w.to(dev), block_m=128, block_n=128)
    q_ref, s_ref = O.quant_block(w, 128, 128, threads=8)
    assert r.dequant_scale.shape == (32, 56)
    assert_same(r, q_ref, s_ref, "config3")


# ---------------------------------------------------------------------------
# dual 1 x 128 + 128 x 1 quantization (one read, both outputs)
# ---------------------------------------------------------------------------
DUAL_CASES = [
    ((256, 384), "bf16", 128, "e4m3", None),          # whole blocks
    ((3, 256, 640), "f16", 128, "e5m2", None),        # batch
    ((200, 520), "bf16", 128, "e4m3", None),          # ragged rows, partial last strip
    ((2, 130, 136), "f32", 128, "e4m3", None),        # fp32 input, ragged both ways
    ((96, 1000), "bf16", 128, "e4m3", "outliers"),
    ((45, 77), "bf16", 128, "e4m3", None),            # n % 8 != 0: the two quantizers in turn
    ((256, 256), "bf16", 64, "e4m3", None),           # other block size: the two quantizers in turn
    ((384, 256), "bf16", 128, "e4m3", "transposed"),  # column-major input: the two quantizers in turn
    ((256, 384), "bf16", 128, "e4m3", "zero_rows"),
    ((2, 256, 384), "bf16", 128, "e4m3", "padded"),   # row pitch 640 (a column slice)
    ((2, 333, 264), "bf16", 128, "e5m2", None),       # partial last row group in a batch, partial strip
    ((1000, 256), "bf16", 128, "e4m3", None),         # partial last row group, several 16-row pieces cut
]


@pytest.mark.parametrize("col_t", [False, True], ids=["col_rows", "col_transposed"])
@pytest.mark.parametrize("shape,dtype,block,fmt,kind", DUAL_CASES)
def test_dual_matches_oracle(dev, shape, dtype, block, fmt, kind, col_t):
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant_dual
    x = make_input(shape, dtype, seed=sum(shape) + block, outliers=0.01 if kind == "outliers" else 0.0)
    if kind == "zero_rows":
        x[5:37] = 0
        x[:, 129:257] = 0
    xd = x.to(dev)
    if kind == "transposed":
        x = x.t().contiguous().t()        # same values, column-major strides
        xd = xd.t().contiguous().t()
    if kind == "padded":
        wide = torch.zeros(*shape[:-1], 640, dtype=x.dtype, device=dev)
        wide[..., :shape[-1]] = xd
        xd = wide[..., :shape[-1]]
    print(f"dual shape={shape} dtype={dtype} block={block} fmt={fmt} kind={kind} col_t={col_t}", flush=True)
    r_row, r_col = hip_per_block_quant_dual(xd, block=block, fp8_dtype=FMT[fmt], col_transposed=col_t)
    if col_t:
        # [.., N, M] storage, rows padded to 16 bytes
        assert r_col.tensor.stride(-2) == 1 and r_col.tensor.stride(-1) == -(-shape[-2] // 16) * 16
    q1, s1 = O.quant_block(x, 1, block, fmt=fmt)
    q2, s2 = O.quant_block(x, block, 1, fmt=fmt)
    assert r_row.meta["block_m"] == 1 and r_row.meta["block_n"] == block
    assert r_col.meta["block_m"] == block and r_col.meta["block_n"] == 1
    assert_same(r_row, q1, s1, "dual 1 x block")
    assert_same(r_col, q2, s2, "dual block x 1")
    # and the same bits as the two separate entry points
    for r, bm, bn in ((r_row, 1, block), (r_col, block, 1)):
        one = hip_per_block_quant(xd, block_m=bm, block_n=bn, fp8_dtype=FMT[fmt])
        assert np.array_equal(qbits(r.tensor), qbits(one.tensor))
        assert np.array_equal(sbits(r.dequant_scale), sbits(one.dequant_scale))
        assert r.dequant_scale.shape == one.dequant_scale.shape



def _tiny_input(dtype, seed):
    """[256, 512] of N(0, 1) in which one 128 x 128 block, row 200 and column
    300 hold only values of magnitude 1.2e-38 .. 2e-38 (normal in fp32 and
    bf16, random signs, no zeros): every kind of group, block, row and column
    has a member whose amax is that small."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((256, 512)).astype(np.float32)
    def tiny(shape):
        return (g.uniform(1.2e-38, 2e-38, shape) * g.choice([-1.0, 1.0], shape)).astype(np.float32)
    x[:128, :128] = tiny((128, 128))
    x[200, :] = tiny((512,))
    x[:, 300] = tiny((256,))
    return torch.from_numpy(x).to(DT[dtype])


TINY_EPS_PATHS = [
    # (kind, dtype, bm, bn)
    ("block", "bf16", 1, 128),      # row groups, flat
    ("block", "f32", 1, 128),
    ("block", "bf16", 128, 128),    # tiles
    ("block", "bf16", 128, 1),      # column groups
    ("block", "bf16", 4, 16),       # generic
    ("channel-2", "bf16", 0, 0),    # one scale per row
    ("channel-1", "bf16", 0, 0),    # one scale per column
    ("dual", "bf16", 0, 0),
    ("dual_t", "bf16", 0, 0),
]


@pytest.mark.parametrize("fmt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("kind,dtype,bm,bn", TINY_EPS_PATHS)
def test_eps_zero_tiny_amax_matches_oracle(dev, kind, dtype, bm, bn, fmt):
    """eps = 0 with groups whose amax is below fp8_max / FLT_MAX: qs = fp8_max /
    amax overflows to inf, x * qs = +-inf, and the reference's clamp makes
    that +-fp8_max. The clamp-free kernel instantiations would emit NaN (e4m3)
    or inf (e5m2) bytes there, so the host keeps the clamp; bit-exact against
    the oracle at the format maximum."""
    fmax = 448.0 if fmt == "e4m3" else 57344.0
    print(f"eps=0 tiny amax {kind} {dtype} {bm}x{bn} {fmt}", flush=True)
    x = _tiny_input(dtype, seed=bm + bn + len(kind))
    xd = x.to(dev)
    fp8 = FMT[fmt]
    if kind == "block":
        q, s = _abi_quant_block(xd, bm, bn, fp8, fmax, eps=0.0)
        _same_bits(q, s, *O.quant_block(x, bm, bn, fmt=fmt, eps=0.0), kind)
    elif kind.startswith("channel"):
        axis = int(kind[len("channel"):])
        q, s = _abi_quant_channel(xd, axis, fp8, fmax, eps=0.0)
        _same_bits(q, s, *O.quant_channel(x, axis, fmt=fmt, eps=0.0), kind)
    else:
        yr, sr, yc, sc = _abi_quant_dual(xd, fp8, fmax, kind == "dual_t", eps=0.0)
        q1, s1 = O.quant_block(x, 1, 128, fmt=fmt, eps=0.0)
        q2, s2 = O.quant_block(x, 128, 1, fmt=fmt, eps=0.0)
        _same_bits(yr, sr, q1, s1, kind + " rows")
        _same_bits(yc, sc, q2, s2, kind + " columns")
    # the tiny elements saturate: no NaN / inf code anywhere
    qb = qbits(q if kind == "block" or kind.startswith("channel") else yr)
    nan_codes = (0x7F, 0xFF) if fmt == "e4m3" else tuple(range(0x7C, 0x80)) + tuple(range(0xFC, 0x100))
    assert not np.isin(qb, nan_codes).any()

def test_dual_full_size(dev):
    """Both quantizations of the config-1 input shape (bf16 [4096, 7168],
    N(0,1) with 0.1% outliers x50) from one kernel, bit-exact."""
    from practice_cuda_amd.impls.hip_per_block import hip_per_block_quant_dual
    g = torch.Generator().manual_seed(2)
    x = torch.randn(4096, 7168, generator=g)
    m = torch.rand(4096, 7168, generator=g) < 0.001
    x[m] *= 50
    x = x.bfloat16()
    r_row, r_col = hip_per_block_quant_dual(x.to(dev), block=128, col_transposed=True)
    q1, s1 = O.quant_block(x, 1, 128, threads=8)
    assert_same(r_row, q1, s1, "dual 1x128 full size")
    q2, s2 = O.quant_block(x, 128, 1, threads=8)
    assert_same(r_col, q2, s2, "dual 128x1 full size")


def test_dual_rejects_aliased_outputs(dev):
    x = torch.randn(128, 128, device=dev).bfloat16()
    y = torch.empty(128, 128, device=dev, dtype=torch.float8_e4m3fn)
    s1 = torch.empty(128, 1, device=dev)
    s2 = torch.empty(1, 128, device=dev)
    rc = _lib.lib().pcamd_quant_block_dual(
        _lib.ptr(x), _lib.BF16, 1, 128, 128, 0, 128, 1, _lib.ptr(y), 0, 128, 1, _lib.ptr(y), 0, 128, 1,
        _lib.E4M3FN, _lib.ptr(s1), 0, 1, 1, _lib.ptr(s2), 0, 128, 1, 128, 448.0, 1e-12, _lib.stream_of(x))
    assert rc == -1 and b"alias" in _lib.lib().pcamd_last_error()


# ---------------------------------------------------------------------------
# per-channel
# ---------------------------------------------------------------------------
CHANNEL_CASES = [
    ((33, 200), "bf16", -2, "e4m3"),        # register-resident rows
    ((2, 40, 7168), "bf16", -2, "e4m3"),    # 14 chunk slots per lane
    ((2, 16, 8200), "bf16", -2, "e4m3"),    # longer than 8192: generic two-pass row
    ((50, 70), "f32", -2, "e4m3"),          # generic (n % 8 != 0)
    ((3, 300, 264), "bf16", -1, "e4m3"),    # row slabs + atomic column maxima, ragged strip
    ((200, 264), "bf16", -1, "e4m3"),       # column strips (<= 256 rows)
    ((50, 70), "f32", -1, "e5m2"),          # generic columns
    ((1, 4096, 512), "f16", -1, "e4m3"),    # row slabs
    ((1000, 136), "f32", -1, "e5m2"),       # row slabs, ragged last slab, fp32
    ((64, 1024), "f32", -2, "e5m2"),        # fp32 rows
]


@pytest.mark.parametrize("shape,dtype,axis,fmt", CHANNEL_CASES)
def test_channel_quant_matches_oracle(dev, shape, dtype, axis, fmt):
    x = make_input(shape, dtype, seed=hash((shape, axis)) & 0xFFFF, scale=0.02, outliers=0.001)
    print(f"channel {shape} {dtype} axis={axis} {fmt}", flush=True)
    r = hip_per_channel_quant(x.to(dev), channel_axis=axis, fp8_dtype=FMT[fmt])
    q_ref, s_ref = O.quant_channel(x, axis, fmt, threads=8)
    assert r.dequant_scale.shape == s_ref.shape
    assert_same(r, q_ref, s_ref, f"{shape} axis {axis}")


def test_channel_one_pass_same_bytes(dev):
    x = make_input((64, 4096), "bf16", seed=11).to(dev)
    a = hip_per_channel_quant(x, channel_axis=-2, one_pass=True)
    b = hip_per_channel_quant(x, channel_axis=-2)
    assert a.meta["quant_strategy"] == "one_pass" and b.meta["quant_strategy"] == "two_pass"
    assert torch.equal(a.tensor.view(torch.uint8), b.tensor.view(torch.uint8))
    assert torch.equal(a.dequant_scale, b.dequant_scale)


def test_columns_full_size(dev):
    """One scale per column (channel_axis=-1, the reference bench's default
    axis and the per-channel BMM's B operand) over the config-2 weight
    [18432, 7168]: 144 row slabs meet in each column's atomic maximum."""
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(18432, 7168, generator=g) * 0.02)
    w[12345, 77] = 9.0                       # a lone column maximum deep in the tensor
    w = w.bfloat16()
    r = hip_per_channel_quant(w.to(dev), channel_axis=-1)
    q_ref, s_ref = O.quant_channel(w, -1, threads=8)
    assert r.dequant_scale.shape == (7168,)
    assert_same(r, q_ref, s_ref, "columns full size")


def test_columns_microbench_shape(dev):
    """The reference's per-channel microbench point
    (fp8_training/microbench/profile_fused_quant.py:27-35): fp32 [80, 2048,
    1280], channel_axis=-1, eps 1e-6; seeded on the CPU (the reference draws
    on the device)."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(80, 2048, 1280, generator=g)
    r = hip_per_channel_quant(x.to(dev), channel_axis=-1, eps=1e-6)
    q_ref, s_ref = O.quant_channel(x, -1, eps=1e-6, threads=8)
    assert r.dequant_scale.shape == (80, 1280)
    assert_same(r, q_ref, s_ref, "microbench per-column")


def test_config2_full_size(dev):
    """bf16 weight [18432, 7168] N(0, 0.02), one scale per row."""
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(18432, 7168, generator=g) * 0.02).bfloat16()
    r = hip_per_channel_quant(w.to(dev), channel_axis=-2)
    q_ref, s_ref = O.quant_channel(w, -2, threads=8)
    assert r.dequant_scale.shape == (18432,)
    assert_same(r, q_ref, s_ref, "config2")


# ---------------------------------------------------------------------------
# per-tensor
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,dtype,fmt", [((3, 17, 33), "bf16", "e4m3"), ((64, 64), "f32", "e4m3"),
                                             ((14, 2048, 512), "f32", "e5m2"), ((128, 256), "f16", "e4m3")])
def test_tensor_quant_matches_oracle(dev, shape, dtype, fmt):
    x = make_input(shape, dtype, seed=7, scale=3.0, outliers=0.001)
    r = hip_per_tensor_quant(x.to(dev), fp8_dtype=FMT[fmt])
    q_ref, ds, _ = O.quant_tensor(x, fmt)
    assert r.dequant_scale.ndim == 0
    assert_same(r, q_ref, np.float32(ds), f"tensor {shape}")


@pytest.mark.parametrize("shape,dtype,fmt,amax", [((3, 40, 72), "bf16", "e4m3", 0.5234375),
                                                  ((2048, 512), "bf16", "e5m2", 0.5390625),
                                                  ((14, 2048, 512), "f32", "e4m3", 3.0),
                                                  ((64, 96), "f16", "e4m3", 0.0)])
def test_tensor_quant_torchao_form(dev, shape, dtype, fmt, amax):
    # scale arithmetic in fp64 (torchao's tensorwise scale, the reference
    # layer's form): the kernels' bytes and scales against the oracle; at
    # the bf16 amax values the fp32 form gives another scale
    print(f"tensor torchao form {shape} {dtype} {fmt} amax={amax}", flush=True)
    x = make_input(shape, dtype, seed=17, scale=0.05, outliers=0.0)
    if amax == 0.0:
        x = torch.zeros_like(x)
    else:
        x.view(-1)[len(x.view(-1)) // 3] = -amax
    q, ds, qs = quant_tensor_raw(x.to(dev), FMT[fmt], 1e-12, scale_dtype=torch.float64)
    q_ref, ds_ref, qs_ref = O.quant_tensor(x, fmt, scale_dt=O.F64)
    torch.cuda.synchronize()
    assert np.array_equal(qbits(q), q_ref)
    assert np.float32(ds.item()) == np.float32(ds_ref) and np.float32(qs.item()) == np.float32(qs_ref)
    if amax in (0.5234375, 0.5390625):
        assert np.float32(qs_ref) != np.float32(O.quant_tensor(x, fmt)[2])


def test_determinism(dev):
    x = make_input((512, 7168), "bf16", seed=9).to(dev)
    a = hip_per_block_quant(x, block_m=1, block_n=128)
    b = hip_per_block_quant(x, block_m=1, block_n=128)
    assert torch.equal(a.tensor.view(torch.uint8), b.tensor.view(torch.uint8))
    assert torch.equal(a.dequant_scale, b.dequant_scale)


def test_dequant_roundtrip(dev):
    # reference fp8_quant_test.py:110-119: |x_hat - x| <= 0.1|x| + 0.05 amax
    x = make_input((32, 2048), "f32", seed=10).to(dev)
    for r in (hip_per_block_quant(x, block_m=1, block_n=128),
              hip_per_channel_quant(x, channel_axis=-2),
              hip_per_tensor_quant(x)):
        xh = r.dequantize()
        assert torch.allclose(xh, x, rtol=1e-1, atol=0.05 * x.abs().max().item())


@pytest.mark.parametrize("axis", [-1, -2])
def test_torch_compile_role_same_bytes(dev, axis):
    """The registry's torch_compile_per_channel entry runs the per-channel
    kernel: bytes and scales identical to hip_per_channel, the reference's
    result fields for that entry (impl name, quant_strategy)."""
    from practice_cuda_amd import get_quant
    g = torch.Generator().manual_seed(11)
    x = torch.randn(3, 96, 160, generator=g).bfloat16().to(dev)
    a = get_quant("torch_compile_per_channel").fn(x, channel_axis=axis)
    b = get_quant("hip_per_channel").fn(x, channel_axis=axis)
    assert torch.equal(a.tensor.view(torch.uint8), b.tensor.view(torch.uint8))
    assert torch.equal(a.dequant_scale, b.dequant_scale)
    assert a.impl == "torch_compile_per_channel" and a.meta["quant_strategy"] == "torch_compile"
    assert a.granularity == "channel" and a.meta["channel_axis"] == axis


# ---------------------------------------------------------------------------
# fp8_max below the format maximum: the clamping kernel instantiations
# ---------------------------------------------------------------------------
def _clamp_witnesses(fmax: float) -> np.ndarray:
    """bf16 values s in [1, 8) with fl(s * fl(fmax / s)) > fmax in fp32: as a
    block's amax, s quantizes to a product just above fmax, so a kernel that
    skipped the clamp would round it one code too far when fmax sits on a
    rounding midpoint."""
    s = (np.arange(0x3F80, 0x4100, dtype=np.uint32) << 16).view(np.float32)
    f = np.float32(fmax)
    return s[s * (f / s) > f]


def _planted_input(shape, dtype, fmax, seed):
    """N(0, 0.3) clipped to |x| < 1, one witness of random sign per row."""
    g = np.random.default_rng(seed)
    x = np.clip(g.standard_normal(shape) * 0.3, -0.99, 0.99).astype(np.float32)
    w = _clamp_witnesses(fmax)
    rows = x.reshape(-1, shape[-1])
    cols = g.integers(0, shape[-1], rows.shape[0])
    rows[np.arange(rows.shape[0]), cols] = w[g.integers(0, len(w), rows.shape[0])] * g.choice([-1.0, 1.0], rows.shape[0])
    return torch.from_numpy(x).to(DT[dtype])


def _abi_quant_block(xd, bm, bn, fp8, fmax, eps=1e-12):
    y = torch.empty_like(xd, dtype=fp8)
    x3, y3 = (xd[None], y[None]) if xd.ndim == 2 else (xd, y)
    b, m, n = x3.shape
    s = torch.empty(b, -(-m // bm), -(-n // bn), device=xd.device)
    _lib.check(_lib.lib().pcamd_quant_block(
        _lib.ptr(x3), _lib.dtype_code(xd.dtype), b, m, n, *x3.stride(), _lib.ptr(y3), _lib.dtype_code(fp8),
        *y3.stride(), _lib.ptr(s), *s.stride(), bm, bn, float(fmax), float(eps), _lib.stream_of(xd)), "quant_block")
    return y, s


def _abi_quant_dual(xd, fp8, fmax, transposed, eps=1e-12):
    x3 = xd[None] if xd.ndim == 2 else xd
    b, m, n = x3.shape
    yr = torch.empty_like(x3, dtype=fp8)
    if transposed:
        pitch = -(-m // 16) * 16
        yc = torch.empty(b, n, pitch, dtype=fp8, device=xd.device)[..., :m].transpose(-1, -2)
    else:
        yc = torch.empty_like(yr)
    sr = torch.empty(b, m, -(-n // 128), device=xd.device)
    sc = torch.empty(b, -(-m // 128), n, device=xd.device)
    _lib.check(_lib.lib().pcamd_quant_block_dual(
        _lib.ptr(x3), _lib.dtype_code(xd.dtype), b, m, n, *x3.stride(), _lib.ptr(yr), *yr.stride(),
        _lib.ptr(yc), *yc.stride(), _lib.dtype_code(fp8), _lib.ptr(sr), *sr.stride(), _lib.ptr(sc),
        *sc.stride(), 128, float(fmax), float(eps), _lib.stream_of(xd)), "quant_block_dual")
    return yr, sr, yc, sc


def _abi_quant_channel(xd, axis, fp8, fmax, eps=1e-12):
    y = torch.empty_like(xd, dtype=fp8)
    x3, y3 = (xd[None], y[None]) if xd.ndim == 2 else (xd, y)
    b, m, n = x3.shape
    s = torch.empty(b, m if axis == -2 else n, device=xd.device)
    _lib.check(_lib.lib().pcamd_quant_channel(
        _lib.ptr(x3), _lib.dtype_code(xd.dtype), b, m, n, *x3.stride(), _lib.ptr(y3), _lib.dtype_code(fp8),
        *y3.stride(), _lib.ptr(s), *s.stride(), axis, float(fmax), float(eps), _lib.stream_of(xd)), "quant_channel")
    return y, s


def _same_bits(q, s, q_ref, s_ref, label):
    torch.cuda.synchronize()
    qg = qbits(q).reshape(np.asarray(q_ref).shape)
    assert np.array_equal(qg, q_ref), f"{label}: {int((qg != q_ref).sum())} fp8 bytes differ"
    sr = np.asarray(s_ref, np.float32).reshape(-1).view(np.uint32)
    assert np.array_equal(sbits(s), sr), f"{label}: scales differ"


# (fmt, fp8_max): e4m3 just below the 240/256 midpoint and on the 96/104
# midpoint, e5m2 on the 32768/40960 midpoint
REDUCED_MAX = [("e4m3", float(np.nextafter(np.float32(248.0), np.float32(0.0)))), ("e4m3", 100.0),
               ("e5m2", 36864.0)]
REDUCED_PATHS = [
    # (kind, shape, dtype, bm, bn)
    ("block", (64, 1024), "bf16", 1, 128),        # row groups, flat
    ("block", (3, 40, 1000), "f32", 1, 128),      # row groups, ragged
    ("block", (256, 384), "bf16", 128, 128),      # tiles, whole
    ("block", (4096, 5120), "bf16", 128, 128),    # tiles, eight blocks per workgroup (160)
    ("block", (200, 300), "f16", 128, 128),       # tiles, partial
    ("block", (300, 256), "bf16", 128, 1),        # column groups
    ("block", (50, 70), "f16", 4, 16),            # generic
    ("channel-2", (64, 2048), "bf16", 0, 0),      # register-resident rows
    ("channel-1", (256, 512), "bf16", 0, 0),      # column strips
    ("dual", (256, 512), "bf16", 0, 0),
    ("dual", (2, 333, 264), "bf16", 0, 0),
    ("dual_t", (256, 512), "bf16", 0, 0),
    ("dual_t", (1000, 256), "bf16", 0, 0),
]


@pytest.mark.parametrize("fmt,fmax", REDUCED_MAX, ids=["e4m3_248m", "e4m3_100", "e5m2_36864"])
@pytest.mark.parametrize("kind,shape,dtype,bm,bn", REDUCED_PATHS)
def test_reduced_fp8_max_matches_oracle(dev, kind, shape, dtype, bm, bn, fmt, fmax):
    print(f"reduced fp8_max {kind} shape={shape} dtype={dtype} {bm}x{bn} {fmt} fp8_max={fmax!r}", flush=True)
    x = _planted_input(shape, dtype, fmax, seed=sum(shape) + bm + bn)
    xd = x.to(dev)
    fp8 = FMT[fmt]
    if kind == "block":
        q, s = _abi_quant_block(xd, bm, bn, fp8, fmax)
        _same_bits(q, s, *O.quant_block(x, bm, bn, fmt=fmt, fp8_max=fmax), kind)
    elif kind.startswith("channel"):
        axis = int(kind[len("channel"):])
        q, s = _abi_quant_channel(xd, axis, fp8, fmax)
        _same_bits(q, s, *O.quant_channel(x, axis, fmt=fmt, fp8_max=fmax), kind)
    else:
        yr, sr, yc, sc = _abi_quant_dual(xd, fp8, fmax, kind == "dual_t")
        q1, s1 = O.quant_block(x, 1, 128, fmt=fmt, fp8_max=fmax)
        q2, s2 = O.quant_block(x, 128, 1, fmt=fmt, fp8_max=fmax)
        _same_bits(yr, sr, q1, s1, kind + " rows")
        _same_bits(yc, sc, q2, s2, kind + " columns")
