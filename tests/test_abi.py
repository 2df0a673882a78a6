"""CPU tests of the C ABI: the library loads, exports every function declared
in include/pcamd_fp8.h, and rejects bad arguments with a status code and a
message (no kernel is launched on these paths)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from practice_cuda_amd import _lib

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(__file__)), "include")
HEADER = os.path.join(INCLUDE, "pcamd_fp8.h")
TEST_HEADER = os.path.join(INCLUDE, "pcamd_fp8_selftest.h")
FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: validation fails first


def declared_functions(path: str = HEADER) -> list[str]:
    text = open(path).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(pcamd_\w+)\s*\(", text, re.M)))


def test_library_exports_header_symbols():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 7
    for name in names:
        assert hasattr(L, name), f"{name} declared in the header but not exported"
    assert sorted(_lib.EXPORTED_SYMBOLS) == names


def test_test_only_symbols_live_in_their_own_header():
    L = _lib.lib()
    names = declared_functions(TEST_HEADER)
    assert names == sorted(_lib.TEST_SYMBOLS)
    assert not set(names) & set(declared_functions())
    for name in names:
        assert hasattr(L, name)
    assert L.pcamd_selftest_fp8_convert(7, FAKE, None) == -1
    assert b"fp8 format" in L.pcamd_last_error()
    assert L.pcamd_selftest_copy16(FAKE, FAKE, 24, None) == -1
    assert b"multiple of 16" in L.pcamd_last_error()
    assert L.pcamd_selftest_copy16(ctypes.c_void_p(0x10008), FAKE, 32, None) == -1
    assert b"aligned" in L.pcamd_last_error()
    assert L.pcamd_selftest_copy16(FAKE, FAKE, 0, None) == 0
    assert L.pcamd_selftest_narrow16(FAKE, FAKE, 24, None) == -1
    assert b"multiple of 16" in L.pcamd_last_error()
    assert L.pcamd_selftest_narrow16(FAKE, ctypes.c_void_p(0x10004), 32, None) == -1
    assert b"aligned" in L.pcamd_last_error()
    assert L.pcamd_selftest_narrow16(None, FAKE, 32, None) == -1
    assert b"null" in L.pcamd_last_error()
    assert L.pcamd_selftest_narrow16(FAKE, FAKE, 0, None) == 0


def test_abi_version_matches_header():
    text = open(HEADER).read()
    version = int(re.search(r"#define PCAMD_ABI_VERSION (\d+)", text).group(1))
    assert _lib.lib().pcamd_abi_version() == version


def _quant_block(**over):
    args = dict(x=FAKE, xd=_lib.BF16, b=1, m=4, n=256, sxb=0, sxm=256, sxn=1, y=FAKE,
                yd=_lib.E4M3FN, syb=0, sym=256, syn=1, s=FAKE, ssb=0, ssm=2, ssn=1, bm=1, bn=128,
                fmax=448.0, eps=1e-12, st=None)
    args.update(over)
    return _lib.lib().pcamd_quant_block(*args.values())


def test_invalid_arguments_are_rejected():
    L = _lib.lib()
    assert _quant_block(xd=7) == -1
    assert b"input dtype" in L.pcamd_last_error()
    assert _quant_block(yd=_lib.BF16) == -1
    assert _quant_block(bm=3) == -1 and b"powers of two" in L.pcamd_last_error()
    assert _quant_block(m=-1) == -1
    assert _quant_block(x=None) == -1 and b"null" in L.pcamd_last_error()
    assert _quant_block(fmax=0.0) == -1
    # empty tensors are valid and launch nothing
    assert _quant_block(m=0) == 0 and L.pcamd_last_error() == b""
    rc = L.pcamd_quant_channel(FAKE, _lib.BF16, 1, 4, 256, 0, 256, 1, FAKE, _lib.E4M3FN, 0, 256, 1,
                               FAKE, 0, 1, 0, 448.0, 1e-12, None)
    assert rc == -1 and b"channel_axis" in L.pcamd_last_error()


def test_quant_ex_flags_are_checked():
    L = _lib.lib()
    head = (FAKE, _lib.BF16, 1, 4, 256, 0, 256, 1)
    rc = L.pcamd_quant_block_ex(*head, FAKE, _lib.E4M3FN, 0, 256, 1, FAKE, 0, 2, 1, 1, 128, 448.0, 1e-12, 2, None)
    assert rc == -1 and b"flags" in L.pcamd_last_error()
    rc = L.pcamd_quant_block_dual_ex(*head, FAKE, 0, 256, 1, FAKE, 0, 256, 1, _lib.E4M3FN, FAKE, 0, 2, 1,
                                     FAKE, 0, 256, 1, 128, 448.0, 1e-12, 4, None)
    assert rc == -1 and b"flags" in L.pcamd_last_error()
    # a valid flag reaches the same validation as the call without _ex
    rc = L.pcamd_quant_block_ex(*head, FAKE, _lib.E4M3FN, 0, 256, 1, FAKE, 0, 2, 1, 3, 128, 448.0, 1e-12,
                                _lib.QUANT_CACHED_OUTPUT, None)
    assert rc == -1 and b"powers of two" in L.pcamd_last_error()
    rc = L.pcamd_quant_block_ex(*head[:3], 0, *head[4:], FAKE, _lib.E4M3FN, 0, 256, 1, FAKE, 0, 2, 1, 1, 128,
                                448.0, 1e-12, _lib.QUANT_CACHED_OUTPUT, None)
    assert rc == 0 and L.pcamd_last_error() == b""


def _bmm(**over):
    args = dict(a=FAKE, b=FAKE, abd=_lib.E4M3FN, B=1, M=128, N=128, K=128,
                sab=0, sam=128, sak=1, sbb=0, sbk=128, sbn=1, c=FAKE, cd=_lib.BF16,
                scb=0, scm=128, scn=1, bias=None, biasd=0, sbb0=0, sbm=0, sbn0=0,
                sa=FAKE, ssab=0, ssa1=1, ssa2=1, sb=FAKE, ssbb=0, ssb1=1, ssb2=1,
                mode=_lib.SCALE_BLOCK, saq=0, qbm=1, qbk=128, qbn=128, act=0, st=None)
    args.update(over)
    return _lib.lib().pcamd_bmm_scaled(*args.values())


@pytest.mark.parametrize("over,msg", [
    (dict(abd=_lib.BF16), b"fp8"),
    (dict(cd=9), b"output dtype"),
    (dict(qbk=64), b"multiple of 128"),
    (dict(qbk=192), b"multiple of 128"),
    (dict(act=5), b"activation"),
    (dict(mode=7), b"scale mode"),
    (dict(sak=2, sam=2), b"contiguous along K or M"),
    (dict(scn=2), b"contiguous along N"),
    (dict(sa=None), b"null"),
])
def test_bmm_invalid_arguments(over, msg):
    assert _bmm(**over) == -1
    assert msg in _lib.lib().pcamd_last_error()


def test_bmm_empty_is_ok():
    assert _bmm(M=0) == 0


def _repack(**over):
    args = dict(x=FAKE, b=1, r=256, c=128, sxb=0, sxr=1, sxc=256, y=FAKE, syb=0, syr=128, syc=1, st=None)
    args.update(over)
    return _lib.lib().pcamd_repack_fp8(*args.values())


@pytest.mark.parametrize("over,rc,msg", [
    (dict(r=-1), -1, b"negative size"),
    (dict(x=None), -1, b"null pointer"),
    (dict(sxr=2), -2, b"contiguous along rows"),
    (dict(syc=4), -2, b"contiguous along columns"),
    (dict(sxc=100), -1, b"overlap"),
    (dict(b=70000), -2, b"grid too large"),
])
def test_repack_invalid_arguments(over, rc, msg):
    assert _repack(**over) == rc
    assert msg in _lib.lib().pcamd_last_error()


def test_repack_empty_is_ok():
    assert _repack(r=0) == 0 and _repack(c=0) == 0 and _repack(b=0) == 0


def _bmm_quant_a(**over):
    args = dict(a=FAKE, ad=_lib.BF16, b=FAKE, abd=_lib.E4M3FN, B=1, M=128, N=128, K=256,
                sab=0, sam=256, sak=1, sbb=0, sbk=128, sbn=1, c=FAKE, cd=_lib.BF16, scb=0, scm=128, scn=1,
                bias=None, biasd=0, sbb0=0, sbm=0, sbn0=0, sb=FAKE, ssbb=0, ssb1=1, ssb2=1, qbn=128,
                qa=None, sqab=0, sqam=0, sqak=0, sa=None, soab=0, soam=0, soak=0,
                fmax=448.0, eps=1e-12, act=0, st=None)
    args.update(over)
    return _lib.lib().pcamd_bmm_quant_a(*args.values())


@pytest.mark.parametrize("over,rc,msg", [
    (dict(ad=_lib.F32), -1, b"bf16"),
    (dict(abd=_lib.BF16), -1, b"fp8"),
    (dict(cd=9), -1, b"output dtype"),
    (dict(bias=FAKE, biasd=_lib.E4M3FN), -1, b"bias dtype"),
    (dict(M=-1), -1, b"negative size"),
    (dict(act=3), -1, b"activation"),
    (dict(fmax=0.0), -1, b"fp8_max"),
    (dict(eps=-1.0), -1, b"eps"),
    (dict(qbn=96), -1, b"power of two"),
    (dict(qa=FAKE), -1, b"together"),
    (dict(sb=None), -1, b"null"),
    (dict(scn=2), -1, b"contiguous along N"),
    # outside the fused envelope: the caller quantizes, then multiplies
    (dict(K=200), -2, b"multiple of 128"),
    (dict(sak=128, sam=1), -2, b"K-major"),
])
def test_bmm_quant_a_invalid_arguments(over, rc, msg):
    assert _bmm_quant_a(**over) == rc
    assert msg in _lib.lib().pcamd_last_error()


def test_bmm_quant_a_empty_is_ok():
    assert _bmm_quant_a(M=0) == 0 and _bmm_quant_a(N=0) == 0 and _bmm_quant_a(B=0) == 0
    assert _lib.lib().pcamd_last_error() == b""


@pytest.mark.parametrize("n,k,qbn,inside", [
    (16, 256, 128, True), (64, 512, 128, True), (192, 4096, 256, True), (256, 256, 128, True),
    (272, 4096, 128, False),   # wider than one workgroup's columns
    (120, 4096, 128, False),   # N not a multiple of 16
    (128, 384, 128, False),    # K not a multiple of 256
    (128, 128, 128, False),    # K below two blocks
    (128, 4096, 64, False),    # quant-N blocks under 128
    (0, 4096, 128, False),
])
def test_fused_streams_envelope(n, k, qbn, inside):
    # the products hip_per_block_bmm_quant_a sends to the fused entry point by
    # default: the streaming kernel's envelope (bmm_fused_stream_ok)
    from practice_cuda_amd.impls.hip_per_block import fused_streams
    assert fused_streams(n, k, qbn) is inside
