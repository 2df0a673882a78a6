/*
 * pcamd_fp8_selftest.h - test and measurement entry points of
 * libpcamd_fp8.so.
 *
 * Not part of the product interface (include/pcamd_fp8.h): the test suite
 * calls them to pin the hardware fp8 conversion the quantizers use, and
 * bench.py to measure the plain-copy and narrowing ceilings the quantizers
 * are compared with. They have no counterpart in the reference (xuOAO/practice_cuda),
 * whose fp8 casts are Triton's `.to(fp8)`
 * (fp8_training/fp8_bench/kernels/quant/per_block.py:47).
 */
#ifndef PCAMD_FP8_SELFTEST_H
#define PCAMD_FP8_SELFTEST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * Device self-test of the fp32 -> fp8 conversion used by the quantizers:
 * compares the gfx950 hardware conversion with an integer restatement of
 * round-to-nearest-even over every fp32 bit pattern with |x| <= fp8 max.
 * result (device, 4 x uint32) receives {mismatches, first mismatching
 * pattern, checked count low 32 bits, 0}. fmt is PCAMD_E4M3FN (3) or
 * PCAMD_E5M2 (4). Returns 0 or a negative status (see pcamd_fp8.h).
 */
int pcamd_selftest_fp8_convert(int fmt, uint32_t *result, void *stream);

/*
 * Plain device copy y[i] = x[i] of `bytes` bytes (a multiple of 16, both
 * pointers 16-byte aligned) in the quantizers' streaming layout: one 16-byte
 * non-temporal load and store per lane, 256-thread workgroups. The 1 : 1
 * read/write ceiling the dual quantizer is measured against. Returns 0 or a
 * negative status.
 */
int pcamd_selftest_copy16(const void *x, void *y, int64_t bytes, void *stream);

/*
 * Plain device narrowing: y receives the high byte of every 16-bit element
 * of x (in_bytes a multiple of 16; x 16-byte and y 8-byte aligned; y holds
 * in_bytes / 2 bytes), in the 1 x 128 quantizer's streaming layout: each
 * lane loads two 16-byte chunks 64 apart (non-temporal) and then stores
 * their 8-byte results (non-temporal), 256-thread workgroups. The
 * quantizers' 2 : 1 read/write mix with no arithmetic, the ceiling they are
 * measured against.
 * Returns 0 or a negative status.
 */
int pcamd_selftest_narrow16(const void *x, void *y, int64_t in_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* PCAMD_FP8_SELFTEST_H */
