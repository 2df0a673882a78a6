// bmm_fast.h - arguments and launcher of the tuned FP8 BMM path (bmm_fast.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pcamd {

struct FastArgs {
  const uint8_t* a;
  const uint8_t* b;
  void* c;
  const void* bias;
  const float* sa;
  const float* sb;
  int32_t m, n, k;
  int64_t sab, sbb;            // batch strides of a / b (bytes)
  uint32_t lda, ldb;           // stride between the rows the kernel walks (bytes):
                               //   A k-major: m rows; A m-major: k rows
                               //   B k-major: n rows; B n-major: k rows
  uint32_t a_extent, b_extent; // bytes addressable in one batch slice (buffer bounds)
  int64_t scb, scm, scn;
  int64_t sbiasb, sbiasm, sbiasn;
  int64_t ssab, ssa1, ssa2, ssbb, ssb1, ssb2;
  int32_t qbk, qbm_shift, qbn_shift;
  int32_t tiles_m, tiles_n, tiles_per_batch, total_tiles;
  int32_t tile_base;           // first tile of a launch that covers a range of tiles
  int32_t c_dtype, bias_dtype, act, scales_are_quant;
  // fused A quantization (bmm_fused_launch only): `a` holds 16-bit values
  // (lda, sab and a_extent in bytes) quantized in the kernel in 1 x 128 groups
  // with fp8_max / eps; qa_out / sa_out (both or neither) receive the fp8
  // bytes and dequant scales, written by the workgroups of the first N tile.
  uint8_t* qa_out;
  float* sa_out;
  int64_t sqab, sqam;          // qa_out strides (elements; contiguous along k)
  int64_t soab, soam, soak;    // sa_out strides (elements)
  float fp8_max, eps;
};

// mode: 0 block, 1 channel, 2 tensor
int bmm_fast_launch(const FastArgs& a, int ab_dtype, bool a_k, bool b_k, int mode, bool sb_col, bool qb1,
                    hipStream_t st);
int bmm_fast_tile_m();
int bmm_fast_tile_n();

// 128 x 256-tile kernel with the A operand quantized inside the K loop:
// a_dtype PCAMD_BF16 / PCAMD_F16 (K-major, 16-byte aligned rows), block
// scales on B with quant_block_k == 128 (sb_col: qbn < 16), fmt the fp8 code
// of B and of the quantized A
int bmm_fused_launch(const FastArgs& a, int a_dtype, int fmt, bool b_k, bool sb_col, hipStream_t st);

// the same product for narrow N (bmm_fused_stream.hip): A streamed once,
// quantized in registers; bmm_fused_stream_ok is its envelope (N <= 256,
// N % 16 == 0, K % 256 == 0, qbn >= 128, C contiguous along N)
bool bmm_fused_stream_ok(const FastArgs& a, int64_t batch, int64_t qbn);
int bmm_fused_stream_launch(const FastArgs& a, int a_dtype, int fmt, bool b_k, int64_t batch, hipStream_t st);

// persistent streaming kernel for K == 128, N == 512, A K-major, B N-major,
// 1 x 128 A scales and column-block B scales, plain bf16 output
// (bmm_stream.hip); bmm_stream_ok is the host-side envelope check
bool bmm_stream_ok(const FastArgs& a, bool a_k, bool b_k, int mode, int64_t batch, int64_t qbm, int64_t qbn,
                   int64_t ssa1, int64_t ssb2);
int bmm_stream_launch(const FastArgs& a, int ab_dtype, int64_t batch, hipStream_t st);

// 256 x 256-tile, 8-wave kernel for two or more K steps (bmm_wide.h,
// bmm_wide*.hip); K a multiple of 4 (a last K step of fewer than 128 is
// masked); block mode requires quant_block_k == 128 and power-of-two qbm /
// qbn. a_fmt / b_fmt: the fp8 format of each operand (PCAMD_FP8_*).
int bmm_wide_launch(const FastArgs& a, int a_fmt, int b_fmt, bool a_k, bool b_k, int mode, hipStream_t st);
int bmm_wide_tile();

}  // namespace pcamd
