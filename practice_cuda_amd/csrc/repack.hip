// repack.hip - transposing byte copy of fp8 tensors behind the C ABI
// (pcamd_repack_fp8 in include/pcamd_fp8.h).
//
// The BMM wrappers' do_transpose_a / do_transpose_b variants turn an M-major
// A or an N-major B into a K-major copy before the GEMM
// (xuOAO/practice_cuda fp8_training/fp8_bench/impls/triton_per_block.py:254-272,
// `.contiguous()` on the strided view). For one-byte elements torch runs that
// copy as a strided elementwise kernel at about 0.5 TB/s on MI355X, 13 times
// slower than a plain copy of the same bytes. This kernel moves the same
// bytes through LDS in 128 x 128 tiles:
//   - a thread loads 16 consecutive rows of four consecutive columns (four
//     16-byte loads along the contiguous row dimension; a wave reads eight
//     columns x 128 contiguous bytes per instruction);
//   - four 4 x 4 byte transposes in registers turn them into 16 rows x 4
//     columns, which go to LDS as dwords ([row][dword column], pitch 33
//     dwords: at most 2-way bank conflicts);
//   - a thread then reads four dwords of one row and stores them as 16
//     contiguous output bytes (a wave writes eight rows x 128 bytes).
// Views whose pointers or byte strides are not 16-byte aligned take the same
// tiles with byte loads and stores; tiles at the ragged edges mask per byte.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "abi_util.h"
#include "fp8_common.h"

namespace pcamd {
namespace repack {

constexpr int NT = 256;
constexpr int TR = 128, TC = 128;  // tile rows (contiguous in x) and columns (contiguous in y)
constexpr int PITCH = TC / 4 + 1;  // LDS dwords per tile row

struct Args {
  const uint8_t* x;
  uint8_t* y;
  int64_t rows, cols;
  int64_t sxb, sxc;  // x: element (r, c) of batch b at b * sxb + c * sxc + r
  int64_t syb, syr;  // y: element (r, c) of batch b at b * syb + r * syr + c
};

// VEC: pointers and byte strides are 16-byte aligned (16-byte loads and
// stores where a whole vector lies inside the matrix)
template <bool VEC>
__global__ __launch_bounds__(NT) void repack_kernel(Args a) {
  __shared__ uint32_t tile[TR * PITCH];
  const int t = threadIdx.x;
  const int64_t b = blockIdx.z;
  const int64_t r0 = int64_t(blockIdx.y) * TR, c0 = int64_t(blockIdx.x) * TC;
  const uint8_t* xb = a.x + b * a.sxb;
  uint8_t* yb = a.y + b * a.syb;

  // load: rows r .. r + 15 of columns c .. c + 3
  const int cq = t >> 3, rb = t & 7;
  const int64_t r = r0 + 16 * rb;
  u32x4_t v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int64_t c = c0 + 4 * cq + j;
    v[j] = u32x4_t{0u, 0u, 0u, 0u};
    if (c >= a.cols || r >= a.rows) continue;
    const uint8_t* src = xb + c * a.sxc + r;
    if (VEC && r + 16 <= a.rows) {
      v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src));
    } else {
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      for (int k = 0; k < 16 && r + k < a.rows; ++k) w[k >> 2] |= uint32_t(src[k]) << (8 * (k & 3));
      v[j] = u32x4_t{w[0], w[1], w[2], w[3]};
    }
  }
  // rows 16 rb + 4 q + k: byte i of dword e[k] is column 4 cq + i
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t e[4];
    byte_transpose4(v[0][q], v[1][q], v[2][q], v[3][q], e);
#pragma unroll
    for (int k = 0; k < 4; ++k) tile[(16 * rb + 4 * q + k) * PITCH + cq] = e[k];
  }
  __syncthreads();

  // store: 16 bytes (columns 16 ch ..) of rows rr = t / 8 + 32 i
  const int ch = t & 7;
  const int64_t col = c0 + 16 * ch;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rr = (t >> 3) + 32 * i;
    const int64_t row = r0 + rr;
    if (row >= a.rows || col >= a.cols) continue;
    const uint32_t* src = tile + rr * PITCH + 4 * ch;
    const u32x4_t o = {src[0], src[1], src[2], src[3]};
    uint8_t* dst = yb + row * a.syr + col;
    if (VEC && col + 16 <= a.cols) {
      __builtin_nontemporal_store(o, reinterpret_cast<u32x4_t*>(dst));
    } else {
      for (int k = 0; k < 16 && col + k < a.cols; ++k) dst[k] = static_cast<uint8_t>(o[k >> 2] >> (8 * (k & 3)));
    }
  }
}

}  // namespace repack
}  // namespace pcamd

extern "C" int pcamd_repack_fp8(const void* x, int64_t batch, int64_t rows, int64_t cols, int64_t sxb, int64_t sxr,
                                int64_t sxc, void* y, int64_t syb, int64_t syr, int64_t syc, void* stream) {
  using namespace pcamd;
  clear_error();
  if (batch < 0 || rows < 0 || cols < 0) return set_error(PCAMD_ERR_INVALID, "negative size");
  if (batch == 0 || rows == 0 || cols == 0) return PCAMD_OK;
  if (!x || !y) return set_error(PCAMD_ERR_INVALID, "null pointer");
  if (sxr != 1 || syc != 1)
    return set_error(PCAMD_ERR_UNSUPPORTED,
                     "repack reads a view contiguous along rows and writes one contiguous along columns "
                     "(got x row stride %lld, y column stride %lld)", (long long)sxr, (long long)syc);
  if (sxb < 0 || sxc < rows || syb < 0 || syr < cols)
    return set_error(PCAMD_ERR_INVALID, "strides overlap the rows / columns they step over");
  if (batch > 65535 || (rows + repack::TR - 1) / repack::TR > 65535 || (cols + repack::TC - 1) / repack::TC > INT32_MAX)
    return set_error(PCAMD_ERR_UNSUPPORTED, "repack: grid too large (batch %lld, rows %lld, cols %lld)",
                     (long long)batch, (long long)rows, (long long)cols);
  repack::Args a{};
  a.x = static_cast<const uint8_t*>(x);
  a.y = static_cast<uint8_t*>(y);
  a.rows = rows;
  a.cols = cols;
  a.sxb = sxb;
  a.sxc = sxc;
  a.syb = syb;
  a.syr = syr;
  const dim3 grid(static_cast<uint32_t>((cols + repack::TC - 1) / repack::TC),
                  static_cast<uint32_t>((rows + repack::TR - 1) / repack::TR), static_cast<uint32_t>(batch));
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0 &&
                   sxb % 16 == 0 && sxc % 16 == 0 && syb % 16 == 0 && syr % 16 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (vec) repack::repack_kernel<true><<<grid, repack::NT, 0, st>>>(a);
  else repack::repack_kernel<false><<<grid, repack::NT, 0, st>>>(a);
  return check_launch("repack_kernel");
}
