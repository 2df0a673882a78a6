// bmm_epilogue.h - LDS-staged 16-bit (bf16 / fp16) output of one wave's 64 x 128 sub-tile.
//
// With the MFMA operands swapped, a lane holds 4 consecutive columns of one
// row per 16 x 16 tile, so direct stores write 32-byte pieces of 16 rows per
// instruction (16 partial-line requests each). Staging through LDS lets each
// lane store 16 contiguous bytes instead: an instruction covers 4 rows x 256
// contiguous bytes, i.e. full 128-byte lines. The stores are non-temporal:
// C is written once and should not evict the operand tiles from L2.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "fp8_common.h"

namespace pcamd {

// Two floats to bf16 (round to nearest even), lo in the low half. Converted
// as a pair so that it is one v_cvt_pk_bf16_f32; converting each float on
// its own costs two of them plus a shift and an OR.
PCAMD_DEV uint32_t pack_bf16_pair(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Two floats to fp16 (round to nearest even), lo in the low half.
PCAMD_DEV uint32_t pack_f16_pair(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));
}

// 16-bit output element: bf16 or fp16 (the dtype codes of fp8_common.h), or
// OUT16_RUNTIME: the one picked by out_f16 at run time
constexpr int OUT16_RUNTIME = -1;
template <int OUT>
PCAMD_DEV uint32_t pack16_pair(float lo, float hi, bool out_f16 = false) {
  if constexpr (OUT == kF16) return pack_f16_pair(lo, hi);
  else if constexpr (OUT == kBF16) return pack_bf16_pair(lo, hi);
  else return out_f16 ? pack_f16_pair(lo, hi) : pack_bf16_pair(lo, hi);
}

// Whether the staged path applies: a 16-bit output (bf16 or fp16), 16-byte
// aligned rows and N a multiple of 8 (a lane's 8 columns never straddle N).
// Bias is applied by the caller's value function.
PCAMD_DEV bool staged_output_ok(const void* c, int64_t scb, int64_t scm, int n, bool out16) {
  return out16 && (n & 7) == 0 && (scm & 7) == 0 && (scb & 7) == 0 && (reinterpret_cast<uintptr_t>(c) & 15) == 0;
}

// stg: 8 KiB of LDS private to this wave. c: the batch's C (OUT elements, row
// pitch scm elements). The sub-tile covers rows row0 .. row0 + 63 and columns
// col0 .. col0 + 127; value(i, j, v) fills the 4 outputs of this lane in
// MFMA tile (i, j): row row0 + 16 i + (lane & 15), columns
// col0 + 16 j + 4 (lane >> 4) + r. The sub-tile goes out in two halves of
// 32 rows; staged chunk c of row r sits at LDS position c ^ (r & 15).
template <int OUT = kBF16, typename ValueFn>
PCAMD_DEV void store_subtile_staged(uint8_t* stg, uint16_t* c, int64_t scm, int m, int n, int row0, int col0,
                                    int lane, ValueFn&& value, bool out_f16 = false) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int il = 0; il < 2; ++il) {
        float v[4];
        value(2 * h + il, j, v);
        const int r = 16 * il + lr;
        const int chunk = 2 * j + (lg >> 1);
        uint2* dst = reinterpret_cast<uint2*>(stg + r * 256 + ((chunk ^ (r & 15)) << 4) + ((lg & 1) << 3));
        *dst = make_uint2(pack16_pair<OUT>(v[0], v[1], out_f16), pack16_pair<OUT>(v[2], v[3], out_f16));
      }
    }
    // LDS operations of one wave complete in order; the wait keeps the
    // compiler from moving the reads above the writes.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int r = 4 * it + (lane >> 4);
      const int chunk = lane & 15;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * 256 + ((chunk ^ (r & 15)) << 4));
      const int mm = row0 + 32 * h + r;
      const int nn = col0 + 8 * chunk;
      if (mm < m && nn < n) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(c + int64_t(mm) * scm + nn));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// Half-width variant: stg is 4 KiB of LDS private to this wave; the region
// covers rows row0 .. row0 + 63 and columns col0 .. col0 + 63, and
// value(i, jj, v) fills the 4 outputs of this lane in MFMA tile (i, jj): row
// row0 + 16 i + (lane & 15), columns col0 + 16 jj + 4 (lane >> 4) + r. Two
// pieces of 32 rows; staged chunk c of row r sits at LDS position c ^ (r & 7).
// Each store instruction writes 8 rows x 128 contiguous bytes.
template <int OUT = kBF16, typename ValueFn>
PCAMD_DEV void store_half_staged(uint8_t* stg, uint16_t* c, int64_t scm, int m, int n, int row0, int col0, int lane,
                                 ValueFn&& value, bool out_f16 = false) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int lr = lane & 15, lg = lane >> 4;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
      for (int il = 0; il < 2; ++il) {
        float v[4];
        value(2 * h + il, jj, v);
        const int r = 16 * il + lr;
        const int chunk = 2 * jj + (lg >> 1);
        uint2* dst = reinterpret_cast<uint2*>(stg + r * 128 + ((chunk ^ (r & 7)) << 4) + ((lg & 1) << 3));
        *dst = make_uint2(pack16_pair<OUT>(v[0], v[1], out_f16), pack16_pair<OUT>(v[2], v[3], out_f16));
      }
    }
    // LDS operations of one wave complete in order; the wait keeps the
    // compiler from moving the reads above the writes.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int r = 8 * it + (lane >> 3);
      const int chunk = lane & 7;
      const u32x4 v = *reinterpret_cast<const u32x4*>(stg + r * 128 + ((chunk ^ (r & 7)) << 4));
      const int mm = row0 + 32 * h + r;
      const int nn = col0 + 8 * chunk;
      if (mm < m && nn < n) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(c + int64_t(mm) * scm + nn));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
}

// Transposed output of one wave's 64 x (16 * JN) sub-tile: the kernel
// computed C' = B^T A^T, and C (the caller's) holds its transpose, so the
// lane's 4 consecutive n' of one m' go to 4 rows of C at one column. stg: 16
// KiB of LDS private to this wave, laid out as the wave's block of C: staged
// row R = n' - col0 (16 * JN rows), 64 m' per row (128 bytes), 16-byte chunk
// q of row R at position q ^ (R & 7). Lanes pair up (lane ^ 1 holds the next
// m'): each lane of a pair writes one dword (two m') to two of the four rows,
// after one DPP swap. Each store instruction then writes 8 rows x 128
// contiguous bytes of C. c: the batch's C, row pitch ld elements; rows n' <
// n and columns m' < m are stored (m a multiple of 8).
template <int OUT, int JN, typename ValueFn>
PCAMD_DEV void store_subtile_staged_t(uint8_t* stg, uint16_t* c, int64_t ld, int m, int n, int row0, int col0,
                                      int lane, ValueFn&& value, bool out_f16 = false) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int lr = lane & 15, lg = lane >> 4;
  const bool odd = lr & 1;
  auto swap1 = [](float x) {  // the value of lane ^ 1 (DPP quad_perm [1, 0, 3, 2])
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0xB1, 0xF, 0xF, false));
  };
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < JN; ++j) {
      float v[4];
      value(i, j, v);
      // the even lane keeps rows 0, 1 of the four, the odd one rows 2, 3;
      // each sends its partner the two values it keeps
      const float r0 = swap1(odd ? v[0] : v[2]), r1 = swap1(odd ? v[1] : v[3]);
      const uint32_t w0 = pack16_pair<OUT>(odd ? r0 : v[0], odd ? v[2] : r0, out_f16);
      const uint32_t w1 = pack16_pair<OUT>(odd ? r1 : v[1], odd ? v[3] : r1, out_f16);
      const int rr = 16 * j + 4 * lg + (odd ? 2 : 0);
      const int byte = 2 * (16 * i + (lr & ~1));  // the pair's even m', 4-byte aligned
      const int q = byte >> 4, within = byte & 15;
      *reinterpret_cast<uint32_t*>(stg + rr * 128 + ((q ^ (rr & 7)) << 4) + within) = w0;
      *reinterpret_cast<uint32_t*>(stg + (rr + 1) * 128 + ((q ^ ((rr + 1) & 7)) << 4) + within) = w1;
    }
  }
  // LDS operations of one wave complete in order; the wait keeps the
  // compiler from moving the reads above the writes.
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int it = 0; it < 2 * JN; ++it) {
    const int rr = 8 * it + (lane >> 3);
    const int q = lane & 7;
    const u32x4 v = *reinterpret_cast<const u32x4*>(stg + rr * 128 + ((q ^ (rr & 7)) << 4));
    const int nn = col0 + rr;
    const int mm = row0 + 8 * q;
    if (nn < n && mm < m) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(c + int64_t(nn) * ld + mm));
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

}  // namespace pcamd
