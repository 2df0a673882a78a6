// bmm_lds.h - direct global -> LDS loading of MN-major FP8 operand tiles and
// their transposing fragment reads, shared by the BMM kernels.
//
// An MN-major operand tile is 128 k-rows of COLS contiguous bytes (256 here),
// copied into LDS row for row by buffer_load_dwordx4 ... lds, 16 B per lane,
// with no VGPR staging. Chunk c (16 B) of k-row k sits at position
// c ^ swz_mn(k). MFMA fragments are read with ds_read_b64_tr_b8: within a
// 16-lane group lane j addresses 8 bytes of k-row (k0 + j / 2) at column
// (col0 + 8 (j & 1)), and lane c receives column (col0 + c) of those eight
// k-rows, i.e. 8 consecutive k of its own m / n.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "fp8_common.h"

namespace pcamd {
namespace lds {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i* lds_v2i_ptr;

constexpr int BK = 128;                       // k-rows per tile (one K step)
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // gfx9-family raw buffer descriptor

// Buffer descriptor in four SGPRs: base, byte size (the hardware returns 0
// for offsets at or past it), raw addressing.
PCAMD_DEV v4i make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  v4i r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = kRsrcWord3;
  return r;
}

PCAMD_DEV uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)p)));
}

// 16 bytes per lane global -> LDS: lane i's bytes land at lds + 16 i. Issued
// from inline asm on purpose: the compiler's wait-count pass cannot tell
// that LDS reads of another stage do not alias these writes and would put a
// vmcnt(0) in front of every ds_read. Kernels order these loads themselves
// (s_waitcnt vmcnt(0) + barrier before a stage is read, barrier before it is
// refilled).
PCAMD_DEV void lds_dma16(v4i rs, uint32_t lds, uint32_t voff) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(lds) : "memory");
}

// MN-major swizzle for 256-byte k-rows: c ^ (k & 7) ^ (8 ((k >> 5) & 1)). A
// 16-lane group reads 8 k-rows k0..k0+7 (k0 % 8 == 0) at one 8-byte half
// pair: k & 7 spreads them over 32 banks, and the group served in the same
// cycle (k-rows 32 further on) lands in the other 32.
PCAMD_DEV int swz_mn(int k) { return (k & 7) ^ (((k >> 5) & 1) << 3); }

// MN-major tile loader for WAVES waves: 128 k-rows (k0 + k, stride ld) x COLS
// bytes from col0. Instruction i of wave w fills k-rows kb = w * PER_WAVE +
// i * R .. + R - 1 (R = 64 / (COLS / 16) rows per instruction); lane l takes
// k-row kb + l / CHUNKS and LDS slot l % CHUNKS, which holds global chunk
// slot ^ swz_mn(k). Bit 5 of k is the wave's (PER_WAVE is 16 or 32, so a
// wave's k-rows never straddle a multiple of 32), and k & 7 repeats every two
// instructions, so two lane offsets per wave serve them all. The per-lane part
// of the offset is computed once; the uniform part (tile origin, K step,
// instruction) in SGPRs, hidden from the optimiser so it cannot hoist one
// loop-invariant VGPR per instruction out of a K loop.
template <int COLS, int WAVES>
struct MNMajorLoader {
  static constexpr int CHUNKS = COLS / 16;
  static constexpr int R = 64 / CHUNKS;
  static constexpr int PER_WAVE = BK / WAVES;
  static constexpr int INSTS = PER_WAVE / R;
  static_assert(COLS == 256 && (PER_WAVE == 16 || PER_WAVE == 32),
                "swizzle assumes 256-byte k-rows, 16 or 32 per wave");
  uint32_t voff[2];
  PCAMD_DEV MNMajorLoader(uint32_t ld, int lane, int wave) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = wave * PER_WAVE + h * R + lane / CHUNKS;
      voff[h] = (lane / CHUNKS) * ld + (((lane % CHUNKS) ^ swz_mn(k)) << 4);
    }
  }
  PCAMD_DEV void issue(v4i rs, uint8_t* tile, uint32_t col0, uint32_t ld, uint32_t k0, int wave) const {
    issue(rs, lds_addr(tile), col0, ld, k0, wave);
  }
  // instruction i of issue() alone (0 <= i < INSTS)
  PCAMD_DEV void issue_one(v4i rs, uint32_t tile_lds, uint32_t col0, uint32_t ld, uint32_t k0, int wave,
                           int i) const {
    const int kb = wave * PER_WAVE + i * R;
    uint32_t u = __builtin_amdgcn_readfirstlane((k0 + kb) * ld + col0);
    asm volatile("" : "+s"(u));
    lds_dma16(rs, tile_lds + kb * COLS, voff[i & 1] + u);
  }
  // tile_lds: LDS byte address of the tile
  PCAMD_DEV void issue(v4i rs, uint32_t tile_lds, uint32_t col0, uint32_t ld, uint32_t k0, int wave) const {
#pragma unroll
    for (int i = 0; i < INSTS; ++i) {
      const int kb = wave * PER_WAVE + i * R;
      uint32_t u = __builtin_amdgcn_readfirstlane((k0 + kb) * ld + col0);
      asm volatile("" : "+s"(u));
      lds_dma16(rs, tile_lds + kb * COLS, voff[i & 1] + u);
    }
  }
};

// fragment of an MN-major tile (COLS bytes per k-row): column block
// [col16, col16 + 16) (16-aligned), lane j = lane & 15, k-group g: lane
// (j, g) receives k bytes [32 g, 32 g + 32) of column col16 + j
template <int COLS>
PCAMD_DEV v8i frag_mn(const uint8_t* tile, int col16, int lane) {
  const int g = lane >> 4, j = lane & 15;
  const int c = col16 >> 4;       // chunk holding the 16 columns
  const int half = (j & 1) << 3;  // lane pairs cover 8 + 8 columns
  v8i f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int k = 32 * g + 8 * q + (j >> 1);
    const uint8_t* p = tile + k * COLS + ((c ^ swz_mn(k)) << 4) + half;
    const v2i v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_ptr)(p));
    f[2 * q] = v[0];
    f[2 * q + 1] = v[1];
  }
  return f;
}

}  // namespace lds
}  // namespace pcamd
