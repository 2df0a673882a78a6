// bmm_wide.h - large-tile scaled FP8 BMM for gfx950 (at least two K steps of
// 128; 16-byte aligned operands). The kernel and its launch templates; the
// translation units bmm_wide*.hip instantiate them per pair of operand
// formats, so those compile in parallel.
//
// Workgroup: 512 threads = 8 waves (4 along M x 2 along N), output tile
// 256 x 256, K step 128, two LDS stages of 64 KiB. Two waves per SIMD, so one
// wave's MFMAs cover the other's LDS reads, waits and scale folding. Each wave
// owns 64 x 128 = 4 x 8 tiles of v_mfma_f32_16x16x128_f8f6f4, issued with the
// operands swapped so a lane holds four consecutive N outputs of one row.
//
// Half tiles: when the last wave of tiles would fill at most half the CUs
// (e.g. 896 tiles on 256 CUs), those tiles run as a second launch of
// 256 x 128 halves, two workgroups per tile, each wave computing 64 x 64
// (JN = 4 sub-tiles instead of 8). A half loads the whole tile's operands -
// the loaders and LDS layout are the same - and reads the B fragments of its
// own 128 columns, so it takes more than half of a whole tile's time.
//
// Both operands go global -> LDS with buffer_load_dwordx4 ... lds (no VGPR
// staging), one K step ahead of the MFMAs. The LDS layout follows the global
// one:
//   K-major operand (rows contiguous along k): [row][8 x 16 B], chunk c of
//     row r at position c ^ swz_k(r) (below); fragments are two
//     ds_read_b128 per lane.
//   MN-major operand (k rows contiguous along m / n): [k][16 x 16 B], chunk c
//     of k-row k at position c ^ swz_mn(k) (bmm_lds.h); fragments are four
//     ds_read_b64_tr_b8 per lane. Within a 16-lane group, lane j addresses
//     8 bytes of k-row (k0 + j / 2) at column (col0 + 8 (j & 1)), and lane c
//     receives column (col0 + c) of those eight k-rows, i.e. 8 consecutive k
//     of its own m / n.
// Either way a lane ends up with k bytes [32 g, 32 g + 32) of its row (g =
// lane / 16), the same k order for both operands.
//
// Scales: block mode (quant_block_k == 128) folds each step's partial,
// acc += P * (sa * sb) (xuOAO/practice_cuda kernels/bmm/per_block.py:99-111),
// with the step's scales staged in LDS; channel / tensor scales are applied
// once in the epilogue (the tile's channel scales are staged in LDS in the
// prologue). Wider quant-K blocks use bmm_fast.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstdint>
#include <type_traits>

#include "abi_util.h"
#include "bmm_epilogue.h"
#include "bmm_fast.h"
#include "bmm_lds.h"
#include "fp8_common.h"

namespace pcamd {
namespace bmmw {

using lds::v8i;
using lds::v4i;
using lds::make_rsrc;
using lds::lds_addr;
using lds::lds_dma16;
using lds::frag_mn;
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int NT = 512;
constexpr int WAVES = NT / 64;
constexpr int BM = 256, BN = 256, BK = 128;
constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;  // 32 KiB each
constexpr int STAGE = A_BYTES + B_BYTES;
template <int COLS>
using MNMajorLoader = lds::MNMajorLoader<COLS, WAVES>;

// LDS swizzles. gfx950's LDS serves 256 bytes (64 banks) per cycle.
// K-major tile (128-byte rows): chunk c of row r sits at position c ^ swz_k(r).
// A fragment read touches rows r0..r0+15 (lanes 16 g + r) at chunk 2 g + h.
// Measured on gfx950, XOR-ing with r & 7 or with (r >> 1) & 7 both leave every
// ds_read_b128 2-way conflicted: the lanes served together are not 16
// consecutive ones but (among the groupings that fit) eight rows of two
// adjacent g. swz_k = 5 * bit1(r) ^ bit2(r) spreads the 16 (row, chunk) pairs
// of each such group over distinct bank groups for all of them.
template <int N>
using IC = std::integral_constant<int, N>;

PCAMD_DEV int swz_k(int r) { return (((r >> 1) & 1) * 5) ^ ((r >> 2) & 1); }
// Direct-to-LDS loads of one operand tile. The per-lane part of the byte
// offset is the same for every K step (and, for a K-major tile, for every
// instruction), so it is computed once; the uniform part - tile origin, K
// step, instruction - is computed in SGPRs each step and added just before the
// load. The whole offset stays in the VGPR operand, which the descriptor's
// range check covers; the uniform part is hidden from the optimiser so it
// cannot hoist one loop-invariant VGPR per instruction out of the K loop.
//
// K-major tile: ROWS rows (row0 + r, stride ld) x 128 k-bytes. Instruction i
// of wave w fills rows rb = w * ROWS / 8 + 8 i .. rb + 7, lane l taking row
// rb + (l >> 3) and LDS slot l & 7, which holds global chunk
// (l & 7) ^ swz_k(r). rb is a multiple of 8 and swz_k reads only bits 1-2 of
// r, so swz_k(r) = swz_k(l >> 3) and one lane offset serves every instruction.
//
// The row part of the offset (tile origin, instruction, lane) is fixed for the
// tile and kept per instruction in VGPRs; the K step's byte offset k0 goes in
// the instruction's SGPR offset, so no VALU work is issued per load. Rows past
// the matrix are out of range through the VGPR part alone; for rows inside
// it, row * ld + k0 + 127 stays below the row's end (k0 < K <= ld).
template <int ROWS>
struct KMajorLoader {
  static constexpr int PER_WAVE = ROWS / WAVES;
  static constexpr int INSTS = PER_WAVE / 8;
  uint32_t voff[INSTS];
  PCAMD_DEV KMajorLoader(uint32_t ld, int lane, int wave, uint32_t row0) {
    const uint32_t lp = (lane >> 3) * ld + (((lane & 7) ^ swz_k(lane >> 3)) << 4);
#pragma unroll
    for (int i = 0; i < INSTS; ++i) voff[i] = (row0 + wave * PER_WAVE + i * 8) * ld + lp;
  }
  // instruction i (0 <= i < INSTS); tile_lds: LDS byte address of the tile
  PCAMD_DEV void issue_one(v4i rs, uint32_t tile_lds, uint32_t k0, int wave, int i) const {
    const uint32_t lds = tile_lds + (wave * PER_WAVE + i * 8) * BK;
    asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff[i]), "s"(rs), "s"(k0), "{m0}"(lds)
                 : "memory");
  }
  PCAMD_DEV void issue(v4i rs, uint32_t tile_lds, uint32_t k0, int wave) const {
#pragma unroll
    for (int i = 0; i < INSTS; ++i) issue_one(rs, tile_lds, k0, wave, i);
  }
};

// fragment of a K-major tile: row `row`, k bytes [32 g, 32 g + 32)
PCAMD_DEV v8i frag_k(const uint8_t* tile, int row, int g) {
  const uint4* l = reinterpret_cast<const uint4*>(tile + row * BK);
  const int s = swz_k(row);
  const uint4 x = l[(2 * g) ^ s];
  const uint4 y = l[(2 * g + 1) ^ s];
  v8i f;
  f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
  f[4] = y.x; f[5] = y.y; f[6] = y.z; f[7] = y.w;
  return f;
}

// The MFMA is issued with the operands swapped (x: B fragment, y: A
// fragment), so the format code of src0 (cbsz) is B's and that of src1
// (blgp) is A's: 0 e4m3fn, 1 e5m2.
template <int FA, int FB>
PCAMD_DEV v4f mfma(const v8i& x, const v8i& y, const v4f& c) {
  constexpr int ca = FA == kE5M2 ? 1 : 0, cb = FB == kE5M2 ? 1 : 0;
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, c, cb, ca, 0, 0, 0, 0);
}

// Block-mode step for one row block: p_new = A x B (fresh 16x16 partial), then
// acc += p_old * f (the partial of the previous sub-tile, produced four MFMAs
// earlier). One asm block fixes that order: scheduled as separate
// instructions, each fold is hoisted next to the MFMA that produces its input
// and the wave stalls on the result. f[r] is the factor of output r (the same
// value four times when it only depends on the row). p_old was written at
// least three MFMAs and twelve VALU instructions earlier, more than the
// XDL-write -> VALU-read wait states of an 8-pass MFMA.
template <int FA, int FB>
PCAMD_DEV void mfma_fold(const v8i& x, const v8i& y, v4f& p_new, const v4f& p_old, float& a0, float& a1, float& a2,
                         float& a3, float f0, float f1, float f2, float f3) {
#define PCAMD_MFMA_FOLD(MOD)                                                                   \
  asm volatile("v_mfma_f32_16x16x128_f8f6f4 %0, %5, %6, 0" MOD "\n\t"                          \
               "v_fmac_f32_e32 %1, %7, %11\n\t"                                                 \
               "v_fmac_f32_e32 %2, %8, %12\n\t"                                                 \
               "v_fmac_f32_e32 %3, %9, %13\n\t"                                                 \
               "v_fmac_f32_e32 %4, %10, %14"                                                    \
               : "=&v"(p_new), "+v"(a0), "+v"(a1), "+v"(a2), "+v"(a3)                           \
               : "v"(x), "v"(y), "v"(p_old[0]), "v"(p_old[1]), "v"(p_old[2]), "v"(p_old[3]),   \
                 "v"(f0), "v"(f1), "v"(f2), "v"(f3))
  if constexpr (FA == kE5M2 && FB == kE5M2) PCAMD_MFMA_FOLD(" cbsz:1 blgp:1");
  else if constexpr (FA == kE5M2) PCAMD_MFMA_FOLD(" blgp:1");
  else if constexpr (FB == kE5M2) PCAMD_MFMA_FOLD(" cbsz:1");
  else PCAMD_MFMA_FOLD("");
#undef PCAMD_MFMA_FOLD
}


PCAMD_DEV float load_bias(const void* p, int dt, int64_t off) {
  if (dt == kF32) return static_cast<const float*>(p)[off];
  if (dt == kBF16) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[off]) << 16);
  return static_cast<float>(static_cast<const _Float16*>(p)[off]);
}

__device__ __attribute__((noinline)) void epilogue_general(void* c, int64_t c_row, int c_dtype, const void* bias,
                                                          int64_t bias_row, int64_t sbiasn, int bias_dtype, int act,
                                                          int nn, int nvalid, float v0, float v1, float v2, float v3) {
  float v[4] = {v0, v1, v2, v3};
  for (int r = 0; r < nvalid; ++r) {
    float x = v[r];
    const int n = nn + r;
    if (bias) x += load_bias(bias, bias_dtype, bias_row + int64_t(n) * sbiasn);
    if (act == PCAMD_ACT_GELU) x = 0.5f * x * (1.0f + erff(x * 0.7071067811865475f));
    if (c_dtype == kBF16) {
      static_cast<__bf16*>(c)[c_row + n] = static_cast<__bf16>(x);
    } else if (c_dtype == kF16) {
      static_cast<_Float16*>(c)[c_row + n] = static_cast<_Float16>(x);
    } else if (c_dtype == kF32) {
      static_cast<float*>(c)[c_row + n] = x;
    } else {
      const float q = clamp_sym(x, c_dtype == kE5M2 ? 57344.0f : 448.0f);
      const uint32_t w = c_dtype == kE5M2 ? hw_pack4<kE5M2>(q, 0.f, 0.f, 0.f) : hw_pack4<kE4M3>(q, 0.f, 0.f, 0.f);
      static_cast<uint8_t*>(c)[c_row + n] = static_cast<uint8_t>(w & 0xFFu);
    }
  }
}

// MODE: 0 block (qbk == 128), 1 channel, 2 tensor. SBK (block mode): how
// the B scales vary over a wave's 128 columns - 0: one scale (qbn >= 128),
// 1: one per 16-column sub-tile (16 <= qbn < 128), 2: one per column.
//
// Block scales are staged through LDS one K step ahead (sa for the tile's
// 256 rows, sb for its 256 columns), so the fold acc += P * (sa * sb) reads
// them with a few ds_reads instead of holding them in registers.
//
// Schedule of one K step (8 sub-tiles j of 4 MFMAs each, one per row block i):
//   - the B fragment of sub-tile j + 1 is read while sub-tile j issues;
//   - block mode: the MFMA (i, j) writes a fresh partial p[i]; just before it,
//     the previous partial p[i] (sub-tile j - 1, or sub-tile 7 of the previous
//     step) is folded, acc += p * factor, so the 4 fold FMAs of each MFMA run
//     in the matrix core's shadow and one set of partials is live;
//   - the step boundary sits in front of sub-tile 7: wait for the next
//     stage's DMA, barrier, start the DMA two steps ahead, read the next
//     step's first B fragment; the next step's A fragment i is read right
//     after MFMA (i, 7) has consumed the current one. The last sub-tile's
//     MFMAs cover the latency of those reads.
// JN: 16-column sub-tiles per wave - 8 (256 x 256 tiles), 4 (half tiles of
// a short last wave) or 7 (256 x 224 tiles). CT: C receives the transpose of
// this product (the launcher computes C^T = B^T A^T when 224-column tiles
// fill the waves better); only plain 16-bit outputs take it.
template <bool A_K, bool B_K, int FA, int FB, int MODE, int SBK, int JN, bool KT, bool CT = false>
__global__ __launch_bounds__(NT, 1) void bmm_wide_kernel(FastArgs a) {
  static_assert(JN == 8 || JN == 7 || JN == 4, "sub-tiles per wave: 8 (whole tiles), 7 (224-column tiles) or "
                "4 (half tiles)");
  static_assert(!CT || JN == 7, "the transposed output goes with 224-column tiles");
  constexpr int TN = JN == 7 ? 224 : BN;  // tile columns
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float* sa_tile = reinterpret_cast<float*>(smem + 2 * STAGE);  // [2][BM]
  float* sb_tile = sa_tile + 2 * BM;                             // [2][BN]
  const int t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave & 3, wn = wave >> 2;  // 4 x 2 waves
  const int lr = lane & 15, lg = lane >> 4;

  // Tile index (tiles ordered as below) and the wave's first column in it.
  // Whole tiles: consecutive tiles land on one XCD (blockIdx % 8 picks it).
  // Half tiles (tiles tile_base ..): the two halves of a tile go to
  // workgroups b and b + 8, on the same XCD, so both read its operands
  // through one L2.
  int pid = blockIdx.x;
  int wcol = wn * 16 * (JN == 4 ? 8 : JN);
  if constexpr (JN != 4) {
    if ((a.total_tiles & 7) == 0) pid = (pid & 7) * (a.total_tiles >> 3) + (pid >> 3);
  } else {
    int hsel;
    if ((gridDim.x & 15) == 0) {
      hsel = (pid >> 3) & 1;
      pid = a.tile_base + ((pid >> 4) << 3) + (pid & 7);
    } else {
      hsel = pid & 1;
      pid = a.tile_base + (pid >> 1);
    }
    wcol = __builtin_amdgcn_readfirstlane(hsel * 128 + wn * 64);
  }
  // (the divisions run on the VALU; the results are workgroup-uniform and are
  // moved back to SGPRs so everything derived from them stays scalar)
  const int bidx = __builtin_amdgcn_readfirstlane(pid / a.tiles_per_batch);
  const int tile = pid - bidx * a.tiles_per_batch;
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * a.tiles_n;
  const int group = tile / per_group;
  const int first_m = group * GROUP_M;
  const int gm = min(a.tiles_m - first_m, GROUP_M);
  const int in_group = tile - group * per_group;
  const int m0 = __builtin_amdgcn_readfirstlane((first_m + in_group % gm) * BM);
  const int n0 = __builtin_amdgcn_readfirstlane((in_group / gm) * TN);

  const v4i rsa = make_rsrc(a.a + bidx * a.sab, a.a_extent);
  const v4i rsb = make_rsrc(a.b + bidx * a.sbb, a.b_extent);
  using LA = typename std::conditional<A_K, KMajorLoader<BM>, MNMajorLoader<BM>>::type;
  using LB = typename std::conditional<B_K, KMajorLoader<BN>, MNMajorLoader<BN>>::type;
  auto make_loader = [&](auto is_k, uint32_t ld, uint32_t origin) {
    if constexpr (decltype(is_k)::value) return KMajorLoader<BM>(ld, lane, wave, origin);
    else return MNMajorLoader<BM>(ld, lane, wave);
  };
  const LA load_a = make_loader(std::integral_constant<bool, A_K>{}, a.lda, m0);
  const LB load_b = make_loader(std::integral_constant<bool, B_K>{}, a.ldb, n0);

  auto issue = [&](int ks, uint8_t* stage) {
    const uint32_t k0 = __builtin_amdgcn_readfirstlane(ks * BK);
    const uint32_t base = lds_addr(stage);  // one generic -> LDS conversion per step
    if constexpr (A_K) load_a.issue(rsa, base, k0, wave);
    else load_a.issue(rsa, base, m0, a.lda, k0, wave);
    if constexpr (B_K) load_b.issue(rsb, base + A_BYTES, k0, wave);
    else load_b.issue(rsb, base + A_BYTES, n0, a.ldb, k0, wave);
  };
  // instruction q of the A / B loads of K step ks into `stage`
  static_assert(LA::INSTS == 4 && LB::INSTS == 4, "DMA schedule assumes four load instructions per operand");
  auto issue_a1 = [&](int ks, const uint8_t* stage, int q) {
    const uint32_t k0 = __builtin_amdgcn_readfirstlane(ks * BK);
    if constexpr (A_K) load_a.issue_one(rsa, lds_addr(stage), k0, wave, q);
    else load_a.issue_one(rsa, lds_addr(stage), m0, a.lda, k0, wave, q);
  };
  auto issue_b1 = [&](int ks, const uint8_t* stage, int q) {
    const uint32_t k0 = __builtin_amdgcn_readfirstlane(ks * BK);
    if constexpr (B_K) load_b.issue_one(rsb, lds_addr(stage) + A_BYTES, k0, wave, q);
    else load_b.issue_one(rsb, lds_addr(stage) + A_BYTES, n0, a.ldb, k0, wave, q);
  };
  auto afrag = [&](const uint8_t* stage, int i) -> v8i {
    if constexpr (A_K) return frag_k(stage, wm * 64 + i * 16 + lr, lg);
    else return frag_mn<BM>(stage, wm * 64 + i * 16, lane);
  };
  auto bfrag = [&](const uint8_t* stage, int j) -> v8i {
    if constexpr (B_K) return frag_k(stage + A_BYTES, wcol + j * 16 + lr, lg);
    else return frag_mn<BN>(stage + A_BYTES, wcol + j * 16, lane);
  };
  // Block scales of K step ks for this thread's slot: waves 0-3 fetch the
  // tile's 256 row scales, waves 4-7 its 256 column scales (the wave index is
  // made scalar so the choice is uniform). Rows / columns past the matrix read
  // the last valid scale; they only feed outputs that are never stored.
  const bool row_scales = wave < 4;
  const int slot = t & 255;
  const int s_idx = row_scales ? min(m0 + slot, a.m - 1) : min(n0 + slot, a.n - 1);
  const int64_t s_off = row_scales ? bidx * a.ssab + int64_t(s_idx >> a.qbm_shift) * a.ssa1
                                   : bidx * a.ssbb + int64_t(s_idx >> a.qbn_shift) * a.ssb2;
  const int64_t s_kstride = row_scales ? a.ssa2 : a.ssb1;
  const float* s_ptr = (row_scales ? a.sa : a.sb) + s_off;
  float* s_tile = (row_scales ? sa_tile : sb_tile) + slot;
  auto load_scale = [&](int ks) -> float { return s_ptr[int64_t(ks) * s_kstride]; };  // qbk == 128
  auto store_scale = [&](int ks, float v) { s_tile[(ks & 1) * 256] = v; };

  v4f acc[4][JN];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < JN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // KT: K is not a multiple of 128. The last K step then holds kt < 128
  // valid k; what its tiles hold past them (the next row's bytes for a K-major
  // operand, zeros past the buffer) is masked out of the fragments.
  const int ksteps = KT ? (a.k + BK - 1) / BK : a.k / BK;  // >= 2
  const int kt = a.k - (ksteps - 1) * BK;
  // Word w of a lane's fragment holds k 32 (lane / 16) + 4 w .. + 3 of the
  // step, for K-major and (transposing reads) MN-major tiles alike; words at
  // or past kt become zero, in both operands, so no product of a stale byte
  // (possibly a NaN pattern) reaches the accumulator. Needs kt % 4 == 0.
  // The block-mode MFMA is inline asm (mfma_fold), which the compiler's
  // hazard checks cannot see into: a VALU write of a VGPR that an MFMA reads
  // as src A / B needs wait states the compiler would otherwise insert. The
  // s_nop takes the masked fragment as an in/out operand, so the masks are
  // complete before it and every MFMA reads its output.
  auto mask_k = [&](v8i& f) {
    const int lim = kt - 32 * lg;
#pragma unroll
    for (int w = 0; w < 8; ++w) f[w] = 4 * w < lim ? f[w] : 0;
    asm volatile("s_nop 4" : "+v"(f));
  };
  // prologue: step 0 resident in stage 0 (step 0's sub-tiles start step 1's DMA)
  issue(0, smem);
  if constexpr (MODE == 0) store_scale(0, load_scale(0));
  if constexpr (MODE == 1) {
    // channel scales of the tile's 256 rows (waves 0-3) and 256 columns
    // (waves 4-7), read by the epilogue from LDS; 0 past the matrix, where
    // no output is stored
    const int idx = (row_scales ? m0 : n0) + slot;
    const bool in = idx < (row_scales ? a.m : a.n);
    const float* sp = row_scales ? a.sa + bidx * a.ssab + int64_t(min(idx, a.m - 1)) * a.ssa1
                                 : a.sb + bidx * a.ssbb + int64_t(min(idx, a.n - 1)) * a.ssb1;
    (row_scales ? sa_tile : sb_tile)[slot] = in ? *sp : 0.0f;
  }
  // tensor scale: loaded here, under the first K step's DMA, rather than
  // after the K loop where the epilogue would wait for it
  float tscale = 1.0f;
  if constexpr (MODE == 2) tscale = a.scales_are_quant ? 1.0f / (a.sa[0] * a.sb[0]) : a.sa[0];
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (MODE == 2) asm volatile("" : "+v"(tscale));  // materialised before the K loop
  __syncthreads();
  float sc_next = 0.0f;
  if constexpr (MODE == 0) sc_next = load_scale(1);

  v8i af[4], bf[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) af[i] = afrag(smem, i);
  bf[0] = bfrag(smem, 0);

  // Block-mode fold state. The factor of output (i, r) of a sub-tile is the
  // row factor f[i] (sa * sb for SBK 0 / 1, sa for SBK 2) times, for SBK 2,
  // the column scale c[r]. p / pf / pc: the pending partials and their
  // factors. Row scales of a step: sa_c (fc = sa_c * sb for SBK 0); column
  // scales of sub-tile j (SBK 1 / 2): cs[j & 1], read one sub-tile ahead.
  v4f p[4];
  float pf[4], pc[4], sa_c[4], fc[4];
  float4 cs[2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    p[i] = v4f{0.f, 0.f, 0.f, 0.f};
    pf[i] = pc[i] = sa_c[i] = fc[i] = 0.0f;
  }
  cs[0] = cs[1] = float4{0.f, 0.f, 0.f, 0.f};
  const int sa_off = wm * 64 + lr;
  const int sb_off = wcol + (SBK == 2 ? 4 * lg : 0);
  auto read_rows = [&](int ks, float (&sa)[4], float (&f)[4]) {
    const float* sat = sa_tile + (ks & 1) * BM + sa_off;
#pragma unroll
    for (int i = 0; i < 4; ++i) sa[i] = sat[16 * i];
    if constexpr (SBK == 0) {
      const float sb = sb_tile[(ks & 1) * BN + sb_off];
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = sa[i] * sb;
    }
  };
  // column scales of sub-tile j of step ks into slot `slot` (default j & 1)
  auto read_cols = [&](int ks, int j, int slot = -1) {
    const float* sbt = sb_tile + (ks & 1) * BN + sb_off + 16 * j;
    const int sl = slot < 0 ? (j & 1) : slot;
    if constexpr (SBK == 1) cs[sl].x = sbt[0];
    if constexpr (SBK == 2) cs[sl] = *reinterpret_cast<const float4*>(sbt);
  };
  if constexpr (MODE == 0) {
    read_rows(0, sa_c, fc);
    read_cols(0, 0);
  }

  using T = std::true_type;
  using F = std::false_type;
  // MFMAs of sub-tile j (B fragment bcur), each preceded by the fold of the
  // pending partial of its row block (sub-tile j - 1, or 7 of the previous
  // step); with af_next, the next step's A fragment i is read right after
  // MFMA (i, j). ds_reads: LDS reads issued in the same scheduling region
  // ahead of the MFMAs (the next B fragment and scales).
  auto subtile = [&](int j, const v8i& bcur, const uint8_t* af_next, auto ds_reads_c, auto next_c) {
    constexpr int ds_reads = decltype(ds_reads_c)::value;
    constexpr bool NEXT = decltype(next_c)::value;
    const int jp = (j + JN - 1) % JN;
    float cf[4], cc[4];
    if constexpr (MODE == 0) {
      const float4 c = cs[j & 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) cf[i] = SBK == 0 ? fc[i] : SBK == 1 ? sa_c[i] * c.x : sa_c[i];
      cc[0] = c.x; cc[1] = c.y; cc[2] = c.z; cc[3] = c.w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (MODE == 0) {
        float f[4], a[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          f[r] = SBK == 2 ? pf[i] * pc[r] : pf[i];
          a[r] = acc[i][jp][r];
        }
        v4f pn;
        mfma_fold<FA, FB>(bcur, af[i], pn, p[i], a[0], a[1], a[2], a[3], f[0], f[1], f[2], f[3]);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[i][jp][r] = a[r];
        p[i] = pn;
      } else {
        acc[i][j] = mfma<FA, FB>(bcur, af[i], acc[i][j]);
      }
      if constexpr (NEXT) af[i] = afrag(af_next, i);
    }
    if constexpr (MODE == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pf[i] = cf[i];
        pc[i] = cc[i];
      }
    }
    // Instruction order of the sub-tile (sched_group_barrier: mask, count,
    // pipeline id; masks 0x2 VALU, 0x8 MFMA, 0x100 DS read): its LDS reads
    // first, then per row block the fold VALU followed by the MFMA, and with
    // af_next the A fragment read behind each MFMA. Pure arithmetic carries no
    // ordering of its own, and without this the folds sink below all MFMAs.
    if constexpr (MODE != 0) {
      if constexpr (ds_reads > 0) __builtin_amdgcn_sched_group_barrier(0x100, ds_reads, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        if constexpr (NEXT) __builtin_amdgcn_sched_group_barrier(0x100, A_K ? 2 : 4, 0);
      }
    }
  };

  // One K step. BOUNDARY: the next step follows (barrier and fragment
  // reads in front of sub-tile 7); DMA: the step's first sub-tiles start the
  // next step's global -> LDS loads; SCALES: fetch the block scales two steps
  // ahead. All three are compile-time so that the main loop body is one basic
  // block: with a branch at the step boundary the compiler sinks the folds of
  // the earlier sub-tiles past it and keeps all their partials live.
  //
  // The next step's DMA goes to the other stage, which every wave has left
  // at the previous boundary's barrier, and the boundary's vmcnt(0) + barrier
  // publish it. Its eight load instructions are spread over the first
  // sub-tiles (A in sub-tiles 0-1, B in 2-3 for whole tiles) rather than
  // issued together at the boundary: the same loads in one burst right
  // after the barrier made the forward GEMM of config 5 17 % slower.
  constexpr int kSchedA[4] = {0, 0, 1, 1};
  constexpr int kSchedB[4] = {JN != 4 ? 2 : 1, JN != 4 ? 2 : 1, JN != 4 ? 3 : 2, JN != 4 ? 3 : 2};
  constexpr int kBReads = B_K ? 2 : 4;  // ds_read instructions per B fragment
  // The B fragment and column scales of sub-tile j sit in slot j & 1. The
  // last sub-tile's slot is LAST; at the step boundary the next step's
  // sub-tile 0 goes to the other slot, and with an odd number of sub-tiles
  // (JN = 7) it is moved to slot 0 after the last sub-tile.
  constexpr int LAST = (JN - 1) & 1, FREE = LAST ^ 1;
  auto step = [&](int ks, auto boundary, auto dma, auto scales) {
    constexpr bool BOUNDARY = decltype(boundary)::value;
    constexpr bool DMA = decltype(dma)::value;
    constexpr bool SCALES = decltype(scales)::value;
    const uint8_t* cur = smem + (ks & 1) * STAGE;
    const uint8_t* nxt = smem + ((ks + 1) & 1) * STAGE;
    constexpr bool MASK = KT && !BOUNDARY;  // the last K step of a ragged K
    if constexpr (MASK) {
#pragma unroll
      for (int i = 0; i < 4; ++i) mask_k(af[i]);
    }
#pragma unroll
    for (int j = 0; j < JN - 1; ++j) {
      if constexpr (DMA) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (j == kSchedA[q]) issue_a1(ks + 1, nxt, q);
          if (j == kSchedB[q]) issue_b1(ks + 1, nxt, q);
        }
      }
      v8i bcur = bf[j & 1];
      if constexpr (MASK) mask_k(bcur);
      bf[(j + 1) & 1] = bfrag(cur, j + 1);
      if constexpr (MODE == 0 && SBK != 0) read_cols(ks, j + 1);
      subtile(j, bcur, nullptr, IC<kBReads + (MODE == 0 && SBK != 0 ? 1 : 0)>{}, F{});
    }
    if constexpr (BOUNDARY) {
      if constexpr (MODE == 0) store_scale(ks + 1, sc_next);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if constexpr (MODE == 0 && SCALES) sc_next = load_scale(ks + 2);
      bf[FREE] = bfrag(nxt, 0);
      if constexpr (MODE == 0) {
        // cs[LAST] (the last sub-tile) is still needed; cs[FREE] takes sub-tile 0 of the next step
        if constexpr (SBK != 0) read_cols(ks + 1, 0, FREE);
        float sa_n[4], fc_n[4];
        read_rows(ks + 1, sa_n, fc_n);
        subtile(JN - 1, bf[LAST], nxt, IC<kBReads + (SBK != 0 ? 1 : 0) + (SBK == 0 ? 3 : 2)>{}, T{});
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sa_c[i] = sa_n[i];
          fc[i] = fc_n[i];
        }
      } else {
        subtile(JN - 1, bf[LAST], nxt, IC<kBReads>{}, T{});
      }
      if constexpr (FREE != 0) {
        bf[0] = bf[FREE];
        if constexpr (MODE == 0 && SBK != 0) cs[0] = cs[FREE];
      }
    } else {
      v8i bcur = bf[LAST];
      if constexpr (MASK) mask_k(bcur);
      subtile(JN - 1, bcur, nullptr, IC<0>{}, F{});
    }
  };
  for (int ks = 0; ks < ksteps - 2; ++ks) step(ks, T{}, T{}, T{});
  step(ksteps - 2, T{}, T{}, F{});
  step(ksteps - 1, F{}, F{}, F{});
  if constexpr (MODE == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][JN - 1][r] += p[i][r] * (SBK == 2 ? pf[i] * pc[r] : pf[i]);
  }

  const int row_base = m0 + wm * 64 + lr;
  const int col_base = n0 + wcol + 4 * lg;

  // ---- epilogue ----
  // SAQ (scales_are_quant, channel mode): the per-element scale is
  // 1 / (sa * sb). It is a compile-time branch of the epilogue: as a runtime
  // condition inside the unrolled element loops it was if-converted, and
  // every output paid for a division it did not use.
  auto epilogue = [&](auto saq_c) {
    constexpr bool SAQ = decltype(saq_c)::value;
    // output value (i, j, r) of this lane with the channel / tensor scales applied
    // column scales of sub-tile column j (channel mode; 1 otherwise)
    auto col_scales = [&](int j, float (&sbv)[4]) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sbv[r] = 1.0f;
        if constexpr (MODE == 1) sbv[r] = sb_tile[wcol + 4 * lg + 16 * j + r];
      }
    };
    auto out_value = [&](int i, int j, int r, float sam_v, const float (&sbv)[4]) -> float {
      float x = acc[i][j][r];
      if constexpr (MODE == 1) {
        float s = sam_v * sbv[r];
        if constexpr (SAQ) s = 1.0f / s;
        x *= s;
      } else if constexpr (MODE == 2) {
        x *= tscale;
      }
      return x;
    };
    auto row_scale = [&](int i) -> float {
      float sam_v = 1.0f;
      if constexpr (MODE == 1) sam_v = sa_tile[wm * 64 + 16 * i + lr];
      return sam_v;
    };
    const bool plain = a.bias == nullptr && a.act == PCAMD_ACT_NONE && a.c_dtype == kBF16;
    // the staged path also takes fp16 output, GELU and a 16-bit bias
    // contiguous along N with 8-byte aligned rows (one load per lane's 4
    // columns); other bias forms and output types take the direct path below
    const bool bias16 = a.bias != nullptr && (a.bias_dtype == kBF16 || a.bias_dtype == kF16) && a.sbiasn == 1 &&
                        (a.sbiasm & 3) == 0 && (a.sbiasb & 3) == 0 && (reinterpret_cast<uintptr_t>(a.bias) & 7) == 0;
    const bool out16 = (a.c_dtype == kBF16 || a.c_dtype == kF16) && (a.bias == nullptr || bias16);
    // (CT: the launcher checked the transposed output's alignment)
    if (CT || staged_output_ok(a.c, a.scb, a.scm, a.n, out16)) {
      // each wave stages its sub-tile in 8 KiB (4 KiB for a half tile) of the
      // LDS stage the last K step did not read (no other wave touches it, so no
      // barrier is needed)
      const float sam_v[4] = {row_scale(0), row_scale(1), row_scale(2), row_scale(3)};
      uint16_t* cb = reinterpret_cast<uint16_t*>(a.c) + bidx * a.scb;
      auto stage = [&](auto out_c, auto&& value) {
        constexpr int OUT = decltype(out_c)::value;
        if constexpr (JN == 8)
          store_subtile_staged<OUT>(smem + (ksteps & 1) * STAGE + wave * 8192, cb, a.scm, a.m, a.n, m0 + wm * 64,
                                    n0 + wcol, lane, value, a.c_dtype == kF16);
        else
          store_half_staged<OUT>(smem + (ksteps & 1) * STAGE + wave * 4096, cb, a.scm, a.m, a.n, m0 + wm * 64,
                                 n0 + wcol, lane, value, a.c_dtype == kF16);
      };
      if constexpr (CT) {
        // every wave's 14 KiB of staging spans both LDS stages: wait until all
        // waves have finished reading the last one
        __syncthreads();
        auto value = [&](int i, int j, float (&v)[4]) {
          float sbv[4];
          col_scales(j, sbv);
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = out_value(i, j, r, sam_v[i], sbv);
        };
        // C^T's rows are C's columns: its row pitch is C's n stride
        store_subtile_staged_t<OUT16_RUNTIME, JN>(smem + wave * 16384, cb, a.scn, a.m, a.n, m0 + wm * 64,
                                                 n0 + wcol, lane, value, a.c_dtype == kF16);
        return;
      } else {
        if (plain) {
          stage(IC<kBF16>{}, [&](int i, int j, float (&v)[4]) {
            float sbv[4];
            col_scales(j, sbv);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = out_value(i, j, r, sam_v[i], sbv);
          });
          return;
        }
        // fp16 output, a 16-bit bias and / or GELU, in the reference's order:
        // scaled product, + bias, activation, one rounding
        // (kernels/bmm/per_block.py:113-137). The output type is picked per
        // element pair at run time (OUT16_RUNTIME), so this path is
        // instantiated once.
        const bool bias_bf16 = a.bias_dtype == kBF16, gelu = a.act == PCAMD_ACT_GELU;
        const uint16_t* bias_b = bias16 ? static_cast<const uint16_t*>(a.bias) + bidx * a.sbiasb : nullptr;
        auto value = [&](int i, int j, float (&v)[4]) {
          float sbv[4];
          col_scales(j, sbv);
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = out_value(i, j, r, sam_v[i], sbv);
          const int mm = row_base + 16 * i, nn = col_base + 16 * j;
          if (bias_b && mm < a.m && nn < a.n) {
            const uint2 h = *reinterpret_cast<const uint2*>(bias_b + int64_t(mm) * a.sbiasm + nn);
            const uint32_t e[4] = {h.x & 0xFFFFu, h.x >> 16, h.y & 0xFFFFu, h.y >> 16};
#pragma unroll
            for (int r = 0; r < 4; ++r)
              v[r] += bias_bf16 ? __uint_as_float(e[r] << 16)
                                : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(e[r])));
          }
          if (gelu) {
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = 0.5f * v[r] * (1.0f + erff(v[r] * 0.7071067811865475f));
          }
        };
        stage(IC<OUT16_RUNTIME>{}, value);
        return;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mm = row_base + 16 * i;
      const float sam_v = row_scale(i);
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int nn = col_base + 16 * j;
        float sbv[4];
        col_scales(j, sbv);
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = out_value(i, j, r, sam_v, sbv);
        if (mm >= a.m || nn >= a.n) continue;
        __bf16* p = reinterpret_cast<__bf16*>(a.c) + bidx * a.scb + int64_t(mm) * a.scm + nn;
        if (plain && nn + 4 <= a.n && (reinterpret_cast<uintptr_t>(p) & 7) == 0) {
          *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16_pair(v[0], v[1]), pack_bf16_pair(v[2], v[3]));
        } else {
          epilogue_general(a.c, bidx * a.scb + int64_t(mm) * a.scm, a.c_dtype, a.bias,
                           bidx * a.sbiasb + int64_t(mm) * a.sbiasm, a.sbiasn, a.bias_dtype, a.act, nn,
                           min(4, a.n - nn), v[0], v[1], v[2], v[3]);
        }
      }
    }
  };
  if constexpr (MODE == 1) {
    if (a.scales_are_quant) epilogue(std::true_type{});
    else epilogue(std::false_type{});
  } else {
    epilogue(std::false_type{});
  }
}

constexpr int LDS_BYTES = 2 * STAGE + 2 * (BM + BN) * 4;

// PCAMD_BMM_T224=0 keeps the 256 x 256 tiling everywhere (read once)
inline bool transposed_disabled() {
  static const bool off = [] {
    const char* e = getenv("PCAMD_BMM_T224");
    return e && e[0] == '0';
  }();
  return off;
}

// PCAMD_BMM_HALVES=0 keeps whole 256 x 256 tiles for small grids (read once)
inline bool halves_disabled() {
  static const bool off = [] {
    const char* e = getenv("PCAMD_BMM_HALVES");
    return e && e[0] == '0';
  }();
  return off;
}

template <bool A_K, bool B_K, int FA, int FB, int MODE, int SBK, int JN, bool KT, bool CT = false>
int launch_tiles(const FastArgs& a, int grid, hipStream_t st) {
  auto kern = bmm_wide_kernel<A_K, B_K, FA, FB, MODE, SBK, JN, KT, CT>;
  static std::atomic<uint64_t> configured{0};  // devices whose LDS limit is set
  const int rc = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), LDS_BYTES, st, configured);
  if (rc != 0) return rc;
  kern<<<grid, NT, LDS_BYTES, st>>>(a);
  return check_launch("bmm_wide_kernel");
}

// One workgroup per tile (one per CU at a time: the LDS stages allow no
// more). When the last wave of tiles would occupy at most half the CUs, it
// runs as a second launch of half tiles instead; a grid of at most half as
// many tiles as CUs runs as half tiles altogether (twice the CUs at work).
template <bool A_K, bool B_K, int FA, int FB, int MODE, int SBK, bool KT>
int launch_one(const FastArgs& a, hipStream_t st) {
  const int cus = device_cu_count(st);
  if (cus > 0 && 2 * a.total_tiles <= cus && !halves_disabled()) {
    FastArgs half = a;
    half.tile_base = 0;
    return launch_tiles<A_K, B_K, FA, FB, MODE, SBK, 4, KT>(half, 2 * a.total_tiles, st);
  }
  const int tail = cus > 0 && a.total_tiles > cus ? a.total_tiles % cus : 0;
  if (tail == 0 || 2 * tail > cus) return launch_tiles<A_K, B_K, FA, FB, MODE, SBK, 8, KT>(a, a.total_tiles, st);
  FastArgs whole = a;
  whole.total_tiles = a.total_tiles - tail;  // the XCD remap spans the whole tiles only
  int rc = launch_tiles<A_K, B_K, FA, FB, MODE, SBK, 8, KT>(whole, whole.total_tiles, st);
  if (rc != 0) return rc;
  FastArgs half = a;
  half.tile_base = a.total_tiles - tail;
  return launch_tiles<A_K, B_K, FA, FB, MODE, SBK, 4, KT>(half, 2 * tail, st);
}

// Tile-count model: 256 x 256 tiles take floor(T / CUs) whole waves and a
// short last wave as half tiles (each about 0.85 of a whole tile) when it
// fills at most half the CUs. The transposed product C^T = B^T A^T on
// 256 x 224 tiles takes ceil(T' / CUs) waves of 224 / 256 of a tile each; it
// is chosen when that is at least 5 % cheaper, e.g. wgrad of config 5
// (14336 x 4096: 896 tiles = 3.85 tile-times, against 1024 = 4 waves of 224-
// column tiles, 3.5).
inline bool transposed_pays(const FastArgs& a, int cus) {
  if (cus <= 0 || a.total_tiles <= cus) return false;
  const int tail = a.total_tiles % cus;
  const double now = a.total_tiles / cus + (tail == 0 ? 0.0 : 2 * tail <= cus ? 0.85 : 1.0);
  const int64_t batch = a.total_tiles / a.tiles_per_batch;
  const int64_t t2 = int64_t((a.n + BM - 1) / BM) * ((a.m + 223) / 224) * batch;
  const double alt = double((t2 + cus - 1) / cus) * (224.0 / 256.0);
  return alt < 0.95 * now;
}

// The transposed launch's arguments: A' = B^T, B' = A^T, C' = C^T (rows of
// C' are C's columns), block scales with their roles swapped. Plain 16-bit C
// only (its staged store writes C's rows of 16-byte chunks), and every offset
// the 224-column tiles form (they load 256 columns) inside 32 bits.
inline bool transposed_args(const FastArgs& a, bool a_k, FastArgs& t) {
  if (a.bias != nullptr || a.act != PCAMD_ACT_NONE || (a.c_dtype != kBF16 && a.c_dtype != kF16)) return false;
  if (a.scn != 1 || (a.scm & 7) || (a.scb & 7) || (a.n & 7) || (reinterpret_cast<uintptr_t>(a.c) & 15))
    return false;
  const int64_t kpad = (a.k + BK - 1) / BK * BK;
  const int64_t rows = int64_t((a.m + 223) / 224) * 224 + 32;  // A's rows (or columns) the tiles reach
  const int64_t amax = a_k ? rows * a.lda + kpad : (kpad - 1) * int64_t(a.lda) + rows;
  if (amax >= (int64_t{1} << 32) - 64) return false;
  t = a;
  t.a = a.b; t.b = a.a;
  t.sab = a.sbb; t.sbb = a.sab;
  t.lda = a.ldb; t.ldb = a.lda;
  t.a_extent = a.b_extent; t.b_extent = a.a_extent;
  t.m = a.n; t.n = a.m;
  t.scm = a.scn; t.scn = a.scm;
  t.sa = a.sb; t.sb = a.sa;
  t.ssab = a.ssbb; t.ssa1 = a.ssb2; t.ssa2 = a.ssb1;  // A' = B^T: rows are B's columns
  t.ssbb = a.ssab; t.ssb1 = a.ssa2; t.ssb2 = a.ssa1;  // B' = A^T: columns are A's rows
  t.qbm_shift = a.qbn_shift; t.qbn_shift = a.qbm_shift;
  t.tiles_m = (t.m + BM - 1) / BM;
  t.tiles_n = (t.n + 223) / 224;
  t.tiles_per_batch = t.tiles_m * t.tiles_n;
  t.total_tiles = t.tiles_per_batch * (a.total_tiles / a.tiles_per_batch);
  t.tile_base = 0;
  return true;
}

// block mode: B-scale kind from the quant block width (qbn = 1 << qbn_shift):
// >= 128 one scale per wave, >= 16 one per 16-column sub-tile, else per column
template <bool A_K, bool B_K, int FA, int FB, bool KT>
int launch_mode(const FastArgs& a, int mode, hipStream_t st) {
  // A with one scale per row (qbm = 1): the transposed kernel's B' has one
  // scale per column, the wgrad recipe's 128 x 1 x 128 x 1 product
  FastArgs t;
  if (mode == 0 && a.qbm_shift == 0 && transposed_pays(a, device_cu_count(st)) && transposed_args(a, A_K, t) &&
      !transposed_disabled())
    return launch_tiles<B_K, A_K, FB, FA, 0, 2, 7, KT, true>(t, t.total_tiles, st);
  if (mode == 1) return launch_one<A_K, B_K, FA, FB, 1, 0, KT>(a, st);
  if (mode == 2) return launch_one<A_K, B_K, FA, FB, 2, 0, KT>(a, st);
  if (a.qbn_shift >= 7) return launch_one<A_K, B_K, FA, FB, 0, 0, KT>(a, st);
  if (a.qbn_shift >= 4) return launch_one<A_K, B_K, FA, FB, 0, 1, KT>(a, st);
  return launch_one<A_K, B_K, FA, FB, 0, 2, KT>(a, st);
}

template <int FA, int FB, bool KT>
int launch_layout(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st) {
  if (a_k && b_k) return launch_mode<true, true, FA, FB, KT>(a, mode, st);
  if (a_k) return launch_mode<true, false, FA, FB, KT>(a, mode, st);
  if (b_k) return launch_mode<false, true, FA, FB, KT>(a, mode, st);
  return launch_mode<false, false, FA, FB, KT>(a, mode, st);
}

// every layout and scale mode for one pair of operand formats; K need not be
// a multiple of 128 (a multiple of 4)
template <int FA, int FB>
int launch_formats(const FastArgs& a, bool a_k, bool b_k, int mode, hipStream_t st) {
  if (a.k % BK != 0) return launch_layout<FA, FB, true>(a, a_k, b_k, mode, st);
  return launch_layout<FA, FB, false>(a, a_k, b_k, mode, st);
}

}  // namespace bmmw
}  // namespace pcamd
