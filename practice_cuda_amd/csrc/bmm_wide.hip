// bmm_wide.hip - large-tile scaled FP8 BMM for gfx950 (K a multiple of 128 and
// at least two K steps; 16-byte aligned operands).
//
// Workgroup: 512 threads = 8 waves (4 along M x 2 along N), output tile
// 256 x 256, K step 128, two LDS stages of 64 KiB. Two waves per SIMD, so one
// wave's MFMAs cover the other's LDS reads, waits and scale folding. Each wave
// owns 64 x 128 = 4 x 8 tiles of v_mfma_f32_16x16x128_f8f6f4, issued with the
// operands swapped so a lane holds four consecutive N outputs of one row.
//
// Both operands go global -> LDS with buffer_load_dwordx4 ... lds (no VGPR
// staging), one K step ahead of the MFMAs. The LDS layout follows the global
// one:
//   K-major operand (rows contiguous along k): [row][8 x 16 B], chunk c of
//     row r at position c ^ ((r ^ r >> 4) & 7); fragments are two
//     ds_read_b128 per lane.
//   MN-major operand (k rows contiguous along m / n): [k][16 x 16 B], chunk c
//     of k-row k at position c ^ (k & 7); fragments are four
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
// once in the epilogue. Wider quant-K blocks use bmm_fast.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "abi_util.h"
#include "bmm_epilogue.h"
#include "bmm_fast.h"
#include "fp8_common.h"

namespace pcamd {
namespace bmmw {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(3))) v2i* lds_v2i_ptr;

constexpr int NT = 512;
constexpr int WAVES = NT / 64;
constexpr int BM = 256, BN = 256, BK = 128;
constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;  // 32 KiB each
constexpr int STAGE = A_BYTES + B_BYTES;
constexpr uint32_t kRsrcWord3 = 0x00020000u;

// LDS swizzles. gfx950's LDS serves 256 bytes (64 banks) per cycle.
// K-major tile (128-byte rows): chunk c of row r sits at position c ^ swz_k(r).
// A fragment read touches rows r0..r0+15 (lanes 16 g + r) at chunk 2 g + h.
// Measured on gfx950, XOR-ing with r & 7 or with (r >> 1) & 7 both leave every
// ds_read_b128 2-way conflicted: the lanes served together are not 16
// consecutive ones but (among the groupings that fit) eight rows of two
// adjacent g. swz_k = 5 * bit1(r) ^ bit2(r) spreads the 16 (row, chunk) pairs
// of each such group over distinct bank groups for all of them.
PCAMD_DEV int swz_k(int r) { return (((r >> 1) & 1) * 5) ^ ((r >> 2) & 1); }
// MN-major tile (256-byte k-rows): chunk c of k-row k sits at position
// c ^ (k & 7) ^ (8 ((k >> 5) & 1)). A 16-lane group reads 8 k-rows k0..k0+7
// (k0 % 8 == 0) at one 8-byte half pair: k & 7 spreads them over 32 banks,
// and the group served in the same cycle (k-rows 32 further on) lands in the
// other 32.
PCAMD_DEV int swz_mn(int k) { return (k & 7) ^ (((k >> 5) & 1) << 3); }

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
// that LDS reads of the other stage do not alias these writes and would put
// a vmcnt(0) in front of every ds_read, serialising prefetch and MFMAs. The
// kernels order these loads themselves (s_waitcnt vmcnt(0) + barrier before
// a stage is read, barrier before it is refilled).
PCAMD_DEV void lds_dma16(v4i rs, uint32_t lds, uint32_t voff) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rs), "{m0}"(lds) : "memory");
}

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
template <int ROWS>
struct KMajorLoader {
  static constexpr int PER_WAVE = ROWS / WAVES;
  static constexpr int INSTS = PER_WAVE / 8;
  uint32_t voff;
  PCAMD_DEV KMajorLoader(uint32_t ld, int lane, int /*wave*/)
      : voff((lane >> 3) * ld + (((lane & 7) ^ swz_k(lane >> 3)) << 4)) {}
  PCAMD_DEV void issue(v4i rs, uint8_t* tile, uint32_t row0, uint32_t ld, uint32_t k0, int wave) const {
#pragma unroll
    for (int i = 0; i < INSTS; ++i) {
      const int rb = wave * PER_WAVE + i * 8;
      uint32_t u = __builtin_amdgcn_readfirstlane((row0 + rb) * ld + k0);
      asm volatile("" : "+s"(u));
      lds_dma16(rs, lds_addr(tile + rb * BK), voff + u);
    }
  }
};

// MN-major tile: 128 k-rows (k0 + k, stride ld) x COLS bytes from col0.
// Instruction i of wave w fills k-rows kb = w * 16 + i * R .. + R - 1 (R = 64 /
// (COLS / 16) rows per instruction); lane l takes k-row kb + l / CHUNKS and LDS
// slot l % CHUNKS, which holds global chunk slot ^ swz_mn(k). Bit 5 of k is
// the wave's (w * 16 + i * R + l / CHUNKS < w * 16 + 16), and k & 7 repeats
// every two instructions, so two lane offsets per wave serve them all.
template <int COLS>
struct MNMajorLoader {
  static constexpr int CHUNKS = COLS / 16;
  static constexpr int R = 64 / CHUNKS;
  static constexpr int PER_WAVE = BK / WAVES;
  static constexpr int INSTS = PER_WAVE / R;
  static_assert(COLS == 256 && PER_WAVE == 16, "swizzle assumes 256-byte k-rows, 16 per wave");
  uint32_t voff[2];
  PCAMD_DEV MNMajorLoader(uint32_t ld, int lane, int wave) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int k = wave * PER_WAVE + h * R + lane / CHUNKS;
      voff[h] = (lane / CHUNKS) * ld + (((lane % CHUNKS) ^ swz_mn(k)) << 4);
    }
  }
  PCAMD_DEV void issue(v4i rs, uint8_t* tile, uint32_t col0, uint32_t ld, uint32_t k0, int wave) const {
#pragma unroll
    for (int i = 0; i < INSTS; ++i) {
      const int kb = wave * PER_WAVE + i * R;
      uint32_t u = __builtin_amdgcn_readfirstlane((k0 + kb) * ld + col0);
      asm volatile("" : "+s"(u));
      lds_dma16(rs, lds_addr(tile + kb * COLS), voff[i & 1] + u);
    }
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

// fragment of an MN-major tile (COLS bytes per k-row): column block
// [col16, col16 + 16) (16-aligned), lane j = lane & 15, k-group g
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

template <int FMT>
PCAMD_DEV v4f mfma(const v8i& x, const v8i& y, const v4f& c) {
  constexpr int code = FMT == kE5M2 ? 1 : 0;
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, c, code, code, 0, 0, 0, 0);
}

PCAMD_DEV uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(lo))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(hi))) << 16);
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

// MODE: 0 block (qbk == 128), 1 channel, 2 tensor. SB_COL: block scales with
// qbn < 16 (one B scale per output column).
//
// Block scales are staged through LDS one K step ahead (sa for the tile's
// 256 rows, sb for its 256 columns), so the fold acc += P * (sa * sb) reads
// them with a few ds_reads instead of holding them in registers.
template <bool A_K, bool B_K, int FMT, int MODE, bool SB_COL>
__global__ __launch_bounds__(NT, 1) void bmm_wide_kernel(FastArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float* sa_tile = reinterpret_cast<float*>(smem + 2 * STAGE);  // [2][BM]
  float* sb_tile = sa_tile + 2 * BM;                             // [2][BN]
  const int t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave & 3, wn = wave >> 2;  // 4 x 2 waves
  const int lr = lane & 15, lg = lane >> 4;

  int pid = blockIdx.x;
  if ((a.total_tiles & 7) == 0) pid = (pid & 7) * (a.total_tiles >> 3) + (pid >> 3);
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
  const int n0 = __builtin_amdgcn_readfirstlane((in_group / gm) * BN);

  const v4i rsa = make_rsrc(a.a + bidx * a.sab, a.a_extent);
  const v4i rsb = make_rsrc(a.b + bidx * a.sbb, a.b_extent);
  using LA = typename std::conditional<A_K, KMajorLoader<BM>, MNMajorLoader<BM>>::type;
  using LB = typename std::conditional<B_K, KMajorLoader<BN>, MNMajorLoader<BN>>::type;
  const LA load_a(a.lda, lane, wave);
  const LB load_b(a.ldb, lane, wave);

  auto issue = [&](int ks, uint8_t* stage) {
    const uint32_t k0 = ks * BK;
    load_a.issue(rsa, stage, m0, a.lda, k0, wave);
    load_b.issue(rsb, stage + A_BYTES, n0, a.ldb, k0, wave);
  };
  auto afrag = [&](const uint8_t* stage, int i) -> v8i {
    if constexpr (A_K) return frag_k(stage, wm * 64 + i * 16 + lr, lg);
    else return frag_mn<BM>(stage, wm * 64 + i * 16, lane);
  };
  auto bfrag = [&](const uint8_t* stage, int j) -> v8i {
    if constexpr (B_K) return frag_k(stage + A_BYTES, wn * 128 + j * 16 + lr, lg);
    else return frag_mn<BN>(stage + A_BYTES, wn * 128 + j * 16, lane);
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

  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // one K step on the stage of step ks
  auto compute = [&](int ks) {
    const uint8_t* cur = smem + (ks & 1) * STAGE;
    v8i af[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = afrag(cur, i);
    if constexpr (MODE != 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const v8i bf = bfrag(cur, j);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = mfma<FMT>(bf, af[i], acc[i][j]);
      }
    } else {
      const float* sat = sa_tile + (ks & 1) * BM + wm * 64 + lr;
      const float* sbt = sb_tile + (ks & 1) * BN + wn * 128 + 4 * lg;
      float sav[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) sav[i] = sat[16 * i];
      // acc[.][j] += P_j * (sa * sb): the MFMAs of sub-tile j are issued, then
      // sub-tile j - 1 is folded while they run, so only two sub-tiles of
      // partials are live at a time.
      auto fold = [&](int j, const v4f (&p)[4]) {
        float sb4[4];
        if constexpr (SB_COL) {
          const float4 v = *reinterpret_cast<const float4*>(sbt + 16 * j);
          sb4[0] = v.x; sb4[1] = v.y; sb4[2] = v.z; sb4[3] = v.w;
        } else {
          sb4[0] = sbt[16 * j];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] += p[i][r] * (sav[i] * sb4[SB_COL ? r : 0]);
      };
      v4f p[2][4];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const v8i bf = bfrag(cur, j);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[j & 1][i] = mfma<FMT>(bf, af[i], v4f{0.f, 0.f, 0.f, 0.f});
        if (j > 0) fold(j - 1, p[(j - 1) & 1]);
        __builtin_amdgcn_sched_barrier(0);
      }
      fold(7, p[1]);
    }
  };

  const int ksteps = a.k / BK;  // >= 2
  issue(0, smem);
  if constexpr (MODE == 0) store_scale(0, load_scale(0));
  for (int ks = 0; ks < ksteps - 1; ++ks) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    float next_scale = 0.0f;
    if constexpr (MODE == 0) next_scale = load_scale(ks + 1);
    issue(ks + 1, smem + ((ks + 1) & 1) * STAGE);
    compute(ks);
    if constexpr (MODE == 0) store_scale(ks + 1, next_scale);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  compute(ksteps - 1);

  const int row_base = m0 + wm * 64 + lr;
  const int col_base = n0 + wn * 128 + 4 * lg;

  // ---- epilogue ----
  float tscale = 1.0f;
  if constexpr (MODE == 2) tscale = a.scales_are_quant ? 1.0f / (a.sa[0] * a.sb[0]) : a.sa[0];
  // output value (i, j, r) of this lane with the channel / tensor scales applied
  // column scales of sub-tile column j (channel mode; 1 otherwise)
  auto col_scales = [&](int j, float (&sbv)[4]) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sbv[r] = 1.0f;
      if constexpr (MODE == 1) {
        const int nn = col_base + 16 * j + r;
        sbv[r] = nn < a.n ? a.sb[bidx * a.ssbb + int64_t(nn) * a.ssb1] : 0.0f;
      }
    }
  };
  auto out_value = [&](int i, int j, int r, float sam_v, const float (&sbv)[4]) -> float {
    float x = acc[i][j][r];
    if constexpr (MODE == 1) {
      float s = sam_v * sbv[r];
      if (a.scales_are_quant) s = 1.0f / s;
      x *= s;
    } else if constexpr (MODE == 2) {
      x *= tscale;
    }
    return x;
  };
  auto row_scale = [&](int i) -> float {
    float sam_v = 1.0f;
    if constexpr (MODE == 1) {
      const int mm = row_base + 16 * i;
      sam_v = mm < a.m ? a.sa[bidx * a.ssab + int64_t(mm) * a.ssa1] : 0.0f;
    }
    return sam_v;
  };
  const bool plain = a.bias == nullptr && a.act == PCAMD_ACT_NONE && a.c_dtype == kBF16;
  if (staged_output_ok(a.c, a.scb, a.scm, a.n, plain)) {
    // each wave stages its sub-tile in 8 KiB of the LDS stage the last K step
    // did not read (no other wave touches it, so no barrier is needed)
    const float sam_v[4] = {row_scale(0), row_scale(1), row_scale(2), row_scale(3)};
    store_subtile_staged(smem + (ksteps & 1) * STAGE + wave * 8192,
                         reinterpret_cast<__bf16*>(a.c) + bidx * a.scb, a.scm, a.m, a.n, m0 + wm * 64,
                         n0 + wn * 128, lane, [&](int i, int j, float (&v)[4]) {
                           float sbv[4];
                           col_scales(j, sbv);
#pragma unroll
                           for (int r = 0; r < 4; ++r) v[r] = out_value(i, j, r, sam_v[i], sbv);
                         });
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int mm = row_base + 16 * i;
    const float sam_v = row_scale(i);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int nn = col_base + 16 * j;
      float sbv[4];
      col_scales(j, sbv);
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = out_value(i, j, r, sam_v, sbv);
      if (mm >= a.m || nn >= a.n) continue;
      __bf16* p = reinterpret_cast<__bf16*>(a.c) + bidx * a.scb + int64_t(mm) * a.scm + nn;
      if (plain && nn + 4 <= a.n && (reinterpret_cast<uintptr_t>(p) & 7) == 0) {
        *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
      } else {
        epilogue_general(a.c, bidx * a.scb + int64_t(mm) * a.scm, a.c_dtype, a.bias,
                         bidx * a.sbiasb + int64_t(mm) * a.sbiasm, a.sbiasn, a.bias_dtype, a.act, nn,
                         min(4, a.n - nn), v[0], v[1], v[2], v[3]);
      }
    }
  }
}

constexpr int LDS_BYTES = 2 * STAGE + 2 * (BM + BN) * 4;

template <bool A_K, bool B_K, int FMT, int MODE, bool SB_COL>
int launch_one(const FastArgs& a, hipStream_t st) {
  auto kern = bmm_wide_kernel<A_K, B_K, FMT, MODE, SB_COL>;
  static bool configured = false;  // benign race: the attribute call is idempotent
  if (!configured) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, LDS_BYTES);
    if (e != hipSuccess) return set_error(PCAMD_ERR_LAUNCH, "hipFuncSetAttribute: %s", hipGetErrorString(e));
    configured = true;
  }
  kern<<<a.total_tiles, NT, LDS_BYTES, st>>>(a);
  return check_launch("bmm_wide_kernel");
}

template <bool A_K, bool B_K, int FMT>
int launch_mode(const FastArgs& a, int mode, bool sb_col, hipStream_t st) {
  if (mode == 1) return launch_one<A_K, B_K, FMT, 1, false>(a, st);
  if (mode == 2) return launch_one<A_K, B_K, FMT, 2, false>(a, st);
  return sb_col ? launch_one<A_K, B_K, FMT, 0, true>(a, st) : launch_one<A_K, B_K, FMT, 0, false>(a, st);
}

template <int FMT>
int launch_layout(const FastArgs& a, bool a_k, bool b_k, int mode, bool sb_col, hipStream_t st) {
  if (a_k && b_k) return launch_mode<true, true, FMT>(a, mode, sb_col, st);
  if (a_k) return launch_mode<true, false, FMT>(a, mode, sb_col, st);
  if (b_k) return launch_mode<false, true, FMT>(a, mode, sb_col, st);
  return launch_mode<false, false, FMT>(a, mode, sb_col, st);
}

}  // namespace bmmw

int bmm_wide_launch(const FastArgs& a, int ab_dtype, bool a_k, bool b_k, int mode, bool sb_col,
                    hipStream_t st) {
  if (ab_dtype == kE5M2) return bmmw::launch_layout<kE5M2>(a, a_k, b_k, mode, sb_col, st);
  return bmmw::launch_layout<kE4M3>(a, a_k, b_k, mode, sb_col, st);
}

int bmm_wide_tile() { return bmmw::BM; }

}  // namespace pcamd
