// bmm_fast.hip - tuned scaled FP8 BMM path for gfx950 (K a multiple of 128,
// 16-byte aligned operands). Shapes outside that envelope use bmm.hip.
//
// Workgroup: 256 threads = 4 waves (2 x 2), output tile 128 (M) x 256 (N),
// K step 128, two LDS stages of 48 KiB (A 16 KiB + B 32 KiB). Each wave owns
// a 64 x 128 tile = 4 x 8 tiles of v_mfma_f32_16x16x128_f8f6f4, issued with
// the operands swapped so a lane holds four consecutive N outputs of one row.
//
// Global -> LDS, both staged one K step ahead of the MFMAs:
//   K-major operand: buffer_load_dwordx4 ... lds (direct to LDS, 16 B per
//     lane, no VGPR staging); the source address of each LDS slot is chosen
//     so the tile lands swizzled.
//   MN-major operand: buffer_load_dwordx4 of 8 k-rows x 16 bytes per thread,
//     4 x 4 byte transposes (v_perm_b32) and ds_write_b64 into the same
//     K-contiguous swizzled layout.
// Buffer resources give hardware bounds checks: rows past M / N read zero.
//
// LDS tile layout (both operands): row r holds 128 k-bytes as 8 chunks of 16
// B; chunk c of row r is stored at position c ^ f(r), f(r) = (r ^ r >> 4) & 7.
// That keeps the fragment reads (two ds_read_b128 per lane), the direct loads
// and the transposed 8-byte writes free of bank conflicts.
//
// Block scales (xuOAO/practice_cuda kernels/bmm/per_block.py:99-111): every
// quant-K block accumulates a partial P in the MFMA, then acc += P * (sa*sb);
// the partials of one N sub-tile are folded while the next sub-tile's MFMAs
// run. Channel / tensor scales accumulate all of K in the MFMA and scale in
// the epilogue (per_channel.py:82-98, per_tensor.py:76).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "abi_util.h"
#include "bmm_epilogue.h"
#include "bmm_fast.h"
#include "bmm_lds.h"
#include "fp8_common.h"

namespace pcamd {
namespace bmmf {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int NT = 256;
constexpr int BM = 128, BN = 256, BK = 128;
constexpr int A_BYTES = BM * BK, B_BYTES = BN * BK;
constexpr int STAGE = A_BYTES + B_BYTES;
constexpr uint32_t kRsrcWord3 = 0x00020000u;  // gfx9-family raw buffer descriptor

PCAMD_DEV int swz(int r) { return (r ^ (r >> 4)) & 7; }

// The descriptor must live in SGPRs: route the (wave-uniform) base and size
// through readfirstlane so the compiler knows they are uniform.
PCAMD_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
  void* ub = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, __builtin_amdgcn_readfirstlane(bytes), kRsrcWord3);
}

PCAMD_DEV uint4 buf_load16(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
  v4i v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// K-major operand: ROWS x 128 bytes from rows (row0 + r) of stride ld.
template <int ROWS>
PCAMD_DEV void issue_kmajor(__amdgpu_buffer_rsrc_t rs, uint8_t* tile, uint32_t row0, uint32_t ld,
                            uint32_t k0, int wave, int lane) {
  constexpr int PER_WAVE = ROWS / 4;
#pragma unroll
  for (int i = 0; i < PER_WAVE / 8; ++i) {
    const int rb = wave * PER_WAVE + i * 8;  // first row of this instruction
    const int r = rb + (lane >> 3);
    const int c = (lane & 7) ^ swz(r);      // chunk that belongs in slot (r, lane & 7)
    const uint32_t off = (row0 + r) * ld + k0 + c * 16;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(tile + rb * BK), 16, off, 0, 0, 0);
  }
}

PCAMD_DEV void transpose4x4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3, uint32_t (&e)[4]) {
  const uint32_t t0 = __builtin_amdgcn_perm(d1, d0, 0x05010400u);
  const uint32_t t1 = __builtin_amdgcn_perm(d1, d0, 0x07030602u);
  const uint32_t t2 = __builtin_amdgcn_perm(d3, d2, 0x05010400u);
  const uint32_t t3 = __builtin_amdgcn_perm(d3, d2, 0x07030602u);
  e[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
  e[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
  e[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
  e[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

PCAMD_DEV uint32_t comp(const uint4& v, int i) { return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w; }

// MN-major operand: the global tile is 128 k-rows of ROWS contiguous bytes.
// Thread t < ROWS owns an 8 (k) x 16 (row) byte block: cb = 16-row group,
// kb = 8-k group, lanes paired by k parity so the 8-byte LDS writes of a
// 16-lane group cover all banks.
template <int ROWS>
struct MNStage {
  static constexpr int NCB = ROWS / 16;
  uint4 r[8];
  PCAMD_DEV void load(__amdgpu_buffer_rsrc_t rs, uint32_t col0, uint32_t ld, uint32_t k0, int t) {
    if (t < ROWS) {
      const int cb = (t >> 1) % NCB, kb = ((t >> 1) / NCB) * 2 + (t & 1);
      const uint32_t base = (k0 + 8 * kb) * ld + col0 + 16 * cb;
#pragma unroll
      for (int j = 0; j < 8; ++j) r[j] = buf_load16(rs, base + j * ld);
    }
  }
  PCAMD_DEV void store(uint8_t* tile, int t) const {
    if (t < ROWS) {
      const int cb = (t >> 1) % NCB, kb = ((t >> 1) / NCB) * 2 + (t & 1);
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint32_t lo[4], hi[4];
        transpose4x4(comp(r[0], w), comp(r[1], w), comp(r[2], w), comp(r[3], w), lo);
        transpose4x4(comp(r[4], w), comp(r[5], w), comp(r[6], w), comp(r[7], w), hi);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * cb + 4 * w + i;
          const int off = row * BK + (((kb >> 1) ^ swz(row)) << 4) + ((kb & 1) << 3);
          *reinterpret_cast<uint2*>(tile + off) = make_uint2(lo[i], hi[i]);
        }
      }
    }
  }
};

// MFMA operand fragment: row `row` of a swizzled tile, k bytes [32 g, 32 g + 32)
PCAMD_DEV v8i frag(const uint8_t* tile, int row, int g) {
  const uint4* l = reinterpret_cast<const uint4*>(tile + row * BK);
  const int s = swz(row);
  const uint4 x = l[(2 * g) ^ s];
  const uint4 y = l[(2 * g + 1) ^ s];
  v8i f;
  f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
  f[4] = y.x; f[5] = y.y; f[6] = y.z; f[7] = y.w;
  return f;
}

// Fused A quantization: the 128 x 128 A tile of a K step arrives as 16-bit
// values (bf16 / fp16) in registers and leaves as fp8 in the swizzled LDS
// layout frag() reads. Lane l of wave w holds, for i = 0..7, chunk l & 15 (8
// elements) of row 32 w + 4 i + l / 16, so the 16 lanes of a DPP row hold one
// row's 128-element group: its amax is group_max<16> and its scales and bytes
// are those of the 1 x 128 quantizer (quant_groups_kernel: the same helpers,
// the reference's per-block math kernels/quant/per_block.py:35-48).
template <int DT>
struct AQStage {
  uint4 r[8];
  PCAMD_DEV static int row_of(int wave, int lane, int i) { return wave * 32 + i * 4 + (lane >> 4); }
  PCAMD_DEV void load(__amdgpu_buffer_rsrc_t rs, uint32_t row0, uint32_t ld, uint32_t k0, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      r[i] = buf_load16(rs, (row0 + row_of(wave, lane, i)) * ld + k0 * 2 + (lane & 15) * 16);
  }
  // tile: the stage's A region; sa: the stage's 128 row scales in LDS. With
  // write_out, rows below m also go to qa_out / sa_out (quant-K block kb).
  template <int FMT>
  PCAMD_DEV void store(uint8_t* tile, float* sa, const FastArgs& a, int bidx, int m0, int kb, bool write_out,
                       int wave, int lane) const {
    const int cg = lane & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      Chunk<DT> c;
      c.r[0] = r[i];
      const float amax = group_max<16>(chunk_amax<DT>(c));
      const Scales sc = block_scales(amax, a.fp8_max, a.eps);
      const uint2 q = quant_chunk<DT, FMT>(c, sc.qs, a.fp8_max);
      const int row = row_of(wave, lane, i);
      *reinterpret_cast<uint2*>(tile + row * BK + (((cg >> 1) ^ swz(row)) << 4) + ((cg & 1) << 3)) = q;
      if (cg == 0) sa[row] = sc.ds;
      if (write_out && m0 + row < a.m) {
        const int64_t mm = m0 + row;
        *reinterpret_cast<uint2*>(a.qa_out + bidx * a.sqab + mm * a.sqam + int64_t(kb) * BK + cg * 8) = q;
        if (cg == 0) a.sa_out[bidx * a.soab + mm * a.soam + int64_t(kb) * a.soak] = sc.ds;
      }
    }
  }
};

template <int FMT>
PCAMD_DEV v4f mfma(const v8i& x, const v8i& y, const v4f& c) {
  constexpr int code = FMT == kE5M2 ? 1 : 0;
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, c, code, code, 0, 0, 0, 0);
}


PCAMD_DEV float load_bias(const void* p, int dt, int64_t off) {
  if (dt == kF32) return static_cast<const float*>(p)[off];
  if (dt == kBF16) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[off]) << 16);
  return static_cast<float>(static_cast<const _Float16*>(p)[off]);
}

// bias, activation, any output dtype, partial coverage (out of line). Takes
// plain values, not the argument struct, so the struct stays in SGPRs.
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

// MODE: 0 block, 1 channel, 2 tensor. SB_COL: block mode with qbn < 16 (one
// B scale per output column). QB1: block mode with qbk == 128. ADT: -1 for an
// fp8 A; kBF16 / kF16 for a 16-bit A quantized 1 x 128 in the kernel (block
// mode, qbk == 128), its row scales kept in LDS behind the two stages.
template <bool A_K, bool B_K, int FMT, int MODE, bool SB_COL, bool QB1, int ADT = -1>
__global__ __launch_bounds__(NT, 1) void bmm_fast_kernel(FastArgs a) {
  constexpr bool AQ = ADT == kBF16 || ADT == kF16;
  static_assert(!AQ || (A_K && MODE == 0 && QB1), "fused A quantization: K-major A, 1 x 128 block scales");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  float* sa_lds = reinterpret_cast<float*>(smem + 2 * STAGE);  // [2][BM], fused A quantization only
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, lg = lane >> 4;

  // tile index: XCD-contiguous remap, then GROUP_M rasterization in a batch
  int pid = blockIdx.x;
  if ((a.total_tiles & 7) == 0) pid = (pid & 7) * (a.total_tiles >> 3) + (pid >> 3);
  const int bidx = pid / a.tiles_per_batch;
  const int tile = pid - bidx * a.tiles_per_batch;
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * a.tiles_n;
  const int group = tile / per_group;
  const int first_m = group * GROUP_M;
  const int gm = min(a.tiles_m - first_m, GROUP_M);
  const int in_group = tile - group * per_group;
  const int m0 = (first_m + in_group % gm) * BM;
  const int n0 = (in_group / gm) * BN;

  const __amdgpu_buffer_rsrc_t rsa = make_rsrc(a.a + bidx * a.sab, a.a_extent);
  const __amdgpu_buffer_rsrc_t rsb = make_rsrc(a.b + bidx * a.sbb, a.b_extent);

  MNStage<BM> ast;  // used when A is M-major
  MNStage<BN> bst;  // used when B is N-major
  AQStage<AQ ? ADT : kBF16> aq;  // used when A is quantized here
  const bool write_q = AQ && a.qa_out != nullptr && n0 == 0;

  auto issue = [&](int ks, uint8_t* stage) {
    const uint32_t k0 = ks * BK;
    if constexpr (A_K && !AQ) issue_kmajor<BM>(rsa, stage, m0, a.lda, k0, wave, lane);
    if constexpr (B_K) issue_kmajor<BN>(rsb, stage + A_BYTES, n0, a.ldb, k0, wave, lane);
  };
  auto load_mn = [&](int ks) {
    const uint32_t k0 = ks * BK;
    if constexpr (AQ) aq.load(rsa, m0, a.lda, k0, wave, lane);
    if constexpr (!A_K) ast.load(rsa, m0, a.lda, k0, t);
    if constexpr (!B_K) bst.load(rsb, n0, a.ldb, k0, t);
  };
  // ks: the K step the stage is filled for
  auto store_mn = [&](uint8_t* stage, int ks) {
    if constexpr (AQ) aq.template store<FMT>(stage, sa_lds + (ks & 1) * BM, a, bidx, m0, ks, write_q, wave, lane);
    if constexpr (!A_K) ast.store(stage, t);
    if constexpr (!B_K) bst.store(stage + A_BYTES, t);
  };

  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  constexpr bool KEEP_P = MODE == 0 && !QB1;
  v4f part[KEEP_P ? 4 : 1][KEEP_P ? 8 : 1];
  if constexpr (KEEP_P) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) part[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  const int ksteps = a.k / BK;
  const int row_base = m0 + wm * 64 + lr;           // + 16 mt
  const int col_base = n0 + wn * 128 + 4 * lg;      // + 16 nt + r

  // prologue: stage 0
  load_mn(0);
  issue(0, smem);
  store_mn(smem, 0);

  for (int ks = 0; ks < ksteps; ++ks) {
    uint8_t* cur = smem + (ks & 1) * STAGE;
    uint8_t* nxt = smem + ((ks + 1) & 1) * STAGE;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();

    // block scales of this step's quant-K block (loaded before the next
    // stage's traffic so waiting on them does not wait on it)
    float sav[4] = {0.f, 0.f, 0.f, 0.f};
    float sbv[8][SB_COL ? 4 : 1];
    bool block_end = true;
    if constexpr (MODE == 0) {
      const int kq = (ks * BK) / a.qbk;
      block_end = QB1 || ((ks + 1) * BK) % a.qbk == 0 || ks + 1 == ksteps;
      if (block_end) {
        const float* sab = a.sa + bidx * a.ssab + int64_t(kq) * a.ssa2;
        const float* sbb = a.sb + bidx * a.ssbb + int64_t(kq) * a.ssb1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int mm = row_base + 16 * i;
          if constexpr (AQ) sav[i] = sa_lds[(ks & 1) * BM + wm * 64 + 16 * i + lr];
          else sav[i] = mm < a.m ? sab[int64_t(mm >> a.qbm_shift) * a.ssa1] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if constexpr (SB_COL) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int nn = col_base + 16 * j + r;
              sbv[j][r] = nn < a.n ? sbb[int64_t(nn >> a.qbn_shift) * a.ssb2] : 0.0f;
            }
          } else {
            const int nn = col_base + 16 * j;
            sbv[j][0] = nn < a.n ? sbb[int64_t(nn >> a.qbn_shift) * a.ssb2] : 0.0f;
          }
        }
      }
    }

    if (ks + 1 < ksteps) {
      load_mn(ks + 1);
      issue(ks + 1, nxt);
    }

    v8i af[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = frag(cur, wm * 64 + i * 16 + lr, lg);

    if constexpr (MODE != 0 || KEEP_P) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const v8i bf = frag(cur + A_BYTES, wn * 128 + j * 16 + lr, lg);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (MODE != 0) acc[i][j] = mfma<FMT>(bf, af[i], acc[i][j]);
          else part[i][j] = mfma<FMT>(bf, af[i], part[i][j]);
        }
      }
      if constexpr (KEEP_P) {
        if (block_end) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                acc[i][j][r] += part[i][j][r] * (sav[i] * sbv[j][SB_COL ? r : 0]);
              part[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
            }
        }
      }
    } else {
      // qbk == 128: a fresh partial per step; fold sub-tile j while the
      // MFMAs of sub-tile j + 1 are in flight
      v4f p[4];
      {
        const v8i bf = frag(cur + A_BYTES, wn * 128 + lr, lg);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = mfma<FMT>(bf, af[i], v4f{0.f, 0.f, 0.f, 0.f});
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v4f q[4];
        if (j + 1 < 8) {
          const v8i bf = frag(cur + A_BYTES, wn * 128 + (j + 1) * 16 + lr, lg);
#pragma unroll
          for (int i = 0; i < 4; ++i) q[i] = mfma<FMT>(bf, af[i], v4f{0.f, 0.f, 0.f, 0.f});
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j][r] += p[i][r] * (sav[i] * sbv[j][SB_COL ? r : 0]);
        if (j + 1 < 8) {
#pragma unroll
          for (int i = 0; i < 4; ++i) p[i] = q[i];
        }
      }
    }

    if (ks + 1 < ksteps) store_mn(nxt, ks + 1);
  }

  // ---- epilogue ----
  // SAQ (scales_are_quant, channel mode): 1 / (sa * sb) per element, a
  // compile-time branch so that the other case carries no division
  auto epilogue = [&](auto saq_c) {
    constexpr bool SAQ = decltype(saq_c)::value;
    float tscale = 1.0f;
    if constexpr (MODE == 2) tscale = a.scales_are_quant ? 1.0f / (a.sa[0] * a.sb[0]) : a.sa[0];
    const bool plain = a.bias == nullptr && a.act == PCAMD_ACT_NONE && a.c_dtype == kBF16;
    float sam[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mm = row_base + 16 * i;
      sam[i] = 1.0f;
      if constexpr (MODE == 1) sam[i] = mm < a.m ? a.sa[bidx * a.ssab + int64_t(mm) * a.ssa1] : 0.0f;
    }
    auto value = [&](int i, int j, float (&v)[4]) {
      const int nn = col_base + 16 * j;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float x = acc[i][j][r];
        if constexpr (MODE == 1) {
          float s = nn + r < a.n ? sam[i] * a.sb[bidx * a.ssbb + int64_t(nn + r) * a.ssb1] : 0.0f;
          if constexpr (SAQ) s = 1.0f / s;
          x *= s;
        } else if constexpr (MODE == 2) {
          x *= tscale;
        }
        v[r] = x;
      }
    };
    if (staged_output_ok(a.c, a.scb, a.scm, a.n, plain)) {
      // the stage the last K step did not read is free (every wave passed the
      // last barrier after its final read of it): 8 KiB of it per wave
      store_subtile_staged(smem + (ksteps & 1) * STAGE + wave * 8192, reinterpret_cast<uint16_t*>(a.c) + bidx * a.scb,
                           a.scm, a.m, a.n, m0 + wm * 64, n0 + wn * 128, lane, value);
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int mm = row_base + 16 * i;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int nn = col_base + 16 * j;
        float v[4];
        value(i, j, v);
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

// K <= 128 (one K step, one quant-K block): a single LDS stage (48 KiB), the
// MFMA result is scaled once in the epilogue (acc = P * sa * sb for block
// scales). This is the output-bound config-4 shape, limited by how many tiles
// are in flight: the wave's 64 x 128 output is computed and stored in two
// 64 x 64 halves, so three workgroups share a CU and one's stores overlap the
// others' loads and MFMAs.
// STAGED: plain bf16 output with aligned rows (staged_output_ok, decided on
// the host); otherwise the direct epilogue (bias, activation, other dtypes).
template <bool A_K, bool B_K, int FMT, int MODE, bool SB_COL, bool STAGED>
__global__ __launch_bounds__(NT, STAGED ? 3 : 2) void bmm_single_kernel(FastArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, lg = lane >> 4;

  int pid = blockIdx.x;
  if ((a.total_tiles & 7) == 0) pid = (pid & 7) * (a.total_tiles >> 3) + (pid >> 3);
  const int bidx = pid / a.tiles_per_batch;
  const int tile = pid - bidx * a.tiles_per_batch;
  constexpr int GROUP_M = 8;
  const int per_group = GROUP_M * a.tiles_n;
  const int group = tile / per_group;
  const int first_m = group * GROUP_M;
  const int gm = min(a.tiles_m - first_m, GROUP_M);
  const int in_group = tile - group * per_group;
  const int m0 = (first_m + in_group % gm) * BM;
  const int n0 = (in_group / gm) * BN;

  const int row_base = m0 + wm * 64 + lr;
  const int col_base = n0 + wn * 128 + 4 * lg;
  // per-row and per-column scales, issued first: the MN-major operand's LDS
  // store below waits for its loads, and would otherwise expose their latency.
  // Indices are clamped to the last row / column instead of branching; values
  // of rows and columns past the matrix are never stored.
  float sav[4], sbv[8][SB_COL || MODE == 1 ? 4 : 1];
  const float* sa_b = a.sa + bidx * a.ssab;
  const float* sb_b = a.sb + bidx * a.ssbb;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int mm = min(row_base + 16 * i, a.m - 1);
    if constexpr (MODE == 0) sav[i] = sa_b[int64_t(mm >> a.qbm_shift) * a.ssa1];
    else if constexpr (MODE == 1) sav[i] = sa_b[int64_t(mm) * a.ssa1];
    else sav[i] = 1.0f;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if constexpr (MODE == 0 && !SB_COL) {
      const int nn = min(col_base + 16 * j, a.n - 1);
      sbv[j][0] = sb_b[int64_t(nn >> a.qbn_shift) * a.ssb2];
    } else if constexpr (MODE == 0 || MODE == 1) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int nn = min(col_base + 16 * j + r, a.n - 1);
        sbv[j][r] = MODE == 0 ? sb_b[int64_t(nn >> a.qbn_shift) * a.ssb2] : sb_b[int64_t(nn) * a.ssb1];
      }
    } else {
      sbv[j][0] = 1.0f;
    }
  }

  const __amdgpu_buffer_rsrc_t rsa = make_rsrc(a.a + bidx * a.sab, a.a_extent);
  // An M-major A goes through registers (loads, then byte transposes into the
  // K-contiguous LDS layout); its loads are issued ahead of the direct-to-LDS
  // ones so the transposes overlap them. B goes straight to LDS either way:
  // K-major rows, or N-major k-rows read back with transposing LDS loads.
  MNStage<BM> sta;
  if constexpr (!A_K) sta.load(rsa, m0, a.lda, 0, t);
  if constexpr (A_K) issue_kmajor<BM>(rsa, smem, m0, a.lda, 0, wave, lane);
  if constexpr (B_K) {
    issue_kmajor<BN>(make_rsrc(a.b + bidx * a.sbb, a.b_extent), smem + A_BYTES, n0, a.ldb, 0, wave, lane);
  } else {
    const lds::MNMajorLoader<BN, NT / 64> lb(a.ldb, lane, wave);
    lb.issue(lds::make_rsrc(a.b + bidx * a.sbb, a.b_extent), smem + A_BYTES, n0, a.ldb, 0, wave);
  }
  if constexpr (!A_K) sta.store(smem, t);

  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  v8i af[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) af[i] = frag(smem, wm * 64 + i * 16 + lr, lg);
  // SAQ (scales_are_quant, channel mode): 1 / (sa * sb) per element, a
  // compile-time branch so that the other case carries no division
  auto epilogue = [&](auto saq_c) {
    constexpr bool SAQ = decltype(saq_c)::value;
    float tscale = 1.0f;
    if constexpr (MODE == 2) tscale = a.scales_are_quant ? 1.0f / (a.sa[0] * a.sb[0]) : a.sa[0];
    const bool plain = a.bias == nullptr && a.act == PCAMD_ACT_NONE && a.c_dtype == kBF16;
    if constexpr (STAGED) {
      // every wave holds its A fragments: the A region becomes the staging area
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      __syncthreads();
    }
    // The wave's 64 x 128 output in two 64 x 64 halves, so only 64
    // accumulators are live and three workgroups fit on a CU.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4f acc[4][4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        v8i bf;
        if constexpr (B_K) bf = frag(smem + A_BYTES, wn * 128 + (4 * h + jj) * 16 + lr, lg);
        else bf = lds::frag_mn<BN>(smem + A_BYTES, wn * 128 + (4 * h + jj) * 16, lane);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][jj] = mfma<FMT>(bf, af[i], v4f{0.f, 0.f, 0.f, 0.f});
      }
      auto value = [&](int i, int jj, float (&v)[4]) {
        const int j = 4 * h + jj;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float s;
          if constexpr (MODE == 0) s = sav[i] * sbv[j][SB_COL ? r : 0];  // (sa * sb), then * P
          else if constexpr (MODE == 1) {
            s = sav[i] * sbv[j][r];
            if constexpr (SAQ) s = 1.0f / s;
          } else s = tscale;
          v[r] = acc[i][jj][r] * s;
        }
      };
      if constexpr (STAGED) {
        store_half_staged(smem + wave * 4096, reinterpret_cast<uint16_t*>(a.c) + bidx * a.scb, a.scm, a.m, a.n,
                          m0 + wm * 64, n0 + wn * 128 + 64 * h, lane, value);
        continue;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int mm = row_base + 16 * i;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int nn = col_base + 16 * (4 * h + jj);
          float v[4];
          value(i, jj, v);
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
    }
  };
  if constexpr (MODE == 1) {
    if (a.scales_are_quant) epilogue(std::true_type{});
    else epilogue(std::false_type{});
  } else {
    epilogue(std::false_type{});
  }
}

template <bool A_K, bool B_K, int FMT, int MODE, bool SB_COL>
int launch_single(const FastArgs& a, hipStream_t st) {
  const bool plain = a.bias == nullptr && a.act == PCAMD_ACT_NONE && a.c_dtype == kBF16;
  const bool staged = plain && (a.n & 7) == 0 && (a.scm & 7) == 0 && (a.scb & 7) == 0 &&
                      (reinterpret_cast<uintptr_t>(a.c) & 15) == 0;  // staged_output_ok on the host
  if (staged) bmm_single_kernel<A_K, B_K, FMT, MODE, SB_COL, true><<<a.total_tiles, NT, STAGE, st>>>(a);
  else bmm_single_kernel<A_K, B_K, FMT, MODE, SB_COL, false><<<a.total_tiles, NT, STAGE, st>>>(a);
  return check_launch("bmm_single_kernel");
}

template <bool A_K, bool B_K, int FMT, int MODE, bool SB_COL, bool QB1>
int launch_one(const FastArgs& a, hipStream_t st) {
  auto kern = bmm_fast_kernel<A_K, B_K, FMT, MODE, SB_COL, QB1>;
  static std::atomic<uint64_t> configured{0};  // devices whose LDS limit is set
  const int rc = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), 2 * STAGE, st, configured);
  if (rc != 0) return rc;
  kern<<<a.total_tiles, NT, 2 * STAGE, st>>>(a);
  return check_launch("bmm_fast_kernel");
}

template <bool A_K, bool B_K, int FMT>
int launch_mode(const FastArgs& a, int mode, bool sb_col, bool qb1, hipStream_t st) {
  if (a.k == BK) {  // one K step: single-stage kernel, two workgroups per CU
    if (mode == 1) return launch_single<A_K, B_K, FMT, 1, false>(a, st);
    if (mode == 2) return launch_single<A_K, B_K, FMT, 2, false>(a, st);
    return sb_col ? launch_single<A_K, B_K, FMT, 0, true>(a, st) : launch_single<A_K, B_K, FMT, 0, false>(a, st);
  }
  if (mode == 1) return launch_one<A_K, B_K, FMT, 1, false, false>(a, st);
  if (mode == 2) return launch_one<A_K, B_K, FMT, 2, false, false>(a, st);
  if (sb_col) {
    return qb1 ? launch_one<A_K, B_K, FMT, 0, true, true>(a, st) : launch_one<A_K, B_K, FMT, 0, true, false>(a, st);
  }
  return qb1 ? launch_one<A_K, B_K, FMT, 0, false, true>(a, st) : launch_one<A_K, B_K, FMT, 0, false, false>(a, st);
}

template <int FMT>
int launch_layout(const FastArgs& a, bool a_k, bool b_k, int mode, bool sb_col, bool qb1, hipStream_t st) {
  if (a_k && b_k) return launch_mode<true, true, FMT>(a, mode, sb_col, qb1, st);
  if (a_k) return launch_mode<true, false, FMT>(a, mode, sb_col, qb1, st);
  if (b_k) return launch_mode<false, true, FMT>(a, mode, sb_col, qb1, st);
  return launch_mode<false, false, FMT>(a, mode, sb_col, qb1, st);
}

template <bool B_K, int FMT, bool SB_COL, int ADT>
int launch_fused(const FastArgs& a, hipStream_t st) {
  auto kern = bmm_fast_kernel<true, B_K, FMT, 0, SB_COL, true, ADT>;
  constexpr int kLds = 2 * STAGE + 2 * BM * 4;  // two stages + the quantized A's row scales
  static std::atomic<uint64_t> configured{0};   // devices whose LDS limit is set
  const int rc = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), kLds, st, configured);
  if (rc != 0) return rc;
  kern<<<a.total_tiles, NT, kLds, st>>>(a);
  return check_launch("bmm_fast_kernel (fused A quantization)");
}

template <int FMT, int ADT>
int launch_fused_layout(const FastArgs& a, bool b_k, bool sb_col, hipStream_t st) {
  if (b_k) return sb_col ? launch_fused<true, FMT, true, ADT>(a, st) : launch_fused<true, FMT, false, ADT>(a, st);
  return sb_col ? launch_fused<false, FMT, true, ADT>(a, st) : launch_fused<false, FMT, false, ADT>(a, st);
}

}  // namespace bmmf

int bmm_fused_launch(const FastArgs& a, int a_dtype, int fmt, bool b_k, bool sb_col, hipStream_t st) {
  if (fmt == kE5M2) {
    if (a_dtype == kF16) return bmmf::launch_fused_layout<kE5M2, kF16>(a, b_k, sb_col, st);
    return bmmf::launch_fused_layout<kE5M2, kBF16>(a, b_k, sb_col, st);
  }
  if (a_dtype == kF16) return bmmf::launch_fused_layout<kE4M3, kF16>(a, b_k, sb_col, st);
  return bmmf::launch_fused_layout<kE4M3, kBF16>(a, b_k, sb_col, st);
}

int bmm_fast_launch(const FastArgs& a, int ab_dtype, bool a_k, bool b_k, int mode, bool sb_col, bool qb1,
                    hipStream_t st) {
  if (ab_dtype == kE5M2) return bmmf::launch_layout<kE5M2>(a, a_k, b_k, mode, sb_col, qb1, st);
  return bmmf::launch_layout<kE4M3>(a, a_k, b_k, mode, sb_col, qb1, st);
}

int bmm_fast_tile_m() { return bmmf::BM; }
int bmm_fast_tile_n() { return bmmf::BN; }

}  // namespace pcamd
