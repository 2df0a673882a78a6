// bmm.hip - scaled FP8 batched GEMM for gfx950 behind the C ABI.
//
// c[b] = act(scale(a[b] @ b[b]) + bias[b]) with fp32 accumulation on the
// CDNA4 matrix cores (v_mfma_f32_16x16x128_f8f6f4: one MFMA spans a full
// 128-wide K step, which is exactly one quant-K block of the block-scaled
// recipe).
//
// Workgroup: 256 threads (4 waves in a 2 x 2 grid), output tile 128 x 128,
// K step 128. Each wave owns 64 x 64 = 4 x 4 MFMA tiles. The MFMA is issued
// with the operands swapped (X = B^T rows, Y = A^T columns) so that every
// lane ends up holding four consecutive N outputs of one M row, which turns
// the epilogue into 8-byte row-contiguous stores.
//
// LDS staging (one 16 KiB tile per operand):
//   K-major operand (A k-major, B k-major): [row][8 x 16 B] with the 16-byte
//     chunk index XOR-swizzled by (row & 7); MFMA fragments are two
//     ds_read_b128 per lane, conflict free.
//   MN-major operand (A m-major, B n-major): the global tile arrives as k rows
//     of contiguous m/n bytes; each thread byte-transposes 4 k x 16 m blocks
//     in registers (v_perm_b32) and stores "k4-interleaved" dwords
//     [k / 4][row], the row index XOR 16 on alternate groups of 8 dword
//     columns so the fragment reads (8 x ds_read_b32) hit distinct banks.
//
// Scale epilogues (xuOAO/practice_cuda):
//   block   kernels/bmm/per_block.py:99-111: acc += P_kq * (sa * sb) per
//           quant-K block (P_kq = fp32 partial of that block)
//   channel kernels/bmm/per_channel.py:82-98: acc *= sa[m] * sb[n]
//           (1 / (sa sb) for quant scales)
//   tensor  kernels/bmm/per_tensor.py:76 and :196-204
// then + bias (fp32), exact-erf GELU (kernels/bmm/activation.py:12-19),
// and the cast to the output dtype (bf16/fp16 RNE, fp32, saturating fp8).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <type_traits>

#include "abi_util.h"
#include "bmm_fast.h"
#include "fp8_common.h"

namespace pcamd {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

namespace bmm {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int NT = 256;

enum Mode { kBlock128 = 0, kBlockWide = 1, kChannel = 2, kTensor = 3 };

struct Args {
  const uint8_t* a;
  const uint8_t* b;
  void* c;
  const void* bias;
  const float* sa;
  const float* sb;
  int64_t m, n, k;
  int64_t sab, sam, sak, sbb, sbk, sbn;
  int64_t scb, scm, scn;
  int64_t sbiasb, sbiasm, sbiasn;
  int64_t ssab, ssa1, ssa2, ssbb, ssb1, ssb2;
  int64_t qbm, qbn, qbk;
  int32_t qbm_shift, qbn_shift;  // log2 of qbm / qbn, or -1 if not a power of two
  int32_t tiles_m, tiles_n;
  int64_t tiles_per_batch, total_tiles;
  int32_t c_dtype, bias_dtype, act, scales_are_quant;
  int32_t vec_a, vec_b;  // 16-byte global loads are aligned for a / b
};

// ---------------------------------------------------------------------------
// 4 x 4 byte transpose: in[j] holds bytes (row j, cols 0..3); out[i] holds
// bytes (col i, rows 0..3).
// ---------------------------------------------------------------------------
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

// Byte-wise masked 16-byte gather: element j at base + j * step, valid while
// j < count (count may be <= 0).
__device__ __attribute__((noinline)) uint4 gather16(const uint8_t* base, int64_t step, int64_t count) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int j = 0; j < 16; ++j)
    if (j < count) w[j >> 2] |= static_cast<uint32_t>(base[j * step]) << (8 * (j & 3));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------------------
// operand stage: global tile (128 rows x 128 k) -> registers -> LDS
// ---------------------------------------------------------------------------
template <bool KMAJOR>
struct Stage;

// rows are contiguous along k (stride s_k == 1)
template <>
struct Stage<true> {
  uint4 r[4];
  PCAMD_DEV void load(const uint8_t* base, int64_t s_row, int64_t s_k, int64_t row0, int64_t rows,
                      int64_t k0, int64_t kt, bool vec, int t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = t + NT * i;
      const int64_t row = row0 + (q >> 3);
      const int64_t kk = k0 + (q & 7) * 16;
      if (row < rows && vec && kk + 16 <= kt) {
        r[i] = *reinterpret_cast<const uint4*>(base + row * s_row + kk);
      } else {
        r[i] = row < rows ? gather16(base + row * s_row + kk * s_k, s_k, kt - kk) : make_uint4(0, 0, 0, 0);
      }
    }
  }
  PCAMD_DEV void store(uint8_t* lds, int t) const {
    uint4* l = reinterpret_cast<uint4*>(lds);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int q = t + NT * i;
      const int row = q >> 3, c = q & 7;
      l[row * 8 + (c ^ (row & 7))] = r[i];
    }
  }
  static PCAMD_DEV v8i frag(const uint8_t* lds, int row, int g) {
    const uint4* l = reinterpret_cast<const uint4*>(lds);
    const uint4 x = l[row * 8 + ((2 * g) ^ (row & 7))];
    const uint4 y = l[row * 8 + ((2 * g + 1) ^ (row & 7))];
    v8i f;
    f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
    f[4] = y.x; f[5] = y.y; f[6] = y.z; f[7] = y.w;
    return f;
  }
};

// k rows are contiguous along the m / n dimension (stride s_row == 1)
template <>
struct Stage<false> {
  uint4 r[4];
  PCAMD_DEV void load(const uint8_t* base, int64_t s_row, int64_t s_k, int64_t row0, int64_t rows,
                      int64_t k0, int64_t kt, bool vec, int t) {
    const int mb = t & 7, kb = t >> 3;
    const int64_t row = row0 + 16 * mb;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t kk = k0 + 4 * kb + j;
      if (kk < kt && vec && row + 16 <= rows) {
        r[j] = *reinterpret_cast<const uint4*>(base + kk * s_k + row);
      } else {
        r[j] = kk < kt ? gather16(base + kk * s_k + row * s_row, s_row, rows - row) : make_uint4(0, 0, 0, 0);
      }
    }
  }
  PCAMD_DEV void store(uint8_t* lds, int t) const {
    uint32_t* l = reinterpret_cast<uint32_t*>(lds);
    const int mb = t & 7, kb = t >> 3;
    const int flip = ((kb >> 3) & 1) << 4;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t e[4];
      transpose4x4(comp(r[0], w), comp(r[1], w), comp(r[2], w), comp(r[3], w), e);
      const int rowp = (16 * mb + 4 * w) ^ flip;
      *reinterpret_cast<uint4*>(l + kb * BM + rowp) = make_uint4(e[0], e[1], e[2], e[3]);
    }
  }
  static PCAMD_DEV v8i frag(const uint8_t* lds, int row, int g) {
    const uint32_t* l = reinterpret_cast<const uint32_t*>(lds);
    const int rowp = row ^ ((g & 1) << 4);
    v8i f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = static_cast<int>(l[(8 * g + j) * BM + rowp]);
    return f;
  }
};

// Format codes per operand (0 = fp8 e4m3, 1 = bf8 e5m2). The operands are
// swapped (x: B fragment, y: A fragment), so src0's code (cbsz) is B's and
// src1's (blgp) is A's.
template <int FA, int FB>
PCAMD_DEV v4f mfma(const v8i& x, const v8i& y, const v4f& c) {
  constexpr int ca = FA == kE5M2 ? 1 : 0, cb = FB == kE5M2 ? 1 : 0;
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, c, cb, ca, 0, 0, 0, 0);
}

PCAMD_DEV int64_t qidx(int64_t v, int32_t shift, int64_t q) { return shift >= 0 ? (v >> shift) : v / q; }

PCAMD_DEV float load_bias(const void* p, int dt, int64_t off) {
  if (dt == kF32) return static_cast<const float*>(p)[off];
  if (dt == kBF16) return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(p)[off]) << 16);
  return static_cast<float>(static_cast<const _Float16*>(p)[off]);
}

PCAMD_DEV float gelu(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865475f)); }

PCAMD_DEV int out_bytes(int dt) { return dt == kF32 ? 4 : (dt == kBF16 || dt == kF16) ? 2 : 1; }

// General epilogue for four consecutive outputs c[b, m, n..n+nvalid): bias,
// activation and any output dtype. Out of line: it only runs for tiles that
// need bias / GELU / non-bf16 output / partial coverage.
__device__ __attribute__((noinline)) void epilogue_general(const Args& a, int64_t bidx, int64_t mm, int64_t nn,
                                                          int nvalid, float v0, float v1, float v2, float v3) {
  float v[4] = {v0, v1, v2, v3};
  for (int r = 0; r < nvalid; ++r) {
    float x = v[r];
    if (a.bias) x += load_bias(a.bias, a.bias_dtype, bidx * a.sbiasb + mm * a.sbiasm + (nn + r) * a.sbiasn);
    if (a.act == PCAMD_ACT_GELU) x = gelu(x);
    v[r] = x;
  }
  const int dt = a.c_dtype;
  char* crow = static_cast<char*>(a.c) + (bidx * a.scb + mm * a.scm) * out_bytes(dt);
  for (int r = 0; r < nvalid; ++r) {
    const int64_t off = (nn + r) * a.scn;
    if (dt == kBF16) {
      reinterpret_cast<__bf16*>(crow)[off] = static_cast<__bf16>(v[r]);
    } else if (dt == kF16) {
      reinterpret_cast<_Float16*>(crow)[off] = static_cast<_Float16>(v[r]);
    } else if (dt == kF32) {
      reinterpret_cast<float*>(crow)[off] = v[r];
    } else {
      // saturating fp8 output: clamp to the format maximum, then RNE
      const float q = clamp_sym(v[r], dt == kE5M2 ? 57344.0f : 448.0f);
      const uint32_t w = dt == kE5M2 ? hw_pack4<kE5M2>(q, 0.f, 0.f, 0.f) : hw_pack4<kE4M3>(q, 0.f, 0.f, 0.f);
      reinterpret_cast<uint8_t*>(crow)[off] = static_cast<uint8_t>(w & 0xFFu);
    }
  }
}

// Two floats to bf16 (round to nearest even) as one v_cvt_pk_bf16_f32.
PCAMD_DEV uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

template <bool A_K, bool B_K, int FA, int FB, int MODE>
__global__ __launch_bounds__(NT) void bmm_kernel(Args a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds_a[BM * BK];
  __shared__ __attribute__((aligned(16))) uint8_t lds_b[BN * BK];

  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, lg = lane >> 4;

  // ---- tile index: XCD-contiguous remap, then grouped rasterization ----
  int64_t pid = blockIdx.x;
  if ((a.total_tiles & 7) == 0) pid = (pid & 7) * (a.total_tiles >> 3) + (pid >> 3);
  const int64_t bidx = pid / a.tiles_per_batch;
  const int64_t tile = pid - bidx * a.tiles_per_batch;
  constexpr int GROUP_M = 8;
  const int64_t per_group = static_cast<int64_t>(GROUP_M) * a.tiles_n;
  const int64_t group = tile / per_group;
  const int64_t first_m = group * GROUP_M;
  const int64_t gm = min(static_cast<int64_t>(a.tiles_m) - first_m, static_cast<int64_t>(GROUP_M));
  const int64_t in_group = tile - group * per_group;
  const int64_t tm = first_m + in_group % gm;
  const int64_t tn = in_group / gm;
  const int64_t m0 = tm * BM, n0 = tn * BN;

  const uint8_t* abase = a.a + bidx * a.sab;
  const uint8_t* bbase = a.b + bidx * a.sbb;

  Stage<A_K> sa_stage;
  Stage<B_K> sb_stage;
  // A rows are m (stride sam) with k stride sak; B rows are n (stride sbn) with k stride sbk.
  sa_stage.load(abase, a.sam, a.sak, m0, a.m, 0, a.k, a.vec_a, t);
  sb_stage.load(bbase, a.sbn, a.sbk, n0, a.n, 0, a.k, a.vec_b, t);

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  v4f part[MODE == kBlockWide ? 4 : 1][MODE == kBlockWide ? 4 : 1];
  if constexpr (MODE == kBlockWide) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) part[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
  }

  const int64_t ksteps = (a.k + BK - 1) / BK;
  for (int64_t ks = 0; ks < ksteps; ++ks) {
    __syncthreads();
    sa_stage.store(lds_a, t);
    sb_stage.store(lds_b, t);
    __syncthreads();
    if (ks + 1 < ksteps) {
      sa_stage.load(abase, a.sam, a.sak, m0, a.m, (ks + 1) * BK, a.k, a.vec_a, t);
      sb_stage.load(bbase, a.sbn, a.sbk, n0, a.n, (ks + 1) * BK, a.k, a.vec_b, t);
    }

    v8i bfr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bfr[j] = Stage<B_K>::frag(lds_b, wn * 64 + j * 16 + lr, lg);

    if constexpr (MODE == kChannel || MODE == kTensor) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v8i afr = Stage<A_K>::frag(lds_a, wm * 64 + i * 16 + lr, lg);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma<FA, FB>(bfr[j], afr, acc[i][j]);
      }
    } else {
      // block scales: quant-K block of this step and whether it ends here
      const int64_t kbeg = ks * BK;
      const int64_t kq = kbeg / a.qbk;
      const bool block_end = (MODE == kBlock128) || ((kbeg + BK) % a.qbk == 0) || (ks + 1 == ksteps);
      float sav[4], sbv[4][4];
      if (block_end) {
        const float* sab = a.sa + bidx * a.ssab + kq * a.ssa2;
        const float* sbb = a.sb + bidx * a.ssbb + kq * a.ssb1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int64_t mm = m0 + wm * 64 + i * 16 + lr;
          sav[i] = mm < a.m ? sab[qidx(mm, a.qbm_shift, a.qbm) * a.ssa1] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int64_t nn = n0 + wn * 64 + j * 16 + 4 * lg + r;
            sbv[j][r] = nn < a.n ? sbb[qidx(nn, a.qbn_shift, a.qbn) * a.ssb2] : 0.0f;
          }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v8i afr = Stage<A_K>::frag(lds_a, wm * 64 + i * 16 + lr, lg);
        if constexpr (MODE == kBlock128) {
          v4f p[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) p[j] = mfma<FA, FB>(bfr[j], afr, v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[i][j][r] += p[j][r] * (sav[i] * sbv[j][r]);
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) part[i][j] = mfma<FA, FB>(bfr[j], afr, part[i][j]);
          if (block_end) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
              for (int r = 0; r < 4; ++r) acc[i][j][r] += part[i][j][r] * (sav[i] * sbv[j][r]);
              part[i][j] = v4f{0.f, 0.f, 0.f, 0.f};
            }
          }
        }
      }
    }
  }

  // ---- epilogue: scales, then bf16 fast path or the general path ----
  // SAQ (scales_are_quant, channel mode): 1 / (sa * sb) per element, a
  // compile-time branch so that the other case carries no division
  auto epilogue = [&](auto saq_c) {
    constexpr bool SAQ = decltype(saq_c)::value;
    float tscale = 1.0f;
    if constexpr (MODE == kTensor) tscale = a.scales_are_quant ? 1.0f / (a.sa[0] * a.sb[0]) : a.sa[0];
    const bool plain = a.bias == nullptr && a.act == PCAMD_ACT_NONE && a.c_dtype == kBF16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t mm = m0 + wm * 64 + i * 16 + lr;
      float sam_v = 1.0f;
      if constexpr (MODE == kChannel) sam_v = mm < a.m ? a.sa[bidx * a.ssab + mm * a.ssa1] : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int64_t nn = n0 + wn * 64 + j * 16 + 4 * lg;
        float v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x = acc[i][j][r];
          if constexpr (MODE == kChannel) {
            float s = nn + r < a.n ? sam_v * a.sb[bidx * a.ssbb + (nn + r) * a.ssb1] : 0.0f;
            if constexpr (SAQ) s = 1.0f / s;
            x *= s;
          } else if constexpr (MODE == kTensor) {
            x *= tscale;
          }
          v[r] = x;
        }
        if (mm >= a.m || nn >= a.n) continue;
        __bf16* p = reinterpret_cast<__bf16*>(a.c) + bidx * a.scb + mm * a.scm + nn;
        if (plain && nn + 4 <= a.n && (reinterpret_cast<uintptr_t>(p) & 7) == 0) {
          *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
        } else {
          const int nvalid = static_cast<int>(min(static_cast<int64_t>(4), a.n - nn));
          epilogue_general(a, bidx, mm, nn, nvalid, v[0], v[1], v[2], v[3]);
        }
      }
    }
  };
  if constexpr (MODE == kChannel) {
    if (a.scales_are_quant) epilogue(std::true_type{});
    else epilogue(std::false_type{});
  } else {
    epilogue(std::false_type{});
  }
}

template <bool A_K, bool B_K, int FA, int FB>
int launch_mode(const Args& a, int mode, hipStream_t st) {
  const int grid = static_cast<int>(a.total_tiles);
  switch (mode) {
    case kBlock128: bmm_kernel<A_K, B_K, FA, FB, kBlock128><<<grid, NT, 0, st>>>(a); break;
    case kBlockWide: bmm_kernel<A_K, B_K, FA, FB, kBlockWide><<<grid, NT, 0, st>>>(a); break;
    case kChannel: bmm_kernel<A_K, B_K, FA, FB, kChannel><<<grid, NT, 0, st>>>(a); break;
    default: bmm_kernel<A_K, B_K, FA, FB, kTensor><<<grid, NT, 0, st>>>(a); break;
  }
  return check_launch("bmm_kernel");
}

template <int FA, int FB>
int launch_layout(const Args& a, bool a_k, bool b_k, int mode, hipStream_t st) {
  if (a_k && b_k) return launch_mode<true, true, FA, FB>(a, mode, st);
  if (a_k && !b_k) return launch_mode<true, false, FA, FB>(a, mode, st);
  if (!a_k && b_k) return launch_mode<false, true, FA, FB>(a, mode, st);
  return launch_mode<false, false, FA, FB>(a, mode, st);
}

inline int launch_formats(const Args& a, int a_fmt, int b_fmt, bool a_k, bool b_k, int mode, hipStream_t st) {
  if (a_fmt == kE4M3 && b_fmt == kE4M3) return launch_layout<kE4M3, kE4M3>(a, a_k, b_k, mode, st);
  if (a_fmt == kE5M2 && b_fmt == kE5M2) return launch_layout<kE5M2, kE5M2>(a, a_k, b_k, mode, st);
  if (a_fmt == kE5M2) return launch_layout<kE5M2, kE4M3>(a, a_k, b_k, mode, st);
  return launch_layout<kE4M3, kE5M2>(a, a_k, b_k, mode, st);
}

inline int log2_or_neg(int64_t v) {
  if (v <= 0 || (v & (v - 1))) return -1;
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}

}  // namespace bmm
}  // namespace pcamd

using namespace pcamd;

// The body of pcamd_bmm_scaled and pcamd_bmm_scaled_mixed: a_fmt / b_fmt
// are each operand's fp8 format.
static int bmm_scaled(const void* a, int a_fmt, const void* b, int b_fmt, int64_t batch, int64_t m, int64_t n,
                      int64_t k, int64_t sab, int64_t sam, int64_t sak, int64_t sbb, int64_t sbk, int64_t sbn,
                      void* c, int c_dtype, int64_t scb, int64_t scm, int64_t scn, const void* bias,
                      int bias_dtype, int64_t sbiasb, int64_t sbiasm, int64_t sbiasn, const float* sa,
                      int64_t ssab, int64_t ssa1, int64_t ssa2, const float* sb, int64_t ssbb, int64_t ssb1,
                      int64_t ssb2, int scale_mode, int scales_are_quant, int64_t qbm, int64_t qbk, int64_t qbn,
                      int activation, void* stream) {
  if (a_fmt != kE4M3 && a_fmt != kE5M2)
    return set_error(PCAMD_ERR_INVALID, "a must be fp8 (code %d or %d), got %d", kE4M3, kE5M2, a_fmt);
  if (b_fmt != kE4M3 && b_fmt != kE5M2)
    return set_error(PCAMD_ERR_INVALID, "b must be fp8 (code %d or %d), got %d", kE4M3, kE5M2, b_fmt);
  const bool same_fmt = a_fmt == b_fmt;
  if (c_dtype != kF32 && c_dtype != kBF16 && c_dtype != kF16 && c_dtype != kE4M3 && c_dtype != kE5M2)
    return set_error(PCAMD_ERR_INVALID, "unsupported output dtype code %d", c_dtype);
  if (bias && bias_dtype != kF32 && bias_dtype != kBF16 && bias_dtype != kF16)
    return set_error(PCAMD_ERR_INVALID, "unsupported bias dtype code %d", bias_dtype);
  if (batch < 0 || m < 0 || n < 0 || k < 0) return set_error(PCAMD_ERR_INVALID, "negative size");
  if (activation != PCAMD_ACT_NONE && activation != PCAMD_ACT_GELU)
    return set_error(PCAMD_ERR_INVALID, "unknown activation %d", activation);
  if (scale_mode < PCAMD_SCALE_BLOCK || scale_mode > PCAMD_SCALE_TENSOR)
    return set_error(PCAMD_ERR_INVALID, "unknown scale mode %d", scale_mode);
  if (batch == 0 || m == 0 || n == 0) return PCAMD_OK;
  if (!c || !sa || (scale_mode != PCAMD_SCALE_TENSOR && !sb) || (k > 0 && (!a || !b)))
    return set_error(PCAMD_ERR_INVALID, "null pointer");
  if (scale_mode == PCAMD_SCALE_TENSOR && scales_are_quant && !sb)
    return set_error(PCAMD_ERR_INVALID, "tensor mode with quant scales needs sb");
  const bool a_k = sak == 1;
  const bool b_k = sbk == 1;
  if (!a_k && sam != 1) return set_error(PCAMD_ERR_INVALID, "A must be contiguous along K or M");
  if (!b_k && sbn != 1) return set_error(PCAMD_ERR_INVALID, "B must be contiguous along N or K");
  if (scn != 1) return set_error(PCAMD_ERR_INVALID, "C must be contiguous along N");
  int mode = bmm::kTensor;
  if (scale_mode == PCAMD_SCALE_BLOCK) {
    if (qbk < 128 || qbk % 128 != 0)
      return set_error(PCAMD_ERR_INVALID, "quant_block_k must be a positive multiple of 128, got %lld",
                       (long long)qbk);
    if (qbm <= 0 || qbn <= 0) return set_error(PCAMD_ERR_INVALID, "quant block sizes must be positive");
    mode = qbk == 128 ? bmm::kBlock128 : bmm::kBlockWide;
  } else if (scale_mode == PCAMD_SCALE_CHANNEL) {
    mode = bmm::kChannel;
  }
  bmm::Args args{};
  args.a = static_cast<const uint8_t*>(a);
  args.b = static_cast<const uint8_t*>(b);
  args.c = c; args.bias = bias; args.sa = sa; args.sb = sb;
  args.m = m; args.n = n; args.k = k;
  args.sab = sab; args.sam = sam; args.sak = sak; args.sbb = sbb; args.sbk = sbk; args.sbn = sbn;
  args.scb = scb; args.scm = scm; args.scn = scn;
  args.sbiasb = sbiasb; args.sbiasm = sbiasm; args.sbiasn = sbiasn;
  args.ssab = ssab; args.ssa1 = ssa1; args.ssa2 = ssa2; args.ssbb = ssbb; args.ssb1 = ssb1; args.ssb2 = ssb2;
  args.qbm = qbm > 0 ? qbm : 1; args.qbn = qbn > 0 ? qbn : 1; args.qbk = qbk > 0 ? qbk : 128;
  args.qbm_shift = bmm::log2_or_neg(args.qbm);
  args.qbn_shift = bmm::log2_or_neg(args.qbn);
  args.tiles_m = static_cast<int32_t>((m + bmm::BM - 1) / bmm::BM);
  args.tiles_n = static_cast<int32_t>((n + bmm::BN - 1) / bmm::BN);
  args.tiles_per_batch = static_cast<int64_t>(args.tiles_m) * args.tiles_n;
  args.total_tiles = args.tiles_per_batch * batch;
  if (args.total_tiles > INT32_MAX) return set_error(PCAMD_ERR_UNSUPPORTED, "too many output tiles");
  args.c_dtype = c_dtype; args.bias_dtype = bias_dtype; args.act = activation;
  args.scales_are_quant = scales_are_quant;
  // 16-byte vector loads need a 16-byte aligned base and row strides
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  args.vec_a = al16(a) && (sab % 16 == 0) && (a_k ? sam % 16 == 0 : sak % 16 == 0);
  args.vec_b = al16(b) && (sbb % 16 == 0) && (b_k ? sbn % 16 == 0 : sbk % 16 == 0);
  hipStream_t st = static_cast<hipStream_t>(stream);

  // tuned path: K a multiple of 128, 16-byte aligned operands and rows,
  // power-of-two block sizes, 32-bit addressable batch slices.
  // PCAMD_BMM_WIDE=0 / PCAMD_BMM_STREAM=0 / PCAMD_BMM_GENERIC select the other
  // kernels (read once)
  static const bool env_no_wide = [] {
    const char* e = getenv("PCAMD_BMM_WIDE");
    return e && e[0] == '0';
  }();
  static const bool env_generic = getenv("PCAMD_BMM_GENERIC") != nullptr;
  static const bool env_no_stream = [] {
    const char* e = getenv("PCAMD_BMM_STREAM");
    return e && e[0] == '0';
  }();
  {
    // K not a multiple of 128: the wide kernel masks its last K step (two
    // steps or more, K a multiple of 4); the other fast kernels need whole steps
    const bool ragged = k % 128 != 0;
    const bool wide = k > 128 && (!ragged || k % 4 == 0) &&
                      (scale_mode != PCAMD_SCALE_BLOCK || args.qbk == 128) && !env_no_wide;
    const int64_t TM = wide ? bmm_wide_tile() : bmm_fast_tile_m();
    const int64_t TN = wide ? bmm_wide_tile() : bmm_fast_tile_n();
    const int64_t tm = (m + TM - 1) / TM, tn = (n + TN - 1) / TN;
    const int64_t lda = a_k ? sam : sak, ldb = b_k ? sbn : sbk;
    // largest byte offset a workgroup can form (rows padded to the tile, K to
    // the step)
    const int64_t kpad = (k + 127) / 128 * 128;
    const int64_t a_max = a_k ? (tm * TM) * lda + kpad : (kpad - 1) * lda + tm * TM;
    const int64_t b_max = b_k ? (tn * TN) * ldb + kpad : (kpad - 1) * ldb + tn * TN;
    const bool block_ok = scale_mode != PCAMD_SCALE_BLOCK ||
                          (args.qbm_shift >= 0 && args.qbn_shift >= 0);
    const bool fast = k > 0 && (!ragged || wide) && args.vec_a && args.vec_b && lda % 16 == 0 && ldb % 16 == 0 &&
                      a_max < (int64_t{1} << 32) - 64 && b_max < (int64_t{1} << 32) - 64 &&
                      m < INT32_MAX && n < INT32_MAX && k < INT32_MAX && tm * tn * batch < INT32_MAX &&
                      block_ok && !env_generic;
    if (fast) {
      FastArgs f{};
      f.a = args.a; f.b = args.b; f.c = c; f.bias = bias; f.sa = sa; f.sb = sb;
      f.m = static_cast<int32_t>(m); f.n = static_cast<int32_t>(n); f.k = static_cast<int32_t>(k);
      f.sab = sab; f.sbb = sbb;
      f.lda = static_cast<uint32_t>(lda); f.ldb = static_cast<uint32_t>(ldb);
      f.a_extent = static_cast<uint32_t>(a_k ? (m - 1) * sam + k : (k - 1) * sak + m);
      f.b_extent = static_cast<uint32_t>(b_k ? (n - 1) * sbn + k : (k - 1) * sbk + n);
      f.scb = scb; f.scm = scm; f.scn = scn;
      f.sbiasb = sbiasb; f.sbiasm = sbiasm; f.sbiasn = sbiasn;
      f.ssab = ssab; f.ssa1 = ssa1; f.ssa2 = ssa2; f.ssbb = ssbb; f.ssb1 = ssb1; f.ssb2 = ssb2;
      f.qbk = static_cast<int32_t>(args.qbk); f.qbm_shift = args.qbm_shift; f.qbn_shift = args.qbn_shift;
      f.tiles_m = static_cast<int32_t>(tm); f.tiles_n = static_cast<int32_t>(tn);
      f.tiles_per_batch = static_cast<int32_t>(tm * tn);
      f.total_tiles = static_cast<int32_t>(tm * tn * batch);
      f.c_dtype = c_dtype; f.bias_dtype = bias_dtype; f.act = activation; f.scales_are_quant = scales_are_quant;
      const int fmode = scale_mode == PCAMD_SCALE_BLOCK ? 0 : scale_mode == PCAMD_SCALE_CHANNEL ? 1 : 2;
      const bool sb_col = scale_mode == PCAMD_SCALE_BLOCK && args.qbn < 16;
      const bool qb1 = scale_mode == PCAMD_SCALE_BLOCK && args.qbk == 128;
      // the streaming (config-4) and 128 x 256 kernels take one format for both operands
      if (same_fmt && !env_no_stream && bmm_stream_ok(f, a_k, b_k, fmode, batch, args.qbm, args.qbn, ssa1, ssb2))
        return bmm_stream_launch(f, a_fmt, batch, st);
      if (wide) return bmm_wide_launch(f, a_fmt, b_fmt, a_k, b_k, fmode, st);
      if (same_fmt) return bmm_fast_launch(f, a_fmt, a_k, b_k, fmode, sb_col, qb1, st);
    }
  }
  return bmm::launch_formats(args, a_fmt, b_fmt, a_k, b_k, mode, st);
}

extern "C" int pcamd_bmm_scaled(const void* a, const void* b, int ab_dtype, int64_t batch, int64_t m,
                                int64_t n, int64_t k, int64_t sab, int64_t sam, int64_t sak,
                                int64_t sbb, int64_t sbk, int64_t sbn, void* c, int c_dtype,
                                int64_t scb, int64_t scm, int64_t scn, const void* bias,
                                int bias_dtype, int64_t sbiasb, int64_t sbiasm, int64_t sbiasn,
                                const float* sa, int64_t ssab, int64_t ssa1, int64_t ssa2,
                                const float* sb, int64_t ssbb, int64_t ssb1, int64_t ssb2,
                                int scale_mode, int scales_are_quant, int64_t qbm, int64_t qbk,
                                int64_t qbn, int activation, void* stream) {
  clear_error();
  return bmm_scaled(a, ab_dtype, b, ab_dtype, batch, m, n, k, sab, sam, sak, sbb, sbk, sbn, c, c_dtype, scb, scm,
                    scn, bias, bias_dtype, sbiasb, sbiasm, sbiasn, sa, ssab, ssa1, ssa2, sb, ssbb, ssb1, ssb2,
                    scale_mode, scales_are_quant, qbm, qbk, qbn, activation, stream);
}

extern "C" int pcamd_bmm_scaled_mixed(const void* a, int a_dtype, const void* b, int b_dtype, int64_t batch,
                                      int64_t m, int64_t n, int64_t k, int64_t sab, int64_t sam, int64_t sak,
                                      int64_t sbb, int64_t sbk, int64_t sbn, void* c, int c_dtype, int64_t scb,
                                      int64_t scm, int64_t scn, const void* bias, int bias_dtype, int64_t sbiasb,
                                      int64_t sbiasm, int64_t sbiasn, const float* sa, int64_t ssab, int64_t ssa1,
                                      int64_t ssa2, const float* sb, int64_t ssbb, int64_t ssb1, int64_t ssb2,
                                      int scale_mode, int scales_are_quant, int64_t qbm, int64_t qbk, int64_t qbn,
                                      int activation, void* stream) {
  clear_error();
  return bmm_scaled(a, a_dtype, b, b_dtype, batch, m, n, k, sab, sam, sak, sbb, sbk, sbn, c, c_dtype, scb, scm, scn,
                    bias, bias_dtype, sbiasb, sbiasm, sbiasn, sa, ssab, ssa1, ssa2, sb, ssbb, ssb1, ssb2, scale_mode,
                    scales_are_quant, qbm, qbk, qbn, activation, stream);
}

// Block-scaled BMM with the A operand quantized inside the kernel (1 x 128
// groups along K, the quantizer's exact bytes and scales); see
// include/pcamd_fp8.h. Layouts outside the fused kernel's envelope return
// PCAMD_ERR_UNSUPPORTED so the caller can quantize and multiply separately.
// PCAMD_BMM_FUSED_STREAM=0 (read once per process): narrow fused products take the 128 x 256 kernel too
static bool fused_stream_disabled() {
  static const bool off = [] {
    const char* e = getenv("PCAMD_BMM_FUSED_STREAM");
    return e && e[0] == '0';
  }();
  return off;
}

extern "C" int pcamd_bmm_quant_a(const void* a, int a_dtype, const void* b, int ab_dtype, int64_t batch,
                                 int64_t m, int64_t n, int64_t k, int64_t sab, int64_t sam, int64_t sak,
                                 int64_t sbb, int64_t sbk, int64_t sbn, void* c, int c_dtype, int64_t scb,
                                 int64_t scm, int64_t scn, const void* bias, int bias_dtype, int64_t sbiasb,
                                 int64_t sbiasm, int64_t sbiasn, const float* sb, int64_t ssbb, int64_t ssb1,
                                 int64_t ssb2, int64_t qbn, void* qa_out, int64_t sqab, int64_t sqam,
                                 int64_t sqak, float* sa_out, int64_t soab, int64_t soam, int64_t soak,
                                 float fp8_max, float eps, int activation, void* stream) {
  clear_error();
  if (a_dtype != kBF16 && a_dtype != kF16)
    return set_error(PCAMD_ERR_INVALID, "A must be bf16 (code %d) or fp16 (code %d), got %d", kBF16, kF16, a_dtype);
  if (ab_dtype != kE4M3 && ab_dtype != kE5M2)
    return set_error(PCAMD_ERR_INVALID, "b must be fp8 (code %d or %d), got %d", kE4M3, kE5M2, ab_dtype);
  if (c_dtype != kF32 && c_dtype != kBF16 && c_dtype != kF16 && c_dtype != kE4M3 && c_dtype != kE5M2)
    return set_error(PCAMD_ERR_INVALID, "unsupported output dtype code %d", c_dtype);
  if (bias && bias_dtype != kF32 && bias_dtype != kBF16 && bias_dtype != kF16)
    return set_error(PCAMD_ERR_INVALID, "unsupported bias dtype code %d", bias_dtype);
  if (batch < 0 || m < 0 || n < 0 || k < 0) return set_error(PCAMD_ERR_INVALID, "negative size");
  if (activation != PCAMD_ACT_NONE && activation != PCAMD_ACT_GELU)
    return set_error(PCAMD_ERR_INVALID, "unknown activation %d", activation);
  if (!(fp8_max > 0.0f) || !(eps >= 0.0f)) return set_error(PCAMD_ERR_INVALID, "need fp8_max > 0 and eps >= 0");
  if (qbn <= 0 || (qbn & (qbn - 1))) return set_error(PCAMD_ERR_INVALID, "qbn must be a power of two");
  if ((qa_out == nullptr) != (sa_out == nullptr))
    return set_error(PCAMD_ERR_INVALID, "qa_out and sa_out are given together or not at all");
  if (batch == 0 || m == 0 || n == 0) return PCAMD_OK;
  if (!c || !sb || (k > 0 && (!a || !b))) return set_error(PCAMD_ERR_INVALID, "null pointer");
  if (scn != 1) return set_error(PCAMD_ERR_INVALID, "C must be contiguous along N");
  const bool b_k = sbk == 1;
  if (!b_k && sbn != 1) return set_error(PCAMD_ERR_INVALID, "B must be contiguous along N or K");
  // the fused kernel's envelope
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int64_t lda = sam * 2, ldb = b_k ? sbn : sbk;
  const int64_t tm = (m + bmm_fast_tile_m() - 1) / bmm_fast_tile_m();
  const int64_t tn = (n + bmm_fast_tile_n() - 1) / bmm_fast_tile_n();
  const int64_t a_max = (tm * bmm_fast_tile_m()) * lda + k * 2;
  const int64_t b_max = b_k ? (tn * bmm_fast_tile_n()) * ldb + k : (k - 1) * ldb + tn * bmm_fast_tile_n();
  const bool ok = k > 0 && k % 128 == 0 && sak == 1 && al16(a) && lda % 16 == 0 && (sab * 2) % 16 == 0 &&
                  al16(b) && ldb % 16 == 0 && sbb % 16 == 0 && a_max < (int64_t{1} << 32) - 64 &&
                  b_max < (int64_t{1} << 32) - 64 && m < INT32_MAX && n < INT32_MAX &&
                  tm * tn * batch < INT32_MAX &&
                  (!qa_out || (sqak == 1 && sqam % 8 == 0 && sqab % 8 == 0 &&
                               (reinterpret_cast<uintptr_t>(qa_out) & 7) == 0));
  if (!ok)
    return set_error(PCAMD_ERR_UNSUPPORTED,
                     "fused A quantization needs a K-major 16-byte aligned A, K a positive multiple of 128, "
                     "an aligned B and 32-bit addressable batch slices");
  FastArgs f{};
  f.a = static_cast<const uint8_t*>(a); f.b = static_cast<const uint8_t*>(b); f.c = c; f.bias = bias;
  f.sa = nullptr; f.sb = sb;
  f.m = static_cast<int32_t>(m); f.n = static_cast<int32_t>(n); f.k = static_cast<int32_t>(k);
  f.sab = sab * 2; f.sbb = sbb;
  f.lda = static_cast<uint32_t>(lda); f.ldb = static_cast<uint32_t>(ldb);
  f.a_extent = static_cast<uint32_t>(((m - 1) * sam + k) * 2);
  f.b_extent = static_cast<uint32_t>(b_k ? (n - 1) * sbn + k : (k - 1) * sbk + n);
  f.scb = scb; f.scm = scm; f.scn = scn;
  f.sbiasb = sbiasb; f.sbiasm = sbiasm; f.sbiasn = sbiasn;
  f.ssbb = ssbb; f.ssb1 = ssb1; f.ssb2 = ssb2;
  f.qbk = 128; f.qbm_shift = 0; f.qbn_shift = bmm::log2_or_neg(qbn);
  f.tiles_m = static_cast<int32_t>(tm); f.tiles_n = static_cast<int32_t>(tn);
  f.tiles_per_batch = static_cast<int32_t>(tm * tn);
  f.total_tiles = static_cast<int32_t>(tm * tn * batch);
  f.c_dtype = c_dtype; f.bias_dtype = bias_dtype; f.act = activation; f.scales_are_quant = 0;
  f.qa_out = static_cast<uint8_t*>(qa_out); f.sa_out = sa_out;
  f.sqab = sqab; f.sqam = sqam; f.soab = soab; f.soam = soam; f.soak = soak;
  f.fp8_max = fp8_max; f.eps = eps;
  // narrow products stream A once (the 128 x 256 kernel quantizes each A
  // row block once per N tile and runs few tiles)
  if (bmm_fused_stream_ok(f, batch, qbn) && !fused_stream_disabled())
    return bmm_fused_stream_launch(f, a_dtype, ab_dtype, b_k, batch, static_cast<hipStream_t>(stream));
  return bmm_fused_launch(f, a_dtype, ab_dtype, b_k, qbn < 16, static_cast<hipStream_t>(stream));
}
