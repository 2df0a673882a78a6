// fp8_common.h - device helpers shared by the gfx950 FP8 kernels.
//
// Element conversions, 8-element "chunk" loads (one 128-bit load for 16-bit
// inputs, two for fp32), wavefront max reductions over aligned lane groups
// (DPP inside a 16-lane row, ds_swizzle/bpermute beyond), and fp32 -> OCP
// fp8 packing through the gfx950 hardware converters.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/pcamd_fp8.h"

#define PCAMD_DEV __device__ __forceinline__

namespace pcamd {

constexpr int kF32 = PCAMD_F32;
constexpr int kBF16 = PCAMD_BF16;
constexpr int kF16 = PCAMD_F16;
constexpr int kE4M3 = PCAMD_E4M3FN;
constexpr int kE5M2 = PCAMD_E5M2;
constexpr int kF64 = PCAMD_F64;  // scale arithmetic only

// ---------------------------------------------------------------------------
// element conversions
// ---------------------------------------------------------------------------
PCAMD_DEV float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
PCAMD_DEV float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
PCAMD_DEV float f16_lo(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xFFFFu)));
}
PCAMD_DEV float f16_hi(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

template <int DT>
PCAMD_DEV float load_one(const void* base, int64_t off) {
  if constexpr (DT == kF32) {
    return static_cast<const float*>(base)[off];
  } else if constexpr (DT == kBF16) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(base)[off]) << 16);
  } else {
    return static_cast<float>(static_cast<const _Float16*>(base)[off]);
  }
}

template <int DT>
constexpr int elem_bytes() {
  return DT == kF32 ? 4 : 2;
}

// Eight consecutive input elements as raw bits.
template <int DT>
struct Chunk {
  uint4 r[DT == kF32 ? 2 : 1];
};

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// 4 x 4 byte transpose: byte j of d[i] -> byte i of e[j]
PCAMD_DEV void byte_transpose4(uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3, uint32_t (&e)[4]) {
  const uint32_t lo01 = __builtin_amdgcn_perm(d1, d0, 0x05010400u);  // d0.b0 d1.b0 d0.b1 d1.b1
  const uint32_t hi01 = __builtin_amdgcn_perm(d1, d0, 0x07030602u);  // d0.b2 d1.b2 d0.b3 d1.b3
  const uint32_t lo23 = __builtin_amdgcn_perm(d3, d2, 0x05010400u);
  const uint32_t hi23 = __builtin_amdgcn_perm(d3, d2, 0x07030602u);
  e[0] = __builtin_amdgcn_perm(lo23, lo01, 0x05040100u);
  e[1] = __builtin_amdgcn_perm(lo23, lo01, 0x07060302u);
  e[2] = __builtin_amdgcn_perm(hi23, hi01, 0x05040100u);
  e[3] = __builtin_amdgcn_perm(hi23, hi01, 0x07060302u);
}

// Input chunks are read once: non-temporal loads.
template <int DT>
PCAMD_DEV void load_chunk(Chunk<DT>& c, const void* p) {
  const u32x4_t* q = static_cast<const u32x4_t*>(p);
  const u32x4_t a = __builtin_nontemporal_load(q);
  c.r[0] = make_uint4(a.x, a.y, a.z, a.w);
  if constexpr (DT == kF32) {
    const u32x4_t b = __builtin_nontemporal_load(q + 1);
    c.r[1] = make_uint4(b.x, b.y, b.z, b.w);
  }
}

// The same with ordinary loads, for input that is read again soon.
template <int DT>
PCAMD_DEV void load_chunk_temporal(Chunk<DT>& c, const void* p) {
  const uint4* q = static_cast<const uint4*>(p);
  c.r[0] = q[0];
  if constexpr (DT == kF32) c.r[1] = q[1];
}

template <int DT>
PCAMD_DEV void zero_chunk(Chunk<DT>& c) {
  c.r[0] = make_uint4(0, 0, 0, 0);
  if constexpr (DT == kF32) c.r[1] = make_uint4(0, 0, 0, 0);
}

template <int DT>
PCAMD_DEV void unpack_chunk(const Chunk<DT>& c, float (&v)[8]) {
  if constexpr (DT == kF32) {
    v[0] = __uint_as_float(c.r[0].x); v[1] = __uint_as_float(c.r[0].y);
    v[2] = __uint_as_float(c.r[0].z); v[3] = __uint_as_float(c.r[0].w);
    v[4] = __uint_as_float(c.r[1].x); v[5] = __uint_as_float(c.r[1].y);
    v[6] = __uint_as_float(c.r[1].z); v[7] = __uint_as_float(c.r[1].w);
  } else if constexpr (DT == kBF16) {
    v[0] = bf16_lo(c.r[0].x); v[1] = bf16_hi(c.r[0].x);
    v[2] = bf16_lo(c.r[0].y); v[3] = bf16_hi(c.r[0].y);
    v[4] = bf16_lo(c.r[0].z); v[5] = bf16_hi(c.r[0].z);
    v[6] = bf16_lo(c.r[0].w); v[7] = bf16_hi(c.r[0].w);
  } else {
    v[0] = f16_lo(c.r[0].x); v[1] = f16_hi(c.r[0].x);
    v[2] = f16_lo(c.r[0].y); v[3] = f16_hi(c.r[0].y);
    v[4] = f16_lo(c.r[0].z); v[5] = f16_hi(c.r[0].z);
    v[6] = f16_lo(c.r[0].w); v[7] = f16_hi(c.r[0].w);
  }
}

// bf16 pairs as raw bits: |x| clears the sign bits, and non-negative bf16
// values order like their bit patterns, so the max of |x| over a chunk is an
// unsigned 16-bit max (v_pk_max_u16 does two per instruction). NaN inputs are
// outside the quantizers' contract.
typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
PCAMD_DEV uint32_t bf16_abs2(uint32_t w) { return w & 0x7FFF7FFFu; }
PCAMD_DEV uint32_t pk_max_u16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(u16x2_t, a), __builtin_bit_cast(u16x2_t, b)));
}
// the larger of the two 16-bit halves, zero-extended
PCAMD_DEV uint32_t max_halves(uint32_t m) { return max(m & 0xFFFFu, m >> 16); }
// bf16 bit pattern (low 16 bits) -> float
PCAMD_DEV float bf16_bits(uint32_t b) { return __uint_as_float(b << 16); }

// max |x| over the 8 elements of a chunk
template <int DT>
PCAMD_DEV float chunk_amax(const Chunk<DT>& c) {
  if constexpr (DT == kBF16) {
    const uint32_t m = pk_max_u16(pk_max_u16(bf16_abs2(c.r[0].x), bf16_abs2(c.r[0].y)),
                                  pk_max_u16(bf16_abs2(c.r[0].z), bf16_abs2(c.r[0].w)));
    return bf16_bits(max_halves(m));
  }
  float v[8];
  unpack_chunk<DT>(c, v);
  float a = fmaxf(fabsf(v[0]), fabsf(v[1]));
  float b = fmaxf(fabsf(v[2]), fabsf(v[3]));
  float d = fmaxf(fabsf(v[4]), fabsf(v[5]));
  float e = fmaxf(fabsf(v[6]), fabsf(v[7]));
  return fmaxf(fmaxf(a, b), fmaxf(d, e));
}

// ---------------------------------------------------------------------------
// wavefront reductions: max over aligned groups of LANES lanes (power of 2)
// ---------------------------------------------------------------------------
template <int CTRL>
PCAMD_DEV float dpp_mov(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// All 64 lanes must be active when this is called. v >= 0 (a max of |x|):
// non-negative floats order like their bit patterns, so the steps are
// unsigned maxima, whose identity 0 lets each DPP move fold into its max.
template <int LANES>
PCAMD_DEV float group_max(float v) {
  uint32_t u = __float_as_uint(v);
  auto dpp = [](uint32_t x, auto ctrl) {
    return max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), decltype(ctrl)::value,
                                                                     0xF, 0xF, false)));
  };
  if constexpr (LANES >= 2) u = dpp(u, std::integral_constant<int, kDppQuadXor1>{});
  if constexpr (LANES >= 4) u = dpp(u, std::integral_constant<int, kDppQuadXor2>{});
  // after the quad steps every lane holds its quad's max; mirroring inside 8
  // (then 16) lanes pairs each quad with the other quad of the half-row (row)
  if constexpr (LANES >= 8) u = dpp(u, std::integral_constant<int, kDppRowHalfMirror>{});
  if constexpr (LANES >= 16) u = dpp(u, std::integral_constant<int, kDppRowMirror>{});
  if constexpr (LANES >= 32) {
    // swap the two 16-lane rows of each 32-lane half (bit-mode swizzle, xor 16)
    u = max(u, static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(u), 0x401F)));
  }
  if constexpr (LANES >= 64) u = max(u, static_cast<uint32_t>(__shfl_xor(static_cast<int>(u), 32, 64)));
  return __uint_as_float(u);
}

// Unsigned max over aligned groups of LANES (<= 16) lanes. 0 is the identity
// of the max, so each step can fold its DPP move into the max.
template <int LANES>
PCAMD_DEV uint32_t group_max_u32(uint32_t v) {
  static_assert(LANES <= 16, "row-local DPP steps only");
  auto step = [](uint32_t x, auto ctrl) {
    return max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), decltype(ctrl)::value,
                                                                     0xF, 0xF, false)));
  };
  if constexpr (LANES >= 2) v = step(v, std::integral_constant<int, kDppQuadXor1>{});
  if constexpr (LANES >= 4) v = step(v, std::integral_constant<int, kDppQuadXor2>{});
  if constexpr (LANES >= 8) v = step(v, std::integral_constant<int, kDppRowHalfMirror>{});
  if constexpr (LANES >= 16) v = step(v, std::integral_constant<int, kDppRowMirror>{});
  return v;
}

// value of lane P of this lane's quad (DPP quad_perm [P, P, P, P])
template <int P>
PCAMD_DEV float quad_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), P * 0x55, 0xF, 0xF, false));
}

// ---------------------------------------------------------------------------
// fp32 -> fp8 (OCP e4m3fn / e5m2), round to nearest even
// ---------------------------------------------------------------------------
// Integer restatement (same algorithm as the CPU oracle); used by the
// conversion self-test and available as a fallback path.
template <int FMT>
PCAMD_DEV uint32_t sw_encode(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7FFFFFFFu;
  if constexpr (FMT == kE4M3) {
    if (a > 0x7F800000u || a >= 0x43F00000u) return sign | 0x7Fu;
    if (a < 0x3C800000u) return sign | static_cast<uint32_t>(__builtin_rintf(__uint_as_float(a) * 512.0f));
    uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
    return sign | ((r >> 20) - ((127u - 7u) << 3));
  } else {
    if (a > 0x7F800000u) return sign | 0x7Fu;
    if (a >= 0x47800000u) return sign | 0x7Cu;
    if (a < 0x38800000u) return sign | static_cast<uint32_t>(__builtin_rintf(__uint_as_float(a) * 65536.0f));
    uint32_t r = a + 0xFFFFFu + ((a >> 21) & 1u);
    return sign | ((r >> 21) - ((127u - 15u) << 2));
  }
}

// gfx950 v_cvt_pk_{fp8,bf8}_f32: two fp32 -> two OCP fp8 in the selected
// 16-bit half of the destination (src0 -> low byte).
template <int FMT>
PCAMD_DEV uint32_t hw_pack4(float a, float b, float c, float d) {
  if constexpr (FMT == kE4M3) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true));
  } else {
    int w = __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false);
    return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(c, d, w, true));
  }
}

template <int FMT>
PCAMD_DEV uint32_t pack4(float a, float b, float c, float d) {
  return hw_pack4<FMT>(a, b, c, d);
}

// tl.clamp(v, -max, max)
PCAMD_DEV float clamp_sym(float v, float hi) { return __builtin_amdgcn_fmed3f(v, -hi, hi); }

// quantize a chunk: 8 elements -> 8 fp8 bytes (little-endian in a uint2);
// CLAMP false: see quant8
template <int DT, int FMT, bool CLAMP = true>
PCAMD_DEV uint2 quant_chunk(const Chunk<DT>& c, float qs, float fp8_max) {
  float v[8];
  unpack_chunk<DT>(c, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = CLAMP ? clamp_sym(v[i] * qs, fp8_max) : v[i] * qs;
  return make_uint2(pack4<FMT>(v[0], v[1], v[2], v[3]), pack4<FMT>(v[4], v[5], v[6], v[7]));
}

// Largest finite value of the format.
template <int FMT>
constexpr float fmt_max() {
  return FMT == kE5M2 ? 57344.0f : 448.0f;
}

// Quantize 8 fp32 values (x * qs, clamped to +-fp8_max when CLAMP). The
// clamp of the reference (tl.clamp before the cast) can be left out when
// fp8_max is the format's largest finite value and qs = fp8_max / s with s at
// least the max |x| of the values it scales: then |fl(x * qs)| <= fp8_max *
// (1 + 2^-23), below the rounding midpoint to the next (non-finite) code
// (464 for e4m3fn, 61440 for e5m2), and round-to-nearest-even gives the
// clamped value's code. The conversion self-test pins the hardware converter
// on every pattern up to 464 (e4m3fn) and 59392 (e5m2), both past
// fp8_max * (1 + 2^-23). The host picks these instantiations only when qs is
// finite as well (clamp_free in quant.hip).
template <int FMT, bool CLAMP>
PCAMD_DEV uint2 quant8(const float (&v)[8], float qs, float fp8_max) {
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = CLAMP ? clamp_sym(v[i] * qs, fp8_max) : v[i] * qs;
  return make_uint2(pack4<FMT>(q[0], q[1], q[2], q[3]), pack4<FMT>(q[4], q[5], q[6], q[7]));
}

template <int DT, int FMT>
PCAMD_DEV uint32_t quant_one(float v, float qs, float fp8_max) {
  float q = clamp_sym(v * qs, fp8_max);
  return hw_pack4<FMT>(q, 0.0f, 0.0f, 0.0f) & 0xFFu;
}

// Scale formulas of the reference kernels (IEEE fp32 division).
// per-block:   dequant = 1 / (fp8_max / max(amax, eps))
// per-channel: dequant = max(amax, eps) / fp8_max
// per-tensor:  dequant = 1 / ((1 / max(amax, eps)) * fp8_max)
//   (torchao's tensorwise form, scale_dt kF64: dequant = 1 / fp32(fp8_max / max(amax, eps)) in fp64)
struct Scales {
  float qs, ds;
};
PCAMD_DEV Scales block_scales(float amax, float fp8_max, float eps) {
  float s = fmaxf(amax, eps);
  float qs = fp8_max / s;
  return {qs, 1.0f / qs};
}
PCAMD_DEV Scales channel_scales(float amax, float fp8_max, float eps) {
  float s = fmaxf(amax, eps);
  return {fp8_max / s, s / fp8_max};
}
// Round an fp32 value to dtype dt (RNE) and back; identity for kF32.
PCAMD_DEV float round_dt(float v, int dt) {
  if (dt == kBF16) {
    uint32_t u = __float_as_uint(v);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return v;
    return __uint_as_float((u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u);
  }
  if (dt == kF16) return static_cast<float>(static_cast<_Float16>(v));
  return v;
}

// per-tensor: the reference evaluates `fp8_max / max_abs` as a torch tensor
// op, i.e. reciprocal(max_abs) * fp8_max (two roundings), then reciprocal.
// scale_dt is the dtype those 0-d tensor ops run in: fp32 for
// fp8_bench/impls/triton_per_tensor.py:40-44, the input's dtype for the
// legacy kernels/fp8_bmm/fp8_warper.py:21-25 (each op evaluated in fp32, then
// rounded to that dtype).
PCAMD_DEV Scales tensor_scales(float amax, float fp8_max, float eps, int scale_dt = kF32) {
  if (scale_dt == kF64) {
    // torchao's amax_to_scale: the division in fp64, rounded once to fp32
    const float qs = static_cast<float>(static_cast<double>(fp8_max) /
                                        fmax(static_cast<double>(amax), static_cast<double>(eps)));
    return {qs, 1.0f / qs};
  }
  const float s = round_dt(fmaxf(round_dt(amax, scale_dt), round_dt(eps, scale_dt)), scale_dt);
  const float qs = round_dt(round_dt(1.0f / s, scale_dt) * fp8_max, scale_dt);
  return {qs, round_dt(1.0f / qs, scale_dt)};
}

}  // namespace pcamd
