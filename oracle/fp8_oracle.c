/*
 * fp8_oracle.c - TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of the reference's FP8 quantizer arithmetic, used as the
 * parity checker for the HIP kernels and as the CPU baseline in bench.py.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it; the product (practice_cuda_amd) never does.
 *
 * Paths cited are relative to the reference repository xuOAO/practice_cuda.
 *
 *   oracle_encode_e4m3fn / _e5m2: the fp32 -> fp8 cast that Triton's
 *     `.to(float8_e4m3fn)` performs at kernels/quant/per_block.py:47 and
 *     per_channel.py:93,194 (round to nearest even, OCP formats). Values are
 *     clamped to +-fp8_max before the cast (per_block.py:46), so only the
 *     in-range behaviour is load-bearing.
 *   oracle_quant_block:   kernels/quant/per_block.py:35-48
 *   oracle_quant_channel: kernels/quant/per_channel.py:136-201 (axis -2),
 *                         :202-267 (axis -1), one-pass :35-102
 *   oracle_quant_tensor:  impls/triton_per_tensor.py:40-44 +
 *                         kernels/quant/per_tensor.py:36-43, and with
 *                         scale_dt = the input dtype the legacy
 *                         kernels/fp8_bmm/fp8_warper.py:21-25 +
 *                         kernel/fp8_quant_kernel.py:56-60
 *                         and with scale_dt = OR_F64 torchao's tensorwise
 *                         scale (fp8_training/fp8_bench/modules/float8/
 *                         float8_utils.py:45-48 + float8_training_tensor.py:
 *                         153-154), which the reference layer quantizes with
 *   oracle_round_dt:      the bf16 / fp16 rounding of torch's 0-d tensor ops
 *
 * Pinning (tests/test_oracle.py): the encoders against torch's CPU cast over
 * every fp32 bit pattern with |x| <= fp8_max; scales against closed forms
 * and hand-derived special cases (zero blocks, power-of-two amax, eps);
 * block/channel structure against brute-force numpy on tiny inputs and the
 * committed golden vectors in tests/golden/.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fno-fast-math). No FMA
 * contraction and IEEE single-precision division are required for the
 * scales to be bit-exact.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

enum { OR_F32 = 0, OR_BF16 = 1, OR_F16 = 2, OR_E4M3 = 3, OR_E5M2 = 4, OR_F64 = 5 };

static inline float bits_to_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}
static inline uint32_t f32_to_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* IEEE binary16 -> binary32, exact. */
static float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0x1F) return bits_to_f32(sign | 0x7F800000u | (man << 13));
  if (exp == 0) {
    /* zero or subnormal: man * 2^-24, exact in fp32 */
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_to_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

/* binary32 -> binary16, round to nearest even (overflow to infinity). */
static uint16_t f32_to_f16_rne(float f) {
  uint32_t x = f32_to_bits(f);
  uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return sign | 0x7E00u;            /* NaN */
  if (ax >= 0x477FF000u) return sign | 0x7C00u;           /* >= 65520: tie or above rounds to inf */
  if (ax < 0x38800000u) {                                 /* below 2^-14: subnormal or zero */
    float r = rintf(bits_to_f32(ax) * 16777216.0f);       /* units of 2^-24, exact scaling */
    return sign | (uint16_t)r;                            /* r == 1024 is the smallest normal */
  }
  uint32_t r = ax + 0xFFFu + ((ax >> 13) & 1u);           /* drop 13 mantissa bits, RNE */
  r -= 112u << 23;                                        /* rebias 127 -> 15 */
  return sign | (uint16_t)(r >> 13);
}

/* Round a binary32 value to `dtype` (RNE) and back; identity for OR_F32. */
float oracle_round_dt(float f, int dtype) {
  if (dtype == OR_BF16) {
    uint32_t u = f32_to_bits(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return f;
    u = (u + 0x7FFFu + ((u >> 16) & 1u)) & 0xFFFF0000u;
    return bits_to_f32(u);
  }
  if (dtype == OR_F16) return f16_to_f32(f32_to_f16_rne(f));
  return f;
}

static inline float load_elem(const void *base, int dtype, int64_t off) {
  switch (dtype) {
    case OR_F32: return ((const float *)base)[off];
    case OR_BF16: return bits_to_f32((uint32_t)((const uint16_t *)base)[off] << 16);
    default: return f16_to_f32(((const uint16_t *)base)[off]);
  }
}

/*
 * fp32 -> e4m3fn, round to nearest even. e4m3fn: bias 7, 3 mantissa bits,
 * largest finite 448 (0x7e), no infinity, NaN 0x7f. Subnormals are m * 2^-9.
 * Magnitudes at or above 480 have no finite encoding and map to NaN (the
 * non-saturating cast); callers clamp to +-448 first.
 */
uint8_t oracle_encode_e4m3fn(float f) {
  uint32_t u = f32_to_bits(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;  /* NaN */
  if (a >= 0x43F00000u) return sign | 0x7Fu; /* |f| >= 480 */
  if (a < 0x3C800000u) {                     /* |f| < 2^-6: subnormal grid */
    /* |f| * 2^9 is exact; rintf rounds half to even in the default mode. */
    uint32_t q = (uint32_t)rintf(bits_to_f32(a) * 512.0f);
    return sign | (uint8_t)q; /* q == 8 is the smallest normal, 0x08 */
  }
  /* keep 3 of 23 mantissa bits: add half-ulp-minus-one plus the lsb (RNE) */
  uint32_t r = a + 0x7FFFFu + ((a >> 20) & 1u);
  return sign | (uint8_t)((r >> 20) - ((127u - 7u) << 3));
}

/*
 * fp32 -> e5m2, round to nearest even. e5m2: bias 15, 2 mantissa bits,
 * largest finite 57344 (0x7b), infinity 0x7c, subnormals m * 2^-16.
 */
uint8_t oracle_encode_e5m2(float f) {
  uint32_t u = f32_to_bits(f);
  uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
  uint32_t a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) return sign | 0x7Fu;  /* NaN */
  if (a >= 0x47800000u) return sign | 0x7Cu; /* |f| >= 65536 -> inf */
  if (a < 0x38800000u) {                     /* |f| < 2^-14 */
    uint32_t q = (uint32_t)rintf(bits_to_f32(a) * 65536.0f);
    return sign | (uint8_t)q;
  }
  uint32_t r = a + 0xFFFFFu + ((a >> 21) & 1u);
  return sign | (uint8_t)((r >> 21) - ((127u - 15u) << 2));
}

static inline uint8_t encode(float v, int fmt) {
  return fmt == OR_E5M2 ? oracle_encode_e5m2(v) : oracle_encode_e4m3fn(v);
}

/* clamp as tl.clamp(v, -max, max) (per_block.py:46) */
static inline float clampf(float v, float lo, float hi) {
  return v < lo ? lo : (v > hi ? hi : v);
}

void oracle_encode_array(const float *in, uint8_t *out, int64_t count, int fmt) {
  for (int64_t i = 0; i < count; ++i) out[i] = encode(in[i], fmt);
}

/*
 * Per-block quantization (kernels/quant/per_block.py:35-48). One program per
 * block_m x block_n tile of x[b]; masked elements load as 0 and cannot raise
 * the amax. Scale stored is 1 / (fp8_max / max(amax, eps)) (:42-45).
 */
int oracle_quant_block(const void *x, int xd, int64_t batch, int64_t m, int64_t n,
                       int64_t sxb, int64_t sxm, int64_t sxn, uint8_t *y,
                       int yfmt, int64_t syb, int64_t sym, int64_t syn,
                       float *scale, int64_t ssb, int64_t ssm, int64_t ssn,
                       int64_t bm, int64_t bn, float fp8_max, float eps,
                       int threads) {
  if (bm <= 0 || bn <= 0) return -1;
  int64_t mb = (m + bm - 1) / bm, nb = (n + bn - 1) / bn;
  int64_t total = batch * mb * nb;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) if (threads > 1)
#endif
  for (int64_t t = 0; t < total; ++t) {
    int64_t b = t / (mb * nb), rem = t % (mb * nb);
    int64_t pm = rem / nb, pn = rem % nb;
    int64_t r0 = pm * bm, c0 = pn * bn;
    int64_t r1 = r0 + bm < m ? r0 + bm : m, c1 = c0 + bn < n ? c0 + bn : n;
    float amax = 0.0f;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t c = c0; c < c1; ++c) {
        float a = fabsf(load_elem(x, xd, b * sxb + r * sxm + c * sxn));
        amax = fmaxf(amax, a);
      }
    float safe = fmaxf(amax, eps); /* tl.maximum(amax, EPS) */
    float qs = fp8_max / safe;
    float ds = 1.0f / qs;
    scale[b * ssb + pm * ssm + pn * ssn] = ds;
    for (int64_t r = r0; r < r1; ++r)
      for (int64_t c = c0; c < c1; ++c) {
        float v = load_elem(x, xd, b * sxb + r * sxm + c * sxn) * qs;
        y[b * syb + r * sym + c * syn] = encode(clampf(v, -fp8_max, fp8_max), yfmt);
      }
  }
  (void)threads;
  return 0;
}

/*
 * Per-channel quantization (kernels/quant/per_channel.py:136-267).
 * axis -2: one scale per row, reduce along n; axis -1: one per column.
 * Scale stored is max(amax, eps) / fp8_max (:159-161, :225-227).
 */
int oracle_quant_channel(const void *x, int xd, int64_t batch, int64_t m, int64_t n,
                         int64_t sxb, int64_t sxm, int64_t sxn, uint8_t *y,
                         int yfmt, int64_t syb, int64_t sym, int64_t syn,
                         float *scale, int64_t ssb, int64_t ssc, int axis,
                         float fp8_max, float eps, int threads) {
  if (axis != -1 && axis != -2) return -1;
  int64_t channels = axis == -2 ? m : n, red = axis == -2 ? n : m;
  int64_t total = batch * channels;
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static) if (threads > 1)
#endif
  for (int64_t t = 0; t < total; ++t) {
    int64_t b = t / channels, ch = t % channels;
    int64_t xo = b * sxb + (axis == -2 ? ch * sxm : ch * sxn);
    int64_t yo = b * syb + (axis == -2 ? ch * sym : ch * syn);
    int64_t xs = axis == -2 ? sxn : sxm, ys = axis == -2 ? syn : sym;
    float amax = 0.0f;
    for (int64_t i = 0; i < red; ++i) {
      float a = fabsf(load_elem(x, xd, xo + i * xs));
      amax = fmaxf(amax, a);
    }
    float safe = fmaxf(amax, eps);
    float qs = fp8_max / safe;
    float ds = safe / fp8_max;
    scale[b * ssb + ch * ssc] = ds;
    for (int64_t i = 0; i < red; ++i) {
      float v = load_elem(x, xd, xo + i * xs) * qs;
      y[yo + i * ys] = encode(clampf(v, -fp8_max, fp8_max), yfmt);
    }
  }
  (void)threads;
  return 0;
}

/*
 * Per-tensor quantization (impls/triton_per_tensor.py:40-44,
 * kernels/quant/per_tensor.py:36-43): amax over everything, clamp_min(eps),
 * qs = reciprocal(s) * fp8_max, dequant = reciprocal(qs).
 *
 * scale_dt is the dtype the scalar scale arithmetic is carried out in. The
 * fp8_bench path computes it in fp32 (OR_F32). The legacy
 * kernels/fp8_bmm/fp8_warper.py:21-25 does the same torch ops on 0-d tensors
 * of the input's dtype, so for a bf16 / fp16 input every step rounds to that
 * dtype: s = max(amax, dt(eps)), r = dt(1 / s), qs = dt(r * fp8_max),
 * dequant = dt(1 / qs) (each op evaluated in fp32, as torch's opmath does,
 * then rounded). The quantization multiplies x (as fp32) by that qs.
 */
int oracle_quant_tensor(const void *x, int xd, int64_t batch, int64_t m, int64_t n,
                        int64_t sxb, int64_t sxm, int64_t sxn, uint8_t *y,
                        int yfmt, int64_t syb, int64_t sym, int64_t syn,
                        float *scale, float *quant_scale, float fp8_max,
                        float eps, int scale_dt) {
  float amax = 0.0f;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t r = 0; r < m; ++r)
      for (int64_t c = 0; c < n; ++c) {
        float a = fabsf(load_elem(x, xd, b * sxb + r * sxm + c * sxn));
        amax = fmaxf(amax, a);
      }
  float qs, ds;
  if (scale_dt == OR_F64) {
    /* torchao amax_to_scale (float8_utils.py:45-48): amax.to(float64),
     * max / clamp(amax, min=EPS) in fp64, .to(float32); its scaled GEMMs
     * take scale.reciprocal() in fp32 */
    qs = (float)((double)fp8_max / fmax((double)amax, (double)eps));
    ds = 1.0f / qs;
  } else {
    float safe = oracle_round_dt(fmaxf(oracle_round_dt(amax, scale_dt), oracle_round_dt(eps, scale_dt)), scale_dt);
    /* `fp8_max / max_abs` with a Python-float numerator is evaluated by torch
     * as max_abs.reciprocal() * fp8_max (torch/_tensor.py __rdiv__): two
     * roundings, unlike the true division of the Triton kernels. */
    qs = oracle_round_dt(oracle_round_dt(1.0f / safe, scale_dt) * fp8_max, scale_dt);
    ds = oracle_round_dt(1.0f / qs, scale_dt); /* quant_scale.reciprocal() */
  }
  *scale = ds;
  if (quant_scale) *quant_scale = qs;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t r = 0; r < m; ++r)
      for (int64_t c = 0; c < n; ++c) {
        float v = load_elem(x, xd, b * sxb + r * sxm + c * sxn) * qs;
        y[b * syb + r * sym + c * syn] = encode(clampf(v, -fp8_max, fp8_max), yfmt);
      }
  return 0;
}

/* fp8 -> fp32 decode, exact (used by tests to dequantize). */
float oracle_decode_fp8(uint8_t v, int fmt) {
  uint32_t sign = (uint32_t)(v & 0x80u) << 24;
  if (fmt == OR_E5M2) {
    uint32_t e = (v >> 2) & 0x1Fu, mnt = v & 0x3u;
    if (e == 0x1F) return bits_to_f32(sign | 0x7F800000u | (mnt ? 0x400000u : 0u));
    if (e == 0) {
      float f = (float)mnt * 1.52587890625e-05f; /* 2^-16 */
      return sign ? -f : f;
    }
    return bits_to_f32(sign | ((e + 112u) << 23) | (mnt << 21));
  }
  uint32_t e = (v >> 3) & 0xFu, mnt = v & 0x7u;
  if (e == 0xF && mnt == 0x7) return bits_to_f32(sign | 0x7FC00000u);
  if (e == 0) {
    float f = (float)mnt * 0.001953125f; /* 2^-9 */
    return sign ? -f : f;
  }
  return bits_to_f32(sign | ((e + 120u) << 23) | (mnt << 20));
}

int oracle_abi_version(void) { return 1; }
