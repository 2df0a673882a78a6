// bmm_fused_stream.hip - block-scaled FP8 GEMM with the activation's 1 x 128
// quantization fused, for narrow products (N <= 256): C = quant(A) B.
//
// A narrow product is bound by reading the 16-bit A (2 bytes per element,
// against N / 64 FLOP per byte of MFMA work), so this kernel streams A once:
// each wave owns 16 rows and every column. A lane loads its own 64 bytes of
// a K step (row lane & 15, k [32 g, 32 g + 32), g = lane / 16: exactly the
// MFMA A fragment's slice) straight into a ring of two pipeline steps of
// registers (a step is one or, where K allows, two K blocks of 128), the
// four lanes of a row meet in a lane-shuffle max (the row's 1 x 128 group),
// and the lane quantizes its 32 values into its own fragment: no LDS round
// trip for A. B ([128 k, N] per K block, shared by the workgroup's 8 waves)
// is copied global -> LDS one step ahead, double buffered. Block scales fold as in the wide kernel: acc += P * (sa * sb)
// per 128-wide K block (xuOAO/practice_cuda kernels/bmm/per_block.py:99-111),
// with two MFMA partials in flight (the one folded was written two MFMAs
// earlier). Bytes and scales of the quantized A, and C, are those of
// pcamd_quant_block(1 x 128) followed by pcamd_bmm_scaled.
//
// Envelope (pcamd_bmm_quant_a checks it; other calls take the 128 x 256
// fused kernel of bmm_fast.hip): N <= 256 and a multiple of 16, K a multiple
// of 256, B's column blocks qbn >= 128, C contiguous along N; any bias,
// activation and output type.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdlib>

#include "abi_util.h"
#include "bmm_fast.h"
#include "bmm_wide.h"
#include "fp8_common.h"

namespace pcamd {
namespace bmmq {

// PCAMD_BMM_FUSED_STEP2=0: one K block per pipeline step at every K
static bool step_pairs_disabled() {
  static const bool v = [] {
    const char* e = getenv("PCAMD_BMM_FUSED_STEP2");
    return e && e[0] == '0';
  }();
  return v;
}

using lds::v4i;
using lds::v8i;
using bmmw::v4f;

constexpr int NT = 512, WAVES = NT / 64, ROWS = WAVES * 16;  // 128 rows per workgroup
constexpr int BK = 128;   // one MFMA / one 1 x 128 group along K
constexpr int RING = 2;   // pipeline steps of A in flight per lane

// The descriptor lives in SGPRs: base and size go through readfirstlane.
PCAMD_DEV __amdgpu_buffer_rsrc_t make_buf(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(p >> 32));
  void* ub = reinterpret_cast<void*>((static_cast<uint64_t>(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(ub, 0, static_cast<int>(__builtin_amdgcn_readfirstlane(bytes)),
                                           lds::kRsrcWord3);
}

// A ring slot: a lane's 64 bytes (32 16-bit values) of each of G K blocks
template <int G>
struct ASlot {
  v4i c[4 * G];
};

// G: K blocks per pipeline step (one A refill, one B copy, one wait and
// barrier per step). Two blocks double the bytes in flight per CU and the
// time each refill has to land.
// WQ: qa_out / sa_out are written (a compile-time choice, so that every step
// issues the same vector-memory instructions: the hand-counted waits below
// rely on it)
// CLAMP: the clamp to +-fp8_max before the cast (left out when it cannot
// change a byte: fp8_max the format's largest value and every quant scale
// finite, as in the quantizers)
template <int DT, int FMT, bool B_K, int JN, int G, bool WQ, bool CLAMP>
__global__ __launch_bounds__(NT, 1) void bmm_fused_stream_kernel(FastArgs a) {
  static_assert(JN == 4 || JN == 8 || JN == 12 || JN == 16, "N up to 64, 128, 192 or 256");
  static_assert(G == 1 || (G == 2 && JN <= 12), "two K blocks per step: N up to 192");
  constexpr int BCOLS = 16 * JN;                   // B columns per stage (K-major B: its rows)
  constexpr int B_BYTES = B_K ? BCOLS * BK : 256 * BK;  // one K block of B in LDS
  constexpr int SB_LOADS = JN > 8 ? 2 : 1;        // B block scales per K block (qbn >= 128)
  constexpr int Q_STORES = WQ ? 5 : 0;             // per K block: 4 x 8 bytes of qa_out + the scale
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int lr = lane & 15, lg = lane >> 4;
  const int bidx = blockIdx.y;
  const int m0 = blockIdx.x * ROWS;
  const int row = m0 + wave * 16 + lr;
  const int steps = a.k / (G * BK);  // even, >= RING

  // A: buffer loads over the batch's slice (rows past M read zero); the row
  // part of the offset per lane, the step in the SGPR offset
  const __amdgpu_buffer_rsrc_t rsa = make_buf(a.a + bidx * a.sab, a.a_extent);
  const uint32_t a_voff = static_cast<uint32_t>(row) * a.lda + 64u * lg;
  auto load_a = [&](ASlot<G>& s, int st) {
    const int k0 = __builtin_amdgcn_readfirstlane(st * G * BK * 2);
#pragma unroll
    for (int c = 0; c < 4 * G; ++c)
      s.c[c] = __builtin_amdgcn_raw_buffer_load_b128(rsa, a_voff + 16 * (c & 3) + 2 * BK * (c >> 2), k0, 0);
  };

  // B: global -> LDS one step ahead (inline asm, ordered by hand); K block
  // kb lands in LDS slot kb % (2 G)
  const v4i rsb = lds::make_rsrc(a.b + bidx * a.sbb, a.b_extent);
  using LB = typename std::conditional<B_K, bmmw::KMajorLoader<BCOLS>, lds::MNMajorLoader<256, WAVES>>::type;
  const LB load_b = [&] {
    if constexpr (B_K) return bmmw::KMajorLoader<BCOLS>(a.ldb, lane, wave, 0);
    else return lds::MNMajorLoader<256, WAVES>(a.ldb, lane, wave);
  }();
  auto issue_b = [&](int kb) {
    const uint32_t k0 = __builtin_amdgcn_readfirstlane(kb * BK);
    const uint32_t base = lds::lds_addr(smem + (kb % (2 * G)) * B_BYTES);
    if constexpr (B_K) load_b.issue(rsb, base, k0, wave);
    else load_b.issue(rsb, base, 0, a.ldb, k0, wave);
  };
  auto bfrag = [&](int kb, int j) -> v8i {
    const uint8_t* st = smem + (kb % (2 * G)) * B_BYTES;
    if constexpr (B_K) return bmmw::frag_k(st, 16 * j + lr, lg);
    else return lds::frag_mn<256>(st, 16 * j, lane);
  };
  // B block scales of K block kb: columns 0-127 and 128-255 (qbn >= 128)
  const float* sb_b = a.sb + bidx * a.ssbb;
  auto load_sb = [&](int kb, float (&v)[2]) {
    v[0] = sb_b[int64_t(kb) * a.ssb1];
    v[1] = SB_LOADS > 1 ? sb_b[int64_t(kb) * a.ssb1 + int64_t(128 >> a.qbn_shift) * a.ssb2] : v[0];
  };

  // qa_out / sa_out through range-checked buffer stores: rows past M (and
  // the scale of lanes other than the row's first) fall outside the range
  // and are dropped, so every step issues the same instructions
  const __amdgpu_buffer_rsrc_t rsq =
      make_buf(WQ ? a.qa_out + bidx * a.sqab : nullptr, WQ ? static_cast<uint32_t>((a.m - 1) * a.sqam + a.k) : 0u);
  const __amdgpu_buffer_rsrc_t rss = make_buf(
      WQ ? a.sa_out + bidx * a.soab : nullptr,
      WQ ? static_cast<uint32_t>(((a.m - 1) * a.soam + (a.k / BK - 1) * a.soak + 1) * 4) : 0u);
  const uint32_t q_voff = row < a.m ? static_cast<uint32_t>(row * a.sqam + 32 * lg) : 0x80000000u;
  const uint32_t s_voff = row < a.m && lg == 0 ? static_cast<uint32_t>(row * a.soam * 4) : 0x80000000u;

  // quantize this lane's slice of K block kb (chunks c0 .. c0 + 3 of the
  // slot) into its MFMA A fragment; the row's 1 x 128 group is its four
  // lanes (16 apart): pcamd_quant_block's math
  auto quantize = [&](const ASlot<G>& s, int c0, int kb, v8i& f) -> float {
    float amax = 0.0f;
    if constexpr (DT == kBF16) {
      // |x| of all 32 values as one unsigned 16-bit max over the raw pairs,
      // then the larger half (non-negative bf16 order like their bits)
      uint32_t m = bf16_abs2(static_cast<uint32_t>(s.c[c0][0]));
#pragma unroll
      for (int w = 1; w < 16; ++w) m = pk_max_u16(m, bf16_abs2(static_cast<uint32_t>(s.c[c0 + w / 4][w % 4])));
      amax = bf16_bits(max_halves(m));
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        Chunk<DT> ch;
        ch.r[0] = make_uint4(s.c[c0 + c][0], s.c[c0 + c][1], s.c[c0 + c][2], s.c[c0 + c][3]);
        amax = fmaxf(amax, chunk_amax<DT>(ch));
      }
    }
    // non-negative floats order like their bits
    uint32_t u = __float_as_uint(amax);
    u = max(u, static_cast<uint32_t>(__builtin_amdgcn_ds_swizzle(static_cast<int>(u), 0x401F)));
    u = max(u, static_cast<uint32_t>(__shfl_xor(static_cast<int>(u), 32, 64)));
    const Scales sc = block_scales(__uint_as_float(u), a.fp8_max, a.eps);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      Chunk<DT> ch;
      ch.r[0] = make_uint4(s.c[c0 + c][0], s.c[c0 + c][1], s.c[c0 + c][2], s.c[c0 + c][3]);
      const uint2 q = quant_chunk<DT, FMT, CLAMP>(ch, sc.qs, a.fp8_max);
      f[2 * c] = static_cast<int>(q.x);
      f[2 * c + 1] = static_cast<int>(q.y);
    }
    if constexpr (WQ) {
      const int kq = __builtin_amdgcn_readfirstlane(kb * BK);
      const int ks4 = __builtin_amdgcn_readfirstlane(static_cast<int>(kb * a.soak * 4));
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        typedef int v2i_t __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64(v2i_t{f[2 * c], f[2 * c + 1]}, rsq, q_voff + 8 * c, kq, 0);
      }
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_int(sc.ds), rss, s_voff, ks4, 0);
    }
    // a VALU write of an MFMA source operand needs wait states the compiler
    // cannot see (the MFMA is inline asm)
    asm volatile("s_nop 4" : "+v"(f));
    return sc.ds;
  };

  v4f acc[JN];
#pragma unroll
  for (int j = 0; j < JN; ++j) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};
  // MFMA partials in flight: MFMA t writes slot t & 1, and MFMA t + 2 folds
  // it (two MFMAs apart: past the XDL -> VALU wait states); the sequence
  // runs on across K blocks and steps
  v4f p[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
  float pf[2] = {0.f, 0.f};  // their factors
  float sbv[G][2];

  // One step (K blocks G st .. G st + G - 1) on ring slot S. RELOAD: refill
  // the slot for step st + RING; NEXT: a step follows (its B and scales are
  // fetched here). Vector-memory issue order per step (the waits count on
  // it; the counter retires in order): next step's scales, next step's B
  // (asm DMA), this step's qa_out stores, the ring refill.
  ASlot<G> ring[RING];
  auto step = [&](int st, auto slot_c, auto reload_c, auto next_c) {
    constexpr int S = decltype(slot_c)::value;
    constexpr bool RELOAD = decltype(reload_c)::value;
    constexpr bool NEXT = decltype(next_c)::value;
    float sb_next[G][2];
    if constexpr (NEXT) {
#pragma unroll
      for (int g = 0; g < G; ++g) load_sb((st + 1) * G + g, sb_next[g]);
#pragma unroll
      for (int g = 0; g < G; ++g) issue_b((st + 1) * G + g);
    }
    v8i af[G];
    float ds[G];
#pragma unroll
    for (int g = 0; g < G; ++g) ds[g] = quantize(ring[S], 4 * g, st * G + g, af[g]);
    asm volatile("" ::: "memory");  // the stores above stay ahead of the refill
    if constexpr (RELOAD) load_a(ring[S], st + RING);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int kb = st * G + g;
      const float f0 = ds[g] * sbv[g][0], f1 = ds[g] * sbv[g][1];
      v8i b_cur = bfrag(kb, 0);
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const v8i b_next = j + 1 < JN ? bfrag(kb, j + 1) : b_cur;
        const int jo = (j + JN - 2) % JN;  // sub-tile of the partial folded now
        float a4[4] = {acc[jo][0], acc[jo][1], acc[jo][2], acc[jo][3]};
        v4f pn;
        const float fo = pf[j & 1];
        bmmw::mfma_fold<FMT, FMT>(b_cur, af[g], pn, p[j & 1], a4[0], a4[1], a4[2], a4[3], fo, fo, fo, fo);
        acc[jo] = v4f{a4[0], a4[1], a4[2], a4[3]};
        p[j & 1] = pn;
        pf[j & 1] = 16 * j < 128 ? f0 : f1;
        b_cur = b_next;
        // keep the next fragments' LDS reads behind this MFMA: left free, the
        // scheduler hoists all of a step's fragment reads and runs out of VGPRs
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if constexpr (NEXT) {
      // step st + 1's scales and B have landed once at most this step's
      // stores and refill are outstanding
      constexpr int AFTER = G * (Q_STORES + (RELOAD ? 4 : 0));
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(AFTER) : "memory");
      __syncthreads();
#pragma unroll
      for (int g = 0; g < G; ++g) {
        sbv[g][0] = sb_next[g][0];
        sbv[g][1] = sb_next[g][1];
      }
    }
  };

  // prologue: step 0's scales and B, then the ring
#pragma unroll
  for (int g = 0; g < G; ++g) load_sb(g, sbv[g]);
#pragma unroll
  for (int g = 0; g < G; ++g) issue_b(g);
#pragma unroll
  for (int r = 0; r < RING; ++r) load_a(ring[r], r);
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * G * RING) : "memory");
  __syncthreads();

  using T = std::true_type;
  using F = std::false_type;
  using IC0 = std::integral_constant<int, 0>;
  using IC1 = std::integral_constant<int, 1>;
  // steps [0, steps - RING) refill their slot, the last RING do not (steps
  // is even: one code path for the tail)
  int st = 0;
  for (; st + RING < steps; st += 2) {
    step(st, IC0{}, T{}, T{});
    step(st + 1, IC1{}, T{}, T{});
  }
  step(st, IC0{}, F{}, T{});
  step(st + 1, IC1{}, F{}, F{});
  // the two partials still pending (sub-tiles JN - 2 and JN - 1), the last
  // written by the final MFMA: wait out the XDL -> VALU latency first
  asm volatile("s_nop 15\n\ts_nop 15" : "+v"(p[0]), "+v"(p[1]));
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int j = JN - 2 + q;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[j][r] += p[j & 1][r] * pf[j & 1];
  }

  // epilogue: row `row`, columns 16 j + 4 lg .. + 3 of each sub-tile, in
  // the reference's order: scaled product, + bias, activation, one rounding
  // to C's type (kernels/bmm/per_block.py:113-137). A 16-bit C (and bias,
  // if any) with 8-byte aligned rows takes 8-byte loads and stores; other
  // types and strides go through the general epilogue.
  if (row < a.m) {
    const bool c16 = (a.c_dtype == kBF16 || a.c_dtype == kF16) && a.scm % 4 == 0 && a.scb % 4 == 0 &&
                     (reinterpret_cast<uintptr_t>(a.c) & 7) == 0;
    const bool b16 = a.bias == nullptr || ((a.bias_dtype == kBF16 || a.bias_dtype == kF16) && a.sbiasn == 1 &&
                                           a.sbiasm % 4 == 0 && a.sbiasb % 4 == 0 &&
                                           (reinterpret_cast<uintptr_t>(a.bias) & 7) == 0);
    if (c16 && b16) {
      uint16_t* crow = reinterpret_cast<uint16_t*>(a.c) + bidx * a.scb + int64_t(row) * a.scm;
      const uint16_t* brow =
          a.bias ? static_cast<const uint16_t*>(a.bias) + bidx * a.sbiasb + int64_t(row) * a.sbiasm : nullptr;
      const bool f16 = a.c_dtype == kF16, bias_bf16 = a.bias_dtype == kBF16, gelu = a.act == PCAMD_ACT_GELU;
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int col = 16 * j + 4 * lg;
        if (col < a.n) {
          float v[4] = {acc[j][0], acc[j][1], acc[j][2], acc[j][3]};
          if (brow) {
            const uint2 h = *reinterpret_cast<const uint2*>(brow + col);
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
          *reinterpret_cast<uint2*>(crow + col) = make_uint2(pack16_pair<OUT16_RUNTIME>(v[0], v[1], f16),
                                                             pack16_pair<OUT16_RUNTIME>(v[2], v[3], f16));
        }
      }
    } else {
      const int64_t c_row = bidx * a.scb + int64_t(row) * a.scm;
      const int64_t bias_row = bidx * a.sbiasb + int64_t(row) * a.sbiasm;
#pragma unroll
      for (int j = 0; j < JN; ++j) {
        const int col = 16 * j + 4 * lg;
        if (col < a.n)
          bmmw::epilogue_general(a.c, c_row, a.c_dtype, a.bias, bias_row, a.sbiasn, a.bias_dtype, a.act, col,
                                 min(4, a.n - col), acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
      }
    }
  }
}

template <int DT, int FMT, bool B_K, int JN, int G, bool WQ, bool CLAMP>
int launch(const FastArgs& a, int64_t batch, hipStream_t st) {
  constexpr int lds_bytes = 2 * G * (B_K ? 16 * JN * BK : 256 * BK);
  auto kern = bmm_fused_stream_kernel<DT, FMT, B_K, JN, G, WQ, CLAMP>;
  static std::atomic<uint64_t> configured{0};  // devices whose LDS limit is set
  const int rc = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), lds_bytes, st, configured);
  if (rc != 0) return rc;
  const dim3 grid(static_cast<uint32_t>((a.m + ROWS - 1) / ROWS), static_cast<uint32_t>(batch));
  kern<<<grid, NT, lds_bytes, st>>>(a);
  return check_launch("bmm_fused_stream_kernel");
}

// two K blocks per step for N <= 128 where K allows (an even number of
// 256-wide steps): with 256 columns the second block's registers do not fit
// (the kernel would spill, and scratch accesses would upset the counted
// waits); the clamped variant (a reduced fp8_max or a tiny eps) keeps one
template <int DT, int FMT, bool B_K, int JN>
int launch_wq(const FastArgs& a, int64_t batch, hipStream_t st) {
  const bool clamp = !(a.fp8_max == fmt_max<FMT>() && a.eps > 0.0f && std::isfinite(a.fp8_max / a.eps));
  if (clamp)
    return a.qa_out ? launch<DT, FMT, B_K, JN, 1, true, true>(a, batch, st)
                    : launch<DT, FMT, B_K, JN, 1, false, true>(a, batch, st);
  if constexpr (JN <= 12) {
    if (a.k % (4 * BK) == 0 && !step_pairs_disabled())
      return a.qa_out ? launch<DT, FMT, B_K, JN, 2, true, false>(a, batch, st)
                      : launch<DT, FMT, B_K, JN, 2, false, false>(a, batch, st);
  }
  return a.qa_out ? launch<DT, FMT, B_K, JN, 1, true, false>(a, batch, st)
                  : launch<DT, FMT, B_K, JN, 1, false, false>(a, batch, st);
}

template <int DT, int FMT>
int launch_dt(const FastArgs& a, bool b_k, int64_t batch, hipStream_t st) {
  // 16-column sub-tiles per wave: the fewest of 4, 8, 12, 16 that cover N
  if (a.n <= 64) return b_k ? launch_wq<DT, FMT, true, 4>(a, batch, st) : launch_wq<DT, FMT, false, 4>(a, batch, st);
  if (a.n <= 128) return b_k ? launch_wq<DT, FMT, true, 8>(a, batch, st) : launch_wq<DT, FMT, false, 8>(a, batch, st);
  if (a.n <= 192) return b_k ? launch_wq<DT, FMT, true, 12>(a, batch, st) : launch_wq<DT, FMT, false, 12>(a, batch, st);
  return b_k ? launch_wq<DT, FMT, true, 16>(a, batch, st) : launch_wq<DT, FMT, false, 16>(a, batch, st);
}

}  // namespace bmmq

bool bmm_fused_stream_ok(const FastArgs& a, int64_t batch, int64_t qbn) {
  return a.n > 0 && a.n <= 256 && a.n % 16 == 0 && a.k >= 256 && a.k % 256 == 0 && qbn >= 128 && a.scn == 1 &&
         batch <= 65535 && a.m <= INT32_MAX - bmmq::ROWS &&
         (!a.qa_out || (a.sqam % 8 == 0 && a.sqab % 8 == 0 && (reinterpret_cast<uintptr_t>(a.qa_out) & 7) == 0 &&
                        a.m * a.sqam + a.k < (int64_t{1} << 31) &&
                        ((a.m - 1) * a.soam + (a.k / 128 - 1) * a.soak + 1) * 4 < (int64_t{1} << 31)));
}

int bmm_fused_stream_launch(const FastArgs& a, int a_dtype, int fmt, bool b_k, int64_t batch, hipStream_t st) {
  if (fmt == kE5M2) {
    if (a_dtype == kF16) return bmmq::launch_dt<kF16, kE5M2>(a, b_k, batch, st);
    return bmmq::launch_dt<kBF16, kE5M2>(a, b_k, batch, st);
  }
  if (a_dtype == kF16) return bmmq::launch_dt<kF16, kE4M3>(a, b_k, batch, st);
  return bmmq::launch_dt<kBF16, kE4M3>(a, b_k, batch, st);
}

}  // namespace pcamd
