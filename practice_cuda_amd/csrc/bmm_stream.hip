// bmm_stream.hip - block-scaled FP8 BMM for one K step (K = 128) with N = 512,
// A K-major and B N-major: the MLA-style head-batched product of config 4
// (A [B, M, 128] with 1 x 128 scales, B [B, 128, 512] with 128 x 128 scales,
// bf16 C [B, M, 512]).
//
// At K = 128 the product is bound by writing C (AI ~ 110 FLOP/B against a
// ridge of ~ 625), so the kernel is organised around a steady stream of full
// C rows:
//   - one workgroup per CU (8 waves, persistent), walking a contiguous range
//     of units; a unit is 128 rows x all 512 columns of one batch, i.e. one
//     contiguous 128 KiB slab of C;
//   - B of the current batch (128 x 512 fp8 = 64 KiB) stays in LDS and is
//     reloaded only when the range crosses into the next batch;
//   - the next unit's A rows (16 KiB) and row scales are loaded straight into
//     the other LDS stage while the current unit computes and stores, so
//     after the first unit no CU waits on a load with no stores in flight;
//   - C leaves through LDS staging as whole 1 KiB rows, one row per store
//     instruction.
// Every global memory access in the loop is inline asm (asynchronous
// global -> LDS copies, and the C stores, which nothing waits for), so the
// compiler tracks none of them and the loop's vmcnt waits are
// written by hand: a unit's loads were issued before the previous unit's
// 16 stores, so vmcnt(16) (vmcnt(0) after a partial unit) means they landed
// without waiting for those stores.
//
// Math (xuOAO/practice_cuda kernels/bmm/per_block.py:99-111 with one K
// block): out = P * (sa * sb), P the fp32 MFMA product, the scale product
// formed first.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>

#include "abi_util.h"
#include "bmm_epilogue.h"
#include "bmm_fast.h"
#include "bmm_lds.h"
#include "fp8_common.h"

namespace pcamd {
namespace bmms {

using lds::v8i;
using lds::v4i;
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int NT = 512;                   // 8 waves: 2 along M x 4 along N
constexpr int WAVES = NT / 64;
constexpr int UM = 128, UN = 512, BK = 128;
constexpr int B_LDS = 0;                  // B: two 256-column halves of [128 k][256 B]
constexpr int A_LDS = UN * BK;            // 64 KiB: two stages of [128 rows][128 B]
constexpr int SA_LDS = A_LDS + 2 * UM * BK;  // two stages of 1 KiB (128 row scales used)
constexpr int SB_LDS = SA_LDS + 2 * 1024;    // 1 KiB: the batch's column-block scales
constexpr int STG_LDS = SB_LDS + 1024;       // output staging: 32 rows of C (1 KiB each)
constexpr int LDS_BYTES = STG_LDS + WAVES * 4096;
constexpr int kRounds = 4;                // staging rounds per unit: one per 16-row block of a wave's 64 rows
constexpr int kRowStoresPerRound = 4;     // whole 1 KiB rows of C stored per wave per round
constexpr int kStoresPerUnit = kRounds * kRowStoresPerRound;  // global store instructions per wave per unit
static_assert(kRounds * 16 == 64, "a round covers one 16-row block of the wave's 64 x 128 output block");
static_assert(WAVES * kRowStoresPerRound == 32, "the staging holds 32 rows of C: every wave stores its share");

// K-major A tile: chunk c (16 B) of row r at position c ^ swz(r)
PCAMD_DEV int swz(int r) { return (r ^ (r >> 4)) & 7; }

PCAMD_DEV v8i frag_k(const uint8_t* tile, int row, int g) {
  const uint4* l = reinterpret_cast<const uint4*>(tile + row * BK);
  const int s = swz(row);
  const uint4 x = l[(2 * g) ^ s];
  const uint4 y = l[(2 * g + 1) ^ s];
  v8i f;
  f[0] = x.x; f[1] = x.y; f[2] = x.z; f[3] = x.w;
  f[4] = y.x; f[5] = y.y; f[6] = y.z; f[7] = y.w;
  return f;
}

template <int FMT>
PCAMD_DEV v4f mfma(const v8i& x, const v8i& y) {
  constexpr int code = FMT == kE5M2 ? 1 : 0;
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, v4f{0.f, 0.f, 0.f, 0.f}, code, code, 0, 0, 0, 0);
}

PCAMD_DEV void barrier() { asm volatile("s_barrier" ::: "memory"); }

// 16 bytes of C: a non-temporal vector store with device scope (nt sc1).
// Measured at config 4 over five alternating runs: 48.1 us against 49.0 us
// for the compiler's non-temporal store (nt alone); stores that allocate in
// L2 (no nt, with or without a scope) took 64 us.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
PCAMD_DEV void store_c(const u32x4& v, __bf16* p) {
  asm volatile("global_store_dwordx4 %0, %1, off nt sc1" ::"v"(p), "v"(v) : "memory");
}
PCAMD_DEV void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

struct StreamArgs {
  FastArgs f;
  uint32_t sa_bytes, sb_bytes;  // buffer bounds of the scale tensors
  int32_t units_per_batch;      // ceil(M / 128)
  int32_t units;                // batch * units_per_batch
};

// A rows of one unit: 128 rows x 128 k-bytes, two instructions per wave.
// Instruction i of wave w fills rows rb = 16 w + 8 i .. rb + 7; lane l takes
// row rb + l / 8 and LDS slot l % 8, which holds global chunk (l % 8) ^ swz.
PCAMD_DEV void issue_a(v4i rs, uint32_t stage_lds, uint32_t m0, uint32_t lda, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int rb = wave * 16 + i * 8;
    const int r = rb + (lane >> 3);
    const uint32_t voff = (m0 + r) * lda + ((((lane & 7) ^ swz(r))) << 4);
    lds::lds_dma16(rs, stage_lds + rb * BK, voff);
  }
}

template <int FMT>
__global__ __launch_bounds__(NT, 1) void bmm_stream_kernel(StreamArgs s) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const FastArgs& a = s.f;
  const int t = threadIdx.x;
  const int lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int lr = lane & 15, lg = lane >> 4;
  const uint32_t base = lds::lds_addr(smem);

  // this workgroup's contiguous range of units
  const int g = gridDim.x, w = blockIdx.x;
  const int u0 = static_cast<int>((int64_t(s.units) * w) / g);
  const int u1 = static_cast<int>((int64_t(s.units) * (w + 1)) / g);
  if (u0 >= u1) return;  // uniform: the whole workgroup leaves

  const lds::MNMajorLoader<256, WAVES> load_b(a.ldb, lane, wave);
  const v4i rs_sa = lds::make_rsrc(a.sa, s.sa_bytes);
  const v4i rs_sb = lds::make_rsrc(a.sb, s.sb_bytes);
  auto issue_b = [&](int bidx) {
    const v4i rs = lds::make_rsrc(a.b + int64_t(bidx) * a.sbb, a.b_extent);
    load_b.issue(rs, base + B_LDS, 0, a.ldb, 0, wave);
    load_b.issue(rs, base + B_LDS + 128 * 256, 256, a.ldb, 0, wave);
    if (wave == 1) lds::lds_dma16(rs_sb, base + SB_LDS, uint32_t(int64_t(bidx) * a.ssbb * 4) + lane * 16);
  };
  auto issue_unit = [&](int u, int stage) {
    const int bidx = u / s.units_per_batch;
    const int m0 = (u - bidx * s.units_per_batch) * UM;
    issue_a(lds::make_rsrc(a.a + int64_t(bidx) * a.sab, a.a_extent), base + A_LDS + stage * UM * BK, m0, a.lda,
            wave, lane);
    if (wave == 0)
      lds::lds_dma16(rs_sa, base + SA_LDS + stage * 1024, uint32_t((int64_t(bidx) * a.ssab + m0) * 4) + lane * 16);
  };

  // prologue: the first batch's B and the first unit's A
  issue_b(u0 / s.units_per_batch);
  issue_unit(u0, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  barrier();

  uint8_t* stg = smem + STG_LDS;
  int st = 0;
  for (int u = u0; u < u1; ++u, st ^= 1) {
    const int bidx = u / s.units_per_batch;
    const int m0 = (u - bidx * s.units_per_batch) * UM;
    const bool has_next = u + 1 < u1;
    const bool new_batch = has_next && (u + 1) / s.units_per_batch != bidx;

    // fragments and scales of this unit
    const uint8_t* at = smem + A_LDS + st * UM * BK;
    v8i af[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) af[i] = frag_k(at, wm * 64 + i * 16 + lr, lg);
    const float* sat = reinterpret_cast<const float*>(smem + SA_LDS + st * 1024);
    float sav[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sav[i] = sat[wm * 64 + i * 16 + lr];
    const float* sbt = reinterpret_cast<const float*>(smem + SB_LDS);
    float sbv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) sbv[j] = sbt[(wn * 128 + 16 * j) >> a.qbn_shift];

    // the next unit's A and row scales into the other stage, which every
    // wave left before the barrier that ended the previous unit
    if (has_next) issue_unit(u + 1, st ^ 1);

    // the wave's eight B fragments (its 128 columns), held for the unit; each
    // epilogue round below issues the MFMAs of its own 16 rows, so the
    // matrix work is spread between the rounds' stores
    v8i bf[8];
    const uint8_t* bt = smem + B_LDS + (wn >> 1) * (128 * 256);
#pragma unroll
    for (int j = 0; j < 8; ++j) bf[j] = lds::frag_mn<256>(bt, (wn & 1) * 128 + 16 * j, lane);

    // crossing into the next batch: once every wave has read this batch's
    // B (its fragment reads complete), load the next one behind the stores
    if (new_batch) {
      wait_lds();
      barrier();
      issue_b((u + 1) / s.units_per_batch);
    }

    // Four rounds through the workgroup's 32 KiB of staging, which holds 32
    // whole rows of C (1 KiB each; 16-byte chunk c of staged row s at
    // position c ^ (s & 15)). In round i, wave (wm, wn) computes rows
    // 16 i .. 16 i + 15 of its 64 x 128 block (8 MFMAs) and stages them as
    // staged rows 16 wm + lr; after a barrier, wave w stores staged rows
    // 4 w .. 4 w + 3, one whole 1 KiB row of C per instruction. Whole rows
    // measured 3 us faster at config 4 than four 256-byte row pieces per
    // instruction, and the MFMAs spread over the rounds 0.6 us faster than
    // all 32 issued before the first.
    __bf16* cb = reinterpret_cast<__bf16*>(a.c) + int64_t(bidx) * a.scb;
#pragma unroll
    for (int i = 0; i < kRounds; ++i) {
      v4f acc[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = mfma<FMT>(bf[j], af[i]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float f = sav[i] * sbv[j];  // (sa * sb), then * P
        const int chunk = wn * 16 + 2 * j + (lg >> 1);
        uint2* dst = reinterpret_cast<uint2*>(stg + (wm * 16 + lr) * 1024 + ((chunk ^ lr) << 4) + ((lg & 1) << 3));
        *dst = make_uint2(pack_bf16_pair(acc[j][0] * f, acc[j][1] * f), pack_bf16_pair(acc[j][2] * f, acc[j][3] * f));
      }
      wait_lds();
      barrier();
#pragma unroll
      for (int it = 0; it < kRowStoresPerRound; ++it) {
        const int srow = kRowStoresPerRound * wave + it;
        const u32x4 v = *reinterpret_cast<const u32x4*>(stg + srow * 1024 + (lane << 4));
        const int chunk = lane ^ (srow & 15);
        const int mm = m0 + (srow >> 4) * 64 + 16 * i + (srow & 15);
        if (mm < a.m) store_c(v, cb + int64_t(mm) * a.scm + 8 * chunk);
      }
      // the next round overwrites the staging: every wave's reads first (the
      // last round's reads are covered by the barrier that ends the unit)
      if (i < kRounds - 1) {
        wait_lds();
        barrier();
      }
    }

    if (has_next) {
      // this wave's loads for the next unit were issued before its
      // kStoresPerUnit stores (before fewer of them if rows past M were
      // skipped: then wait for all); the immediate is that same constant
      if (m0 + UM <= a.m) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kStoresPerUnit) : "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      wait_lds();
      barrier();
    }
  }
}

template <int FMT>
int launch(const StreamArgs& s, hipStream_t st) {
  auto kern = bmm_stream_kernel<FMT>;
  static std::atomic<uint64_t> configured{0};  // devices whose LDS limit is set
  const int rc = ensure_dynamic_lds(reinterpret_cast<const void*>(kern), LDS_BYTES, st, configured);
  if (rc != 0) return rc;
  const int cus = device_cu_count(st);
  const int grid = std::max(1, std::min(s.units, cus > 0 ? cus : 256));
  kern<<<grid, NT, LDS_BYTES, st>>>(s);
  return check_launch("bmm_stream_kernel");
}

}  // namespace bmms

bool bmm_stream_ok(const FastArgs& a, bool a_k, bool b_k, int mode, int64_t batch, int64_t qbm, int64_t qbn,
                   int64_t ssa1, int64_t ssb2) {
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool plain = a.bias == nullptr && a.act == PCAMD_ACT_NONE && a.c_dtype == kBF16;
  return a.k == bmms::BK && a.n == bmms::UN && a_k && !b_k && mode == 0 && qbm == 1 && qbn >= 16 && qbn <= 512 &&
         ssa1 == 1 && ssb2 == 1 && al16(a.sa) && al16(a.sb) && (batch == 1 || (a.ssab % 4 == 0 && a.ssbb % 4 == 0)) &&
         plain && (a.scm & 7) == 0 && (a.scb & 7) == 0 && al16(a.c) && batch * ((a.m + 127) / 128) < INT32_MAX &&
         (batch - 1) * a.ssab + a.m < (int64_t{1} << 29) && (batch - 1) * a.ssbb + 512 < (int64_t{1} << 29);
}

int bmm_stream_launch(const FastArgs& a, int ab_dtype, int64_t batch, hipStream_t st) {
  bmms::StreamArgs s{};
  s.f = a;
  s.units_per_batch = (a.m + bmms::UM - 1) / bmms::UM;
  s.units = static_cast<int32_t>(batch * s.units_per_batch);
  // scale tensors: [B, M, 1] rows and [B, 1, 512 / qbn] column blocks, read
  // 1 KiB at a time from 16-byte aligned offsets (the range check returns
  // zeros past the end)
  s.sa_bytes = static_cast<uint32_t>(((batch - 1) * a.ssab + a.m) * 4);
  s.sb_bytes = static_cast<uint32_t>(((batch - 1) * a.ssbb + (bmms::UN >> a.qbn_shift)) * 4);
  if (ab_dtype == kE5M2) return bmms::launch<kE5M2>(s, st);
  return bmms::launch<kE4M3>(s, st);
}

}  // namespace pcamd
