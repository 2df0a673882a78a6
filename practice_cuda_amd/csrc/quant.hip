// quant.hip - gfx950 FP8 quantizers behind the C ABI (include/pcamd_fp8.h).
//
// Kernels (all HBM-bound; each element is read once, except on the per-tensor
// and whole-column paths, whose amax pass reads it first). The streaming
// kernels are non-persistent: one wave (or workgroup) per unit, all of its
// loads issued up front. Measured on MI355X this streams faster than
// persistent grids that prefetch the next unit in registers (the hardware
// keeps more requests in flight across many short-lived waves).
//   quant_groups_kernel row-contiguous 1 x G groups: a wave owns CPL * 64
//                       consecutive 8-element chunks of one row (one 128-bit
//                       load each for bf16/fp16); groups of G/8 lanes reduce
//                       their amax with DPP.
//   quant_waverow_kernel   per-channel along rows (channel_axis = -2), rows
//                       of up to 2048 elements: one wave per row.
//   quant_rowblock_kernel  per-channel along rows, 2048 to 16384 elements: one
//                       workgroup per row sized to two (rows up to 4096
//                       elements) or four chunks per lane, DPP + one LDS max.
//   quant_tile_kernel   one workgroup per block_m x block_n block held in
//                       registers (e.g. 128 x 128 = 8 chunks per thread);
//                       wave DPP max, then an LDS max across the 4 waves.
//   quant_colgroup_kernel  row-contiguous input with column groups
//                       (block_n = 1, 16 <= block_m <= 256): one 128-column
//                       strip of one row group per workgroup, held in registers.
//   quant_dual_kernel   1 x 128 and 128 x 1 groups of one tensor from a
//                       single read: one 128 x 128 block per workgroup,
//                       row maxima by DPP, column maxima as above.
//   colchan_*_kernel    whole columns of tall tensors (channel_axis = -1):
//                       column maxima of 128-row slabs by atomic max into
//                       the scale slots (temporal loads, so the next pass
//                       finds part of the tensor in cache), then a quantize
//                       pass per slab.
//   quant_cols_kernel   whole columns of up to 256 rows (channel_axis = -1,
//                       two passes over the strip), and column groups on grids
//                       too large for the column-group kernel's 3-D grid.
//   quant_*_generic     any strides / block shape; one workgroup per block or
//                       channel, two passes (second read served by L2).
//   per-tensor          amax kernel (workgroup max + one atomic max on the
//                       fp32 bit pattern), quantize kernel, finalize kernel;
//                       contiguous tensors as one run of 16-byte chunks.
//
// Reference semantics (xuOAO/practice_cuda):
//   kernels/quant/per_block.py:35-48, kernels/quant/per_channel.py:136-267,
//   impls/triton_per_tensor.py:40-44 + kernels/quant/per_tensor.py:36-43.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdlib>

#include "abi_util.h"
#include "fp8_common.h"

namespace pcamd {

constexpr int kThreads = 256;
constexpr int kMaxSlots = 16;  // chunk slots held in registers per lane

// ===========================================================================
// row-contiguous kernels: one wave or one workgroup per unit
// ===========================================================================
// Field order: everything the flat group kernel reads sits in the first 48
// bytes, one 64-byte line of the kernel-argument segment. Its waves test
// `units` before loading anything else, so with the fields spread over two
// lines the first wave on a CU waited for two scalar-cache misses in a row:
// config 1 15.90-15.97 us against 15.56-15.65 us packed (16 rotating buffer
// sets, same kernel code).
struct RowArgs {
  const char* x;
  uint8_t* y;
  float* scale;
  int64_t total;    // chunks of the whole tensor (flat group kernel)
  uint32_t units;   // rows * segs
  int32_t chunks;   // 8-element chunks per row
  float fp8_max, eps;
  uint32_t m;       // rows per batch
  uint32_t segs;    // segments per row (group kernel)
  int32_t cpl;      // chunk slots per lane (wave-per-row kernel)
  int64_t sxb, sxm; // input strides (elements)
  int64_t syb, sym; // output strides (bytes == elements)
  int64_t ssb, ssm, ssn;  // scale strides (elements)
};
static_assert(offsetof(RowArgs, eps) + sizeof(float) <= 64, "flat group kernel fields in one 64-byte line");

typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int DT, bool NTS>
PCAMD_DEV void store8(uint8_t* p, uint2 v) {
  if constexpr (NTS) {
    u32x2 w = {v.x, v.y};
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(p));
  } else {
    *reinterpret_cast<uint2*>(p) = v;
  }
}

// 1 x (8 * LPG) groups along a row. A unit is CPL * 64 consecutive chunks of
// one row; each wave quantizes one unit (kGroupThreads / 64 units per
// workgroup). FLAT: input, output and scales are contiguous and the row
// length is a multiple of the group, so the tensor is one run of chunks
// (units may span rows, groups never do) and no row index is needed.
// 256-thread workgroups: config 1 ([4096, 7168] bf16, 16 rotating buffer
// sets) 16.04-16.14 -> 15.57-15.67 us against 128 threads; 64 and 512
// threads sat in between.
constexpr int kGroupThreads = 256;
// the per-tensor quantize pass keeps its measured 128-thread workgroups
constexpr int kTensorFlatThreads = 128;

template <int DT, int FMT, int LPG, int CPL, bool NTS, bool FLAT, bool CLAMP>
__global__ __launch_bounds__(kGroupThreads) void quant_groups_kernel(RowArgs a) {
  constexpr int EB = elem_bytes<DT>();
  const int lane = threadIdx.x & 63;
  const uint32_t u = blockIdx.x * (kGroupThreads / 64) + (threadIdx.x >> 6);
  if (u >= a.units) return;  // whole waves exit together
  Chunk<DT> cur[CPL];
  if constexpr (FLAT) {
    const int64_t ch0 = int64_t(u) * (CPL * 64) + lane;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int64_t ch = ch0 + c * 64;
      if (ch < a.total) load_chunk<DT>(cur[c], a.x + ch * 8 * EB);
      else zero_chunk<DT>(cur[c]);
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int64_t ch = ch0 + c * 64;
      const float amax = group_max<LPG>(chunk_amax<DT>(cur[c]));
      const Scales s = block_scales(amax, a.fp8_max, a.eps);
      if (ch < a.total) {
        if ((lane & (LPG - 1)) == 0) a.scale[ch / LPG] = s.ds;
        store8<DT, NTS>(a.y + ch * 8, quant_chunk<DT, FMT, CLAMP>(cur[c], s.qs, a.fp8_max));
      }
    }
    return;
  }
  const uint32_t row = u / a.segs;
  const uint32_t seg = u - row * a.segs;
  const uint32_t b = row / a.m, mi = row - b * a.m;
  const int chunk0 = static_cast<int>(seg) * CPL * 64 + lane;
  const char* xrow = a.x + (int64_t(b) * a.sxb + int64_t(mi) * a.sxm) * EB;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = chunk0 + c * 64;
    if (ch < a.chunks) load_chunk<DT>(cur[c], xrow + int64_t(ch) * 8 * EB);
    else zero_chunk<DT>(cur[c]);
  }
  uint8_t* yrow = a.y + int64_t(b) * a.syb + int64_t(mi) * a.sym;
  float* srow = a.scale + int64_t(b) * a.ssb + int64_t(mi) * a.ssm;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int ch = chunk0 + c * 64;
    const float amax = group_max<LPG>(chunk_amax<DT>(cur[c]));
    const Scales s = block_scales(amax, a.fp8_max, a.eps);
    if (ch < a.chunks) {
      if ((lane & (LPG - 1)) == 0) srow[int64_t(ch / LPG) * a.ssn] = s.ds;
      store8<DT, NTS>(yrow + int64_t(ch) * 8, quant_chunk<DT, FMT, CLAMP>(cur[c], s.qs, a.fp8_max));
    }
  }
}

// Per-channel along the row, one wave per row: the row (up to 64 * MAXC
// chunks) is held in registers and read from HBM once.
template <int DT, int FMT, int MAXC, bool NTS>
__global__ __launch_bounds__(kThreads) void quant_waverow_kernel(RowArgs a) {
  constexpr int EB = elem_bytes<DT>();
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (row >= a.units) return;  // whole waves exit together
  const uint32_t b = row / a.m, mi = row - b * a.m;
  const char* xrow = a.x + (int64_t(b) * a.sxb + int64_t(mi) * a.sxm) * EB;
  Chunk<DT> raw[MAXC];
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int ch = lane + c * 64;
    if (c < a.cpl && ch < a.chunks) load_chunk<DT>(raw[c], xrow + int64_t(ch) * 8 * EB);
    else zero_chunk<DT>(raw[c]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) amax = fmaxf(amax, chunk_amax<DT>(raw[c]));
  amax = group_max<64>(amax);
  const Scales s = channel_scales(amax, a.fp8_max, a.eps);
  if (lane == 0) a.scale[int64_t(b) * a.ssb + int64_t(mi) * a.ssm] = s.ds;
  uint8_t* yrow = a.y + int64_t(b) * a.syb + int64_t(mi) * a.sym;
#pragma unroll
  for (int c = 0; c < MAXC; ++c) {
    const int ch = lane + c * 64;
    if (c < a.cpl && ch < a.chunks)
      store8<DT, NTS>(yrow + int64_t(ch) * 8, quant_chunk<DT, FMT>(raw[c], s.qs, a.fp8_max));
  }
}

// Per-channel along the row: one workgroup of nt threads per row, thread t
// owning chunks t, t + nt, ... (CPT of them, nt * CPT >= chunks). Wave DPP
// max, then one LDS exchange across the waves.
// GRID2: grid (rows, batch), so the row and batch come from the workgroup
// index with no division ahead of the loads; otherwise a 1-D grid of
// batch * rows.
template <int DT, int FMT, int CPT, bool NTS, bool GRID2, bool CLAMP>
__global__ __launch_bounds__(1024) void quant_rowblock_kernel(RowArgs a) {
  constexpr int EB = elem_bytes<DT>();
  __shared__ float red[1024 / 64];
  const int t = threadIdx.x, nt = blockDim.x;  // nt: a multiple of 64, CPT * nt >= chunks
  uint32_t b, mi;
  if constexpr (GRID2) {
    b = blockIdx.y;
    mi = blockIdx.x;
  } else {
    b = blockIdx.x / a.m;
    mi = blockIdx.x - b * a.m;
  }
  const char* xrow = a.x + (int64_t(b) * a.sxb + int64_t(mi) * a.sxm) * EB;
  Chunk<DT> cur[CPT];
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = t + c * nt;
    if (ch < a.chunks) load_chunk<DT>(cur[c], xrow + int64_t(ch) * 8 * EB);
    else zero_chunk<DT>(cur[c]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < CPT; ++c) amax = fmaxf(amax, chunk_amax<DT>(cur[c]));
  amax = group_max<64>(amax);
  if ((t & 63) == 0) red[t >> 6] = amax;
  __syncthreads();
  amax = red[0];
  for (int w = 1; w < (nt >> 6); ++w) amax = fmaxf(amax, red[w]);
  const Scales s = channel_scales(amax, a.fp8_max, a.eps);
  if (t == 0) a.scale[int64_t(b) * a.ssb + int64_t(mi) * a.ssm] = s.ds;
  uint8_t* yrow = a.y + int64_t(b) * a.syb + int64_t(mi) * a.sym;
#pragma unroll
  for (int c = 0; c < CPT; ++c) {
    const int ch = t + c * nt;
    if (ch < a.chunks)
      store8<DT, NTS>(yrow + int64_t(ch) * 8, quant_chunk<DT, FMT, CLAMP>(cur[c], s.qs, a.fp8_max));
  }
}

// ===========================================================================
// tile kernel: one block_m x block_n block per workgroup step (persistent,
// the next block prefetched in registers)
// ===========================================================================
struct TileArgs {
  const char* x;
  uint8_t* y;
  float* scale;
  int64_t m, n;
  int64_t sxb, sxm, syb, sym, ssb, ssm, ssn;
  uint32_t mb, nb;   // blocks along m, n
  uint32_t blocks;   // batch * mb * nb
  int32_t block_m;
  int32_t cpt;       // chunks per thread = block_m * lpr / 256
  int32_t lpr, lpr_shift;  // lanes per block row (block_n / 8) and its log2
  int32_t wide;      // H > 0: 128 x 128 blocks, 4 H per workgroup (quant_tile_wide_kernel)
  float fp8_max, eps;
};

// One block per workgroup. GRID3: the grid is (blocks along n, blocks along
// m, batch) and the block comes from the workgroup index; otherwise the grid
// is 1-D (capped) and workgroups stride over the flattened block index. FULL:
// m and n are multiples of the block, so no row / column bounds checks.
template <int DT, int FMT, int CPT, bool NTS, bool GRID3, bool FULL, bool CLAMP>
__global__ __launch_bounds__(kThreads) void quant_tile_kernel(TileArgs a) {
  constexpr int EB = elem_bytes<DT>();
  __shared__ float red[2][kThreads / 64];
  const int t = threadIdx.x;
  const int lr = t & (a.lpr - 1), rp = t >> a.lpr_shift;  // lane in row, row in pass
  const int rpp = kThreads >> a.lpr_shift;                 // rows per pass
  // block (pm, pn) of batch b; rd: this block's slot of the cross-wave maxima
  auto block = [&](uint32_t b, uint32_t pm, uint32_t pn, float* rd) {
    const int64_t r0 = int64_t(pm) * a.block_m;
    const int64_t col = int64_t(pn) * (a.lpr * 8) + lr * 8;
    const char* xb = a.x + int64_t(b) * a.sxb * EB;
    Chunk<DT> cur[CPT];
#pragma unroll
    for (int p = 0; p < CPT; ++p) {
      const int64_t r = r0 + p * rpp + rp;
      if (FULL || (r < a.m && col < a.n)) load_chunk<DT>(cur[p], xb + (r * a.sxm + col) * EB);
      else zero_chunk<DT>(cur[p]);
    }
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < CPT; ++p) amax = fmaxf(amax, chunk_amax<DT>(cur[p]));
    amax = group_max<64>(amax);
    if ((t & 63) == 0) rd[t >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(rd[0], rd[1]), fmaxf(rd[2], rd[3]));
    const Scales s = block_scales(amax, a.fp8_max, a.eps);
    if (t == 0) a.scale[int64_t(b) * a.ssb + int64_t(pm) * a.ssm + int64_t(pn) * a.ssn] = s.ds;
    uint8_t* yb = a.y + int64_t(b) * a.syb;
#pragma unroll
    for (int p = 0; p < CPT; ++p) {
      const int64_t r = r0 + p * rpp + rp;
      if (FULL || (r < a.m && col < a.n))
        store8<DT, NTS>(yb + r * a.sym + col, quant_chunk<DT, FMT, CLAMP>(cur[p], s.qs, a.fp8_max));
    }
  };
  if constexpr (GRID3) {
    // no loop: nothing to load before the block's own loads are issued
    block(blockIdx.z, blockIdx.y, blockIdx.x, red[0]);
  } else {
    int it = 0;
    for (uint32_t blk = blockIdx.x; blk < a.blocks; blk += gridDim.x, ++it) {
      const uint32_t b = blk / (a.mb * a.nb);
      const uint32_t rem = blk - b * a.mb * a.nb;
      const uint32_t pm = rem / a.nb;
      block(b, pm, rem - pm * a.nb, red[it & 1]);  // alternating slots: one barrier per block
    }
  }
}

// 128 x 128 blocks of 16-bit row-contiguous input, 4 H side by side per
// 1024-thread workgroup (128 rows x 512 H columns; m a multiple of 128, n of
// 512 H). Wave w owns rows w, w + 16, ..., and each lane H chunks of a row
// 512 columns apart, so one row piece of a wave is H KiB read by H load
// instructions of 1 KiB (64 lanes x 16 bytes; lanes 16 q .. 16 q + 15 of
// instruction h in block q + 4 h) and written by H stores of 512 bytes. The
// lanes of a block reduce in their 16-lane row by DPP, the 16 waves through
// LDS. Grid (n / (512 H), m / 128, batch). Config 3 ([4096, 7168] bf16, 16
// rotating buffer sets), against one block per 256-thread workgroup (4 rows x
// 256 bytes per load instruction) at 15.9-16.1 us: H = 1 (1 KiB row pieces)
// 15.9-16.1 us, H = 2 (2 KiB) 14.66-14.72 us. The host takes it only for
// grids of at most one workgroup per CU (pcamd_quant_block).
constexpr int kTileWideThreads = 1024;

template <int DT, int FMT, int H, bool NTS, bool CLAMP>
__global__ __launch_bounds__(kTileWideThreads) void quant_tile_wide_kernel(TileArgs a) {
  static_assert(DT == kBF16 || DT == kF16, "16-bit inputs: one 16-byte load per chunk");
  static_assert(H == 1 || H == 2, "four or eight blocks per workgroup");
  constexpr int EB = elem_bytes<DT>();
  constexpr int WAVES = kTileWideThreads / 64, ROWS = 128 / WAVES;  // 8 rows x H chunks per thread
  __shared__ uint32_t red[WAVES][4 * H];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, q = lane >> 4;
  const int64_t r0 = int64_t(blockIdx.y) * 128 + wave;
  const int64_t col = int64_t(blockIdx.x) * (512 * H) + lane * 8;
  const char* xb = a.x + (int64_t(blockIdx.z) * a.sxb + col) * EB;
  Chunk<DT> cur[ROWS][H];
#pragma unroll
  for (int p = 0; p < ROWS; ++p)
#pragma unroll
    for (int h = 0; h < H; ++h) load_chunk<DT>(cur[p][h], xb + ((r0 + p * WAVES) * a.sxm + h * 512) * EB);
  float qs[H];
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float amax = 0.0f;
#pragma unroll
    for (int p = 0; p < ROWS; ++p) amax = fmaxf(amax, chunk_amax<DT>(cur[p][h]));
    const uint32_t u = __float_as_uint(group_max<16>(amax));
    if ((lane & 15) == 0) red[wave][4 * h + q] = u;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < H; ++h) {
    uint32_t mx = red[0][4 * h + q];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) mx = max(mx, red[w][4 * h + q]);  // non-negative floats order like their bits
    const Scales s = block_scales(__uint_as_float(mx), a.fp8_max, a.eps);
    qs[h] = s.qs;
    if (wave == 0 && (lane & 15) == 0)
      a.scale[int64_t(blockIdx.z) * a.ssb + int64_t(blockIdx.y) * a.ssm +
              int64_t(blockIdx.x * 4 * H + 4 * h + q) * a.ssn] = s.ds;
  }
  uint8_t* yb = a.y + int64_t(blockIdx.z) * a.syb + col;
#pragma unroll
  for (int p = 0; p < ROWS; ++p)
#pragma unroll
    for (int h = 0; h < H; ++h)
      store8<DT, NTS>(yb + (r0 + p * WAVES) * a.sym + h * 512,
                      quant_chunk<DT, FMT, CLAMP>(cur[p][h], qs[h], a.fp8_max));
}

// ===========================================================================
// column kernel: 128-column strips, column groups or whole columns
// ===========================================================================
struct ColArgs {
  const char* x;
  uint8_t* y;
  float* scale;
  int64_t m, n;
  int64_t sxb, sxm, syb, sym;
  int64_t ssb, ssm, ssn;  // group mode: scale[b, group, col]; channel: scale[b, col] via ssb, ssn
  int64_t strips;         // ceil(n / 128)
  int64_t groups;         // row groups per batch (group mode), 1 for channel mode
  int64_t units;          // batch * groups * strips
  int32_t group_rows;     // rows per group (group mode)
  int32_t rpt;            // rows per thread (group mode) = group_rows / 16
  float fp8_max, eps;
};

template <int DT, int FMT, bool CHANNEL>
__global__ __launch_bounds__(kThreads) void quant_cols_kernel(ColArgs a) {
  constexpr int EB = elem_bytes<DT>();
  constexpr int SLICES = kThreads / 16;  // 16 threads x 8 columns = 128 columns
  __shared__ float part[SLICES][128];
  __shared__ float qsv[128];
  const int t = threadIdx.x;
  const int lc = t & 15, rs = t >> 4;
  for (int64_t u = blockIdx.x; u < a.units; u += gridDim.x) {
    const int64_t b = u / (a.groups * a.strips);
    const int64_t rem = u - b * a.groups * a.strips;
    const int64_t g = rem / a.strips, strip = rem - g * a.strips;
    const int64_t col = strip * 128 + lc * 8;
    const bool col_ok = col < a.n;
    const char* xb = a.x + b * a.sxb * EB;
    uint8_t* yb = a.y + b * a.syb;
    float cmax[8] = {0, 0, 0, 0, 0, 0, 0, 0};

    if constexpr (CHANNEL) {
      for (int64_t r = rs; r < a.m; r += SLICES) {
        if (col_ok) {
          Chunk<DT> c;
          load_chunk<DT>(c, xb + (r * a.sxm + col) * EB);
          float v[8];
          unpack_chunk<DT>(c, v);
#pragma unroll
          for (int i = 0; i < 8; ++i) cmax[i] = fmaxf(cmax[i], fabsf(v[i]));
        }
      }
    } else {
      Chunk<DT> raw[kMaxSlots];
      const int64_t r0 = g * a.group_rows;
#pragma unroll
      for (int p = 0; p < kMaxSlots; ++p) {
        if (p < a.rpt) {
          const int64_t r = r0 + p * SLICES + rs;
          if (r < a.m && col_ok) load_chunk<DT>(raw[p], xb + (r * a.sxm + col) * EB);
          else zero_chunk<DT>(raw[p]);
          float v[8];
          unpack_chunk<DT>(raw[p], v);
#pragma unroll
          for (int i = 0; i < 8; ++i) cmax[i] = fmaxf(cmax[i], fabsf(v[i]));
        }
      }
      // column maxima across the 16 row slices
#pragma unroll
      for (int i = 0; i < 8; ++i) part[rs][lc * 8 + i] = cmax[i];
      __syncthreads();
      if (t < 128) {
        float mx = 0.0f;
#pragma unroll
        for (int s = 0; s < SLICES; ++s) mx = fmaxf(mx, part[s][t]);
        const Scales sc = block_scales(mx, a.fp8_max, a.eps);
        qsv[t] = sc.qs;
        const int64_t c = strip * 128 + t;
        if (c < a.n) a.scale[b * a.ssb + g * a.ssm + c * a.ssn] = sc.ds;
      }
      __syncthreads();
#pragma unroll
      for (int p = 0; p < kMaxSlots; ++p) {
        if (p < a.rpt) {
          const int64_t r = r0 + p * SLICES + rs;
          if (r < a.m && col_ok) {
            float v[8];
            unpack_chunk<DT>(raw[p], v);
            float q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) q[i] = clamp_sym(v[i] * qsv[lc * 8 + i], a.fp8_max);
            *reinterpret_cast<uint2*>(yb + r * a.sym + col) =
                make_uint2(pack4<FMT>(q[0], q[1], q[2], q[3]), pack4<FMT>(q[4], q[5], q[6], q[7]));
          }
        }
      }
      __syncthreads();
      continue;
    }

    // channel mode: reduce, then a second pass over the strip
#pragma unroll
    for (int i = 0; i < 8; ++i) part[rs][lc * 8 + i] = cmax[i];
    __syncthreads();
    if (t < 128) {
      float mx = 0.0f;
#pragma unroll
      for (int s = 0; s < SLICES; ++s) mx = fmaxf(mx, part[s][t]);
      const Scales sc = channel_scales(mx, a.fp8_max, a.eps);
      qsv[t] = sc.qs;
      const int64_t c = strip * 128 + t;
      if (c < a.n) a.scale[b * a.ssb + c * a.ssn] = sc.ds;
    }
    __syncthreads();
    float qs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) qs[i] = qsv[lc * 8 + i];
    for (int64_t r = rs; r < a.m; r += SLICES) {
      if (col_ok) {
        Chunk<DT> c;
        load_chunk<DT>(c, xb + (r * a.sxm + col) * EB);
        float v[8];
        unpack_chunk<DT>(c, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = clamp_sym(v[i] * qs[i], a.fp8_max);
        *reinterpret_cast<uint2*>(yb + r * a.sym + col) =
            make_uint2(pack4<FMT>(v[0], v[1], v[2], v[3]), pack4<FMT>(v[4], v[5], v[6], v[7]));
      }
    }
    __syncthreads();
  }
}

// ===========================================================================
// generic kernels: any strides, any block shape
// ===========================================================================
struct GenArgs {
  const char* x;
  uint8_t* y;
  float* scale;
  int64_t m, n;
  int64_t sxb, sxm, sxn, syb, sym, syn;
  int64_t ssb, ssm, ssn;
  int64_t bm, bn;     // block shape (block mode); channel mode: see kernel
  int64_t mb, nb;
  int64_t units;
  float fp8_max, eps;
};

PCAMD_DEV float block_reduce_max(float v, float* red) {
  v = group_max<64>(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}

// MODE 0: per block (bm x bn); MODE 1: per channel along rows (one row per
// unit, reduce over n); MODE 2: per channel along columns (reduce over m).
template <int DT, int FMT, int MODE>
__global__ __launch_bounds__(kThreads) void quant_generic_kernel(GenArgs a) {
  __shared__ float red[kThreads / 64];
  for (int64_t u = blockIdx.x; u < a.units; u += gridDim.x) {
    int64_t b, r0, r1, c0, c1, pm = 0, pn = 0;
    if constexpr (MODE == 0) {
      b = u / (a.mb * a.nb);
      const int64_t rem = u - b * a.mb * a.nb;
      pm = rem / a.nb;
      pn = rem - pm * a.nb;
      r0 = pm * a.bm; r1 = min(r0 + a.bm, a.m);
      c0 = pn * a.bn; c1 = min(c0 + a.bn, a.n);
    } else if constexpr (MODE == 1) {
      b = u / a.m; pm = u - b * a.m;
      r0 = pm; r1 = pm + 1; c0 = 0; c1 = a.n;
    } else {
      b = u / a.n; pn = u - b * a.n;
      r0 = 0; r1 = a.m; c0 = pn; c1 = pn + 1;
    }
    const int64_t w = c1 - c0;
    const int64_t cnt = (r1 - r0) * w;
    float amax = 0.0f;
    for (int64_t i = threadIdx.x; i < cnt; i += kThreads) {
      const int64_t r = r0 + i / w, c = c0 + i % w;
      amax = fmaxf(amax, fabsf(load_one<DT>(a.x, b * a.sxb + r * a.sxm + c * a.sxn)));
    }
    amax = block_reduce_max(amax, red);
    const Scales s = MODE == 0 ? block_scales(amax, a.fp8_max, a.eps)
                               : channel_scales(amax, a.fp8_max, a.eps);
    if (threadIdx.x == 0) {
      if constexpr (MODE == 0) a.scale[b * a.ssb + pm * a.ssm + pn * a.ssn] = s.ds;
      else if constexpr (MODE == 1) a.scale[b * a.ssb + pm * a.ssm] = s.ds;
      else a.scale[b * a.ssb + pn * a.ssn] = s.ds;
    }
    for (int64_t i = threadIdx.x; i < cnt; i += kThreads) {
      const int64_t r = r0 + i / w, c = c0 + i % w;
      const float v = load_one<DT>(a.x, b * a.sxb + r * a.sxm + c * a.sxn);
      a.y[b * a.syb + r * a.sym + c * a.syn] = static_cast<uint8_t>(quant_one<DT, FMT>(v, s.qs, a.fp8_max));
    }
  }
}

// ===========================================================================
// per-tensor
// ===========================================================================
__global__ void fill_zero_u32_kernel(uint32_t* p) { *p = 0u; }

struct TensorArgs {
  const char* x;
  uint8_t* y;
  float* scale;        // holds amax bits between the kernels, then 1 / qs
  float* quant_scale;  // optional
  int64_t batch, m, n;
  int64_t sxb, sxm, sxn, syb, sym, syn;
  int64_t total;       // batch * m * n
  float fp8_max, eps;
  int scale_dt;        // scalar scale arithmetic: kF32 / kBF16 / kF16 steps, or kF64 (torchao's form)
};

template <int DT>
__global__ __launch_bounds__(kThreads) void tensor_amax_kernel(TensorArgs a) {
  __shared__ float red[kThreads / 64];
  float amax = 0.0f;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < a.total; i += stride) {
    const int64_t b = i / (a.m * a.n);
    const int64_t rem = i - b * a.m * a.n;
    const int64_t r = rem / a.n, c = rem - r * a.n;
    amax = fmaxf(amax, fabsf(load_one<DT>(a.x, b * a.sxb + r * a.sxm + c * a.sxn)));
  }
  amax = block_reduce_max(amax, red);
  // non-negative fp32 order equals uint32 order of the bit patterns
  if (threadIdx.x == 0) atomicMax(reinterpret_cast<uint32_t*>(a.scale), __float_as_uint(amax));
}

template <int DT, int FMT>
__global__ __launch_bounds__(kThreads) void tensor_quant_kernel(TensorArgs a) {
  const float amax = __uint_as_float(*reinterpret_cast<const uint32_t*>(a.scale));
  const Scales s = tensor_scales(amax, a.fp8_max, a.eps, a.scale_dt);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kThreads;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < a.total; i += stride) {
    const int64_t b = i / (a.m * a.n);
    const int64_t rem = i - b * a.m * a.n;
    const int64_t r = rem / a.n, c = rem - r * a.n;
    const float v = load_one<DT>(a.x, b * a.sxb + r * a.sxm + c * a.sxn);
    a.y[b * a.syb + r * a.sym + c * a.syn] = static_cast<uint8_t>(quant_one<DT, FMT>(v, s.qs, a.fp8_max));
  }
}

// Contiguous input and output (total % 8 == 0, 16-byte aligned): the tensor
// as one run of 8-element chunks. amax: at most 256 workgroups of 512 threads
// striding over units of 8 chunks per lane, one atomic max per workgroup (one
// atomic per workgroup on the single slot is the limit: 1792 non-persistent
// workgroups finishing together took 27 us at [4096, 7168] against 13 us
// here, and a device-scope read before the atomic does not help when they all
// read an empty slot). quantize: units of two chunks per lane (the flat 1 x G
// layout).
constexpr int kAmaxThreads = 512;
constexpr int kAmaxGrid = 256;

template <int DT>
__global__ __launch_bounds__(kAmaxThreads) void tensor_amax_flat_kernel(TensorArgs a) {
  constexpr int EB = elem_bytes<DT>(), CPT = 8, W = kAmaxThreads / 64;
  __shared__ float red[W];
  const int64_t chunks = a.total / 8;
  constexpr int64_t kUnit = int64_t(kAmaxThreads) * CPT;
  float amax = 0.0f;
  for (int64_t base = int64_t(blockIdx.x) * kUnit; base < chunks; base += int64_t(gridDim.x) * kUnit) {
    Chunk<DT> c[CPT];
#pragma unroll
    for (int p = 0; p < CPT; ++p) {
      const int64_t ch = base + p * kAmaxThreads + threadIdx.x;
      if (ch < chunks) load_chunk<DT>(c[p], a.x + ch * 8 * EB);
      else zero_chunk<DT>(c[p]);
    }
#pragma unroll
    for (int p = 0; p < CPT; ++p) amax = fmaxf(amax, chunk_amax<DT>(c[p]));
  }
  amax = group_max<64>(amax);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < W; ++w) amax = fmaxf(amax, red[w]);
    atomicMax(reinterpret_cast<uint32_t*>(a.scale), __float_as_uint(amax));
  }
}

template <int DT, int FMT, bool NTS>
__global__ __launch_bounds__(kTensorFlatThreads) void tensor_quant_flat_kernel(TensorArgs a) {
  constexpr int EB = elem_bytes<DT>(), CPL = 2;
  const int64_t chunks = a.total / 8;
  const int lane = threadIdx.x & 63;
  const int64_t u = int64_t(blockIdx.x) * (kTensorFlatThreads / 64) + (threadIdx.x >> 6);
  const int64_t ch0 = u * (CPL * 64) + lane;
  Chunk<DT> cur[CPL];
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int64_t ch = ch0 + c * 64;
    if (ch < chunks) load_chunk<DT>(cur[c], a.x + ch * 8 * EB);
    else zero_chunk<DT>(cur[c]);
  }
  const Scales s = tensor_scales(__uint_as_float(*reinterpret_cast<const uint32_t*>(a.scale)), a.fp8_max, a.eps,
                                 a.scale_dt);
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int64_t ch = ch0 + c * 64;
    if (ch < chunks) store8<DT, NTS>(a.y + ch * 8, quant_chunk<DT, FMT>(cur[c], s.qs, a.fp8_max));
  }
}

__global__ void tensor_finalize_kernel(TensorArgs a) {
  const float amax = __uint_as_float(*reinterpret_cast<const uint32_t*>(a.scale));
  const Scales s = tensor_scales(amax, a.fp8_max, a.eps, a.scale_dt);
  *a.scale = s.ds;
  if (a.quant_scale) *a.quant_scale = s.qs;
}

// ===========================================================================
// conversion self-test
// ===========================================================================
template <int FMT>
__global__ __launch_bounds__(kThreads) void selftest_convert_kernel(uint32_t* result, uint32_t limit) {
  // Every pattern p in [0, limit] (limit: bits of 464.0 for e4m3fn, the
  // rounding midpoint above its max, and of 59392.0 for e5m2, below the
  // midpoint 61440) is converted
  // in lane position 0 of a packed quadruple (x, y, -x, w) with y and w drawn
  // from other patterns of the range, so sign handling and the byte order of
  // the packed result are checked along with the rounding.
  uint32_t bad = 0, first = 0xFFFFFFFFu;
  const uint32_t stride = gridDim.x * kThreads;
  for (uint32_t p = blockIdx.x * kThreads + threadIdx.x; p <= limit; p += stride) {
    const float x = __uint_as_float(p);
    const float y = -__uint_as_float(limit - p);
    const float w = (p ^ 1u) <= limit ? __uint_as_float(p ^ 1u) : 0.0f;
    const uint32_t hw = hw_pack4<FMT>(x, y, -x, w);
    const uint32_t sw = sw_encode<FMT>(x) | (sw_encode<FMT>(y) << 8) | (sw_encode<FMT>(-x) << 16) |
                        (sw_encode<FMT>(w) << 24);
    if (hw != sw) {
      ++bad;
      first = min(first, p);
    }
  }
  if (bad) {
    atomicAdd(&result[0], bad);
    atomicMin(&result[1], first);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&result[2], limit + 1u);
}

__global__ void selftest_init_kernel(uint32_t* result) {
  result[0] = 0u;
  result[1] = 0xFFFFFFFFu;
  result[2] = 0u;
  result[3] = 0u;
}

// ===========================================================================
// column-group kernel: block_m x 1 groups (block_m = 16 .. 256), one
// 128-column strip of one row group per workgroup
// ===========================================================================
// Grid (strips, row groups, batch). Lane l of a 16-lane row slice takes
// columns 8 l .. 8 l + 7 of the strip, slice s (16 per workgroup) rows
// s, s + 16, ... of the group: CPT = block_m / 16 chunks per lane, loaded up
// front and held in registers. Column maxima: the four slices of a wave meet
// through lane shuffles (xor 16, 32), the four waves through LDS; 128 lanes
// then form one column's scales each. FULL: m and n are multiples of the
// group and the strip, so no bounds checks.
template <int DT, int FMT, int CPT, bool NTS, bool FULL>
__global__ __launch_bounds__(kThreads) void quant_colgroup_kernel(ColArgs a) {
  constexpr int EB = elem_bytes<DT>();
  constexpr int WAVES = kThreads / 64;
  __shared__ float part[WAVES][128];
  __shared__ float qsv[128];
  const int t = threadIdx.x;
  const int lc = t & 15, rs = t >> 4;
  const int64_t b = blockIdx.z, g = blockIdx.y, strip = blockIdx.x;
  const int64_t col = strip * 128 + lc * 8;
  const int64_t r0 = g * (CPT * 16);
  const char* xb = a.x + b * a.sxb * EB;
  Chunk<DT> raw[CPT];
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    const int64_t r = r0 + p * 16 + rs;
    if (FULL || (r < a.m && col < a.n)) load_chunk<DT>(raw[p], xb + (r * a.sxm + col) * EB);
    else zero_chunk<DT>(raw[p]);
  }
  float cmax[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    float v[8];
    unpack_chunk<DT>(raw[p], v);
#pragma unroll
    for (int i = 0; i < 8; ++i) cmax[i] = fmaxf(cmax[i], fabsf(v[i]));
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 16));
    cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 32));
  }
  if ((t & 63) < 16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) part[t >> 6][lc * 8 + i] = cmax[i];
  }
  __syncthreads();
  if (t < 128) {
    float mx = part[0][t];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) mx = fmaxf(mx, part[w][t]);
    const Scales sc = block_scales(mx, a.fp8_max, a.eps);
    qsv[t] = sc.qs;
    const int64_t c = strip * 128 + t;
    if (FULL || c < a.n) a.scale[b * a.ssb + g * a.ssm + c * a.ssn] = sc.ds;
  }
  __syncthreads();
  float qs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qs[i] = qsv[lc * 8 + i];
  uint8_t* yb = a.y + b * a.syb;
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    const int64_t r = r0 + p * 16 + rs;
    if (FULL || (r < a.m && col < a.n)) {
      float v[8];
      unpack_chunk<DT>(raw[p], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = clamp_sym(v[i] * qs[i], a.fp8_max);
      store8<DT, NTS>(yb + r * a.sym + col,
                      make_uint2(pack4<FMT>(v[0], v[1], v[2], v[3]), pack4<FMT>(v[4], v[5], v[6], v[7])));
    }
  }
}

// ===========================================================================
// per-column scales (channel_axis = -1) of tall tensors: column maxima over
// 128-row slabs meet through atomic max in the scale slots, then a second
// kernel quantizes each slab and a third turns the maxima into scales
// ===========================================================================
// scale[b, c] = 0 (the bit pattern the atomic maxima start from)
__global__ __launch_bounds__(kThreads) void colchan_zero_kernel(ColArgs a) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= (a.units / a.strips) * a.n) return;  // units / strips = batch
  const int64_t b = i / a.n, c = i - b * a.n;
  reinterpret_cast<uint32_t*>(a.scale)[b * a.ssb + c * a.ssn] = 0u;
}

// Grid (128-column strips, 128-row slabs, batch), 256 threads: lane t takes
// columns 8 (t % 16) .. + 7 of rows t / 16 + 16 p (p < 8) of its slab. The
// slab's column maxima (lane shuffles, then LDS across the waves) go to the
// scale slots by atomic max on the fp32 bit patterns (for non-negative
// values their uint32 order is the float order). The input is read with
// ordinary (temporal) loads, unlike the other kernels: the apply kernel
// reads it again right after, and what the caches keep of it saves HBM
// reads ([18432, 7168] bf16: 117 -> 106 us for the pair).
template <int DT>
__global__ __launch_bounds__(kThreads) void colchan_amax_kernel(ColArgs a) {
  constexpr int EB = elem_bytes<DT>();
  constexpr int CPT = 8, WAVES = kThreads / 64;
  __shared__ float part[WAVES][128];
  const int t = threadIdx.x;
  const int lc = t & 15, rs = t >> 4;
  const int64_t b = blockIdx.z, strip = blockIdx.x;
  const int64_t col = strip * 128 + lc * 8;
  const int64_t r0 = int64_t(blockIdx.y) * 128;
  const char* xb = a.x + b * a.sxb * EB;
  Chunk<DT> raw[CPT];
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    const int64_t r = r0 + p * 16 + rs;
    if (r < a.m && col < a.n) load_chunk_temporal<DT>(raw[p], xb + (r * a.sxm + col) * EB);
    else zero_chunk<DT>(raw[p]);
  }
  float cmax[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    float v[8];
    unpack_chunk<DT>(raw[p], v);
#pragma unroll
    for (int i = 0; i < 8; ++i) cmax[i] = fmaxf(cmax[i], fabsf(v[i]));
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 16));
    cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 32));
  }
  if ((t & 63) < 16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) part[t >> 6][lc * 8 + i] = cmax[i];
  }
  __syncthreads();
  if (t < 128) {
    float mx = part[0][t];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) mx = fmaxf(mx, part[w][t]);
    const int64_t c = strip * 128 + t;
    if (c < a.n) atomicMax(reinterpret_cast<uint32_t*>(a.scale) + b * a.ssb + c * a.ssn, __float_as_uint(mx));
  }
}

// Same grid: quantize the slab with the finished column maxima.
template <int DT, int FMT, bool NTS>
__global__ __launch_bounds__(kThreads) void colchan_apply_kernel(ColArgs a) {
  constexpr int EB = elem_bytes<DT>();
  constexpr int CPT = 8;
  const int t = threadIdx.x;
  const int lc = t & 15, rs = t >> 4;
  const int64_t b = blockIdx.z, strip = blockIdx.x;
  const int64_t col = strip * 128 + lc * 8;
  const int64_t r0 = int64_t(blockIdx.y) * 128;
  const bool col_ok = col < a.n;
  const char* xb = a.x + b * a.sxb * EB;
  Chunk<DT> raw[CPT];
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    const int64_t r = r0 + p * 16 + rs;
    if (r < a.m && col_ok) load_chunk<DT>(raw[p], xb + (r * a.sxm + col) * EB);
    else zero_chunk<DT>(raw[p]);
  }
  // one division per column of the strip (lanes t < 128), shared through LDS
  __shared__ float qsv[128];
  if (t < 128) {
    const int64_t c = strip * 128 + t;
    const uint32_t* amax_bits = reinterpret_cast<const uint32_t*>(a.scale) + b * a.ssb;
    qsv[t] = c < a.n ? channel_scales(__uint_as_float(amax_bits[c * a.ssn]), a.fp8_max, a.eps).qs : 0.0f;
  }
  __syncthreads();
  float qs[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qs[i] = qsv[lc * 8 + i];
  uint8_t* yb = a.y + b * a.syb;
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    const int64_t r = r0 + p * 16 + rs;
    if (r < a.m && col_ok) {
      float v[8];
      unpack_chunk<DT>(raw[p], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = clamp_sym(v[i] * qs[i], a.fp8_max);
      store8<DT, NTS>(yb + r * a.sym + col,
                      make_uint2(pack4<FMT>(v[0], v[1], v[2], v[3]), pack4<FMT>(v[4], v[5], v[6], v[7])));
    }
  }
}

// scale[b, c]: column maximum -> dequant scale max(amax, eps) / fp8_max
__global__ __launch_bounds__(kThreads) void colchan_finalize_kernel(ColArgs a) {
  const int64_t i = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  if (i >= (a.units / a.strips) * a.n) return;
  const int64_t b = i / a.n, c = i - b * a.n;
  float* s = a.scale + b * a.ssb + c * a.ssn;
  *s = channel_scales(__uint_as_float(*reinterpret_cast<const uint32_t*>(s)), a.fp8_max, a.eps).ds;
}

// ===========================================================================
// dual block quantization: 1 x 128 groups along n and 128 x 1 groups along m
// of one row-contiguous tensor from a single read
// ===========================================================================
struct DualArgs {
  const char* x;
  uint8_t* yr;            // fp8 output of the 1 x 128 groups
  uint8_t* yc;            // fp8 output of the 128 x 1 groups
  float* sr;              // row-group scales [b, row, strip]
  float* sc;              // column-group scales [b, row group, col]
  int64_t m, n;
  int64_t sxb, sxm, syb, sym;
  int64_t ycb, ycn;       // yc strides (bytes) when it is stored transposed (element (r, c) at c * ycn + r)
  int64_t srb, srm, srn, scb, scm, scn;
  float fp8_max, eps;
};

// Grid (128-column strips, 128-row groups, batch), NT threads. Lane t holds
// columns 8 (t % 16) .. + 7 of rows t / 16 + (NT / 16) p (p < 2048 / NT) of
// the 128 x 128 block, loaded up front (TCOL: rows 4 (t / 16) + p, p < 4).
// TCOL: the 128 x 1 output is stored transposed (element (r, c) at
// c * ycn + r): each lane turns its 4 rows x 8 columns of fp8 bytes into 8
// words of 4 rows (byte transposes), the block passes through 16 KiB of LDS,
// and the transposed rows leave as 16-byte stores (ycn a multiple of 16);
// in a partial block the 16 rows of a piece that straddle m go out byte by
// byte and columns past n are skipped. Each
// row's 128 columns sit in one aligned 16-lane row of the wave (DPP max);
// column maxima meet through lane shuffles, then LDS across the waves. The
// results are those of the 1 x 128 and 128 x 1 quantizers run separately.
// FULL: m and n are multiples of 128, so no bounds checks. CLAMP: clamp
// x * qs to +-fp8_max before the cast (needed only when fp8_max is not the
// format's largest finite value, see quant8).
//
// bf16 input with four rows per lane (PK) works on the raw bits: |x| maxima
// are packed unsigned 16-bit maxima (two per instruction), and of the four
// row groups a 16-lane row slice holds, lane (t % 16) forms the scales of
// group (t % 4) only - one division pair per lane instead of four - which
// its quad then broadcasts back. Same bits as the float path.
template <int DT, int FMT, int NT, bool NTS, bool FULL, bool TCOL, bool CLAMP>
__global__ __launch_bounds__(NT) void quant_dual_kernel(DualArgs a) {
  constexpr int EB = elem_bytes<DT>();
  constexpr int CPT = 2048 / NT, WAVES = NT / 64, RPP = NT / 16;
  constexpr bool PK = DT == kBF16 && CPT == 4;
  static_assert(!TCOL || CPT == 4, "transposed column output: four rows per lane");
  __shared__ float part[WAVES][128];  // PK: [WAVES][64] packed column-pair maxima
  __shared__ float qsv[128];
  // transposed block: 128 columns x 32 words of 4 rows; the 16-byte groups of
  // column c sit XOR-ed with (c / 8) % 8 so that the word writes are at most
  // 2-way bank conflicted and the reads are whole 16-byte groups
  __shared__ __attribute__((aligned(16))) uint32_t tt[TCOL ? 128 * 32 : 1];
  const int t = threadIdx.x;
  const int lc = t & 15, rs = t >> 4;
  // XCD-aware block order. Workgroups go to the 8 XCDs in turn (linear id
  // % 8); remapped, XCD x takes the x-th eighth of the blocks in
  // strip-fastest order, so all strips of a row group run on one XCD and the
  // row scales of its rows (one float per row and strip, a row pitch of
  // n / 128 floats apart) fill their cache lines in one L2 instead of
  // reaching HBM as partial lines from eight. A bijection on the grid.
  const uint64_t gx = gridDim.x, gy = gridDim.y;
  const uint64_t total = gx * gy * gridDim.z, per = total / 8;
  const uint64_t lin = (uint64_t(blockIdx.z) * gy + blockIdx.y) * gx + blockIdx.x;
  const uint64_t blk = lin < per * 8 ? (lin % 8) * per + lin / 8 : lin;
  const int64_t strip = static_cast<int64_t>(blk % gx), g = static_cast<int64_t>((blk / gx) % gy),
                b = static_cast<int64_t>(blk / (gx * gy));
  const int64_t col = strip * 128 + lc * 8;
  const int64_t r0 = g * 128;
  auto row_of = [&](int p) -> int64_t { return TCOL ? r0 + 4 * rs + p : r0 + p * RPP + rs; };
  const char* xb = a.x + b * a.sxb * EB;
  Chunk<DT> raw[CPT];
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    const int64_t r = row_of(p);
    if (FULL || (r < a.m && col < a.n)) load_chunk<DT>(raw[p], xb + (r * a.sxm + col) * EB);
    else zero_chunk<DT>(raw[p]);
  }
  float rq[CPT];
  uint32_t* partu = reinterpret_cast<uint32_t*>(&part[0][0]);
  if constexpr (PK) {
    uint32_t ab[CPT][4];
#pragma unroll
    for (int p = 0; p < CPT; ++p) {
      ab[p][0] = bf16_abs2(raw[p].r[0].x); ab[p][1] = bf16_abs2(raw[p].r[0].y);
      ab[p][2] = bf16_abs2(raw[p].r[0].z); ab[p][3] = bf16_abs2(raw[p].r[0].w);
    }
    // 1 x 128: one group per row of the strip
    uint32_t rm[CPT];
#pragma unroll
    for (int p = 0; p < CPT; ++p)
      rm[p] = group_max_u32<16>(max_halves(pk_max_u16(pk_max_u16(ab[p][0], ab[p][1]), pk_max_u16(ab[p][2], ab[p][3]))));
    const int sel = lc & 3;
    const uint32_t ms = sel == 0 ? rm[0] : sel == 1 ? rm[1] : sel == 2 ? rm[2] : rm[3];
    const Scales s = block_scales(bf16_bits(ms), a.fp8_max, a.eps);
    rq[0] = quad_bcast<0>(s.qs); rq[1] = quad_bcast<1>(s.qs);
    rq[2] = quad_bcast<2>(s.qs); rq[3] = quad_bcast<3>(s.qs);
    if (lc < CPT) {
      const int64_t r = row_of(lc);
      if (FULL || r < a.m) a.sr[b * a.srb + r * a.srm + strip * a.srn] = s.ds;
    }
    // 128 x 1: column-pair maxima over this lane's rows, the 4 row slices of
    // the wave (lane shuffles), then the waves (LDS)
    uint32_t cm[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      cm[w] = pk_max_u16(pk_max_u16(ab[0][w], ab[1][w]), pk_max_u16(ab[2][w], ab[3][w]));
      cm[w] = pk_max_u16(cm[w], static_cast<uint32_t>(__shfl_xor(static_cast<int>(cm[w]), 16)));
      cm[w] = pk_max_u16(cm[w], static_cast<uint32_t>(__shfl_xor(static_cast<int>(cm[w]), 32)));
    }
    if ((t & 63) < 16) {
#pragma unroll
      for (int w = 0; w < 4; ++w) partu[(t >> 6) * 64 + lc * 4 + w] = cm[w];
    }
  } else {
    // 1 x 128: one group per row of the strip
#pragma unroll
    for (int p = 0; p < CPT; ++p) {
      const Scales s = block_scales(group_max<16>(chunk_amax<DT>(raw[p])), a.fp8_max, a.eps);
      rq[p] = s.qs;
      const int64_t r = row_of(p);
      if (lc == 0 && (FULL || r < a.m)) a.sr[b * a.srb + r * a.srm + strip * a.srn] = s.ds;
    }
    // 128 x 1: one group per column of the strip
    float cmax[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int p = 0; p < CPT; ++p) {
      float v[8];
      unpack_chunk<DT>(raw[p], v);
#pragma unroll
      for (int i = 0; i < 8; ++i) cmax[i] = fmaxf(cmax[i], fabsf(v[i]));
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 16));
      cmax[i] = fmaxf(cmax[i], __shfl_xor(cmax[i], 32));
    }
    if ((t & 63) < 16) {
#pragma unroll
      for (int i = 0; i < 8; ++i) part[t >> 6][lc * 8 + i] = cmax[i];
    }
  }
  __syncthreads();
  if (t < 128) {
    float mx;
    if constexpr (PK) {
      // column t: dword t / 2 of each wave's row, its low half for even t
      uint32_t m = 0;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) m = max(m, (partu[w * 64 + (t >> 1)] >> ((t & 1) * 16)) & 0xFFFFu);
      mx = bf16_bits(m);
    } else {
      mx = part[0][t];
#pragma unroll
      for (int w = 1; w < WAVES; ++w) mx = fmaxf(mx, part[w][t]);
    }
    const Scales sc = block_scales(mx, a.fp8_max, a.eps);
    qsv[t] = sc.qs;
    const int64_t c = strip * 128 + t;
    if (FULL || c < a.n) a.sc[b * a.scb + g * a.scm + c * a.scn] = sc.ds;
  }
  __syncthreads();
  float qc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qc[i] = qsv[lc * 8 + i];
  uint8_t* yrb = a.yr + b * a.syb;
  uint2 qcol[CPT];
#pragma unroll
  for (int p = 0; p < CPT; ++p) {
    const int64_t r = row_of(p);
    qcol[p] = make_uint2(0u, 0u);
    if (FULL || (r < a.m && col < a.n)) {
      float v[8];
      unpack_chunk<DT>(raw[p], v);
      store8<DT, NTS>(yrb + r * a.sym + col, quant8<FMT, CLAMP>(v, rq[p], a.fp8_max));
      float w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) w[i] = CLAMP ? clamp_sym(v[i] * qc[i], a.fp8_max) : v[i] * qc[i];
      qcol[p] = make_uint2(pack4<FMT>(w[0], w[1], w[2], w[3]), pack4<FMT>(w[4], w[5], w[6], w[7]));
      if constexpr (!TCOL) store8<DT, NTS>(a.yc + b * a.syb + r * a.sym + col, qcol[p]);
    }
  }
  if constexpr (TCOL) {
    // word w[i] of this lane: rows 4 rs .. 4 rs + 3 of column lc * 8 + i
    uint32_t w[8];
    byte_transpose4(qcol[0].x, qcol[1].x, qcol[2].x, qcol[3].x, reinterpret_cast<uint32_t(&)[4]>(w[0]));
    byte_transpose4(qcol[0].y, qcol[1].y, qcol[2].y, qcol[3].y, reinterpret_cast<uint32_t(&)[4]>(w[4]));
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = lc * 8 + i;
      tt[c * 32 + (((rs >> 2) ^ (lc & 7)) << 2) + (rs & 3)] = w[i];
    }
    __syncthreads();
    uint8_t* ycb = a.yc + b * a.ycb + (strip * 128) * a.ycn + r0;
    const int64_t rows = FULL ? 128 : min(int64_t(128), a.m - r0);  // valid rows of the block
#pragma unroll
    for (int j = 0; j < 1024 / NT; ++j) {
      const int q = t + j * NT;           // 16-byte piece: column q / 8, rows 16 (q % 8) .. + 15
      const int ct = q >> 3, seg = q & 7;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(tt + ct * 32 + ((seg ^ ((ct >> 3) & 7)) << 2));
      uint8_t* dst = ycb + ct * a.ycn + seg * 16;
      if (FULL || (strip * 128 + ct < a.n && 16 * seg + 16 <= rows)) {
        if constexpr (NTS) __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(dst));
        else *reinterpret_cast<u32x4_t*>(dst) = v;
      } else if (strip * 128 + ct < a.n) {
        // the piece straddling row m: its first rows - 16 seg bytes
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int k = 0; k < 16; ++k)
          if (16 * seg + k < rows) dst[k] = static_cast<uint8_t>(wv[k >> 2] >> (8 * (k & 3)));
      }
    }
  }
}

// ===========================================================================
// host dispatch helpers
// ===========================================================================
inline int grid_for(int64_t units, int64_t per_block = 1, int64_t cap = 1 << 20) {
  int64_t g = (units + per_block - 1) / per_block;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(g, cap)));
}

template <template <int, int> class Launch, typename... Args>
int dispatch_dt_fmt(int dt, int fmt, Args&&... args) {
  if (fmt == kE4M3) {
    if (dt == kBF16) return Launch<kBF16, kE4M3>::run(args...);
    if (dt == kF16) return Launch<kF16, kE4M3>::run(args...);
    return Launch<kF32, kE4M3>::run(args...);
  }
  if (dt == kBF16) return Launch<kBF16, kE5M2>::run(args...);
  if (dt == kF16) return Launch<kF16, kE5M2>::run(args...);
  return Launch<kF32, kE5M2>::run(args...);
}

// Quantized outputs are written once and not re-read by this kernel:
// non-temporal stores measured 3-6% faster on MI355X for a quantization on
// its own. A caller whose next kernel reads the outputs (the training
// layer's GEMMs) asks for ordinary stores with PCAMD_QUANT_CACHED_OUTPUT
// (the _ex entry points), which leave them in the 256 MB MALL: the
// config-5 layer step 1601 -> 1533 us, its forward GEMM 437 -> 414 us.
// The policy of the current call lives in a thread-local that the _ex entry
// points set for the duration of the call (calls on other threads keep
// their own). PCAMD_QUANT_NT=0 selects ordinary stores everywhere.
thread_local bool tl_cached_output = false;

struct CachedOutputScope {
  bool saved;
  explicit CachedOutputScope(bool on) : saved(tl_cached_output) { tl_cached_output = on; }
  ~CachedOutputScope() { tl_cached_output = saved; }
};

inline bool nt_stores() {
  static const int v = [] {
    const char* e = getenv("PCAMD_QUANT_NT");
    return e && e[0] == '0' ? 0 : 1;
  }();
  return v != 0 && !tl_cached_output;
}

// The clamp of the reference (tl.clamp before the cast) is left out of the
// quantizers (quant8 in fp8_common.h) only when it cannot change a byte: at
// the format's largest value, and with every quant scale qs = fp8_max /
// max(amax, eps) finite, which holds for all amax when fp8_max / eps does.
// Below that eps (fp8_max / FLT_MAX, about 1.3e-36 for e4m3fn) a group whose
// amax is under the bound gets qs = inf, x * qs = +-inf, and only the clamp
// turns that into +-fp8_max; eps <= 0 or NaN keeps the clamp too.
template <int FMT>
inline bool clamp_free(float fp8_max, float eps) {
  return fp8_max == fmt_max<FMT>() && eps > 0.0f && std::isfinite(fp8_max / eps);
}

template <int DT, int FMT>
struct LaunchGroups {
  template <int LPG, int CPL, bool NTS>
  static int go(const RowArgs& a, hipStream_t st) {
    return clamp_free<FMT>(a.fp8_max, a.eps) ? go2<LPG, CPL, NTS, false>(a, st) : go2<LPG, CPL, NTS, true>(a, st);
  }
  template <int LPG, int CPL, bool NTS, bool CLAMP>
  static int go2(const RowArgs& a, hipStream_t st) {
    constexpr int kWaves = kGroupThreads / 64;
    const int grid = static_cast<int>((int64_t(a.units) + kWaves - 1) / kWaves);
    if (a.total > 0) quant_groups_kernel<DT, FMT, LPG, CPL, NTS, true, CLAMP><<<grid, kGroupThreads, 0, st>>>(a);
    else quant_groups_kernel<DT, FMT, LPG, CPL, NTS, false, CLAMP><<<grid, kGroupThreads, 0, st>>>(a);
    return check_launch("quant_groups_kernel");
  }
  template <int LPG, bool NTS>
  static int by_cpl(const RowArgs& a, int cpl, hipStream_t st) {
    if (cpl == 4) return go<LPG, 4, NTS>(a, st);
    if (cpl == 2) return go<LPG, 2, NTS>(a, st);
    return go<LPG, 1, NTS>(a, st);
  }
  template <bool NTS>
  static int by_lpg(const RowArgs& a, int lpg, int cpl, hipStream_t st) {
    switch (lpg) {
      case 1: return by_cpl<1, NTS>(a, cpl, st);
      case 2: return by_cpl<2, NTS>(a, cpl, st);
      case 4: return by_cpl<4, NTS>(a, cpl, st);
      case 8: return by_cpl<8, NTS>(a, cpl, st);
      case 16: return by_cpl<16, NTS>(a, cpl, st);
      case 32: return by_cpl<32, NTS>(a, cpl, st);
      case 64: return by_cpl<64, NTS>(a, cpl, st);
      default: return set_error(PCAMD_ERR_UNSUPPORTED, "row kernel: unsupported lanes per group %d", lpg);
    }
  }
  static int run(const RowArgs& a, int lpg, int cpl, hipStream_t st) {
    return nt_stores() ? by_lpg<true>(a, lpg, cpl, st) : by_lpg<false>(a, lpg, cpl, st);
  }
};

template <int DT, int FMT>
struct LaunchRowBlock {
  template <int CPT, bool NTS>
  static int go(const RowArgs& a, int threads, hipStream_t st) {
    return clamp_free<FMT>(a.fp8_max, a.eps) ? go2<CPT, NTS, false>(a, threads, st)
                                             : go2<CPT, NTS, true>(a, threads, st);
  }
  template <int CPT, bool NTS, bool CLAMP>
  static int go2(const RowArgs& a, int threads, hipStream_t st) {
    const uint32_t batch = a.units / a.m;
    if (batch <= 65535 && a.m <= 0x7FFFFFFFu)
      quant_rowblock_kernel<DT, FMT, CPT, NTS, true, CLAMP><<<dim3(a.m, batch), threads, 0, st>>>(a);
    else
      quant_rowblock_kernel<DT, FMT, CPT, NTS, false, CLAMP><<<a.units, threads, 0, st>>>(a);
    return check_launch("quant_rowblock_kernel");
  }
  template <int MAXC, bool NTS>
  static int wave(const RowArgs& a, hipStream_t st) {
    const int grid = static_cast<int>((int64_t(a.units) + 3) / 4);
    quant_waverow_kernel<DT, FMT, MAXC, NTS><<<grid, kThreads, 0, st>>>(a);
    return check_launch("quant_waverow_kernel");
  }
  template <bool NTS>
  static int pick(const RowArgs& a, hipStream_t st) {
    // Rows shorter than 2048 elements: one wave per row. Longer (up to 16384):
    // one workgroup per row, the workgroup size the smallest multiple of 64
    // that covers the row with two chunks per lane up to 4096 elements and
    // four beyond. A sweep over 2048-16384 elements (non-temporal loads, 2, 3
    // or 4 chunks per lane): four per lane 2-6 % faster from 5120 elements
    // on, equal at 4096 and 8192, two per lane 1 % faster at 2048 (7168: 256
    // threads, 63.4 -> 61.5 us on the config-2 tensor).
    if (a.chunks < 256) return wave<4, NTS>(a, st);
    if (a.chunks <= 512) return go<2, NTS>(a, ((a.chunks + 1) / 2 + 63) / 64 * 64, st);
    return go<4, NTS>(a, ((a.chunks + 3) / 4 + 63) / 64 * 64, st);  // <= 512 threads: chunks <= 2048
  }
  static int run(const RowArgs& a, hipStream_t st) { return nt_stores() ? pick<true>(a, st) : pick<false>(a, st); }
};

template <int DT, int FMT>
struct LaunchTile {
  template <int CPT, bool NTS>
  static int go(const TileArgs& a, hipStream_t st) {
    return clamp_free<FMT>(a.fp8_max, a.eps) ? go2<CPT, NTS, false>(a, st) : go2<CPT, NTS, true>(a, st);
  }
  // 128 x 128 blocks of 16-bit input, 4 H per workgroup (m % 128 == 0,
  // n % (512 H) == 0; the host checked the grid limits)
  template <int H, bool NTS, bool CLAMP>
  static int wide(const TileArgs& a, hipStream_t st) {
    const dim3 grid(static_cast<uint32_t>(a.n / (512 * H)), a.mb, a.blocks / (a.mb * a.nb));
    quant_tile_wide_kernel<DT, FMT, H, NTS, CLAMP><<<grid, kTileWideThreads, 0, st>>>(a);
    return check_launch("quant_tile_wide_kernel");
  }
  template <int H>
  static int run_wide(const TileArgs& a, hipStream_t st) {
    if constexpr (DT == kF32) {
      return set_error(PCAMD_ERR_UNSUPPORTED, "wide tile kernel: 16-bit inputs only");
    } else {
      const bool cf = clamp_free<FMT>(a.fp8_max, a.eps);
      if (nt_stores()) return cf ? wide<H, true, false>(a, st) : wide<H, true, true>(a, st);
      return cf ? wide<H, false, false>(a, st) : wide<H, false, true>(a, st);
    }
  }
  template <int CPT, bool NTS, bool CLAMP>
  static int go2(const TileArgs& a, hipStream_t st) {
    const uint32_t batch = a.blocks / (a.mb * a.nb);
    const bool full = a.m % a.block_m == 0 && a.n % (a.lpr * 8) == 0;
    if (a.mb <= 65535 && batch <= 65535) {
      const dim3 grid(a.nb, a.mb, batch);
      if (full) quant_tile_kernel<DT, FMT, CPT, NTS, true, true, CLAMP><<<grid, kThreads, 0, st>>>(a);
      else quant_tile_kernel<DT, FMT, CPT, NTS, true, false, CLAMP><<<grid, kThreads, 0, st>>>(a);
    } else {
      quant_tile_kernel<DT, FMT, CPT, NTS, false, false, CLAMP><<<grid_for(a.blocks), kThreads, 0, st>>>(a);
    }
    return check_launch("quant_tile_kernel");
  }
  template <bool NTS>
  static int by_cpt(const TileArgs& a, hipStream_t st) {
    switch (a.cpt) {
      case 1: return go<1, NTS>(a, st);
      case 2: return go<2, NTS>(a, st);
      case 4: return go<4, NTS>(a, st);
      case 8: return go<8, NTS>(a, st);
      case 16: return go<16, NTS>(a, st);
      default: return set_error(PCAMD_ERR_UNSUPPORTED, "tile kernel: unsupported chunks per thread %d", a.cpt);
    }
  }
  static int run(const TileArgs& a, hipStream_t st) {
    if (a.wide == 2) return run_wide<2>(a, st);
    if (a.wide == 1) return run_wide<1>(a, st);
    return nt_stores() ? by_cpt<true>(a, st) : by_cpt<false>(a, st);
  }
};

template <int DT, int FMT>
struct LaunchColGroups {
  template <int CPT, bool NTS>
  static int go(const ColArgs& a, hipStream_t st) {
    const dim3 grid(static_cast<uint32_t>(a.strips), static_cast<uint32_t>(a.groups),
                    static_cast<uint32_t>(a.units / (a.groups * a.strips)));
    const bool full = a.m % (CPT * 16) == 0 && a.n % 128 == 0;
    if (full) quant_colgroup_kernel<DT, FMT, CPT, NTS, true><<<grid, kThreads, 0, st>>>(a);
    else quant_colgroup_kernel<DT, FMT, CPT, NTS, false><<<grid, kThreads, 0, st>>>(a);
    return check_launch("quant_colgroup_kernel");
  }
  template <bool NTS>
  static int by_cpt(const ColArgs& a, hipStream_t st) {
    switch (a.rpt) {
      case 1: return go<1, NTS>(a, st);
      case 2: return go<2, NTS>(a, st);
      case 4: return go<4, NTS>(a, st);
      case 8: return go<8, NTS>(a, st);
      case 16: return go<16, NTS>(a, st);
      default: return set_error(PCAMD_ERR_UNSUPPORTED, "column groups: unsupported rows per lane %d", a.rpt);
    }
  }
  static int run(const ColArgs& a, hipStream_t st) { return nt_stores() ? by_cpt<true>(a, st) : by_cpt<false>(a, st); }
};

template <int DT, int FMT>
struct LaunchDual {
  template <bool NTS>
  static int go(const DualArgs& a, int64_t batch, bool tcol, hipStream_t st) {
    const dim3 grid(static_cast<uint32_t>((a.n + 127) / 128), static_cast<uint32_t>((a.m + 127) / 128),
                    static_cast<uint32_t>(batch));
    const bool full = a.m % 128 == 0 && a.n % 128 == 0;
    if (clamp_free<FMT>(a.fp8_max, a.eps)) return go2<NTS, false>(a, grid, full, tcol, st);
    return go2<NTS, true>(a, grid, full, tcol, st);
  }
  template <bool NTS, bool CLAMP>
  static int go2(const DualArgs& a, dim3 grid, bool full, bool tcol, hipStream_t st) {
    constexpr int NT = 512;  // 256: 3 % slower at [8192, 14336]; 1024: 4 % slower
    if (tcol && full) quant_dual_kernel<DT, FMT, NT, NTS, true, true, CLAMP><<<grid, NT, 0, st>>>(a);
    else if (tcol) quant_dual_kernel<DT, FMT, NT, NTS, false, true, CLAMP><<<grid, NT, 0, st>>>(a);
    else if (full) quant_dual_kernel<DT, FMT, NT, NTS, true, false, CLAMP><<<grid, NT, 0, st>>>(a);
    else quant_dual_kernel<DT, FMT, NT, NTS, false, false, CLAMP><<<grid, NT, 0, st>>>(a);
    return check_launch("quant_dual_kernel");
  }
  static int run(const DualArgs& a, int64_t batch, bool tcol, hipStream_t st) {
    return nt_stores() ? go<true>(a, batch, tcol, st) : go<false>(a, batch, tcol, st);
  }
};

template <int DT, int FMT>
struct LaunchColChan {
  template <bool NTS>
  static int go(const ColArgs& a, int64_t batch, hipStream_t st) {
    const int lin = static_cast<int>((batch * a.n + kThreads - 1) / kThreads);
    const dim3 grid(static_cast<uint32_t>(a.strips), static_cast<uint32_t>((a.m + 127) / 128),
                    static_cast<uint32_t>(batch));
    colchan_zero_kernel<<<lin, kThreads, 0, st>>>(a);
    colchan_amax_kernel<DT><<<grid, kThreads, 0, st>>>(a);
    colchan_apply_kernel<DT, FMT, NTS><<<grid, kThreads, 0, st>>>(a);
    colchan_finalize_kernel<<<lin, kThreads, 0, st>>>(a);
    return check_launch("per-column kernels");
  }
  static int run(const ColArgs& a, int64_t batch, hipStream_t st) {
    return nt_stores() ? go<true>(a, batch, st) : go<false>(a, batch, st);
  }
};

template <int DT, int FMT>
struct LaunchCols {
  static int run(const ColArgs& a, bool channel, hipStream_t st) {
    const int grid = grid_for(a.units);
    if (channel) quant_cols_kernel<DT, FMT, true><<<grid, kThreads, 0, st>>>(a);
    else quant_cols_kernel<DT, FMT, false><<<grid, kThreads, 0, st>>>(a);
    return check_launch("quant_cols_kernel");
  }
};

template <int DT, int FMT>
struct LaunchGeneric {
  static int run(const GenArgs& a, int mode, hipStream_t st) {
    const int grid = grid_for(a.units);
    if (mode == 0) quant_generic_kernel<DT, FMT, 0><<<grid, kThreads, 0, st>>>(a);
    else if (mode == 1) quant_generic_kernel<DT, FMT, 1><<<grid, kThreads, 0, st>>>(a);
    else quant_generic_kernel<DT, FMT, 2><<<grid, kThreads, 0, st>>>(a);
    return check_launch("quant_generic_kernel");
  }
};

template <int DT, int FMT>
struct LaunchTensor {
  static int run(const TensorArgs& a, bool flat, hipStream_t st) {
    fill_zero_u32_kernel<<<1, 1, 0, st>>>(reinterpret_cast<uint32_t*>(a.scale));
    if (a.total > 0 && flat) {
      const int64_t chunks = a.total / 8;
      tensor_amax_flat_kernel<DT><<<grid_for(chunks, kAmaxThreads * 8, kAmaxGrid), kAmaxThreads, 0, st>>>(a);
      const int64_t waves = (chunks + 127) / 128;
      const int grid = static_cast<int>((waves + kTensorFlatThreads / 64 - 1) / (kTensorFlatThreads / 64));
      if (nt_stores()) tensor_quant_flat_kernel<DT, FMT, true><<<grid, kTensorFlatThreads, 0, st>>>(a);
      else tensor_quant_flat_kernel<DT, FMT, false><<<grid, kTensorFlatThreads, 0, st>>>(a);
    } else if (a.total > 0) {
      const int grid = grid_for(a.total, kThreads, 4096);
      tensor_amax_kernel<DT><<<grid, kThreads, 0, st>>>(a);
      tensor_quant_kernel<DT, FMT><<<grid, kThreads, 0, st>>>(a);
    }
    tensor_finalize_kernel<<<1, 1, 0, st>>>(a);
    return check_launch("per-tensor kernels");
  }
};

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

// row-contiguous fast-path eligibility: unit element stride, rows made of
// whole 8-element chunks, 16-byte aligned input chunks, 8-byte output chunks
inline bool row_fast_ok(const void* x, int dt, const void* y, int64_t n, int64_t sxb, int64_t sxm,
                        int64_t sxn, int64_t syb, int64_t sym, int64_t syn) {
  const int64_t vec = dt == kF32 ? 4 : 8;  // elements per 16 bytes
  return sxn == 1 && syn == 1 && n % 8 == 0 && aligned(x, 16) && aligned(y, 8) && sxb % vec == 0 &&
         sxm % vec == 0 && syb % 8 == 0 && sym % 8 == 0;
}

int validate_common(const void* x, int x_dtype, int64_t batch, int64_t m, int64_t n, const void* y,
                    int y_dtype, const void* scale, float fp8_max) {
  if (x_dtype != kF32 && x_dtype != kBF16 && x_dtype != kF16)
    return set_error(PCAMD_ERR_INVALID, "unsupported input dtype code %d", x_dtype);
  if (y_dtype != kE4M3 && y_dtype != kE5M2)
    return set_error(PCAMD_ERR_INVALID, "unsupported fp8 dtype code %d", y_dtype);
  if (batch < 0 || m < 0 || n < 0) return set_error(PCAMD_ERR_INVALID, "negative size");
  if (!(fp8_max > 0.0f)) return set_error(PCAMD_ERR_INVALID, "fp8_max must be positive");
  if (batch * m * n > 0 && (!x || !y || !scale)) return set_error(PCAMD_ERR_INVALID, "null pointer");
  return PCAMD_OK;
}

}  // namespace pcamd

using namespace pcamd;

extern "C" int pcamd_quant_block(const void* x, int x_dtype, int64_t batch, int64_t m, int64_t n,
                                 int64_t sxb, int64_t sxm, int64_t sxn, void* y, int y_dtype,
                                 int64_t syb, int64_t sym, int64_t syn, float* scale, int64_t ssb,
                                 int64_t ssm, int64_t ssn, int64_t block_m, int64_t block_n,
                                 float fp8_max, float eps, void* stream) {
  clear_error();
  int rc = validate_common(x, x_dtype, batch, m, n, y, y_dtype, scale, fp8_max);
  if (rc) return rc;
  if (!is_pow2(block_m) || !is_pow2(block_n))
    return set_error(PCAMD_ERR_INVALID, "block sizes must be powers of two, got %lld x %lld",
                     (long long)block_m, (long long)block_n);
  if (batch == 0 || m == 0 || n == 0) return PCAMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool fast = row_fast_ok(x, x_dtype, y, n, sxb, sxm, sxn, syb, sym, syn);
  const int64_t mb = (m + block_m - 1) / block_m, nb = (n + block_n - 1) / block_n;

  if (fast && block_m == 1 && block_n >= 8 && block_n <= 512 && batch * m < UINT32_MAX / 64 &&
      m < UINT32_MAX && n / 8 < INT32_MAX / 2) {
    RowArgs a{};
    a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
    a.m = static_cast<uint32_t>(m); a.sxb = sxb; a.sxm = sxm; a.syb = syb; a.sym = sym;
    a.ssb = ssb; a.ssm = ssm; a.ssn = ssn;
    a.chunks = static_cast<int32_t>(n / 8);
    const int lpg = static_cast<int>(block_n / 8);
    // largest unit (chunk slots per lane) that wastes at most 1/16 of the lanes
    int cpl = 1;
    for (int c : {4, 2}) {
      const int64_t span = 64LL * c, padded = (a.chunks + span - 1) / span * span;
      if ((padded - a.chunks) * 16 <= a.chunks) { cpl = c; break; }
    }
    // contiguous input, output and scales with whole groups per row: one flat
    // run of chunks, units of two chunks per lane (fastest measured)
    const int64_t gpr = n / block_n;  // groups per row
    const bool flat = n % block_n == 0 && sxm == n && sym == n && ssn == 1 && ssm == gpr &&
                      (batch == 1 || (sxb == m * n && syb == m * n && ssb == m * gpr));
    if (flat) {
      cpl = 2;
      a.total = batch * m * a.chunks;
      a.units = static_cast<uint32_t>((a.total + 127) / 128);
      a.segs = 1;
    } else {
      a.segs = static_cast<uint32_t>((a.chunks + 64LL * cpl - 1) / (64LL * cpl));
      a.units = static_cast<uint32_t>(batch * m * a.segs);
    }
    a.cpl = cpl;
    a.fp8_max = fp8_max; a.eps = eps;
    const int64_t units = flat ? (a.total + 127) / 128 : int64_t(batch) * m * a.segs;
    if (units < UINT32_MAX) return dispatch_dt_fmt<LaunchGroups>(x_dtype, y_dtype, a, lpg, cpl, st);
  }
  const int64_t lpr = block_n / 8;
  if (fast && block_n >= 32 && lpr <= 64 && (block_m * lpr) % kThreads == 0 &&
      block_m * lpr / kThreads <= kMaxSlots && batch * mb * nb < UINT32_MAX) {
    TileArgs a{};
    a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
    a.m = m; a.n = n; a.sxb = sxb; a.sxm = sxm; a.syb = syb; a.sym = sym;
    a.ssb = ssb; a.ssm = ssm; a.ssn = ssn;
    a.mb = static_cast<uint32_t>(mb); a.nb = static_cast<uint32_t>(nb);
    a.blocks = static_cast<uint32_t>(batch * mb * nb);
    a.block_m = static_cast<int32_t>(block_m);
    a.cpt = static_cast<int32_t>(block_m * lpr / kThreads);
    a.lpr = static_cast<int32_t>(lpr);
    a.lpr_shift = 0;
    while ((1 << a.lpr_shift) < a.lpr) ++a.lpr_shift;
    a.fp8_max = fp8_max; a.eps = eps;
    // 128 x 128 blocks of 16-bit input: the 1024-thread kernel with 4 H blocks
    // per workgroup when its grid puts at most one workgroup on each CU and
    // fills at least 60 % of them (the whole tensor in flight at once, every
    // CU streaming one 128-row strip piece). Measured on [4096, n] bf16: H = 2
    // 8-14 % faster than one block per 256-thread workgroup at n = 5120-7168
    // (160-224 workgroups), H = 1 9-15 % faster at n = 3072 and 4096 (192 and
    // 256); with more workgroups than CUs (n >= 9216 for H = 2) both were
    // 4-23 % slower, and H = 2 with rows of a multiple of 8 KiB ([8192, 4096])
    // 19 % slower at one workgroup per CU.
    if (block_m == 128 && block_n == 128 && x_dtype != kF32 && m % 128 == 0 && mb <= 65535 && batch <= 65535 &&
        n / 512 <= INT32_MAX) {
      const int64_t cus = device_cu_count(st);
      auto fits = [&](int64_t wgs) { return cus > 0 && wgs <= cus && 10 * wgs >= 6 * cus; };
      const int64_t strips = batch * mb;
      if (n % 1024 == 0 && (sxm * 2) % 8192 != 0 && fits(strips * (n / 1024))) a.wide = 2;
      else if (n % 512 == 0 && fits(strips * (n / 512))) a.wide = 1;
    }
    return dispatch_dt_fmt<LaunchTile>(x_dtype, y_dtype, a, st);
  }
  if (fast && block_n == 1 && block_m >= 16 && block_m <= 256) {
    ColArgs a{};
    a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
    a.m = m; a.n = n; a.sxb = sxb; a.sxm = sxm; a.syb = syb; a.sym = sym;
    a.ssb = ssb; a.ssm = ssm; a.ssn = ssn;
    a.strips = (n + 127) / 128; a.groups = mb; a.units = batch * mb * a.strips;
    a.group_rows = static_cast<int32_t>(block_m);
    a.rpt = static_cast<int32_t>(block_m / 16);
    a.fp8_max = fp8_max; a.eps = eps;
    if (a.strips <= INT32_MAX && mb <= 65535 && batch <= 65535)
      return dispatch_dt_fmt<LaunchColGroups>(x_dtype, y_dtype, a, st);
    return dispatch_dt_fmt<LaunchCols>(x_dtype, y_dtype, a, false, st);
  }
  GenArgs a{};
  a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
  a.m = m; a.n = n; a.sxb = sxb; a.sxm = sxm; a.sxn = sxn; a.syb = syb; a.sym = sym; a.syn = syn;
  a.ssb = ssb; a.ssm = ssm; a.ssn = ssn; a.bm = block_m; a.bn = block_n; a.mb = mb; a.nb = nb;
  a.units = batch * mb * nb; a.fp8_max = fp8_max; a.eps = eps;
  return dispatch_dt_fmt<LaunchGeneric>(x_dtype, y_dtype, a, 0, st);
}

extern "C" int pcamd_quant_block_dual(const void* x, int x_dtype, int64_t batch, int64_t m, int64_t n,
                                      int64_t sxb, int64_t sxm, int64_t sxn, void* y_row, int64_t syb,
                                      int64_t sym, int64_t syn, void* y_col, int64_t ycb, int64_t ycm,
                                      int64_t ycn, int y_dtype, float* scale_row, int64_t srb, int64_t srm,
                                      int64_t srn, float* scale_col, int64_t scb, int64_t scm, int64_t scn,
                                      int64_t block, float fp8_max, float eps, void* stream) {
  clear_error();
  int rc = validate_common(x, x_dtype, batch, m, n, y_row, y_dtype, scale_row, fp8_max);
  if (rc) return rc;
  if (batch * m * n > 0 && (!y_col || !scale_col)) return set_error(PCAMD_ERR_INVALID, "null pointer");
  if (batch * m * n > 0 && (y_row == y_col || scale_row == scale_col))
    return set_error(PCAMD_ERR_INVALID, "the two outputs (and the two scale tensors) must not alias");
  if (!is_pow2(block))
    return set_error(PCAMD_ERR_INVALID, "block size must be a power of two, got %lld", (long long)block);
  if (batch == 0 || m == 0 || n == 0) return PCAMD_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool fast = row_fast_ok(x, x_dtype, y_row, n, sxb, sxm, sxn, syb, sym, syn) && block == 128 &&
                    batch <= 65535 && (m + 127) / 128 <= 65535 && (n + 127) / 128 <= INT32_MAX;
  const bool same_layout = ycb == syb && ycm == sym && ycn == syn && aligned(y_col, 8);
  // transposed 128 x 1 output (element (r, c) at c * ycn + r), 16-byte aligned rows
  const bool transposed = ycm == 1 && ycn >= m && ycn % 16 == 0 && (batch == 1 || ycb % 16 == 0) &&
                          aligned(y_col, 16);
  if (fast && (same_layout || transposed)) {
    DualArgs a{};
    a.x = static_cast<const char*>(x);
    a.yr = static_cast<uint8_t*>(y_row); a.yc = static_cast<uint8_t*>(y_col);
    a.sr = scale_row; a.sc = scale_col;
    a.m = m; a.n = n; a.sxb = sxb; a.sxm = sxm; a.syb = syb; a.sym = sym; a.ycb = ycb; a.ycn = ycn;
    a.srb = srb; a.srm = srm; a.srn = srn; a.scb = scb; a.scm = scm; a.scn = scn;
    a.fp8_max = fp8_max; a.eps = eps;
    return dispatch_dt_fmt<LaunchDual>(x_dtype, y_dtype, a, batch, !same_layout, st);
  }
  // other layouts and block sizes: the two quantizers one after the other
  rc = pcamd_quant_block(x, x_dtype, batch, m, n, sxb, sxm, sxn, y_row, y_dtype, syb, sym, syn, scale_row,
                         srb, srm, srn, 1, block, fp8_max, eps, stream);
  if (rc) return rc;
  return pcamd_quant_block(x, x_dtype, batch, m, n, sxb, sxm, sxn, y_col, y_dtype, ycb, ycm, ycn, scale_col,
                           scb, scm, scn, block, 1, fp8_max, eps, stream);
}

extern "C" int pcamd_quant_block_ex(const void* x, int x_dtype, int64_t batch, int64_t m, int64_t n,
                                    int64_t sxb, int64_t sxm, int64_t sxn, void* y, int y_dtype, int64_t syb,
                                    int64_t sym, int64_t syn, float* scale, int64_t ssb, int64_t ssm, int64_t ssn,
                                    int64_t block_m, int64_t block_n, float fp8_max, float eps, int flags,
                                    void* stream) {
  if (flags & ~PCAMD_QUANT_CACHED_OUTPUT) {
    clear_error();
    return set_error(PCAMD_ERR_INVALID, "unknown quantizer flags 0x%x", flags);
  }
  CachedOutputScope scope((flags & PCAMD_QUANT_CACHED_OUTPUT) != 0);
  return pcamd_quant_block(x, x_dtype, batch, m, n, sxb, sxm, sxn, y, y_dtype, syb, sym, syn, scale, ssb, ssm,
                           ssn, block_m, block_n, fp8_max, eps, stream);
}

extern "C" int pcamd_quant_block_dual_ex(const void* x, int x_dtype, int64_t batch, int64_t m, int64_t n,
                                         int64_t sxb, int64_t sxm, int64_t sxn, void* y_row, int64_t syb,
                                         int64_t sym, int64_t syn, void* y_col, int64_t ycb, int64_t ycm,
                                         int64_t ycn, int y_dtype, float* scale_row, int64_t srb, int64_t srm,
                                         int64_t srn, float* scale_col, int64_t scb, int64_t scm, int64_t scn,
                                         int64_t block, float fp8_max, float eps, int flags, void* stream) {
  if (flags & ~PCAMD_QUANT_CACHED_OUTPUT) {
    clear_error();
    return set_error(PCAMD_ERR_INVALID, "unknown quantizer flags 0x%x", flags);
  }
  CachedOutputScope scope((flags & PCAMD_QUANT_CACHED_OUTPUT) != 0);
  return pcamd_quant_block_dual(x, x_dtype, batch, m, n, sxb, sxm, sxn, y_row, syb, sym, syn, y_col, ycb, ycm,
                                ycn, y_dtype, scale_row, srb, srm, srn, scale_col, scb, scm, scn, block, fp8_max,
                                eps, stream);
}

extern "C" int pcamd_quant_channel(const void* x, int x_dtype, int64_t batch, int64_t m, int64_t n,
                                   int64_t sxb, int64_t sxm, int64_t sxn, void* y, int y_dtype,
                                   int64_t syb, int64_t sym, int64_t syn, float* scale, int64_t ssb,
                                   int64_t ssc, int channel_axis, float fp8_max, float eps,
                                   void* stream) {
  clear_error();
  int rc = validate_common(x, x_dtype, batch, m, n, y, y_dtype, scale, fp8_max);
  if (rc) return rc;
  if (channel_axis != -1 && channel_axis != -2)
    return set_error(PCAMD_ERR_INVALID, "channel_axis must be -1 or -2, got %d", channel_axis);
  const int64_t channels = channel_axis == -2 ? m : n;
  if (batch == 0 || channels == 0) return PCAMD_OK;
  if (!scale) return set_error(PCAMD_ERR_INVALID, "null scale pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool fast = row_fast_ok(x, x_dtype, y, n, sxb, sxm, sxn, syb, sym, syn);
  if (channel_axis == -2 && n == 0) {
    // empty reduction: every row scale is eps / fp8_max (nothing to quantize)
    GenArgs a{};
    a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
    a.m = m; a.n = 0; a.ssb = ssb; a.ssm = ssc; a.units = batch * m;
    a.fp8_max = fp8_max; a.eps = eps;
    return dispatch_dt_fmt<LaunchGeneric>(x_dtype, y_dtype, a, 1, st);
  }
  if (channel_axis == -1 && m == 0) {
    GenArgs a{};
    a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
    a.m = 0; a.n = n; a.ssb = ssb; a.ssn = ssc; a.units = batch * n;
    a.fp8_max = fp8_max; a.eps = eps;
    return dispatch_dt_fmt<LaunchGeneric>(x_dtype, y_dtype, a, 2, st);
  }
  if (channel_axis == -2 && fast && n / 8 <= 8LL * kThreads && batch * m < INT32_MAX && m < UINT32_MAX) {
    RowArgs a{};
    a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
    a.m = static_cast<uint32_t>(m); a.sxb = sxb; a.sxm = sxm; a.syb = syb; a.sym = sym;
    a.ssb = ssb; a.ssm = ssc; a.ssn = 0;
    a.chunks = static_cast<int32_t>(n / 8);
    a.cpl = static_cast<int32_t>((a.chunks + 63) / 64);  // chunk slots per lane, wave-per-row
    a.segs = 1;
    a.units = static_cast<uint32_t>(batch * m);
    a.fp8_max = fp8_max; a.eps = eps;
    return dispatch_dt_fmt<LaunchRowBlock>(x_dtype, y_dtype, a, st);
  }
  if (channel_axis == -1 && fast) {
    ColArgs a{};
    a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
    a.m = m; a.n = n; a.sxb = sxb; a.sxm = sxm; a.syb = syb; a.sym = sym;
    a.ssb = ssb; a.ssm = 0; a.ssn = ssc;
    a.strips = (n + 127) / 128; a.groups = 1; a.units = batch * a.strips;
    a.group_rows = static_cast<int32_t>(std::min<int64_t>(m, INT32_MAX)); a.rpt = 0;
    a.fp8_max = fp8_max; a.eps = eps;
    // Tall tensors: 128-row slabs in parallel (column maxima by atomic max in
    // the scale slots, then a quantize pass). Up to 256 rows one workgroup
    // per strip reads its rows twice.
    if (m > 256 && a.strips <= INT32_MAX && (m + 127) / 128 <= 65535 && batch <= 65535 &&
        (batch * n + kThreads - 1) / kThreads <= INT32_MAX)
      return dispatch_dt_fmt<LaunchColChan>(x_dtype, y_dtype, a, batch, st);
    return dispatch_dt_fmt<LaunchCols>(x_dtype, y_dtype, a, true, st);
  }
  GenArgs a{};
  a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
  a.m = m; a.n = n; a.sxb = sxb; a.sxm = sxm; a.sxn = sxn; a.syb = syb; a.sym = sym; a.syn = syn;
  a.ssb = ssb;
  if (channel_axis == -2) { a.ssm = ssc; a.units = batch * m; }
  else { a.ssn = ssc; a.units = batch * n; }
  a.fp8_max = fp8_max; a.eps = eps;
  return dispatch_dt_fmt<LaunchGeneric>(x_dtype, y_dtype, a, channel_axis == -2 ? 1 : 2, st);
}

extern "C" int pcamd_quant_tensor(const void* x, int x_dtype, int64_t batch, int64_t m, int64_t n,
                                  int64_t sxb, int64_t sxm, int64_t sxn, void* y, int y_dtype,
                                  int64_t syb, int64_t sym, int64_t syn, float* scale,
                                  float* quant_scale_out, float fp8_max, float eps, int scale_dtype,
                                  void* stream) {
  clear_error();
  int rc = validate_common(x, x_dtype, batch, m, n, y, y_dtype, scale, fp8_max);
  if (rc) return rc;
  if (!scale) return set_error(PCAMD_ERR_INVALID, "null scale pointer");
  if (scale_dtype != kF32 && scale_dtype != kBF16 && scale_dtype != kF16 && scale_dtype != kF64)
    return set_error(PCAMD_ERR_INVALID, "scale_dtype must be f32, bf16, f16 or f64 (got %d)", scale_dtype);
  TensorArgs a{};
  a.x = static_cast<const char*>(x); a.y = static_cast<uint8_t*>(y); a.scale = scale;
  a.quant_scale = quant_scale_out;
  a.batch = batch; a.m = m; a.n = n; a.sxb = sxb; a.sxm = sxm; a.sxn = sxn;
  a.syb = syb; a.sym = sym; a.syn = syn; a.total = batch * m * n;
  a.fp8_max = fp8_max; a.eps = eps; a.scale_dt = scale_dtype;
  // one contiguous run of whole chunks in and out
  const bool flat = row_fast_ok(x, x_dtype, y, n, sxb, sxm, sxn, syb, sym, syn) && sxm == n && sym == n &&
                    (batch == 1 || (sxb == m * n && syb == m * n)) && (a.total / 8 + 127) / 128 < (1LL << 31);
  return dispatch_dt_fmt<LaunchTensor>(x_dtype, y_dtype, a, flat, static_cast<hipStream_t>(stream));
}

// plain 16-byte-per-lane streaming copy (measurement of the 1 : 1 ceiling)
__global__ __launch_bounds__(kGroupThreads) void copy16_kernel(const u32x4_t* __restrict__ x,
                                                             u32x4_t* __restrict__ y, int64_t chunks) {
  const int64_t ch = int64_t(blockIdx.x) * kGroupThreads + threadIdx.x;
  if (ch < chunks) __builtin_nontemporal_store(__builtin_nontemporal_load(x + ch), y + ch);
}

extern "C" int pcamd_selftest_copy16(const void* x, void* y, int64_t bytes, void* stream) {
  clear_error();
  if (bytes < 0 || bytes % 16) return set_error(PCAMD_ERR_INVALID, "bytes must be a non-negative multiple of 16");
  if (bytes == 0) return PCAMD_OK;
  if (!x || !y) return set_error(PCAMD_ERR_INVALID, "null pointer");
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15)
    return set_error(PCAMD_ERR_INVALID, "pointers must be 16-byte aligned");
  const int64_t chunks = bytes / 16, grid = (chunks + kGroupThreads - 1) / kGroupThreads;
  if (grid > INT32_MAX) return set_error(PCAMD_ERR_UNSUPPORTED, "copy too large");
  copy16_kernel<<<static_cast<uint32_t>(grid), kGroupThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4_t*>(x), static_cast<u32x4_t*>(y), chunks);
  return check_launch("copy16_kernel");
}

// plain 2 : 1 streaming narrowing, y = the high byte of every 16-bit
// element of x (measurement of the quantizers' read : write ceiling), in the
// flat 1 x G quantizer's streaming layout: a wave owns 128 consecutive
// 16-byte chunks, each lane loads chunks lane and lane + 64 (non-temporal)
// before it stores their 8-byte results (non-temporal); 256-thread
// workgroups
__global__ __launch_bounds__(kGroupThreads) void narrow16_kernel(const u32x4_t* __restrict__ x,
                                                              u32x2_t* __restrict__ y, int64_t chunks) {
  const int64_t ch0 = (int64_t(blockIdx.x) * (kGroupThreads / 64) + (threadIdx.x >> 6)) * 128 + (threadIdx.x & 63);
  u32x4_t v[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) v[c] = ch0 + 64 * c < chunks ? __builtin_nontemporal_load(x + ch0 + 64 * c) : u32x4_t{};
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    // v_perm_b32: bytes 1 and 3 of the second operand, then of the first
    const u32x2_t o = {__builtin_amdgcn_perm(v[c][1], v[c][0], 0x07050301u),
                       __builtin_amdgcn_perm(v[c][3], v[c][2], 0x07050301u)};
    if (ch0 + 64 * c < chunks) __builtin_nontemporal_store(o, y + ch0 + 64 * c);
  }
}

extern "C" int pcamd_selftest_narrow16(const void* x, void* y, int64_t in_bytes, void* stream) {
  clear_error();
  if (in_bytes < 0 || in_bytes % 16) return set_error(PCAMD_ERR_INVALID, "in_bytes must be a non-negative multiple of 16");
  if (in_bytes == 0) return PCAMD_OK;
  if (!x || !y) return set_error(PCAMD_ERR_INVALID, "null pointer");
  if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(y) & 7))
    return set_error(PCAMD_ERR_INVALID, "x must be 16-byte and y 8-byte aligned");
  const int64_t chunks = in_bytes / 16, grid = (chunks + 2 * kGroupThreads - 1) / (2 * kGroupThreads);
  if (grid > INT32_MAX) return set_error(PCAMD_ERR_UNSUPPORTED, "narrowing too large");
  narrow16_kernel<<<static_cast<uint32_t>(grid), kGroupThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4_t*>(x), static_cast<u32x2_t*>(y), chunks);
  return check_launch("narrow16_kernel");
}

extern "C" int pcamd_selftest_fp8_convert(int fmt, uint32_t* result, void* stream) {
  clear_error();
  if (!result) return set_error(PCAMD_ERR_INVALID, "null result pointer");
  if (fmt != kE4M3 && fmt != kE5M2) return set_error(PCAMD_ERR_INVALID, "unknown fp8 format %d", fmt);
  hipStream_t st = static_cast<hipStream_t>(stream);
  selftest_init_kernel<<<1, 1, 0, st>>>(result);
  // every pattern up to 464 for e4m3fn (the rounding midpoint above 448) and
  // up to 59392 for e5m2 (below its midpoint 61440); both bounds round to
  // the max and lie past max * (1 + 2^-23), the most x * qs can reach where
  // the quantizers leave out the clamp
  if (fmt == kE4M3) selftest_convert_kernel<kE4M3><<<4096, kThreads, 0, st>>>(result, 0x43E80000u);
  else selftest_convert_kernel<kE5M2><<<4096, kThreads, 0, st>>>(result, 0x47680000u);
  return check_launch("selftest_convert_kernel");
}
