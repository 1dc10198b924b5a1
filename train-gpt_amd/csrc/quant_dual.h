// Dual quantization: _quantize_to_fp8 of x along its rows AND of x.T (the two
// operands the FP8 backward needs from dY, /root/reference/fp8.py:39-47) from
// one read of x.  Included by quant.hip (the product kernels) and by the
// measurement probe csrc/probe/quant_floor.hip, which instantiates the same
// kernel with its arithmetic taken out (IO = true) so that the I/O floor of
// this exact access pattern can be timed.
//
// Tile = 128 x 128 bf16, one workgroup of kDualThreads = 512 threads.  Lanes
// 16r .. 16r+15 of a wave hold one 128-element row block (as in
// quant_rows_kernel; 4 row blocks per lane), quantize it and keep the raw tile
// in LDS (row pitch 272 B); then groups of 8 lanes own column pairs (16 rows
// per lane), quantize them and store 128 contiguous bytes per column.  The
// bytes and scales equal those of the two separate kernels.  Eight waves per
// tile rather than four halve each wave's arithmetic, which is what the last
// workgroups of a launch (and a launch of one round, such as C1's) wait for.
//
// LDS banks (gfx950, measured with SQ_LDS_BANK_CONFLICT): a 32-bit access
// serves 32 lanes at a time over 32 banks of 4 bytes; a 128-bit read serves
// 16 lanes at a time over 64 banks, the quads {0, 3, 5, 6} or {1, 2, 4, 7} of
// a half-wave.  Both swizzles below leave every LDS instruction of the kernel
// free of bank conflicts:
//  - raw tile: 32-bit word w of row r sits at r * 68 + (w ^ (4 * ((r >> 3) & 3))).
//    The column reads take rows 4j + const for the eight lanes j of a group,
//    and a pitch of 68 words alone puts j, j + 2, j + 4 and j + 6 on the same
//    banks; the xor moves them 4 words apart.  The 16-byte row stores only
//    permute chunks within aligned groups of four.
//  - transposed bytes: column n is 128 bytes at n * 32 words, its 16-byte
//    chunk c at position c ^ (2 * ((n >> 1) & 3)), so that the words the four
//    column pairs of a half-wave write at once land on distinct banks.
//
// ROWS = false gives the column quantization alone (tg_quantize_cols for
// 16-byte-aligned rows); GUARD handles a last tile narrower than 128 columns.
//
// Scales.  With K-block-major scales (skm) a tile's 128 row scales are 512
// contiguous bytes (s[tx * rows + r0 ..]) and so are its 128 column scales
// (st[ty * cols + c0 ..]): they are gathered in LDS and written by two
// waves each, 64 contiguous floats (two whole 128-byte lines) per store
// instruction, instead of 4-byte stores from the lanes that own a block.  The reference's
// row-major layout puts every scale of a tile in a different line, so those
// stay single stores.
//
// Tile order.  Launch slots go round-robin to the 8 XCDs (slot % 8), each
// with its own L2.  A line of row scales (32 tiles along x) and a line of
// column scales (32 tiles along y) are each written 4 bytes at a time by 32
// workgroups in the row-major layout; on one XCD the pieces merge in its L2,
// spread over eight they leave as partial-line writes.  The identity order
// keeps the column-scale lines on one XCD (the XCD of a slot is tx % 8 when
// gridDim.x % 8 == 0) and spreads the row-scale lines over all eight.  With
// xcd_blocks the tiles are dealt to XCDs in blocks of 32 x 16 (each XCD a
// contiguous run of whole blocks), which keeps a row-scale line on one XCD
// and a column-scale line on two.  The host sets it when gridDim.x % 32 == 0,
// gridDim.y % 16 == 0 and each XCD's share is a multiple of 512 tiles.
//
// One launch may carry two tensors (DualJobs): slots [0, nblk0) take the tiles
// of job 0 and the rest those of job 1, each in its own row-major tile order
// (gx tiles along x).  Two 1024-tile tensors (C3's x and W) then fill the
// machine twice over and the second tensor's loads overlap the first one's
// stores, where two launches each run one wave of workgroups.
#pragma once
#include <stdio.h>

#include "row_ops.h"
#include "tg_device.h"
#include "tg_host.h"

namespace tg {

struct DualJob {
  const uint4* x;
  int64_t rows, cols;
  uint2* q;
  float* s;
  uint8_t* qt;
  float* st;
  int gx, gy, xcd_blocks;
  int skm;   // scales K-block-major: s[kb * rows + row], st[kb * cols + col]
  int part;  // 0: rows and x.T; 1: rows only; 2: x.T only (with ROWS)
};
struct DualJobs {
  DualJob job[2];
  int nblk0;   // tiles of job 0; gridDim.x - nblk0 are job 1's
};

constexpr int kDualThreads = 512;

// Word offset of 16-byte chunk c of transposed column n (128 bytes per column).
__device__ __forceinline__ int dual_tq_at(int n, int c) { return n * 32 + 4 * (c ^ (2 * ((n >> 1) & 3))); }

// max over the 8 lanes of a DPP half-row (all lanes receive the result)
__device__ __forceinline__ uint32_t oct_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));    // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));    // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));   // row_half_mirror
  return v;
}

// IO: the probe's variant.  Every load, LDS access and store of the product
// kernel stays (same addresses, same order, same widths); the values stored
// are bit mixes of the loaded words instead of e4m3 bytes and scales, and
// the amax reductions and divides are gone.  IO_SCALES = false also drops
// the scale stores.
template <bool ROWS, bool GUARD, bool IO = false, bool IO_SCALES = true>
__global__ __launch_bounds__(kDualThreads) void quant_dual_kernel(DualJobs jobs) {
  // the raw tile (row pitch 272 B); once every column is in registers the
  // same memory stages the transposed bytes (column pitch 128 B)
  __shared__ uint32_t tile[128 * 68];
  __shared__ float sgather[2][128];   // skm: the tile's row and column scales
  uint32_t* tq = tile;
  constexpr bool kScales = !IO || IO_SCALES;
  const int tid = threadIdx.x;
  const bool second = (int)blockIdx.x >= jobs.nblk0;
  const DualJob& J = second ? jobs.job[1] : jobs.job[0];
  const uint4* __restrict__ x = J.x;
  const int64_t rows = J.rows, cols = J.cols;
  uint2* __restrict__ q = J.q;
  float* __restrict__ s = J.s;
  uint8_t* __restrict__ qt = J.qt;
  float* __restrict__ st = J.st;
  const bool skm = J.skm != 0;
  const int slot = (int)blockIdx.x - (second ? jobs.nblk0 : 0);
  int tx = slot % J.gx, ty = slot / J.gx;
  if (J.xcd_blocks) {
    // slot % 8 is the XCD: the host sets xcd_blocks only on a job that
    // starts at a multiple of 8
    const int per_xcd = J.gx * J.gy / 8;
    const int t = (slot & 7) * per_xcd + (slot >> 3);     // position in XCD-contiguous order
    const int blk = t >> 9, w = t & 511;
    tx = (blk % (J.gx / 32)) * 32 + (w & 31);
    ty = (blk / (J.gx / 32)) * 16 + (w >> 5);
  }
  const int64_t c0 = (int64_t)tx * 128, r0 = (int64_t)ty * 128;
  const int ch = tid & 15, rr = tid >> 4;
  const int64_t cchunks = cols >> 3;
  const bool ch_ok = !GUARD || (c0 >> 3) + ch < cchunks;
  // the job's parts (workgroup-uniform)
  const bool do_rows = ROWS && J.part != 2, do_cols = J.part != 1;
  uint4 v[4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
    v[u] = ch_ok ? ldg_stream(x + (r0 + rr + 32 * u) * cchunks + (c0 >> 3) + ch) : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int row = rr + 32 * u;
    if (do_rows) {
      float sc;
      if constexpr (IO) {
        sc = __uint_as_float(v[u].x);
        q[(r0 + row) * cchunks + (c0 >> 3) + ch] = make_uint2(v[u].x ^ v[u].z, v[u].y ^ v[u].w);
      } else {
        float f[8];
        f[0] = bf16lo(v[u].x); f[1] = bf16hi(v[u].x); f[2] = bf16lo(v[u].y); f[3] = bf16hi(v[u].y);
        f[4] = bf16lo(v[u].z); f[5] = bf16hi(v[u].z); f[6] = bf16lo(v[u].w); f[7] = bf16hi(v[u].w);
        sc = block_scale_bf16(row16_max_u32(absmax8(f)));
        q[(r0 + row) * cchunks + (c0 >> 3) + ch] = quant8<true>(f, sc);
      }
      if (kScales && ch == 0) {
        if (skm) sgather[0][row] = sc;
        else s[(r0 + row) * (cols >> 7) + tx] = sc;
      }
    }
    if (do_cols) *reinterpret_cast<uint4*>(&tile[row * 68 + ((ch * 4) ^ (4 * ((row >> 3) & 3)))]) = v[u];
  }
  const bool rows_gathered = kScales && do_rows && skm;
  if (!do_cols && !rows_gathered) return;
  __syncthreads();
  if (rows_gathered && tid < 128) s[(int64_t)tx * rows + r0 + tid] = sgather[0][tid];
  if (!do_cols) return;

  // columns: the 8 lanes tid >> 3 own the column pair 2c, 2c + 1 (one 32-bit
  // LDS word per row); lane j of the group holds rows 32t + 4j + r, i.e. the
  // 4-row words g = 8t + j of each column
  const int j = tid & 7, cp = tid >> 3;
  const int cpw = cp ^ (4 * ((j >> 1) & 3));   // the pair's word in rows 32t + 4j + r
  auto put_scale = [&](float sc, int n) {
    if (kScales && j == 0 && (!GUARD || c0 + n < cols)) {
      if (skm) sgather[1][n] = sc;
      else st[(c0 + n) * (rows >> 7) + ty] = sc;
    }
  };
  // word g = 8t + j of column n: chunk (g >> 2) = 2t + (j >> 2), word j & 3 of it
  const int jc = j >> 2, jw = j & 3;
  if constexpr (IO) {
    uint32_t wd[16];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) wd[t * 4 + r] = tile[(32 * t + 4 * j + r) * 68 + cpw];
    __syncthreads();   // every lane has read its columns: the tile becomes tq
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      tq[dual_tq_at(2 * cp, 2 * t + jc) + jw] = wd[4 * t] ^ wd[4 * t + 1];
      tq[dual_tq_at(2 * cp + 1, 2 * t + jc) + jw] = wd[4 * t + 2] ^ wd[4 * t + 3];
    }
    put_scale(__uint_as_float(wd[0]), 2 * cp);
    put_scale(__uint_as_float(wd[1]), 2 * cp + 1);
  } else {
    float f0[16], f1[16];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t w = tile[(32 * t + 4 * j + r) * 68 + cpw];
        f0[t * 4 + r] = __uint_as_float(w << 16);
        f1[t * 4 + r] = __uint_as_float(w & 0xFFFF0000u);
      }
    uint32_t m0 = 0, m1 = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      m0 = max(m0, __float_as_uint(f0[i]) & 0x7FFFFFFFu);
      m1 = max(m1, __float_as_uint(f1[i]) & 0x7FFFFFFFu);
    }
    const float sc0 = block_scale_bf16(oct_max_u32(m0));
    const float sc1 = block_scale_bf16(oct_max_u32(m1));
    __syncthreads();   // every lane has read its columns: the tile becomes tq
    auto col_words = [&](const float (&f)[16], float sc, int n) {
      Divider d(sc);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint32_t w;
        if (d.fast) {
          w = e4m3x4(d.div(f[4 * t]), d.div(f[4 * t + 1]), d.div(f[4 * t + 2]), d.div(f[4 * t + 3]));
        } else {
          w = e4m3_nonfinite_scale(f[4 * t], sc) | (e4m3_nonfinite_scale(f[4 * t + 1], sc) << 8) |
              (e4m3_nonfinite_scale(f[4 * t + 2], sc) << 16) |
              (e4m3_nonfinite_scale(f[4 * t + 3], sc) << 24);
        }
        tq[dual_tq_at(n, 2 * t + jc) + jw] = w;
      }
      put_scale(sc, n);
    };
    col_words(f0, sc0, 2 * cp);
    col_words(f1, sc1, 2 * cp + 1);
  }
  __syncthreads();
  // eight lanes per column, lane k writing bytes 16k .. 16k + 15: each store
  // instruction writes eight whole 128-byte columns (full lines).  Ordinary
  // (not non-temporal) stores: the transposed operands are read by the next
  // GEMMs (W.T by the forward's, x.T and dY.T by dW), and written around the
  // Infinity Cache they came back from HBM with each dY.T panel read by one
  // XCD only, which left dW ~15% slower than dX inside the C3 step.
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int n = (tid >> 3) + 64 * p, k = tid & 7;
    if (GUARD && c0 + n >= cols) continue;
    const uint4 val = *reinterpret_cast<const uint4*>(&tq[dual_tq_at(n, k)]);
    *(reinterpret_cast<uint4*>(qt + (c0 + n) * rows + r0) + k) = val;
  }
  if (kScales && skm && tid >= 128 && tid < 256 && (!GUARD || c0 + tid - 128 < cols))
    st[(int64_t)ty * cols + c0 + tid - 128] = sgather[1][tid - 128];
}

// One DualJob over x (rows, cols) in 128 x 128 tiles (a narrower last tile
// along cols).  xcd_ok: the job's first slot is a multiple of 8, so the
// XCD-blocked order may be used (when the tile grid has its shape).
constexpr int64_t kDualMaxTiles = int64_t(1) << 23;   // slots fit one 1-D grid of 256-thread groups

inline int dual_job(DualJob& j, const char* who, const void* x, int64_t rows, int64_t cols, uint8_t* q,
                    float* s, uint8_t* q_t, float* s_t, bool xcd_ok, bool skm) {
  const int64_t gx = (cols + 127) / 128, gy = rows / 128;
  if (gx * gy > kDualMaxTiles) {
    char msg[160];
    snprintf(msg, sizeof msg, "%s: (rows / 128) x (cols / 128) must be <= %lld tiles", who,
             (long long)kDualMaxTiles);
    return einval(msg);
  }
  j.x = reinterpret_cast<const uint4*>(x);
  j.rows = rows;
  j.cols = cols;
  j.q = reinterpret_cast<uint2*>(q);
  j.s = s;
  j.qt = q_t;
  j.st = s_t;
  j.gx = (int)gx;
  j.gy = (int)gy;
  j.xcd_blocks = xcd_ok && gx % 32 == 0 && gy % 16 == 0 && (gx * gy / 8) % 512 == 0;
  j.skm = skm ? 1 : 0;
  j.part = 0;
  return TG_OK;
}

}  // namespace tg
