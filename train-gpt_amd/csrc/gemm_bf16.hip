// bf16 GEMM ("NT": both operands K-contiguous, fp32 accumulation, bf16 out)
// and the straight-through backward of block_scaled_matmul built on it.
//
// The reference's backward (/root/reference/fp8.py:85-98) ignores the FP8
// forward and differentiates the plain product in bf16:
//   da = bf16(g) @ bf16(b).T      -> (M, K)      fp8.py:95
//   db = bf16(a).T @ bf16(g)      -> (K, N)      fp8.py:96
// Both dots take bf16 operands, accumulate in fp32 and round once to bf16.
//
// Design (gfx950, wave64):
//   * v_mfma_f32_16x16x32_bf16, accumulating in place: no per-block scales,
//     so the K loop is MFMA work only.
//   * Workgroup tile 256 x 256, 8 waves as 4 (M) x 2 (N), wave tile 64 x 128
//     = 4 x 8 MFMA tiles, 128 fp32 accumulators per lane.
//   * Operands travel HBM -> LDS by buffer_load ... lds through a ring of four
//     K32 stages (one barrier per stage), issued by one wave per SIMD.
//   * dW contracts over the token axis, which is the row axis of both a and
//     g, so the backward first packs a.T and g.T (bf16, rows padded to a
//     multiple of 64 with zeros) and runs the same NT kernel.
#include "tg_device.h"
#include "tg_host.h"
#include "gemm_tile.h"

namespace tg {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_bf16_16x16x32(const uint4& a, const uint4& b, const v4f& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a),
                                                 __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// Four-stage pipeline.  A stage is one K32 slice of the workgroup tile: 256
// rows x 64 B of A and of B, 32 KiB; four stages ring through 128 KiB of LDS,
// so three slices (96 KiB per CU) are in flight while one is computed.  (With
// two stages of K64, one 64 KiB step in flight, the copy stream was capped by
// the ~1.4 us round trip to L2 / Infinity Cache at ~45 B/ns per CU; the MFMAs
// consume a K64 step in ~0.9 us.)
//   step s: loader waves wait for their copies of slice s (vmcnt(16): the 16
//           DMA instructions of slices s+1 and s+2 stay outstanding); barrier
//           (slice s complete, slice s-1 read by every wave); the loader waves
//           issue slice s+3 into slice s-1's stage; every wave computes s.
// Loads: waves 0-3 (one per SIMD) issue all copies, 8 per slice (rows
// 64w .. 64w+63 of A and of B), so the other wave of each SIMD never stalls at
// a DMA issue; loader and compute waves run separate copies of the loop.  The
// copies are issued unconditionally: past the last slice the offset is out of
// range and the loads read zero, which keeps the vmcnt arithmetic exact.  The
// main loop runs whole rounds of four slices with no exit inside (with exits,
// the compiler's wait analysis merges paths at the loop header and drains
// every outstanding copy there).  The barrier is a bare s_barrier (a fence
// would wait for every outstanding copy).
// LDS rows are 64 B, 16-byte chunk c of row r at c ^ ((r >> 1) & 3): the
// fragment reads (16 rows x 4 chunks per instruction) then run without bank
// conflicts on gfx950 (measured: c ^ ((r >> 2) & 3) doubled every read's
// LDS cycles).  Tiles are computed as
// B . A^T so that a lane holds one output row and four consecutive columns
// (8-byte bf16 pieces for the epilogue).
// ---------------------------------------------------------------------------
__shared__ __attribute__((aligned(16))) uint8_t q4_a0[256 * 64];
__shared__ __attribute__((aligned(16))) uint8_t q4_b0[256 * 64];
__shared__ __attribute__((aligned(16))) uint8_t q4_a1[256 * 64];
__shared__ __attribute__((aligned(16))) uint8_t q4_b1[256 * 64];
__shared__ __attribute__((aligned(16))) uint8_t q4_a2[256 * 64];
__shared__ __attribute__((aligned(16))) uint8_t q4_b2[256 * 64];
__shared__ __attribute__((aligned(16))) uint8_t q4_a3[256 * 64];
__shared__ __attribute__((aligned(16))) uint8_t q4_b3[256 * 64];

template <int S> __device__ __forceinline__ uint8_t* q4_a() {
  return S == 0 ? q4_a0 : S == 1 ? q4_a1 : S == 2 ? q4_a2 : q4_a3;
}
template <int S> __device__ __forceinline__ uint8_t* q4_b() {
  return S == 0 ? q4_b0 : S == 1 ? q4_b1 : S == 2 ? q4_b2 : q4_b3;
}

struct Q4Ctx {
  __amdgpu_buffer_rsrc_t ra, rb;
  uint32_t voa, vob;       // NT: loader lane's byte offsets of slice 0, part 0
  uint32_t row16;          // NT: 16 rows in bytes
  int wave, nks;
  uint32_t fa, fb;         // NT: LDS byte offsets of this lane's fragment chunk (tile 0)
  // TN (operands contraction-major, see gemm_bf16_tn_q4_kernel)
  uint32_t voa4[4], vob4[4];   // loader lane's byte offsets of slice 0, part p
  uint32_t sla, slb;           // bytes of one 32-row slice of A and of B
  uint32_t tro[2];             // LDS byte offset of the row of this lane's transpose read h
  uint32_t trx[2];             // chunk XOR of that row
  uint32_t tca, tcb, tin;      // logical chunk of this lane's columns in subtile 0 of A / B, byte within it
};

// TN stage layout: 32 contraction rows of 512 bytes (the tile's 256 output
// indices); 16-byte chunk c of row r sits at chunk c ^ tn_swz(r).  The XOR
// moves whole 32-byte pieces (a transposed fragment read's 4 lanes of one row)
// and differs over the 8 rows that 32 lanes of one read touch.
__device__ __forceinline__ uint32_t tn_swz(uint32_t r) { return ((r & 3u) | (((r >> 3) & 1u) << 2)) << 1; }

// slice ks into the stage at (la, lb).  NT: loader wave w fills rows
// 64w .. 64w+63 of A and of B, 16 rows per instruction; TN: contraction rows
// 8w .. 8w+7, 2 rows per instruction.
template <bool LOADER, bool TN>
__device__ __forceinline__ void q4_issue(const Q4Ctx& c, uint8_t* la, uint8_t* lb, int ks) {
  if (!LOADER) return;
  if constexpr (TN) {
    const bool in = ks < c.nks;
    const uint32_t soa = in ? (uint32_t)ks * c.sla : 0x80000000u;   // out of range: zeros
    const uint32_t sob = in ? (uint32_t)ks * c.slb : 0x80000000u;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(c.ra, la + c.wave * 4096 + p * 1024, 16, c.voa4[p], soa, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rb, lb + c.wave * 4096 + p * 1024, 16, c.vob4[p], sob, 0, 0);
    }
  } else {
    const uint32_t so = ks < c.nks ? (uint32_t)ks * 64u : 0x80000000u;   // out of range: zeros
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(c.ra, la + c.wave * 4096 + p * 1024, 16, c.voa,
                                               so + p * c.row16, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rb, lb + c.wave * 4096 + p * 1024, 16, c.vob,
                                               so + p * c.row16, 0, 0);
    }
  }
}

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

// TN fragment of subtile t (16 output indices at column chunk base cb + 2t):
// lane (fr, fg) gets contraction rows 8 fg .. 8 fg + 7 of output index
// (subtile start) + fr, as the NT fragment holds them, from two transposed
// reads (ds_read_b64_tr_b16: in each 16-lane group, lane i receives element
// i % 4 of the 8-byte pieces lanes 4j + i / 4 read, j = 0..3); lane 4j + q
// of a group reads row 8 fg + j (+4) at columns 4q .. 4q+3 of the subtile.
__device__ __forceinline__ uint4 tn_frag(const uint8_t* l, const Q4Ctx& c, uint32_t cb, int t) {
  const uint32_t ch = cb + 2u * (uint32_t)t;
  const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4s_t*)(l + c.tro[0] + ((ch ^ c.trx[0]) << 4) + c.tin));
  const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_v4s_t*)(l + c.tro[1] + ((ch ^ c.trx[1]) << 4) + c.tin));
  return make_uint4(((uint32_t)(uint16_t)lo[0]) | ((uint32_t)(uint16_t)lo[1] << 16),
                    ((uint32_t)(uint16_t)lo[2]) | ((uint32_t)(uint16_t)lo[3] << 16),
                    ((uint32_t)(uint16_t)hi[0]) | ((uint32_t)(uint16_t)hi[1] << 16),
                    ((uint32_t)(uint16_t)hi[2]) | ((uint32_t)(uint16_t)hi[3] << 16));
}

// s_waitcnt vmcnt(16) as the builtin (gfx9 encoding: vmcnt bits 15:14 = 1,
// expcnt and lgkmcnt not waited), which the compiler's own wait insertion
// takes into account; an inline-asm wait is opaque to it.
constexpr int kWaitVm16 = (1 << 14) | (0xF << 8) | (0x7 << 4);

template <int S, bool LOADER, bool TN>
__device__ __forceinline__ void q4_step(const Q4Ctx& c, int ks, v4f (&acc)[4][8]) {
  if (LOADER) __builtin_amdgcn_s_waitcnt(kWaitVm16);
  __builtin_amdgcn_s_barrier();
  constexpr int kRefill = (S + 3) & 3;   // the stage slice ks - 1 occupied
  q4_issue<LOADER, TN>(c, q4_a<kRefill>(), q4_b<kRefill>(), ks + 3);
  const uint8_t* la = q4_a<S>();
  const uint8_t* lb = q4_b<S>();
  uint4 af[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    af[i] = TN ? tn_frag(la, c, c.tca, i) : *reinterpret_cast<const uint4*>(la + c.fa + i * 1024);
  uint4 bn = TN ? tn_frag(lb, c, c.tcb, 0) : *reinterpret_cast<const uint4*>(lb + c.fb);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint4 bf = bn;
    if (j + 1 < 8)
      bn = TN ? tn_frag(lb, c, c.tcb, j + 1) : *reinterpret_cast<const uint4*>(lb + c.fb + (j + 1) * 1024);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16_16x16x32(bf, af[i], acc[i][j]);
  }
}

template <bool LOADER, bool TN>
__device__ __forceinline__ void q4_main_loop(const Q4Ctx& c, v4f (&acc)[4][8]) {
  q4_issue<LOADER, TN>(c, q4_a0, q4_b0, 0);
  q4_issue<LOADER, TN>(c, q4_a1, q4_b1, 1);
  q4_issue<LOADER, TN>(c, q4_a2, q4_b2, 2);
  int ks = 0;
  for (; ks + 4 <= c.nks; ks += 4) {
    q4_step<0, LOADER, TN>(c, ks, acc);
    q4_step<1, LOADER, TN>(c, ks + 1, acc);
    q4_step<2, LOADER, TN>(c, ks + 2, acc);
    q4_step<3, LOADER, TN>(c, ks + 3, acc);
  }
  if (ks < c.nks) {
    q4_step<0, LOADER, TN>(c, ks, acc);
    if (ks + 1 < c.nks) {
      q4_step<1, LOADER, TN>(c, ks + 1, acc);
      if (ks + 2 < c.nks) q4_step<2, LOADER, TN>(c, ks + 2, acc);
    }
  }
}

// Epilogue of the 256 x 256 bf16 kernels: lane (fr, fg) holds row i * 16 + fr
// and columns j * 16 + 4 fg .. +3 of the wave tile; stage it in this wave's
// 16 KiB (256-byte rows, chunk c of row r at c ^ (r & 15)), then 16 lanes
// store each row's 256 bytes.
__device__ __forceinline__ void q4_store_tile(const v4f (&acc)[4][8], __bf16* __restrict__ C, int M, int N, int m0,
                                              int n0, int wm, int wn, int wave, int lane) {
  const int fr = lane & 15, fg = lane >> 4;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  uint8_t* wbuf = wave == 0 ? q4_a0 : wave == 1 ? q4_b0 : wave == 2 ? q4_a1 : wave == 3 ? q4_b1
                : wave == 4 ? q4_a2 : wave == 5 ? q4_b2 : wave == 6 ? q4_a3 : q4_b3;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = i * 16 + fr;
      const int chunk = (j * 2 + (fg >> 1)) ^ (r & 15);
      const v4f v = acc[i][j];
      *reinterpret_cast<uint2*>(wbuf + r * 256 + chunk * 16 + (fg & 1) * 8) =
          make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
    }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const bool vec_ok = (N % 8) == 0;
  const int k = lane & 15;
#pragma unroll
  for (int q = 0; q < 16; ++q) {
    const int r = q * 4 + (lane >> 4);
    const int m = m0 + wm * 64 + r;
    const int n = n0 + wn * 128 + k * 8;
    const uint4 v = *reinterpret_cast<const uint4*>(wbuf + r * 256 + ((k ^ (r & 15)) * 16));
    if (m < M && n < N) {
      __bf16* dst = C + (int64_t)m * N + n;
      if (vec_ok) {
        *reinterpret_cast<uint4*>(dst) = v;
      } else {
        const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
        for (int t = 0; t < 8; ++t)
          if (n + t < N) reinterpret_cast<uint16_t*>(dst)[t] = e[t];
      }
    }
  }
}

__global__ __launch_bounds__(512, 1) void gemm_bf16_nt_q4_kernel(const __bf16* __restrict__ A,
                                                                 const __bf16* __restrict__ B,
                                                                 __bf16* __restrict__ C, int M, int N,
                                                                 int K, int tiles_m, int tiles_n) {
  Q4Ctx c;
  const int tid = threadIdx.x, lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  c.nks = K >> 5;
  const int fr = lane & 15, fg = lane >> 4;
  const int wm = c.wave >> 1, wn = c.wave & 1;
  int tmi, tni;
  tile_of(blockIdx.x, tiles_m, tiles_n, tmi, tni);
  const int m0 = tmi * 256, n0 = tni * 256;
  const uint32_t rowb = 2u * (uint32_t)K;
  c.ra = make_rsrc(A, (uint32_t)M * rowb);
  c.rb = make_rsrc(B, (uint32_t)N * rowb);
  c.row16 = 16u * rowb;
  // DMA lane L lands at byte 16 L of its 1 KiB slot: row slot + L / 4,
  // physical chunk L % 4, which holds logical chunk (L % 4) ^ ((L >> 3) & 3)
  const int lrow = c.wave * 64 + (lane >> 2);   // loader waves 0-3
  const uint32_t lch = (uint32_t)((lane & 3) ^ ((lane >> 3) & 3)) * 16u;
  c.voa = (uint32_t)(m0 + lrow) * rowb + lch;
  c.vob = (uint32_t)(n0 + lrow) * rowb + lch;
  // fragment: lane (fr, fg) reads logical chunk fg (k 8fg .. 8fg+7) of row
  // (wave tile row) + 16 t + fr, at physical chunk fg ^ ((fr >> 1) & 3)
  const uint32_t ch = (uint32_t)(fg ^ ((fr >> 1) & 3)) * 16u;
  c.fa = (uint32_t)(wm * 64 + fr) * 64u + ch;
  c.fb = (uint32_t)(wn * 128 + fr) * 64u + ch;

  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  if (c.wave < 4) q4_main_loop<true, false>(c, acc);
  else q4_main_loop<false, false>(c, acc);

  q4_store_tile(acc, C, M, N, m0, n0, wm, wn, c.wave, lane);
}

// C (M, N) = A^T B on contraction-major operands: A (Kc, M) and B (Kc, N)
// row-major with row pitches lda and ldb elements, C[m][n] = sum_c A[c][m] B[c][n].
// This is the straight-through backward's db = a.T @ g (fp8.py:96) read
// straight from a and g, with no transposed copies.  The pipeline, tiles and
// epilogue are the NT kernel's; a stage holds 32 contraction rows of the
// tile's 256 m (A) or n (B) indices, 512 bytes each (stored with tn_swz), and
// the MFMA fragments come from transposed LDS reads (tn_frag).  Contraction
// rows past Kc read zero; tile columns past M or N read neighbouring memory
// that only reaches discarded outputs.
__global__ __launch_bounds__(512, 1) void gemm_bf16_tn_q4_kernel(const __bf16* __restrict__ A,
                                                                 const __bf16* __restrict__ B,
                                                                 __bf16* __restrict__ C, int M, int N, int Kc,
                                                                 int lda, int ldb, int tiles_m, int tiles_n) {
  Q4Ctx c;
  const int tid = threadIdx.x, lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  c.nks = (Kc + 31) >> 5;
  const int fr = lane & 15, fg = lane >> 4;
  const int wm = c.wave >> 1, wn = c.wave & 1;
  int tmi, tni;
  tile_of(blockIdx.x, tiles_m, tiles_n, tmi, tni);
  const int m0 = tmi * 256, n0 = tni * 256;
  const uint32_t pa = 2u * (uint32_t)lda, pb = 2u * (uint32_t)ldb;
  c.ra = make_rsrc(A, (uint32_t)Kc * pa);
  c.rb = make_rsrc(B, (uint32_t)Kc * pb);
  c.sla = 32u * pa;
  c.slb = 32u * pb;
  // DMA: instruction p of loader wave w fills slice rows r = 8w + 2p + L / 32;
  // lane L lands at physical chunk L % 32 of row r, which holds logical chunk
  // (L % 32) ^ tn_swz(r)
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const uint32_t r = (uint32_t)(8 * c.wave + 2 * p + (lane >> 5));
    const uint32_t lc = (uint32_t)(lane & 31) ^ tn_swz(r);
    c.voa4[p] = r * pa + (uint32_t)m0 * 2u + lc * 16u;
    c.vob4[p] = r * pb + (uint32_t)n0 * 2u + lc * 16u;
  }
  // transposed reads: lane (fr, fg) reads row 8 fg + fr / 4 (+ 4) at columns
  // 4 (fr % 4) .. +3 of a subtile: chunk (fr % 4) / 2 of it, byte 8 (fr % 2)
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t r = (uint32_t)(8 * fg + 4 * h + (fr >> 2));
    c.tro[h] = r * 512u;
    c.trx[h] = tn_swz(r);
  }
  c.tca = (uint32_t)(wm * 8 + ((fr & 3) >> 1));
  c.tcb = (uint32_t)(wn * 16 + ((fr & 3) >> 1));
  c.tin = 8u * (uint32_t)(fr & 1);

  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  if (c.wave < 4) q4_main_loop<true, true>(c, acc);
  else q4_main_loop<false, true>(c, acc);

  q4_store_tile(acc, C, M, N, m0, n0, wm, wn, c.wave, lane);
}

// ---------------------------------------------------------------------------
// Packing: y = bf16(x) (RNE for f32 input), optionally transposed, with every
// output row padded with zeros to `pitch` elements.
//   transpose = 0: x (rows, cols) -> y (rows, pitch),  pitch >= cols
//   transpose = 1: x (rows, cols) -> y (cols, pitch),  pitch >= rows
// A 64 x 64 tile goes through LDS so that both the reads and the writes are
// row-contiguous; the LDS tile has one padding element per row.
// ---------------------------------------------------------------------------
template <bool F32_IN, bool TRANSPOSE>
__global__ __launch_bounds__(256) void pack_bf16_kernel(const void* __restrict__ xv,
                                                        __bf16* __restrict__ y, int rows, int cols,
                                                        int pitch) {
  __shared__ uint16_t tile[64][65];
  const int tid = threadIdx.x;
  // tile origin in x coordinates
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  // read 64 x 64 of x: thread covers column c0 + (tid & 63), rows (tid >> 6) + 4t
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int rr = (tid >> 6) + 4 * t, cc = tid & 63;
    const int r = r0 + rr, col = c0 + cc;
    uint16_t v = 0;
    if (r < rows && col < cols) {
      if (F32_IN) {
        const float f = reinterpret_cast<const float*>(xv)[(int64_t)r * cols + col];
        v = __builtin_bit_cast(uint16_t, (__bf16)f);
      } else {
        v = reinterpret_cast<const uint16_t*>(xv)[(int64_t)r * cols + col];
      }
    }
    if (TRANSPOSE) tile[cc][rr] = v; else tile[rr][cc] = v;
  }
  __syncthreads();
  // write: output row (tile row) ty, output column tx; outputs past the
  // data but inside the pitch are the zero padding read above
  const int out_rows = TRANSPOSE ? cols : rows;
  const int or0 = TRANSPOSE ? c0 : r0, oc0 = TRANSPOSE ? r0 : c0;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int ty = (tid >> 6) + 4 * t, tx = tid & 63;
    const int orow = or0 + ty, ocol = oc0 + tx;
    if (orow < out_rows && ocol < pitch)
      reinterpret_cast<uint16_t*>(y)[(int64_t)orow * pitch + ocol] = tile[ty][tx];
  }
}

// Transposing pack of 16-byte-aligned bf16 rows (the common case, x_dtype bf16,
// cols % 8 == 0): a 128 x 128 tile is loaded with 16-byte row loads into LDS
// (pitch 272 B); lane p of a wave reads the column pair 2p, 2p + 1 one 32-bit
// word per row (conflict-free), the tile is re-staged in LDS as output rows
// (pitch 264 B) and 16 lanes write each output row's 256 bytes, so every store
// instruction covers four whole row segments.  (Writing each lane's 16-byte
// pieces straight out left every output line to be assembled from sixteen
// stores of four waves: 2.4 TB/s instead of 4.5 at 8192 x 50304.)  NT: non-
// temporal stores, for outputs larger than the Infinity Cache.
template <bool NT>
__global__ __launch_bounds__(256) void pack_bf16_t128_kernel(const uint4* __restrict__ x,
                                                             uint16_t* __restrict__ y, int rows,
                                                             int cols, int pitch) {
  __shared__ uint32_t tile[128 * 68];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.y * 128, c0 = blockIdx.x * 128;
  const int ch = tid & 15, rr = tid >> 4;
  const int cchunks = cols >> 3;
  const bool ch_ok = (c0 >> 3) + ch < cchunks;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int r = r0 + rr + 16 * u;
    const uint4 v = (ch_ok && r < rows) ? ldg_stream(x + (int64_t)r * cchunks + (c0 >> 3) + ch)
                                        : make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4*>(&tile[(rr + 16 * u) * 68 + ch * 4]) = v;
  }
  __syncthreads();
  // lane p: input columns 2p, 2p + 1 (output rows), input rows 32g + 8c .. +7
  const int p = tid & 63, g = tid >> 6;
  uint32_t lo[4][4], hi[4][4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int rb = 32 * g + 8 * c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t w0 = tile[(rb + 2 * e) * 68 + p], w1 = tile[(rb + 2 * e + 1) * 68 + p];
      lo[c][e] = (w0 & 0xFFFFu) | (w1 << 16);
      hi[c][e] = (w0 >> 16) | (w1 & 0xFFFF0000u);
    }
  }
  __syncthreads();   // every lane has read the tile: the same memory stages the output rows
  uint32_t* tq = tile;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int rb = 32 * g + 8 * c;
    *reinterpret_cast<uint4*>(&tq[(2 * p) * 66 + rb / 2]) = make_uint4(lo[c][0], lo[c][1], lo[c][2], lo[c][3]);
    *reinterpret_cast<uint4*>(&tq[(2 * p + 1) * 66 + rb / 2]) = make_uint4(hi[c][0], hi[c][1], hi[c][2], hi[c][3]);
  }
  __syncthreads();
  const int k = tid & 15;            // elements 8k .. 8k+7 of output row n
  const int oc = r0 + 8 * k;
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int n = (tid >> 4) + 16 * q;
    if (c0 + n < cols && oc < pitch) {
      const uint4 v = *reinterpret_cast<const uint4*>(&tq[n * 66 + 4 * k]);
      uint4* dst = reinterpret_cast<uint4*>(y + (int64_t)(c0 + n) * pitch + oc);
      if (NT) stg_stream(dst, v);
      else *dst = v;
    }
  }
}

int launch_pack_bf16(const void* x, int x_dtype, int64_t rows, int64_t cols, int transpose,
                     __bf16* y, int64_t pitch, hipStream_t st) {
  if (rows == 0 || cols == 0) return TG_OK;
  // the grid covers the padded extent so the zero padding is written too
  const int64_t ext_r = transpose ? pitch : rows, ext_c = transpose ? cols : pitch;
  const dim3 grid((unsigned)((ext_c + 63) / 64), (unsigned)((ext_r + 63) / 64));
  const int r = (int)rows, c = (int)cols, p = (int)pitch;
  if (transpose && x_dtype == TG_DTYPE_BF16 && cols % 8 == 0 && pitch % 8 == 0 &&
      (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(y) & 15) == 0) {
    const dim3 g128((unsigned)((cols + 127) / 128), (unsigned)((pitch + 127) / 128));
    auto X = reinterpret_cast<const uint4*>(x);
    auto Y = reinterpret_cast<uint16_t*>(y);
    if ((uint64_t)cols * (uint64_t)pitch * 2 > (256ull << 20))   // larger than the Infinity Cache
      hipLaunchKernelGGL(pack_bf16_t128_kernel<true>, g128, dim3(256), 0, st, X, Y, r, c, p);
    else
      hipLaunchKernelGGL(pack_bf16_t128_kernel<false>, g128, dim3(256), 0, st, X, Y, r, c, p);
    return check_launch("pack_bf16_t128");
  }
  if (x_dtype == TG_DTYPE_F32) {
    if (transpose) hipLaunchKernelGGL((pack_bf16_kernel<true, true>), grid, dim3(256), 0, st, x, y, r, c, p);
    else hipLaunchKernelGGL((pack_bf16_kernel<true, false>), grid, dim3(256), 0, st, x, y, r, c, p);
  } else {
    if (transpose) hipLaunchKernelGGL((pack_bf16_kernel<false, true>), grid, dim3(256), 0, st, x, y, r, c, p);
    else hipLaunchKernelGGL((pack_bf16_kernel<false, false>), grid, dim3(256), 0, st, x, y, r, c, p);
  }
  return check_launch("pack_bf16");
}

__global__ void fill_zero_u16_kernel(uint16_t* __restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0;
}

int launch_fill_zero_bf16(void* p, int64_t n, hipStream_t st) {
  if (n == 0) return TG_OK;
  const int64_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(fill_zero_u16_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0,
                     st, reinterpret_cast<uint16_t*>(p), n);
  return check_launch("fill_zero_bf16");
}

// C (M, N) = A^T B, A (Kc, M) pitch lda, B (Kc, N) pitch ldb (gemm_bf16_tn_q4_kernel)
int launch_gemm_bf16_tn(const __bf16* a, int64_t lda, const __bf16* b, int64_t ldb, __bf16* c, int64_t M,
                        int64_t N, int64_t Kc, hipStream_t st) {
  if (M == 0 || N == 0) return TG_OK;
  const int tiles_m = (int)((M + 255) / 256), tiles_n = (int)((N + 255) / 256);
  hipLaunchKernelGGL(gemm_bf16_tn_q4_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, st, a, b, c,
                     (int)M, (int)N, (int)Kc, (int)lda, (int)ldb, tiles_m, tiles_n);
  return check_launch("gemm_bf16_tn_256");
}

int launch_gemm_bf16(const __bf16* a, const __bf16* b, __bf16* c, int64_t M, int64_t N, int64_t K,
                     hipStream_t st) {
  if (M == 0 || N == 0) return TG_OK;
  const int tiles_m = (int)((M + 255) / 256), tiles_n = (int)((N + 255) / 256);
  hipLaunchKernelGGL(gemm_bf16_nt_q4_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, st,
                     a, b, c, (int)M, (int)N, (int)K, tiles_m, tiles_n);
  return check_launch("gemm_bf16_nt_256");
}

}  // namespace tg

using namespace tg;

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
static inline int64_t round64(int64_t x) { return (x + 63) & ~(int64_t)63; }

static int check_bf16_gemm(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K <= 0) return einval("bad GEMM shape");
  if (K % 64) return einval("gemm_bf16_nt: K must be a multiple of 64");
  // buffer offsets are 32-bit: each operand must stay below 2 GiB
  if ((uint64_t)M * (uint64_t)K * 2 >= (1ull << 31) || (uint64_t)N * (uint64_t)K * 2 >= (1ull << 31))
    return einval("gemm_bf16_nt: operand larger than 2 GiB");
  if (M > 0x7FFFFFFF || N > 0x7FFFFFFF) return einval("GEMM dimension too large");
  return TG_OK;
}

extern "C" int tg_gemm_bf16_nt(const void* a, const void* b, void* c, int64_t M, int64_t N,
                               int64_t K, void* stream) {
  TG_TRY(check_bf16_gemm(M, N, K));
  if (M == 0 || N == 0) return TG_OK;
  if (!a || !b || !c) return einval("gemm_bf16_nt: null pointer");
  if (!aligned(a, 16) || !aligned(b, 16)) return einval("gemm_bf16_nt: operands must be 16-byte aligned");
  return launch_gemm_bf16(reinterpret_cast<const __bf16*>(a), reinterpret_cast<const __bf16*>(b),
                          reinterpret_cast<__bf16*>(c), M, N, K, as_stream(stream));
}

extern "C" int tg_pack_bf16(const void* x, int x_dtype, int64_t rows, int64_t cols, int transpose,
                            void* y, int64_t pitch, void* stream) {
  if (x_dtype != TG_DTYPE_BF16 && x_dtype != TG_DTYPE_F32) return einval("pack_bf16: bad x_dtype");
  if (rows < 0 || cols < 0 || rows > 0x7FFFFFFF || cols > 0x7FFFFFFF) return einval("pack_bf16: bad shape");
  if (pitch < (transpose ? rows : cols) || pitch > 0x7FFFFFFF) return einval("pack_bf16: pitch too small");
  if (rows == 0 || cols == 0) return TG_OK;
  if (!x || !y) return einval("pack_bf16: null pointer");
  if ((transpose ? pitch : rows) > 65535LL * 64) return einval("pack_bf16: too many rows");
  return launch_pack_bf16(x, x_dtype, rows, cols, transpose, reinterpret_cast<__bf16*>(y), pitch,
                          as_stream(stream));
}

extern "C" size_t tg_block_scaled_matmul_bwd_bf16_workspace(int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0) return 0;
  const size_t np = (size_t)round64(N), mp = (size_t)round64(M);
  return align256((size_t)M * np * 2) + align256((size_t)K * np * 2) +   // g, b packed along N
         align256((size_t)K * mp * 2) + align256((size_t)N * mp * 2);    // a.T, g.T packed along M
}

extern "C" int tg_block_scaled_matmul_bwd_bf16(const void* a, int a_dtype, const void* b,
                                               int b_dtype, const void* g, int g_dtype, void* da,
                                               void* db, int64_t M, int64_t N, int64_t K,
                                               void* workspace, size_t workspace_bytes,
                                               void* stream) {
  for (int d : {a_dtype, b_dtype, g_dtype})
    if (d != TG_DTYPE_BF16 && d != TG_DTYPE_F32) return einval("block_scaled_matmul_bwd_bf16: bad dtype");
  if (M < 0 || N < 0 || K < 0) return einval("block_scaled_matmul_bwd_bf16: bad shape");
  if (M == 0 || N == 0 || K == 0) {
    // an empty contraction gives zero gradients; an empty output is a no-op
    if ((M * K && !da) || (K * N && !db)) return einval("block_scaled_matmul_bwd_bf16: null pointer");
    TG_TRY(launch_fill_zero_bf16(da, M * K, as_stream(stream)));
    return launch_fill_zero_bf16(db, K * N, as_stream(stream));
  }
  const int64_t np = round64(N), mp = round64(M);
  TG_TRY(check_bf16_gemm(M, K, np));    // dX = g . b.T   contracts N
  TG_TRY(check_bf16_gemm(K, N, mp));    // dW = a.T . g   contracts M
  if (!a || !b || !g || !da || !db || !workspace) return einval("block_scaled_matmul_bwd_bf16: null pointer");
  if (workspace_bytes < tg_block_scaled_matmul_bwd_bf16_workspace(M, N, K))
    return einval("block_scaled_matmul_bwd_bf16: workspace too small");
  if (!aligned(workspace, 256)) return einval("block_scaled_matmul_bwd_bf16: workspace must be 256-byte aligned");
  hipStream_t st = as_stream(stream);
  uint8_t* p = reinterpret_cast<uint8_t*>(workspace);
  __bf16* gp = reinterpret_cast<__bf16*>(p);   p += align256((size_t)M * np * 2);
  __bf16* bp = reinterpret_cast<__bf16*>(p);   p += align256((size_t)K * np * 2);
  __bf16* at = reinterpret_cast<__bf16*>(p);   p += align256((size_t)K * mp * 2);
  __bf16* gt = reinterpret_cast<__bf16*>(p);
  // dX operands: used in place when already bf16, 64-aligned along N and 16-byte aligned
  const __bf16* gx = reinterpret_cast<const __bf16*>(g);
  const __bf16* bx = reinterpret_cast<const __bf16*>(b);
  if (g_dtype != TG_DTYPE_BF16 || np != N || !aligned(g, 16)) {
    TG_TRY(launch_pack_bf16(g, g_dtype, M, N, 0, gp, np, st));
    gx = gp;
  }
  if (b_dtype != TG_DTYPE_BF16 || np != N || !aligned(b, 16)) {
    TG_TRY(launch_pack_bf16(b, b_dtype, K, N, 0, bp, np, st));
    bx = bp;
  }
  TG_TRY(launch_gemm_bf16(gx, bx, reinterpret_cast<__bf16*>(da), M, K, np, st));   // fp8.py:95
  if (a_dtype == TG_DTYPE_BF16 && g_dtype == TG_DTYPE_BF16 && K % 8 == 0 && N % 8 == 0 && aligned(a, 16) &&
      aligned(g, 16))
    // db = a.T . g read straight from a and g (contraction-major operands)
    return launch_gemm_bf16_tn(reinterpret_cast<const __bf16*>(a), K, reinterpret_cast<const __bf16*>(g), N,
                               reinterpret_cast<__bf16*>(db), K, N, M, st);                // fp8.py:96
  TG_TRY(launch_pack_bf16(a, a_dtype, M, K, 1, at, mp, st));
  TG_TRY(launch_pack_bf16(g, g_dtype, M, N, 1, gt, mp, st));
  return launch_gemm_bf16(at, gt, reinterpret_cast<__bf16*>(db), K, N, mp, st);      // fp8.py:96
}
