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
//   * Workgroup tile 256 x 256 x 64 (128 bytes of every row per K step, the
//     same LDS geometry as the FP8 kernel), 8 waves as 4 (M) x 2 (N), wave
//     tile 64 x 128 = 4 x 8 MFMA tiles, 128 fp32 accumulators per lane.
//   * Operands travel HBM -> LDS by buffer_load ... lds into two stages (one
//     barrier per K step); every wave issues 1/8 of the next stage, one
//     1 KiB part per compute region.
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

__shared__ __attribute__((aligned(16))) uint8_t h256_a0[256 * 128];
__shared__ __attribute__((aligned(16))) uint8_t h256_b0[256 * 128];
__shared__ __attribute__((aligned(16))) uint8_t h256_a1[256 * 128];
__shared__ __attribute__((aligned(16))) uint8_t h256_b1[256 * 128];

template <int S> __device__ __forceinline__ uint8_t* h256_a() { return S ? h256_a1 : h256_a0; }
template <int S> __device__ __forceinline__ uint8_t* h256_b() { return S ? h256_b1 : h256_b0; }

struct H256Ctx {
  __amdgpu_buffer_rsrc_t ra, rb;
  uint32_t voa[2], vob[2];    // per-lane byte offsets (k step 0) for even / odd u
  uint32_t row8;              // 8 rows in bytes
  int wave, nks;
  uint32_t fa0, fa1, fb0, fb1;   // LDS byte offsets of this lane's fragment chunks
};

// One K step is 64 parts of 1 KiB (8 rows x 128 B): wave w issues parts 0-3
// for A rows 32w .. 32w+31 and parts 4-7 for the same B rows.
__device__ __forceinline__ void h256_issue_part(const H256Ctx& c, uint8_t* la, uint8_t* lb, int ks,
                                                int part) {
  const uint32_t sofs = (uint32_t)ks * 128u + (uint32_t)(part & 3) * c.row8;
  const int u = part & 3;
  if (part < 4)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.ra, la + c.wave * 4096 + u * 1024, 16, c.voa[u & 1],
                                             sofs, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rb, lb + c.wave * 4096 + u * 1024, 16, c.vob[u & 1],
                                             sofs, 0, 0);
}

template <int S>
__device__ __forceinline__ void h256_compute(const H256Ctx& c, v4f (&acc)[4][8], int ks_next) {
  const uint8_t* la = h256_a<S>();
  const uint8_t* lb = h256_b<S>();
  uint4 a0[4], a1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a0[i] = *reinterpret_cast<const uint4*>(la + c.fa0 + i * 2048);
    a1[i] = *reinterpret_cast<const uint4*>(la + c.fa1 + i * 2048);
  }
  uint4 b0 = *reinterpret_cast<const uint4*>(lb + c.fb0);
  uint4 b1 = *reinterpret_cast<const uint4*>(lb + c.fb1);
  const bool pf = ks_next < c.nks;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint4 cb0 = b0, cb1 = b1;
    if (j + 1 < 8) {   // next region's B fragment one region ahead
      b0 = *reinterpret_cast<const uint4*>(lb + c.fb0 + (j + 1) * 2048);
      b1 = *reinterpret_cast<const uint4*>(lb + c.fb1 + (j + 1) * 2048);
    }
    if (pf) h256_issue_part(c, h256_a<S ^ 1>(), h256_b<S ^ 1>(), ks_next, j);
    // lo halves of all four tiles, then hi halves: dependent MFMAs on one
    // accumulator are four instructions apart
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16_16x16x32(a0[i], cb0, acc[i][j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i][j] = mfma_bf16_16x16x32(a1[i], cb1, acc[i][j]);
  }
}

template <int S>
__device__ __forceinline__ void h256_step(const H256Ctx& c, int ks, v4f (&acc)[4][8]) {
  h256_compute<S>(c, acc, ks + 1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// C[M, N] = bf16(A[M, K] . B[N, K]^T); K % 64 == 0, K-contiguous rows.
__global__ __launch_bounds__(512, 1) void gemm_bf16_nt_256_kernel(const __bf16* __restrict__ A,
                                                                  const __bf16* __restrict__ B,
                                                                  __bf16* __restrict__ C, int M,
                                                                  int N, int K, int tiles_m,
                                                                  int tiles_n) {
  H256Ctx c;
  const int tid = threadIdx.x, lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  c.nks = K >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const int wm = c.wave >> 1, wn = c.wave & 1;
  int tmi, tni;
  tile_of(blockIdx.x, tiles_m, tiles_n, tmi, tni);
  const int m0 = tmi * 256, n0 = tni * 256;
  const uint32_t rowb = 2u * (uint32_t)K;   // row pitch in bytes
  c.ra = make_rsrc(A, (uint32_t)M * rowb);
  c.rb = make_rsrc(B, (uint32_t)N * rowb);
  c.row8 = 8u * rowb;
  // loader rows wave*32 + u*8 + lane/8; physical chunk lane%8 holds logical
  // chunk (lane%8) ^ swz(row), which depends on lane/8 and the parity of u
  const int lrow = c.wave * 32 + (lane >> 3);
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int lch = (lane & 7) ^ g256_swz(lrow + par * 8);
    c.voa[par] = (uint32_t)(m0 + lrow) * rowb + lch * 16;
    c.vob[par] = (uint32_t)(n0 + lrow) * rowb + lch * 16;
  }
  // fragments: lane (fr, fg) reads logical chunks fg and fg + 4 of row
  // (wave tile row) + 16t + fr (k elements 8fg .. 8fg+7 and 32+8fg ..
  // 32+8fg+7 of the step; A and B lanes agree).  Chunk pairs {2fg, 2fg + 1}
  // make the four lane groups of a read collide in LDS (~30% slower reads).
  const uint32_t ch0 = (uint32_t)(fg ^ g256_swz(fr)) * 16u;
  c.fa0 = (uint32_t)(wm * 64 + fr) * 128u + ch0;
  c.fa1 = c.fa0 ^ 64u;
  c.fb0 = (uint32_t)(wn * 128 + fr) * 128u + ch0;
  c.fb1 = c.fb0 ^ 64u;

  v4f acc[4][8];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int p = 0; p < 8; ++p) h256_issue_part(c, h256_a0, h256_b0, 0, p);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  int ks = 0;
  for (; ks + 1 < c.nks; ks += 2) {
    h256_step<0>(c, ks, acc);
    h256_step<1>(c, ks + 1, acc);
  }
  if (ks < c.nks) h256_step<0>(c, ks, acc);

  // bf16 epilogue through LDS: each wave stages its 64 x 128 tile as two
  // 32-row halves of 256 B rows, then stores 16 bytes per lane.
  uint8_t* ep = (c.wave < 4 ? h256_a0 + c.wave * 8192 : h256_b0 + (c.wave - 4) * 8192);
  uint8_t* ep2 = (c.wave < 4 ? h256_a1 + c.wave * 8192 : h256_b1 + (c.wave - 4) * 8192);
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = i * 16 + 4 * fg + r, col = j * 16 + fr;
        uint8_t* base = row < 32 ? ep : ep2;
        *reinterpret_cast<__bf16*>(base + (row & 31) * 256 + col * 2) = (__bf16)acc[i][j][r];
      }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const bool vec_ok = (N % 8) == 0;
#pragma unroll
  for (int t = 0; t < 16; ++t) {
    const int row = t * 4 + (lane >> 4), chunk = lane & 15;
    const uint8_t* base = row < 32 ? ep : ep2;
    const uint4 v = *reinterpret_cast<const uint4*>(base + (row & 31) * 256 + chunk * 16);
    const int m = m0 + wm * 64 + row, n = n0 + wn * 128 + chunk * 8;
    if (m < M) {
      __bf16* dst = C + (int64_t)m * N + n;
      if (vec_ok && n + 8 <= N) {
        *reinterpret_cast<uint4*>(dst) = v;
      } else {
        const uint16_t* e = reinterpret_cast<const uint16_t*>(&v);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          if (n + k < N) reinterpret_cast<uint16_t*>(dst)[k] = e[k];
      }
    }
  }
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

int launch_gemm_bf16(const __bf16* a, const __bf16* b, __bf16* c, int64_t M, int64_t N, int64_t K,
                     hipStream_t st) {
  if (M == 0 || N == 0) return TG_OK;
  const int tiles_m = (int)((M + 255) / 256), tiles_n = (int)((N + 255) / 256);
  hipLaunchKernelGGL(gemm_bf16_nt_256_kernel, dim3((unsigned)(tiles_m * tiles_n)), dim3(512), 0, st,
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
  TG_TRY(launch_pack_bf16(a, a_dtype, M, K, 1, at, mp, st));
  TG_TRY(launch_pack_bf16(g, g_dtype, M, N, 1, gt, mp, st));
  return launch_gemm_bf16(at, gt, reinterpret_cast<__bf16*>(db), K, N, mp, st);      // fp8.py:96
}
