// Block-scaled FP8 for any block_k that divides the contracted extent: the
// reference's block_scaled_matmul takes block_k as an argument
// (/root/reference/fp8.py:30-36, 55-56), while the tuned kernels of this
// library fix it at 128 (one scale block per FP8 MFMA K step pair).  These
// kernels are the general path the C ABI takes for every other block size.
// They follow the same numeric contract as the 128 path, written per element:
//   scale = max(amax / 448, 1e-30)  (IEEE divide; amax NaN-propagating)
//   q     = e4m3fn(x / scale)       (IEEE divide, RNE; the non-finite-scale
//                                    rule of e4m3_nonfinite_scale)
// so a block's bytes and scale are those the 128 kernels give for the same
// block, and the GEMM forms each block's partial dot product P as an f32 fma
// chain in k order (which rounds once the block's products span more than
// f32's 24 bits) and adds it as acc = fma(P, sa * sb, acc) in block order
// (fp8.py:70-76), in f32 on the VALU.
// The quantizers: for bf16 x with bk % 16 == 0 one lane per 16-byte chunk
// (rows, bk <= 512) and LDS-transposed tiles (columns, bk <= 1024); otherwise
// one thread per block.  The GEMM for sizes the tuned kernels cannot take
// (block sizes not a multiple or divisor of 128) is a 64 x 64 LDS-tiled VALU
// GEMM.
#include <mutex>

#include "tg_device.h"
#include "tg_host.h"

namespace tg {

__device__ __forceinline__ float gb_load(const void* x, int64_t i, bool f32) {
  return f32 ? reinterpret_cast<const float*>(x)[i]
             : __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(x)[i] << 16);
}

// e4m3fn byte of x / s
__device__ __forceinline__ uint8_t gb_quant1(float x, float s, bool finite_scale) {
  return (uint8_t)(finite_scale ? (e4m3x4(x / s, 0.0f, 0.0f, 0.0f) & 0xFFu) : e4m3_nonfinite_scale(x, s));
}

__device__ __forceinline__ bool gb_finite(float s) { return (__float_as_uint(s) & 0x7F800000u) != 0x7F800000u; }

// Index of scale copy t of block b of output row r (srep copies per block):
// row-major (r, b * srep + t), or K-block-major (b * srep + t, r) with skm,
// the layout of the tuned GEMM's _km entry points.
__device__ __forceinline__ int64_t gb_sidx(bool skm, int64_t r, int64_t b, int t, int64_t nrows, int64_t nb,
                                           int srep) {
  return skm ? (b * srep + t) * nrows + r : (r * nb + b) * srep + t;
}

// one thread per (row, block): q (rows, cols * pf), s (rows, cols / bk * srep).
// Two layouts for the tuned GEMM: each block's scale written srep times
// (srep = bk / 128: 128-wide blocks that share their scale), or each block's
// bytes at the start of a 128-byte slot followed by zeros (pf = 128 / bk: one
// block per 128-wide block, the zeros adding nothing to any product).
template <bool F32_IN>
__global__ __launch_bounds__(256) void quant_rows_gb_kernel(const void* __restrict__ x, int64_t rows,
                                                            int64_t cols, int bk, uint8_t* __restrict__ q,
                                                            float* __restrict__ s, int srep, int pf, bool skm) {
  const int64_t nb = cols / bk;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * nb) return;
  const int64_t r = i / nb, b = i - r * nb;
  const int64_t base = r * cols + b * bk;
  uint32_t m = 0;
  for (int k = 0; k < bk; ++k) m = max(m, __float_as_uint(gb_load(x, base + k, F32_IN)) & 0x7FFFFFFFu);
  const float sc = block_scale(m);
  for (int t = 0; t < srep; ++t) s[gb_sidx(skm, r, b, t, rows, nb, srep)] = sc;
  const bool fin = gb_finite(sc);
  uint8_t* qo = q + base * pf;
  for (int k = 0; k < bk; ++k) qo[k] = gb_quant1(gb_load(x, base + k, F32_IN), sc, fin);
  for (int k = bk; k < bk * pf; ++k) qo[k] = 0;
}

// four e4m3fn bytes of (a, b, c, d) / s, packed little-endian
__device__ __forceinline__ uint32_t gb_quant4(float a, float b, float c, float d, float s, bool finite_scale) {
  if (finite_scale) return e4m3x4(a / s, b / s, c / s, d / s);
  return e4m3_nonfinite_scale(a, s) | (e4m3_nonfinite_scale(b, s) << 8) | (e4m3_nonfinite_scale(c, s) << 16) |
         (e4m3_nonfinite_scale(d, s) << 24);
}
__device__ __forceinline__ uint32_t gb_quant4_bf16(uint32_t lo, uint32_t hi, float s, bool fin) {
  return gb_quant4(bf16lo(lo), bf16hi(lo), bf16lo(hi), bf16hi(hi), s, fin);
}

// The same for bf16 x, bk % 16 == 0, x and q 16-byte aligned: 16-byte loads
// and stores (a thread's block is contiguous in x and in q).
__global__ __launch_bounds__(256) void quant_rows_gb16_kernel(const uint16_t* __restrict__ x, int64_t rows,
                                                              int64_t cols, int bk, uint8_t* __restrict__ q,
                                                              float* __restrict__ s, int srep, int pf, bool skm) {
  const int64_t nb = cols / bk;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * nb) return;
  const int64_t r = i / nb, b = i - r * nb;
  const int64_t base = r * cols + b * bk;
  const uint4* xv = reinterpret_cast<const uint4*>(x + base);
  uint32_t m = 0;
  for (int k = 0; k < bk / 8; ++k) {
    const uint4 v = xv[k];
    m = max(max(max(m, bf16_amax2(v.x)), bf16_amax2(v.y)), max(bf16_amax2(v.z), bf16_amax2(v.w)));
  }
  const float sc = block_scale(m);
  for (int t = 0; t < srep; ++t) s[gb_sidx(skm, r, b, t, rows, nb, srep)] = sc;
  const bool fin = gb_finite(sc);
  uint4* qo = reinterpret_cast<uint4*>(q + base * pf);
  for (int k = 0; k < bk / 16; ++k) {
    const uint4 u = xv[2 * k], v = xv[2 * k + 1];
    qo[k] = make_uint4(gb_quant4_bf16(u.x, u.y, sc, fin), gb_quant4_bf16(u.z, u.w, sc, fin),
                       gb_quant4_bf16(v.x, v.y, sc, fin), gb_quant4_bf16(v.z, v.w, sc, fin));
  }
  for (int k = bk / 16; k < bk * pf / 16; ++k) qo[k] = make_uint4(0u, 0u, 0u, 0u);
}

// x (R, C) bf16 or f32 -> the quantization of x.T along R: q_t (C, R),
// s_t (C, R / bk); one thread per (row block, column), columns fastest
// (coalesced reads of x)
template <bool VEC, bool F32_IN>
__global__ __launch_bounds__(256) void quant_cols_gb_kernel(const void* __restrict__ x, int64_t R, int64_t C,
                                                            int bk, uint8_t* __restrict__ qt,
                                                            float* __restrict__ st, int srep, int pf, bool skm) {
  const int64_t nb = R / bk;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= nb * C) return;
  const int64_t b = i / C, c = i - b * C;
  const int64_t r0 = b * bk;
  auto xf = [&](int k) { return gb_load(x, (r0 + k) * C + c, F32_IN); };
  uint32_t m = 0;
  for (int k = 0; k < bk; ++k) m = max(m, __float_as_uint(xf(k)) & 0x7FFFFFFFu);
  const float sc = block_scale(m);
  for (int t = 0; t < srep; ++t) st[gb_sidx(skm, c, b, t, C, nb, srep)] = sc;
  const bool fin = gb_finite(sc);
  uint8_t* qo = qt + (c * R + r0) * pf;
  if (VEC) {   // bk % 16 == 0, q_t 16-byte aligned: a thread's bytes in 16-byte stores
    uint4* qv = reinterpret_cast<uint4*>(qo);
    for (int k = 0; k < bk; k += 16) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = gb_quant4(xf(k + 4 * j), xf(k + 4 * j + 1), xf(k + 4 * j + 2), xf(k + 4 * j + 3), sc, fin);
      qv[k / 16] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    for (int k = bk / 16; k < bk * pf / 16; ++k) qv[k] = make_uint4(0u, 0u, 0u, 0u);
    return;
  }
  for (int k = 0; k < bk; ++k) qo[k] = gb_quant1(xf(k), sc, fin);
  for (int k = bk; k < bk * pf; ++k) qo[k] = 0;
}

// Wave-cooperative forms of the two quantizers for bf16 x and bk % 16 == 0,
// with the bytes and scales of the one-thread-per-block kernels above (same
// scale and quotient functions).
//
// Rows, bk <= 512: one 16-byte chunk (8 elements) per lane; the L = bk / 8
// lanes of a block are an aligned lane group (a block's first chunk index is
// a multiple of L, since cols % bk == 0), which reduces the block's amax by
// xor shuffles.  Each lane stores its 8 bytes, and the zeros of its column
// of the block's 128-byte slot when pf > 1.
template <int L>
__global__ __launch_bounds__(256) void quant_rows_gbw_kernel(const uint16_t* __restrict__ x, int64_t nchunks,
                                                             int64_t cols, int bk, uint8_t* __restrict__ q,
                                                             float* __restrict__ s, int srep, int pf, bool skm) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const bool in = i < nchunks;                       // whole lane groups are in or out
  const uint4 v = in ? *reinterpret_cast<const uint4*>(x + i * 8) : make_uint4(0u, 0u, 0u, 0u);
  uint32_t m = max(max(bf16_amax2(v.x), bf16_amax2(v.y)), max(bf16_amax2(v.z), bf16_amax2(v.w)));
#pragma unroll
  for (int o = L / 2; o >= 1; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o));
  if (!in) return;
  const float sc = block_scale(m);
  const int64_t e = i * 8, r = e / cols, col = e - r * cols, b = col / bk, within = col - b * bk;
  if (within == 0)
    for (int t = 0; t < srep; ++t) s[gb_sidx(skm, r, b, t, nchunks * 8 / cols, cols / bk, srep)] = sc;
  const bool fin = gb_finite(sc);
  uint8_t* qo = q + (r * cols + b * bk) * pf + within;
  *reinterpret_cast<uint2*>(qo) = make_uint2(gb_quant4_bf16(v.x, v.y, sc, fin), gb_quant4_bf16(v.z, v.w, sc, fin));
  for (int j = 1; j < pf; ++j) *reinterpret_cast<uint2*>(qo + j * bk) = make_uint2(0u, 0u);
}

// Columns (x.T along R), bk <= 1024: a workgroup takes one row block (bk rows)
// x 64 columns.  It copies the tile to LDS with coalesced 16-byte loads (row
// pitch 144 B) and keeps per-thread column maxima, reduces them to the 64
// column scales, then each lane quantizes its column's bytes 16 rows at a time
// from LDS and stores them as 16-byte pieces of q_t's row.
constexpr int kGbtPitch = 64 * 2 + 16;
__global__ __launch_bounds__(256) void quant_cols_gbt_kernel(const uint16_t* __restrict__ x, int64_t R, int64_t C,
                                                             int bk, uint8_t* __restrict__ qt,
                                                             float* __restrict__ st, int srep, int pf, bool skm) {
  extern __shared__ __attribute__((aligned(16))) uint8_t gbt_lds[];
  uint32_t* pam = reinterpret_cast<uint32_t*>(gbt_lds + (size_t)bk * kGbtPitch);   // [32][64] partial maxima
  __shared__ float scol[64];
  const int tid = threadIdx.x, ch = tid & 7, rg = tid >> 3;
  const int64_t c0 = (int64_t)blockIdx.x * 64, r0 = (int64_t)blockIdx.y * bk;
  const bool cin = c0 + ch * 8 < C;                   // C % 8 == 0: a chunk is in or out
  uint32_t m[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  for (int r = rg; r < bk; r += 32) {
    const uint4 v = cin ? *reinterpret_cast<const uint4*>(x + (r0 + r) * C + c0 + ch * 8) : make_uint4(0u, 0u, 0u, 0u);
    *reinterpret_cast<uint4*>(gbt_lds + r * kGbtPitch + ch * 16) = v;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      m[2 * k] = max(m[2 * k], (w[k] << 16) & 0x7FFFFFFFu);
      m[2 * k + 1] = max(m[2 * k + 1], w[k] & 0x7FFF0000u);
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) pam[rg * 64 + ch * 8 + k] = m[k];
  __syncthreads();
  const int64_t nb = R / bk, b = blockIdx.y;
  if (tid < 64) {
    uint32_t a = 0u;
    for (int g = 0; g < 32; ++g) a = max(a, pam[g * 64 + tid]);
    const float sc = block_scale(a);
    scol[tid] = sc;
    if (c0 + tid < C)
      for (int t = 0; t < srep; ++t) st[gb_sidx(skm, c0 + tid, b, t, C, nb, srep)] = sc;
  }
  __syncthreads();
  const int lane = tid & 63, wv = tid >> 6;
  const int64_t c = c0 + lane;
  if (c >= C) return;
  const float sc = scol[lane];
  const bool fin = gb_finite(sc);
  uint8_t* qo = qt + (c * R + r0) * pf;
  for (int p = wv; p < bk / 16; p += 4) {
    float f[16];
#pragma unroll
    for (int k = 0; k < 16; ++k)
      f[k] = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(gbt_lds + (p * 16 + k) * kGbtPitch +
                                                                          lane * 2) << 16);
    *reinterpret_cast<uint4*>(qo + p * 16) =
        make_uint4(gb_quant4(f[0], f[1], f[2], f[3], sc, fin), gb_quant4(f[4], f[5], f[6], f[7], sc, fin),
                   gb_quant4(f[8], f[9], f[10], f[11], sc, fin), gb_quant4(f[12], f[13], f[14], f[15], sc, fin));
  }
  for (int p = bk / 16 + wv; p < bk * pf / 16; p += 4) *reinterpret_cast<uint4*>(qo + p * 16) = make_uint4(0u, 0u, 0u, 0u);
}

// C (M, N) = sum over K blocks b of (A_b . B_b^T) * sa[m][b] * sb[n / bn][b];
// A (M, K), B (N, K) e4m3fn bytes.  Workgroup tile 64 x 64, thread (tx, ty)
// owns rows 4 ty .. +3 and columns 4 tx .. +3.  K walks in 32-byte chunks
// staged through LDS transposed ([k][row], so a thread's 4 rows at one k are
// one 32-bit read); the block's partial sums P run in k order and are folded
// into the accumulator at each block end.
constexpr int kGbTile = 64, kGbKc = 32, kGbPitch = kGbTile + 4;

template <bool OUT_F32>
__global__ __launch_bounds__(256) void gemm_gb_kernel(const uint8_t* __restrict__ A, const float* __restrict__ SA,
                                                      const uint8_t* __restrict__ B, const float* __restrict__ SB,
                                                      int bn, void* __restrict__ Cout, int M, int N, int K,
                                                      int bk) {
  __shared__ __attribute__((aligned(16))) uint8_t at[kGbKc][kGbPitch];
  __shared__ __attribute__((aligned(16))) uint8_t bt[kGbKc][kGbPitch];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int m0 = blockIdx.y * kGbTile, n0 = blockIdx.x * kGbTile;
  const int nb = K / bk;
  const int nsb_rows = (N + bn - 1) / bn;
  // chunk loader: thread t copies 8 bytes of row t / 4 (bytes 8 (t % 4) ..)
  const int lr = tid >> 2, lk = (tid & 3) * 8;
  float acc[4][4], P[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = P[i][j] = 0.0f;
  int kin = 0, blk = 0;   // position inside the current K block, its index
  for (int k0 = 0; k0 < K; k0 += kGbKc) {
    __syncthreads();   // the previous chunk is read by every thread
    {
      const int ma = m0 + lr, nbr = n0 + lr;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int k = k0 + lk + e;
        at[lk + e][lr] = (ma < M && k < K) ? A[(int64_t)ma * K + k] : (uint8_t)0;
        bt[lk + e][lr] = (nbr < N && k < K) ? B[(int64_t)nbr * K + k] : (uint8_t)0;
      }
    }
    __syncthreads();
    const int kn = K - k0 < kGbKc ? K - k0 : kGbKc;
    for (int kk = 0; kk < kn; ++kk) {
      const uint32_t a4 = *reinterpret_cast<const uint32_t*>(&at[kk][ty * 4]);
      const uint32_t b4 = *reinterpret_cast<const uint32_t*>(&bt[kk][tx * 4]);
      typedef float v2f_t __attribute__((ext_vector_type(2)));
      const v2f_t a01 = __builtin_amdgcn_cvt_pk_f32_fp8(a4, false), a23 = __builtin_amdgcn_cvt_pk_f32_fp8(a4, true);
      const v2f_t b01 = __builtin_amdgcn_cvt_pk_f32_fp8(b4, false), b23 = __builtin_amdgcn_cvt_pk_f32_fp8(b4, true);
      const float av[4] = {a01.x, a01.y, a23.x, a23.y}, bv[4] = {b01.x, b01.y, b23.x, b23.y};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) P[i][j] = __builtin_fmaf(av[i], bv[j], P[i][j]);
      if (++kin == bk) {   // block end (uniform over the workgroup)
        float sa[4], sb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + ty * 4 + i;
          sa[i] = m < M ? SA[(int64_t)m * nb + blk] : 0.0f;
          const int n = n0 + tx * 4 + i;
          const int sr = n < N ? n / bn : 0;
          sb[i] = n < N && sr < nsb_rows ? SB[(int64_t)sr * nb + blk] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[i][j] = __builtin_fmaf(P[i][j], sa[i] * sb[j], acc[i][j]);
            P[i][j] = 0.0f;
          }
        kin = 0;
        ++blk;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int m = m0 + ty * 4 + i;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int n = n0 + tx * 4 + j;
      if (n >= N) continue;
      if (OUT_F32) reinterpret_cast<float*>(Cout)[(int64_t)m * N + n] = acc[i][j];
      else reinterpret_cast<uint16_t*>(Cout)[(int64_t)m * N + n] = (uint16_t)pack_bf16x2(acc[i][j], 0.0f);
    }
  }
}

static unsigned gb_grid(int64_t threads) { return (unsigned)((threads + 255) / 256); }

int launch_quant_rows_gb(const void* x, int x_dtype, int64_t rows, int64_t cols, int bk, uint8_t* q, float* s,
                         hipStream_t st, int srep, int pf, bool skm) {
  const int64_t n = rows * (cols / bk);
  if (n == 0) return TG_OK;
  if (n / 256 >= 0x7FFFFFFF) return einval("quantize_rows: too many blocks");
  const bool vec = bk % 16 == 0 && ((uintptr_t)x & 15) == 0 && ((uintptr_t)q & 15) == 0;
  if (x_dtype != TG_DTYPE_F32 && vec && bk <= 512 && (bk & (bk - 1)) == 0) {
    const int64_t nchunks = rows * cols / 8;
    if (nchunks / 256 >= 0x7FFFFFFF) return einval("quantize_rows: too many blocks");
    auto go = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(gb_grid(nchunks)), dim3(256), 0, st, reinterpret_cast<const uint16_t*>(x),
                         nchunks, cols, bk, q, s, srep, pf, skm);
    };
    switch (bk) {
      case 16: go(quant_rows_gbw_kernel<2>); break;
      case 32: go(quant_rows_gbw_kernel<4>); break;
      case 64: go(quant_rows_gbw_kernel<8>); break;
      case 128: go(quant_rows_gbw_kernel<16>); break;
      case 256: go(quant_rows_gbw_kernel<32>); break;
      default: go(quant_rows_gbw_kernel<64>); break;
    }
  } else if (x_dtype != TG_DTYPE_F32 && vec)
    hipLaunchKernelGGL(quant_rows_gb16_kernel, dim3(gb_grid(n)), dim3(256), 0, st,
                       reinterpret_cast<const uint16_t*>(x), rows, cols, bk, q, s, srep, pf, skm);
  else if (x_dtype == TG_DTYPE_F32)
    hipLaunchKernelGGL(quant_rows_gb_kernel<true>, dim3(gb_grid(n)), dim3(256), 0, st, x, rows, cols, bk, q, s,
                       srep, pf, skm);
  else
    hipLaunchKernelGGL(quant_rows_gb_kernel<false>, dim3(gb_grid(n)), dim3(256), 0, st, x, rows, cols, bk, q, s,
                       srep, pf, skm);
  return check_launch("quantize_rows (block_k != 128)");
}

int launch_quant_cols_gb(const void* x, bool x_f32, int64_t rows, int64_t cols, int bk, uint8_t* q_t,
                         float* s_t, hipStream_t st, int srep, int pf, bool skm) {
  const int64_t n = (rows / bk) * cols;
  if (n == 0) return TG_OK;
  if (n / 256 >= 0x7FFFFFFF) return einval("quantize_cols: too many blocks");
  const bool vec = bk % 16 == 0 && ((uintptr_t)q_t & 15) == 0;
  if (!x_f32 && vec && bk <= 1024 && cols % 8 == 0 && ((uintptr_t)x & 15) == 0 && (cols + 63) / 64 <= 0x7FFFFFFF &&
      rows / bk <= 65535) {
    const size_t lds = (size_t)bk * kGbtPitch + 32 * 64 * 4;
    // the dynamic-LDS limit is a per-device function attribute: set once per
    // device, for the largest tile (bk = 1024)
    constexpr int kMaxDev = 64;
    static std::once_flag once[kMaxDev];
    static hipError_t attr_rc[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) dev = 0;
    std::call_once(once[dev], [&] {
      attr_rc[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(quant_cols_gbt_kernel),
                                         hipFuncAttributeMaxDynamicSharedMemorySize,
                                         (int)((size_t)1024 * kGbtPitch + 32 * 64 * 4));
    });
    if (attr_rc[dev] != hipSuccess) {
      set_error("quantize_cols (set LDS size): %s", hipGetErrorString(attr_rc[dev]));
      return TG_EHIP;
    }
    hipLaunchKernelGGL(quant_cols_gbt_kernel, dim3((unsigned)((cols + 63) / 64), (unsigned)(rows / bk)), dim3(256),
                       lds, st, reinterpret_cast<const uint16_t*>(x), rows, cols, bk, q_t, s_t, srep, pf, skm);
    return check_launch("quantize_cols (general, transposed tile)");
  }
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(gb_grid(n)), dim3(256), 0, st, x, rows, cols, bk, q_t, s_t, srep, pf, skm);
  };
  if (x_f32) {
    if (vec) go(quant_cols_gb_kernel<true, true>); else go(quant_cols_gb_kernel<false, true>);
  } else {
    if (vec) go(quant_cols_gb_kernel<true, false>); else go(quant_cols_gb_kernel<false, false>);
  }
  return check_launch("quantize_cols (general)");
}

int launch_gemm_gb(const uint8_t* a_q, const float* a_s, const uint8_t* b_q, const float* b_s, int bn, void* c,
                   int c_dtype, int64_t M, int64_t N, int64_t K, int bk, hipStream_t st) {
  if (M == 0 || N == 0) return TG_OK;
  if ((M + kGbTile - 1) / kGbTile > 65535) return einval("gemm_fp8_nt (block_k != 128): M too large");
  const dim3 grid((unsigned)((N + kGbTile - 1) / kGbTile), (unsigned)((M + kGbTile - 1) / kGbTile));
  if (c_dtype == TG_DTYPE_F32)
    hipLaunchKernelGGL(gemm_gb_kernel<true>, grid, dim3(256), 0, st, a_q, a_s, b_q, b_s, bn, c, (int)M, (int)N,
                       (int)K, bk);
  else
    hipLaunchKernelGGL(gemm_gb_kernel<false>, grid, dim3(256), 0, st, a_q, a_s, b_q, b_s, bn, c, (int)M, (int)N,
                       (int)K, bk);
  return check_launch("gemm_fp8_nt (block_k != 128)");
}

}  // namespace tg
