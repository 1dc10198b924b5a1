// RMSNorm and fused RMSNorm -> FP8 quantize for gfx950 (HBM-bound).
//
// Semantics are _rms_norm_pure (/root/reference/kernels.py:30-33) op by op:
//   var = mean(f32(x)^2)            sum of f32 squares accumulated in f64
//                                   (order-free far below one f32 ulp), rounded
//                                   to f32, divided by D in f32 (jnp.mean)
//   r   = bf16(rsqrt(var + eps))    rsqrt correctly rounded (f64 1/sqrt)
//   y   = bf16(bf16(x * r) * g)     each bf16 x bf16 product is exact in f32
// and the fused variant quantizes the bf16 y exactly as fp8.py:39-47 would
// (what block_scaled_matmul(y, W) does first, fp8.py:66).
//
// One wave64 owns one row at a time.  Lane l holds 16-byte chunks l + 64j, so
// every load instruction of the wave reads 1 KiB of contiguous HBM and a
// 128-element scale block is one 16-lane DPP row.  gamma stays in registers
// while the wave walks rows with a grid stride.  x is read once; y, q and the
// scales are written once.
#include <type_traits>

#include "gemm_tile.h"
#include "row_ops.h"
#include "tg_device.h"
#include "tg_host.h"

namespace tg {

// FULL: every lane owns exactly J chunks of every row (dim == 512 * J), so
// no per-chunk guards are emitted.  Each wave walks rows with a stride of the
// grid's wave count and prefetches the next row's x while it computes the
// current one.
// ADD: the input row is the residual sum x + delta, rounded to bf16 (a bf16
// tensor add) and written to xout (which may be x itself) before the norm.
// y may be null when only the FP8 rows are wanted.
template <int J, bool QUANT, bool FULL, bool ADD = false>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint4* __restrict__ x,
                                                      const uint4* __restrict__ gamma,
                                                      uint4* __restrict__ y,
                                                      uint2* __restrict__ q,
                                                      float* __restrict__ s, int64_t rows,
                                                      int nch, float dimf, float eps,
                                                      const uint4* __restrict__ delta = nullptr,
                                                      uint4* xout = nullptr) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * 4;

  float g[J][8];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = lane + 64 * j;
    uint4 w = (FULL || c < nch) ? gamma[c] : make_uint4(0, 0, 0, 0);
    g[j][0] = bf16lo(w.x); g[j][1] = bf16hi(w.x); g[j][2] = bf16lo(w.y); g[j][3] = bf16hi(w.y);
    g[j][4] = bf16lo(w.z); g[j][5] = bf16hi(w.z); g[j][6] = bf16lo(w.w); g[j][7] = bf16hi(w.w);
  }

  auto load_row = [&](const uint4* src, int64_t row, uint4 (&xv)[J]) {
    const uint4* xr = src + row * nch;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      xv[j] = (FULL || c < nch) ? ldg_stream(xr + c) : make_uint4(0, 0, 0, 0);
    }
  };

  uint4 nxt[J], nd[J];
  if (wave0 < rows) {
    load_row(x, wave0, nxt);
    if (ADD) load_row(delta, wave0, nd);
  }
  for (int64_t row = wave0; row < rows; row += wstride) {
    uint4 cur[J], cd[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      cur[j] = nxt[j];
      cd[j] = ADD ? nd[j] : make_uint4(0, 0, 0, 0);
    }
    if (row + wstride < rows) {                                // prefetch the next row
      load_row(x, row + wstride, nxt);
      if (ADD) load_row(delta, row + wstride, nd);
    }
    uint4 yo[J];
    uint2 qo[J];
    float so[J];
    norm_row<J, QUANT, FULL, ADD>(cur, cd, g, lane, nch, dimf, eps, yo, qo, so);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      if (FULL || c < nch) {
        if (ADD) xout[row * nch + c] = cur[j];   // residual sum in bf16
        if (y) stg_stream(&y[row * nch + c], yo[j]);
        if (QUANT) {
          stg_stream(&q[row * nch + c], qo[j]);
          if ((lane & 15) == 0) s[row * (nch >> 4) + (c >> 4)] = so[j];
        }
      }
    }
  }
}

template <bool QUANT, bool ADD = false>
static int launch_rmsnorm(const void* x, const void* gamma, void* y, uint8_t* q, float* s,
                          int64_t rows, int64_t dim, float eps, hipStream_t st,
                          const void* delta = nullptr, void* xout = nullptr) {
  const int nch = (int)(dim / 8);
  const int jneed = (nch + 63) / 64;
#ifndef TG_NORM_ROWS_PER_WAVE
#define TG_NORM_ROWS_PER_WAVE 2
#endif
  // a few rows per wave so that each wave overlaps the load of the next row
  // with the arithmetic of the current one; at least 2 workgroups per CU
  constexpr int RPW = TG_NORM_ROWS_PER_WAVE;
  int64_t grid = (rows + 4 * RPW - 1) / (4 * RPW);
  if (grid < 512) grid = (rows + 3) / 4 < 512 ? (rows + 3) / 4 : 512;
  if (grid > 16384) grid = 16384;
  const dim3 gdim((unsigned)grid), b(256);
  auto X = reinterpret_cast<const uint4*>(x);
  auto G = reinterpret_cast<const uint4*>(gamma);
  auto Y = reinterpret_cast<uint4*>(y);
  auto Q = reinterpret_cast<uint2*>(q);
  const float dimf = (float)dim;
  auto D = reinterpret_cast<const uint4*>(delta);
  auto XO = reinterpret_cast<uint4*>(xout);
#define TG_NORM_CASE(JJ)                                                                        \
  if (jneed <= JJ) {                                                                             \
    if (nch == JJ * 64)                                                                          \
      hipLaunchKernelGGL((rmsnorm_kernel<JJ, QUANT, true, ADD>), gdim, b, 0, st, X, G, Y, Q, s,  \
                         rows, nch, dimf, eps, D, XO);                                           \
    else                                                                                         \
      hipLaunchKernelGGL((rmsnorm_kernel<JJ, QUANT, false, ADD>), gdim, b, 0, st, X, G, Y, Q, s, \
                         rows, nch, dimf, eps, D, XO);                                           \
    return check_launch("rmsnorm");                                                              \
  }
  TG_NORM_CASE(1)
  TG_NORM_CASE(2)
  TG_NORM_CASE(4)
  TG_NORM_CASE(8)
  TG_NORM_CASE(16)
  TG_NORM_CASE(32)
#undef TG_NORM_CASE
  return einval("rms_norm: dim must be <= 16384");
}

// ---------------------------------------------------------------------------
// Backward of rms_norm: the custom VJP of /root/reference/kernels.py:104-118.
//   rnorm  = rsqrt(mean(x^2) + eps)            (f32, recomputed from x)
//   normed = x * rnorm,  gs = dy * scale
//   dx     = bf16(rnorm * (gs - normed * mean(gs * normed)))
//   dscale = bf16(sum over rows of dy * normed)
// One pass over a row's registers gives both sums (sum x^2 accumulated in
// f64 as in the forward, and sum gs * x, since mean(gs * normed) = rnorm *
// mean(gs * x)); a second pass writes dx.  Same row walk as the forward (one
// wave per row, lane l owns 16-byte chunks l + 64j): x and dy are read once,
// dx written once.  The dscale column sums stay in registers across all rows
// a wave visits; the four waves of a workgroup add theirs into LDS in wave
// order and the workgroup writes one partial row (slice-major, see
// kNormBwdSlice), which rmsnorm_bwd_reduce_sm adds up in a fixed order.
// Both orders are fixed, so dscale is the same on every run.
// GREG: gamma in registers (J <= 4); PF: two rows' loads in flight per wave
// (J <= 4).
// ---------------------------------------------------------------------------
__device__ __forceinline__ void unpack_bf16x8(const uint4& v, float (&f)[8]) {
  f[0] = bf16lo(v.x); f[1] = bf16hi(v.x); f[2] = bf16lo(v.y); f[3] = bf16hi(v.y);
  f[4] = bf16lo(v.z); f[5] = bf16hi(v.z); f[6] = bf16lo(v.w); f[7] = bf16hi(v.w);
}

#ifndef TG_NBWD_GRID
#define TG_NBWD_GRID 256
#endif
#ifndef TG_NBWD_SLICE
#define TG_NBWD_SLICE 32
#endif
constexpr int kNormBwdMaxGrid = TG_NBWD_GRID;
// The row kernel's partial dscale rows are stored slice-major: slice k holds
// columns 32k .. 32k + 31 of every partial row, one 128-byte line per row,
// the rows of a slice contiguous, so that the reduction of a slice reads one
// contiguous run.
constexpr int kNormBwdSlice = TG_NBWD_SLICE;

template <int J, bool FULL>
__global__ __launch_bounds__(256) void rmsnorm_bwd_kernel(const uint4* __restrict__ x,
                                                          const uint4* __restrict__ gamma,
                                                          const uint4* __restrict__ dy,
                                                          uint4* __restrict__ dx,
                                                          float* __restrict__ partial,
                                                          int64_t rows, int nch, float dimf,
                                                          float eps) {
  constexpr bool GREG = J <= 4, PF = J <= 4;
  extern __shared__ float colsum[];   // nch * 8 floats
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t wave0 = (int64_t)blockIdx.x * 4 + wave;
  const int64_t wstride = (int64_t)gridDim.x * 4;

  auto gamma_chunk = [&](int j, float (&f)[8]) {
    const int c = lane + 64 * j;
    unpack_bf16x8((FULL || c < nch) ? gamma[c] : make_uint4(0, 0, 0, 0), f);
  };
  float greg[GREG ? J : 1][8];
  if (GREG) {
#pragma unroll
    for (int j = 0; j < (GREG ? J : 1); ++j) gamma_chunk(j, greg[j]);
  }
  float dg[J][8];
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) dg[j][e] = 0.0f;

  // the row's rnorm and mean(gs * normed) from its unpacked registers
  auto row_stats = [&](const float (&xf)[J][8], const float (&d)[J][8], float& rn, float& dot) {
    double sq = 0.0;
    float gx = 0.0f;   // this lane's part of sum(gs * x)
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float gl[8];
      if (!GREG) gamma_chunk(j, gl);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float gm = GREG ? greg[GREG ? j : 0][e] : gl[e];
        sq += (double)(xf[j][e] * xf[j][e]);
        gx = __builtin_fmaf(d[j][e] * gm, xf[j][e], gx);   // dy * scale is exact in f32
      }
    }
    sq = wave_sum_f64(sq);
    const double gxs = wave_sum_f64((double)gx);
    const float var = (float)sq / dimf;
    rn = (float)(1.0 / __builtin_sqrt((double)(var + eps)));
    dot = rn * ((float)gxs / dimf);
  };
  // dx chunk j of the row (bf16 x 8), and the row's dscale terms when it is real
  auto row_out = [&](int j, const float (&xf)[J][8], const float (&d)[J][8], float rn, float dot, bool real) {
    float gl[8];
    if (!GREG) gamma_chunk(j, gl);
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float gm = GREG ? greg[GREG ? j : 0][e] : gl[e];
      const float nrm = xf[j][e] * rn;
      o[e] = rn * (d[j][e] * gm - nrm * dot);
      const float t = __builtin_fmaf(d[j][e], nrm, dg[j][e]);
      dg[j][e] = real ? t : dg[j][e];
    }
    u32x4_t ov;
    ov.x = pack_bf16x2(o[0], o[1]); ov.y = pack_bf16x2(o[2], o[3]);
    ov.z = pack_bf16x2(o[4], o[5]); ov.w = pack_bf16x2(o[6], o[7]);
    return ov;
  };
  // Row loads and stores are raw buffer accesses over the row's own bytes:
  // lanes past the row's end, and every lane of a row past the last, read
  // zero and write nothing, without a memory access.
  auto row_rsrc = [&](const uint4* base, int64_t row) {
    const bool in = row < rows;
    return make_rsrc(base + (in ? row : 0) * nch, in ? (uint32_t)nch * 16u : 0u);
  };

  if constexpr (PF) {
    // Two rows' loads in flight per wave, and each row's dx held in registers
    // and stored one row later, after the wait for the next row's loads: every
    // access is unconditional (rows past the end are phantoms that touch no
    // memory and add nothing to dscale), so the compiler's waits are for the
    // loads consumed and never for the stores.  With the prefetch behind a
    // branch it waited at the loop head for every outstanding access, the
    // previous row's stores included.
    u32x4_t bx[2][J], bd[2][J], pend[J];
    int64_t pend_row = rows;   // none yet: its stores are dropped
#pragma unroll
    for (int j = 0; j < J; ++j) pend[j] = u32x4_t{0u, 0u, 0u, 0u};
    auto load_slot = [&](auto slot, int64_t row) {
      constexpr int S = decltype(slot)::value;
      const __amdgpu_buffer_rsrc_t rx = row_rsrc(x, row), rd = row_rsrc(dy, row);
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t off = (uint32_t)(lane + 64 * j) * 16u;
        bx[S][j] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, kAuxNT);
        bd[S][j] = __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, kAuxNT);
      }
    };
    auto store_pend = [&]() {
      const __amdgpu_buffer_rsrc_t ro = row_rsrc(dx, pend_row);
#pragma unroll
      for (int j = 0; j < J; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(pend[j], ro, (uint32_t)(lane + 64 * j) * 16u, 0, kAuxNT);
    };
    auto step = [&](auto slot, int64_t row) {
      constexpr int S = decltype(slot)::value;
      float xf[J][8], d[J][8];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        unpack_bf16x8(make_uint4(bx[S][j].x, bx[S][j].y, bx[S][j].z, bx[S][j].w), xf[j]);
        unpack_bf16x8(make_uint4(bd[S][j].x, bd[S][j].y, bd[S][j].z, bd[S][j].w), d[j]);
      }
      store_pend();
      load_slot(slot, row + 2 * wstride);
      // keep the accesses here: the scheduler otherwise sinks the prefetch
      // below the next row's arithmetic, to the end of the loop
      __builtin_amdgcn_sched_barrier(0);
      float rn, dot;
      row_stats(xf, d, rn, dot);
#pragma unroll
      for (int j = 0; j < J; ++j) pend[j] = row_out(j, xf, d, rn, dot, row < rows);
      pend_row = row;
    };
    load_slot(std::integral_constant<int, 0>{}, wave0);
    __builtin_amdgcn_sched_barrier(0);   // the first row's loads strictly before the second's
    load_slot(std::integral_constant<int, 1>{}, wave0 + wstride);
    __builtin_amdgcn_sched_barrier(0);
    for (int64_t row = wave0; row < rows; row += 2 * wstride) {
      step(std::integral_constant<int, 0>{}, row);
      step(std::integral_constant<int, 1>{}, row + wstride);
    }
    store_pend();
  } else {
    for (int64_t row = wave0; row < rows; row += wstride) {
      const __amdgpu_buffer_rsrc_t rx = row_rsrc(x, row), rd = row_rsrc(dy, row);
      float xf[J][8], d[J][8];
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const uint32_t off = (uint32_t)(lane + 64 * j) * 16u;
        const u32x4_t vx = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, kAuxNT);
        const u32x4_t vd = __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, kAuxNT);
        unpack_bf16x8(make_uint4(vx.x, vx.y, vx.z, vx.w), xf[j]);
        unpack_bf16x8(make_uint4(vd.x, vd.y, vd.z, vd.w), d[j]);
      }
      float rn, dot;
      row_stats(xf, d, rn, dot);
      const __amdgpu_buffer_rsrc_t ro = row_rsrc(dx, row);
#pragma unroll
      for (int j = 0; j < J; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(row_out(j, xf, d, rn, dot, true), ro, (uint32_t)(lane + 64 * j) * 16u,
                                               0, kAuxNT);
    }
  }

  // workgroup column sums in wave order, then one partial row per workgroup
  for (int w = 0; w < 4; ++w) {
    if (wave == w) {
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = lane + 64 * j;
        if (FULL || c < nch) {
          float4* p = reinterpret_cast<float4*>(colsum + c * 8);
          float4 a = w ? p[0] : make_float4(0.f, 0.f, 0.f, 0.f);
          float4 b = w ? p[1] : make_float4(0.f, 0.f, 0.f, 0.f);
          a.x += dg[j][0]; a.y += dg[j][1]; a.z += dg[j][2]; a.w += dg[j][3];
          b.x += dg[j][4]; b.y += dg[j][5]; b.z += dg[j][6]; b.w += dg[j][7];
          p[0] = a;
          p[1] = b;
        }
      }
    }
    __syncthreads();
  }
  // slice-major: the partial rows' columns c .. c + kNormBwdSlice - 1 are
  // contiguous across workgroups (see rmsnorm_bwd_reduce_sm)
  const int dim = nch * 8;
  for (int i = threadIdx.x; i < dim; i += 256)
    partial[((int64_t)(i / kNormBwdSlice) * gridDim.x + blockIdx.x) * kNormBwdSlice + i % kNormBwdSlice] =
        colsum[i];
}

// ---------------------------------------------------------------------------
// General path: any width and any of bf16, f16, f32 for x, scale and the
// gradients, with _rms_norm_pure's op-by-op rounding in x's dtype
// (kernels.py:30-33: r = rsqrt(var + eps).astype(x.dtype), x_n = x * r in
// x.dtype, y = x_n * scale in the promoted dtype).  Rows are walked by one
// wave each, two passes over the row (statistics, then output), so no row
// has to fit in registers.  Not the hot path: the bf16 kernels above cover
// bf16 widths up to 16384 (forward) and 4096 (backward).
// ---------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ float ld_f32(const T* p, int64_t i);
template <> __device__ __forceinline__ float ld_f32<uint16_t>(const uint16_t* p, int64_t i) {
  return __uint_as_float((uint32_t)p[i] << 16);
}
template <> __device__ __forceinline__ float ld_f32<float>(const float* p, int64_t i) { return p[i]; }
template <typename T> __device__ __forceinline__ void st_f32(T* p, int64_t i, float v);
template <> __device__ __forceinline__ void st_f32<uint16_t>(uint16_t* p, int64_t i, float v) {
  p[i] = __builtin_bit_cast(uint16_t, (__bf16)v);   // RNE
}
template <> __device__ __forceinline__ void st_f32<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ float ld_f32<_Float16>(const _Float16* p, int64_t i) { return (float)p[i]; }
template <> __device__ __forceinline__ void st_f32<_Float16>(_Float16* p, int64_t i, float v) {
  p[i] = (_Float16)v;   // RNE, f16 subnormals kept
}
template <typename T> constexpr bool is_bf16() { return std::is_same<T, uint16_t>::value; }
// v rounded to T's precision (the .astype(x.dtype) of kernels.py:32), as f32.
template <typename T> __device__ __forceinline__ float round_to(float v) {
  if constexpr (std::is_same<T, uint16_t>::value) return round_bf16(v);
  else if constexpr (std::is_same<T, _Float16>::value) return (float)(_Float16)v;
  else return v;
}

// var = fl32(sum fl32(x)^2) / D (f64 accumulation), rnorm = fl32(1 / sqrt(var + eps)).
template <typename XT>
__device__ __forceinline__ float row_rnorm(const XT* xr, int dim, int lane, float eps) {
  double sq = 0.0;
  for (int c = lane; c < dim; c += 64) {
    const float v = ld_f32(xr, c);
    sq += (double)(v * v);
  }
  sq = wave_sum_f64(sq);
  const float var = (float)sq / (float)dim;
  return (float)(1.0 / __builtin_sqrt((double)(var + eps)));
}

template <typename XT, typename GT, typename YT>
__global__ __launch_bounds__(256) void rmsnorm_gen_kernel(const XT* __restrict__ x,
                                                          const GT* __restrict__ gamma,
                                                          YT* __restrict__ y, int64_t rows, int dim,
                                                          float eps) {
  const int lane = threadIdx.x & 63;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows;
       row += (int64_t)gridDim.x * 4) {
    const XT* xr = x + row * dim;
    const float r = round_to<XT>(row_rnorm(xr, dim, lane, eps));      // .astype(x.dtype)
    for (int c = lane; c < dim; c += 64) {
      const float t = round_to<XT>(ld_f32(xr, c) * r);                  // x * r in x.dtype
      st_f32(y + row * dim, c, t * ld_f32(gamma, c));                   // x_n * scale
    }
  }
}

// Backward statistics per row: (rnorm, rnorm * mean(dy * scale * x)).
template <typename XT, typename GT, typename DT>
__global__ __launch_bounds__(256) void rmsnorm_gen_stats_kernel(const XT* __restrict__ x,
                                                                const GT* __restrict__ gamma,
                                                                const DT* __restrict__ dy,
                                                                float2* __restrict__ stats,
                                                                int64_t rows, int dim, float eps) {
  const int lane = threadIdx.x & 63;
  for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows;
       row += (int64_t)gridDim.x * 4) {
    const XT* xr = x + row * dim;
    const DT* dr = dy + row * dim;
    const float rn = row_rnorm(xr, dim, lane, eps);
    float gx = 0.0f;
    for (int c = lane; c < dim; c += 64)
      gx = __builtin_fmaf(ld_f32(dr, c) * ld_f32(gamma, c), ld_f32(xr, c), gx);
    const double gxs = wave_sum_f64((double)gx);
    if (lane == 0) stats[row] = make_float2(rn, rn * ((float)gxs / (float)dim));
  }
}

// dx = rnorm * (dy * scale - normed * dot) and one partial dscale row per
// row group: block (column tile of 256, row group); each thread owns a column.
constexpr int kGenRowsPerGroup = 16;
template <typename XT, typename GT, typename DT>
__global__ __launch_bounds__(256) void rmsnorm_gen_bwd_kernel(const XT* __restrict__ x,
                                                              const GT* __restrict__ gamma,
                                                              const DT* __restrict__ dy,
                                                              const float2* __restrict__ stats,
                                                              XT* __restrict__ dx,
                                                              float* __restrict__ partial,
                                                              int64_t rows, int dim, int groups) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= dim) return;
  const float gm = ld_f32(gamma, c);
  for (int grp = blockIdx.y; grp < groups; grp += gridDim.y) {
    float dg = 0.0f;
    const int64_t r0 = (int64_t)grp * kGenRowsPerGroup;
    for (int64_t row = r0; row < rows && row < r0 + kGenRowsPerGroup; ++row) {
      const float2 st = stats[row];
      const float d = ld_f32(dy + row * dim, c);
      const float nrm = ld_f32(x + row * dim, c) * st.x;
      st_f32(dx + row * dim, c, st.x * (d * gm - nrm * st.y));
      dg = __builtin_fmaf(d, nrm, dg);
    }
    partial[(int64_t)grp * dim + c] = dg;
  }
}

// dscale[c] = bf16(sum over b of partial[b][c]) with f64 accumulation in a
// fixed order: workgroup = 64 columns x 16 waves; wave w adds partial rows
// w, w + 16, w + 32, ... in that order, and the 16 wave sums are added in
// wave order.  A lane keeps 32 loads in flight, all of its rows for up to 512
// partial rows: the reduction runs on few workgroups (dim / 64), so its time
// is the number of dependent round trips to L2.
template <typename OT>
__global__ __launch_bounds__(1024) void rmsnorm_bwd_reduce(const float* __restrict__ partial,
                                                           int nparts, int dim,
                                                           OT* __restrict__ dscale) {
  constexpr int W = 16, U = 32;
  __shared__ double wsum[W][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  double acc = 0.0;
  if (c < dim) {
    int b = wave;
    for (; b + (U - 1) * W < nparts; b += U * W) {
      float v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) v[u] = partial[(int64_t)(b + u * W) * dim + c];
#pragma unroll
      for (int u = 0; u < U; ++u) acc += (double)v[u];
    }
    for (; b < nparts; b += W) acc += (double)partial[(int64_t)b * dim + c];
  }
  wsum[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && c < dim) {
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < W; ++w) t += wsum[w][lane];
    st_f32(dscale, c, (float)t);
  }
}

// dscale[c] = bf16(sum over b of the slice-major partial rows) with f64
// accumulation in a fixed order: one workgroup per slice of kNormBwdSlice
// columns; thread (pg, cl) adds partial rows pg, pg + PG, ... of column cl
// (16 loads in flight), then the PG group sums are added in group order.  A
// wave's load covers 64 / kNormBwdSlice consecutive partial rows of the slice,
// i.e. one contiguous 256-byte piece.
#ifndef TG_NBWD_RTHREADS
#define TG_NBWD_RTHREADS 1024
#endif
template <typename OT, int U>
__global__ __launch_bounds__(TG_NBWD_RTHREADS) void rmsnorm_bwd_reduce_sm(const float* __restrict__ partial,
                                                                          int nparts, int dim,
                                                                          OT* __restrict__ dscale) {
  constexpr int SW = kNormBwdSlice, PG = TG_NBWD_RTHREADS / SW;
  __shared__ double gsum[PG][SW];
  const int cl = threadIdx.x % SW, pg = threadIdx.x / SW;
  const int c = blockIdx.x * SW + cl;
  const float* __restrict__ base = partial + (int64_t)blockIdx.x * nparts * SW + cl;
  double acc = 0.0;
  int b = pg;
  for (; b + (U - 1) * PG < nparts; b += U * PG) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = base[(int64_t)(b + u * PG) * SW];
#pragma unroll
    for (int u = 0; u < U; ++u) acc += (double)v[u];
  }
  for (; b < nparts; b += PG) acc += (double)base[(int64_t)b * SW];
  gsum[pg][cl] = acc;
  __syncthreads();
  if (pg == 0 && c < dim) {
    double t = 0.0;
#pragma unroll
    for (int g = 0; g < PG; ++g) t += gsum[g][cl];
    st_f32(dscale, c, (float)t);
  }
}

static int64_t norm_bwd_slices(int64_t dim) { return (dim + kNormBwdSlice - 1) / kNormBwdSlice; }

static int64_t norm_bwd_grid(int64_t rows) {
  // about four rows per wave, at most one workgroup per CU (256 partial rows
  // at C2's 8192: 0.5 us less than 512 over both kernels, measured)
  int64_t g = (rows + 15) / 16;
  if (g > kNormBwdMaxGrid) g = kNormBwdMaxGrid;
  return g;
}

static int launch_rmsnorm_bwd(const void* x, const void* gamma, const void* dy, void* dx,
                              void* dscale, float* partial, int64_t rows, int64_t dim, float eps,
                              hipStream_t st) {
  const int nch = (int)(dim / 8);
  const int jneed = (nch + 63) / 64;
  const int64_t grid = norm_bwd_grid(rows);
  auto X = reinterpret_cast<const uint4*>(x);
  auto G = reinterpret_cast<const uint4*>(gamma);
  auto DY = reinterpret_cast<const uint4*>(dy);
  auto DX = reinterpret_cast<uint4*>(dx);
  const float dimf = (float)dim;
  const size_t lds = (size_t)dim * 4;
  if (grid > 0) {
    bool launched = false;
#define TG_NORM_BWD_CASE(JJ)                                                                       \
    if (!launched && jneed <= JJ) {                                                                \
      if (nch == JJ * 64)                                                                          \
        hipLaunchKernelGGL((rmsnorm_bwd_kernel<JJ, true>), dim3((unsigned)grid), dim3(256), lds, st, \
                           X, G, DY, DX, partial, rows, nch, dimf, eps);                           \
      else                                                                                         \
        hipLaunchKernelGGL((rmsnorm_bwd_kernel<JJ, false>), dim3((unsigned)grid), dim3(256), lds,  \
                           st, X, G, DY, DX, partial, rows, nch, dimf, eps);                       \
      launched = true;                                                                             \
    }
    TG_NORM_BWD_CASE(1)
    TG_NORM_BWD_CASE(2)
    TG_NORM_BWD_CASE(4)
    TG_NORM_BWD_CASE(8)
#undef TG_NORM_BWD_CASE
    if (!launched) return einval("rms_norm_bwd: dim must be <= 4096");
    TG_TRY(check_launch("rmsnorm_bwd"));
  }
  // no rows: no partial rows, and the reduction writes dscale = 0
  // U: partial rows per thread in flight at once (every one of them at C2's 512)
  constexpr int kPG = TG_NBWD_RTHREADS / kNormBwdSlice;
  const dim3 rgrid((unsigned)norm_bwd_slices(dim)), rblock(TG_NBWD_RTHREADS);
  auto ds = reinterpret_cast<uint16_t*>(dscale);
  if (grid >= 16 * kPG)
    hipLaunchKernelGGL((rmsnorm_bwd_reduce_sm<uint16_t, 16>), rgrid, rblock, 0, st, partial, (int)grid, (int)dim, ds);
  else if (grid >= 8 * kPG)
    hipLaunchKernelGGL((rmsnorm_bwd_reduce_sm<uint16_t, 8>), rgrid, rblock, 0, st, partial, (int)grid, (int)dim, ds);
  else
    hipLaunchKernelGGL((rmsnorm_bwd_reduce_sm<uint16_t, 4>), rgrid, rblock, 0, st, partial, (int)grid, (int)dim, ds);
  return check_launch("rmsnorm_bwd_reduce");
}

static int64_t gen_groups(int64_t rows) {
  const int64_t g = (rows + kGenRowsPerGroup - 1) / kGenRowsPerGroup;
  return g < 1 ? 1 : g;
}
static size_t gen_bwd_workspace(int64_t rows, int64_t dim) {
  return (((size_t)rows * 8 + 255) & ~(size_t)255) + (size_t)gen_groups(rows) * (size_t)dim * 4;
}
static unsigned row_grid(int64_t rows) {
  const int64_t g = (rows + 3) / 4;
  return (unsigned)(g < 1 ? 1 : g > 16384 ? 16384 : g);
}

// Calls f(T{}) with T the element type of dtype code d: bf16 as its uint16_t
// bits, _Float16, float.  Codes are validated by the entry points.
template <typename F> static int with_dtype(int d, F&& f) {
  switch (d) {
    case TG_DTYPE_BF16: return f(uint16_t{});
    case TG_DTYPE_F16: return f(_Float16{});
    default: return f(float{});
  }
}

static bool valid_float_dtype(int d) { return d == TG_DTYPE_BF16 || d == TG_DTYPE_F16 || d == TG_DTYPE_F32; }

template <typename XT, typename GT>
static int launch_gen_fwd(const void* x, const void* g, void* y, int y_dtype, int64_t rows, int64_t dim,
                          float eps, hipStream_t st) {
  auto X = reinterpret_cast<const XT*>(x);
  auto G = reinterpret_cast<const GT*>(g);
  return with_dtype(y_dtype, [&](auto yt) {
    using YT = decltype(yt);
    hipLaunchKernelGGL((rmsnorm_gen_kernel<XT, GT, YT>), dim3(row_grid(rows)), dim3(256), 0, st, X, G,
                       reinterpret_cast<YT*>(y), rows, (int)dim, eps);
    return check_launch("rmsnorm_gen");
  });
}

template <typename XT, typename GT, typename DT>
static int launch_gen_bwd(const void* x, const void* g, const void* dy, void* dx, void* dscale,
                          int64_t rows, int64_t dim, float eps, void* ws, hipStream_t st) {
  auto X = reinterpret_cast<const XT*>(x);
  auto G = reinterpret_cast<const GT*>(g);
  auto DY = reinterpret_cast<const DT*>(dy);
  float2* stats = reinterpret_cast<float2*>(ws);
  float* partial = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(ws) +
                                            (((size_t)rows * 8 + 255) & ~(size_t)255));
  const int64_t groups = gen_groups(rows);
  if (rows > 0) {
    hipLaunchKernelGGL((rmsnorm_gen_stats_kernel<XT, GT, DT>), dim3(row_grid(rows)), dim3(256), 0, st, X,
                       G, DY, stats, rows, (int)dim, eps);
    TG_TRY(check_launch("rmsnorm_gen_stats"));
    const unsigned gy = (unsigned)(groups < 1024 ? groups : 1024);
    hipLaunchKernelGGL((rmsnorm_gen_bwd_kernel<XT, GT, DT>), dim3((unsigned)((dim + 255) / 256), gy),
                       dim3(256), 0, st, X, G, DY, stats, reinterpret_cast<XT*>(dx), partial, rows,
                       (int)dim, (int)groups);
    TG_TRY(check_launch("rmsnorm_gen_bwd"));
  } else {
    // no rows: dscale = 0 (one zero partial row)
    hipLaunchKernelGGL((rmsnorm_gen_bwd_kernel<XT, GT, DT>), dim3((unsigned)((dim + 255) / 256), 1),
                       dim3(256), 0, st, X, G, DY, stats, reinterpret_cast<XT*>(dx), partial, rows,
                       (int)dim, 1);
    TG_TRY(check_launch("rmsnorm_gen_bwd"));
  }
  hipLaunchKernelGGL(rmsnorm_bwd_reduce<GT>, dim3((unsigned)((dim + 63) / 64)), dim3(1024), 0, st, partial,
                     (int)groups, (int)dim, reinterpret_cast<GT*>(dscale));
  return check_launch("rmsnorm_bwd_reduce");
}

}  // namespace tg

using namespace tg;

extern "C" int tg_rms_norm(const void* x, const void* scale, void* y, int64_t rows, int64_t dim,
                           float eps, void* stream) {
  if (rows < 0 || dim <= 0) return einval("rms_norm: bad shape");
  if (dim % 8) return einval("rms_norm: dim must be a multiple of 8");
  if (rows == 0) return TG_OK;
  if (!x || !scale || !y) return einval("rms_norm: null pointer");
  if (!aligned(x, 16) || !aligned(scale, 16) || !aligned(y, 16))
    return einval("rms_norm: x, scale and y must be 16-byte aligned");
  return launch_rmsnorm<false>(x, scale, y, nullptr, nullptr, rows, dim, eps, as_stream(stream));
}

extern "C" int tg_rms_norm_fp8(const void* x, const void* scale, void* y, uint8_t* q, float* s,
                               int64_t rows, int64_t dim, float eps, int block_k, void* stream) {
  if (block_k != 128) return einval("rms_norm_fp8: block_k must be 128");
  if (rows < 0 || dim <= 0) return einval("rms_norm_fp8: bad shape");
  if (dim % block_k) return einval("rms_norm_fp8: dim not divisible by block_k");
  if (rows == 0) return TG_OK;
  if (!x || !scale || !y || !q || !s) return einval("rms_norm_fp8: null pointer");
  if (!aligned(x, 16) || !aligned(scale, 16) || !aligned(y, 16) || !aligned(q, 8))
    return einval("rms_norm_fp8: x, scale, y must be 16-byte and q 8-byte aligned");
  return launch_rmsnorm<true>(x, scale, y, q, s, rows, dim, eps, as_stream(stream));
}

extern "C" int tg_add_rms_norm_fp8(const void* x, const void* delta, const void* scale,
                                   void* x_out, void* y, uint8_t* q, float* s, int64_t rows,
                                   int64_t dim, float eps, int block_k, void* stream) {
  if (block_k != 128) return einval("add_rms_norm_fp8: block_k must be 128");
  if (rows < 0 || dim <= 0) return einval("add_rms_norm_fp8: bad shape");
  if (dim % block_k) return einval("add_rms_norm_fp8: dim not divisible by block_k");
  if (rows == 0) return TG_OK;
  if (!x || !delta || !scale || !x_out || !q || !s) return einval("add_rms_norm_fp8: null pointer");
  if (!aligned(x, 16) || !aligned(delta, 16) || !aligned(scale, 16) || !aligned(x_out, 16) ||
      (y && !aligned(y, 16)) || !aligned(q, 8))
    return einval("add_rms_norm_fp8: x, delta, scale, x_out, y must be 16-byte and q 8-byte aligned");
  return launch_rmsnorm<true, true>(x, scale, y, q, s, rows, dim, eps, as_stream(stream), delta, x_out);
}

extern "C" size_t tg_rms_norm_bwd_workspace(int64_t rows, int64_t dim) {
  if (rows < 0 || dim <= 0) return 0;
  const size_t fast = (size_t)norm_bwd_grid(rows) * (size_t)norm_bwd_slices(dim) * kNormBwdSlice * 4;
  const size_t gen = gen_bwd_workspace(rows, dim);
  return fast > gen ? fast : gen;
}

extern "C" int tg_rms_norm_bwd(const void* x, const void* scale, const void* dy, void* dx,
                               void* dscale, int64_t rows, int64_t dim, float eps,
                               void* workspace, size_t workspace_bytes, void* stream) {
  if (rows < 0 || dim <= 0) return einval("rms_norm_bwd: bad shape");
  if (dim % 8) return einval("rms_norm_bwd: dim must be a multiple of 8");
  if (!scale || !dscale) return einval("rms_norm_bwd: null pointer");
  if (rows > 0 && (!x || !dy || !dx || !workspace)) return einval("rms_norm_bwd: null pointer");
  if (workspace_bytes < tg_rms_norm_bwd_workspace(rows, dim)) return einval("rms_norm_bwd: workspace too small");
  if (!aligned(x, 16) || !aligned(scale, 16) || !aligned(dy, 16) || !aligned(dx, 16) || !aligned(workspace, 16))
    return einval("rms_norm_bwd: x, scale, dy, dx and workspace must be 16-byte aligned");
  if (dim > 4096 || dim > 0x7FFFFFFF)
    return launch_gen_bwd<uint16_t, uint16_t, uint16_t>(x, scale, dy, dx, dscale, rows, dim, eps,
                                                        workspace, as_stream(stream));
  return launch_rmsnorm_bwd(x, scale, dy, dx, dscale, reinterpret_cast<float*>(workspace), rows, dim,
                            eps, as_stream(stream));
}

extern "C" int tg_rms_norm_ex(const void* x, int x_dtype, const void* scale, int scale_dtype, void* y,
                              int64_t rows, int64_t dim, float eps, void* stream) {
  if (rows < 0 || dim <= 0 || dim > 0x7FFFFFFF) return einval("rms_norm_ex: bad shape");
  if (!valid_float_dtype(x_dtype) || !valid_float_dtype(scale_dtype))
    return einval("rms_norm_ex: dtypes must be TG_DTYPE_BF16, TG_DTYPE_F16 or TG_DTYPE_F32");
  if (rows == 0) return TG_OK;
  if (!x || !scale || !y) return einval("rms_norm_ex: null pointer");
  hipStream_t st = as_stream(stream);
  if (x_dtype == TG_DTYPE_BF16 && scale_dtype == TG_DTYPE_BF16 && dim % 8 == 0 && dim <= 16384 &&
      aligned(x, 16) && aligned(scale, 16) && aligned(y, 16))
    return launch_rmsnorm<false>(x, scale, y, nullptr, nullptr, rows, dim, eps, st);
  // jnp's promotion of x_n * scale: the common dtype, else f32 (bf16 with f16 included)
  const int y_dtype = x_dtype == scale_dtype ? x_dtype : TG_DTYPE_F32;
  return with_dtype(x_dtype, [&](auto xt) {
    return with_dtype(scale_dtype, [&](auto gt) {
      return launch_gen_fwd<decltype(xt), decltype(gt)>(x, scale, y, y_dtype, rows, dim, eps, st);
    });
  });
}

extern "C" int tg_rms_norm_bwd_ex(const void* x, int x_dtype, const void* scale, int scale_dtype,
                                  const void* dy, int dy_dtype, void* dx, void* dscale, int64_t rows,
                                  int64_t dim, float eps, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  if (rows < 0 || dim <= 0 || dim > 0x7FFFFFFF) return einval("rms_norm_bwd_ex: bad shape");
  for (int d : {x_dtype, scale_dtype, dy_dtype})
    if (!valid_float_dtype(d))
      return einval("rms_norm_bwd_ex: dtypes must be TG_DTYPE_BF16, TG_DTYPE_F16 or TG_DTYPE_F32");
  if (!scale || !dscale) return einval("rms_norm_bwd_ex: null pointer");
  if (rows > 0 && (!x || !dy || !dx || !workspace)) return einval("rms_norm_bwd_ex: null pointer");
  if (workspace_bytes < tg_rms_norm_bwd_workspace(rows, dim))
    return einval("rms_norm_bwd_ex: workspace too small");
  if (!aligned(workspace, 16)) return einval("rms_norm_bwd_ex: workspace must be 16-byte aligned");
  const bool all_bf16 = x_dtype == TG_DTYPE_BF16 && scale_dtype == TG_DTYPE_BF16 && dy_dtype == TG_DTYPE_BF16;
  if (all_bf16 && dim % 8 == 0 && aligned(x, 16) && aligned(scale, 16) && aligned(dy, 16) && aligned(dx, 16))
    return tg_rms_norm_bwd(x, scale, dy, dx, dscale, rows, dim, eps, workspace, workspace_bytes, stream);
  hipStream_t st = as_stream(stream);
  return with_dtype(x_dtype, [&](auto xt) {
    return with_dtype(scale_dtype, [&](auto gt) {
      return with_dtype(dy_dtype, [&](auto dt) {
        return launch_gen_bwd<decltype(xt), decltype(gt), decltype(dt)>(x, scale, dy, dx, dscale, rows, dim,
                                                                          eps, workspace, st);
      });
    });
  });
}
