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
#include "tg_device.h"
#include "tg_host.h"

namespace tg {

// max(|a|, |b|, |c|) with NaN propagation (IEEE maximum: v_maximum3_f32)
__device__ __forceinline__ float amax3(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(__builtin_fabsf(a), __builtin_fabsf(b)),
                                       __builtin_fabsf(c));
}

// FULL: every lane owns exactly J chunks of every row (dim == 512 * J), so
// no per-chunk guards are emitted.  Each wave walks rows with a stride of the
// grid's wave count and prefetches the next row's x while it computes the
// current one.
template <int J, bool QUANT, bool FULL>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint4* __restrict__ x,
                                                      const uint4* __restrict__ gamma,
                                                      uint4* __restrict__ y,
                                                      uint2* __restrict__ q,
                                                      float* __restrict__ s, int64_t rows,
                                                      int nch, float dimf, float eps) {
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

  auto load_row = [&](int64_t row, uint4 (&xv)[J]) {
    const uint4* xr = x + row * nch;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      xv[j] = (FULL || c < nch) ? ldg_stream(xr + c) : make_uint4(0, 0, 0, 0);
    }
  };

  uint4 nxt[J];
  if (wave0 < rows) load_row(wave0, nxt);
  for (int64_t row = wave0; row < rows; row += wstride) {
    float xf[J][8];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      xf[j][0] = bf16lo(nxt[j].x); xf[j][1] = bf16hi(nxt[j].x);
      xf[j][2] = bf16lo(nxt[j].y); xf[j][3] = bf16hi(nxt[j].y);
      xf[j][4] = bf16lo(nxt[j].z); xf[j][5] = bf16hi(nxt[j].z);
      xf[j][6] = bf16lo(nxt[j].w); xf[j][7] = bf16hi(nxt[j].w);
    }
    if (row + wstride < rows) load_row(row + wstride, nxt);   // prefetch the next row

    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < J; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (double)(xf[j][e] * xf[j][e]);
    acc = wave_sum_f64(acc);
    const float var = (float)acc / dimf;
    const float ve = var + eps;
    const float rb = round_bf16((float)(1.0 / __builtin_sqrt((double)ve)));

#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      float yv[8];
      uint4 o;
      uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t tp = pack_bf16x2(xf[j][2 * e] * rb, xf[j][2 * e + 1] * rb);
        const uint32_t yp = pack_bf16x2(bf16lo(tp) * g[j][2 * e], bf16hi(tp) * g[j][2 * e + 1]);
        ow[e] = yp;
        yv[2 * e] = bf16lo(yp);
        yv[2 * e + 1] = bf16hi(yp);
      }
      if (FULL || c < nch) stg_stream(&y[row * nch + c], o);
      if (QUANT) {
        const float m = amax3(amax3(yv[0], yv[1], yv[2]), amax3(yv[3], yv[4], yv[5]),
                              __builtin_elementwise_maximum(__builtin_fabsf(yv[6]), __builtin_fabsf(yv[7])));
        // wave-uniform: all lanes take part in the DPP reduction
        const uint32_t mb = row16_max_u32(__float_as_uint(m));
        const float sc = block_scale_bf16(mb);
        if (FULL || c < nch) {
          Divider d(sc);
          uint2 qo;
          if (d.fast) {
            qo.x = e4m3x4(d.div(yv[0]), d.div(yv[1]), d.div(yv[2]), d.div(yv[3]));
            qo.y = e4m3x4(d.div(yv[4]), d.div(yv[5]), d.div(yv[6]), d.div(yv[7]));
          } else {
            uint32_t b[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = e4m3_nonfinite_scale(yv[e], sc);
            qo.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
            qo.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
          }
          stg_stream(&q[row * nch + c], qo);
          if ((lane & 15) == 0) s[row * (nch >> 4) + (c >> 4)] = sc;
        }
      }
    }
  }
}

template <bool QUANT>
static int launch_rmsnorm(const void* x, const void* gamma, void* y, uint8_t* q, float* s,
                          int64_t rows, int64_t dim, float eps, hipStream_t st) {
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
#define TG_NORM_CASE(JJ)                                                                        \
  if (jneed <= JJ) {                                                                             \
    if (nch == JJ * 64)                                                                          \
      hipLaunchKernelGGL((rmsnorm_kernel<JJ, QUANT, true>), gdim, b, 0, st, X, G, Y, Q, s, rows, \
                         nch, dimf, eps);                                                        \
    else                                                                                         \
      hipLaunchKernelGGL((rmsnorm_kernel<JJ, QUANT, false>), gdim, b, 0, st, X, G, Y, Q, s,      \
                         rows, nch, dimf, eps);                                                  \
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
