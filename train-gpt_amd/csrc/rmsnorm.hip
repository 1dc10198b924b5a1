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

template <int J, bool QUANT>
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
    uint4 w = c < nch ? gamma[c] : make_uint4(0, 0, 0, 0);
    g[j][0] = bf16lo(w.x); g[j][1] = bf16hi(w.x); g[j][2] = bf16lo(w.y); g[j][3] = bf16hi(w.y);
    g[j][4] = bf16lo(w.z); g[j][5] = bf16hi(w.z); g[j][6] = bf16lo(w.w); g[j][7] = bf16hi(w.w);
  }

  for (int64_t row = wave0; row < rows; row += wstride) {
    const uint4* xr = x + row * nch;
    uint4 xv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      xv[j] = c < nch ? ldg_stream(xr + c) : make_uint4(0, 0, 0, 0);
    }
    double acc = 0.0;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = bf16lo(w[e]), b = bf16hi(w[e]);
        acc += (double)(a * a);
        acc += (double)(b * b);
      }
    }
    acc = wave_sum_f64(acc);
    const float var = (float)acc / dimf;
    const float ve = var + eps;
    const float rb = round_bf16((float)(1.0 / __builtin_sqrt((double)ve)));

#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      const uint32_t w[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
      float yv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        yv[2 * e] = round_bf16(round_bf16(bf16lo(w[e]) * rb) * g[j][2 * e]);
        yv[2 * e + 1] = round_bf16(round_bf16(bf16hi(w[e]) * rb) * g[j][2 * e + 1]);
      }
      if (c < nch) {
        uint4 o;
        o.x = pack_bf16x2(yv[0], yv[1]);
        o.y = pack_bf16x2(yv[2], yv[3]);
        o.z = pack_bf16x2(yv[4], yv[5]);
        o.w = pack_bf16x2(yv[6], yv[7]);
        y[row * nch + c] = o;
      }
      if (QUANT) {
        uint32_t m = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) m = max(m, __float_as_uint(yv[e]) & 0x7FFFFFFFu);
        m = row16_max_u32(m);                        // wave-uniform: all lanes take part
        const float sc = block_scale(m);
        if (c < nch) {
          Divider d(sc);
          uint2 o;
          if (d.fast) {
            o.x = e4m3x4(d.div(yv[0]), d.div(yv[1]), d.div(yv[2]), d.div(yv[3]));
            o.y = e4m3x4(d.div(yv[4]), d.div(yv[5]), d.div(yv[6]), d.div(yv[7]));
          } else {
            uint32_t b[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = e4m3_nonfinite_scale(yv[e], sc);
            o.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
            o.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
          }
          q[row * nch + c] = o;
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
  int64_t grid = (rows + 3) / 4;
  if (grid > 16384) grid = 16384;
  const dim3 g((unsigned)grid), b(256);
  auto X = reinterpret_cast<const uint4*>(x);
  auto G = reinterpret_cast<const uint4*>(gamma);
  auto Y = reinterpret_cast<uint4*>(y);
  auto Q = reinterpret_cast<uint2*>(q);
  const float dimf = (float)dim;
#define TG_NORM_CASE(JJ)                                                                   \
  if (jneed <= JJ) {                                                                        \
    hipLaunchKernelGGL((rmsnorm_kernel<JJ, QUANT>), g, b, 0, st, X, G, Y, Q, s, rows, nch, \
                       dimf, eps);                                                          \
    return check_launch("rmsnorm");                                                         \
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
