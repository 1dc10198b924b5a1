// Per-row device routines shared by the norm, quantization and decode GEMV
// kernels, so that a fused kernel produces the same bits as the stand-alone
// ones:
//   norm_row   rmsnorm of one row by one wave (/root/reference/kernels.py:30-33),
//              optionally after the bf16 residual add, and its FP8 rows
//              (/root/reference/fp8.py:39-47); norm_row_rb + norm_chunk are its
//              two halves (row statistics by one wave, then any 8-element chunk)
//   quant8     8 values of one 128-element block -> e4m3fn bytes
//   relu2_bf16 bf16(relu(x)^2) (/root/reference/model.py:72 on bf16 tensors)
#pragma once
#include "tg_device.h"

namespace tg {

// max(|a|, |b|, |c|) with NaN propagation (IEEE maximum: v_maximum3_f32)
__device__ __forceinline__ float amax3(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(__builtin_fabsf(a), __builtin_fabsf(b)),
                                       __builtin_fabsf(c));
}

__device__ __forceinline__ uint32_t absmax8(const float (&v)[8]) {
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = max(m, __float_as_uint(v[i]) & 0x7FFFFFFFu);
  return m;
}

// Quantize 8 values of one block with scale sc; bf16-valued inputs use the
// exact reciprocal-refinement divide, f32 inputs the IEEE divide.
template <bool BF16_VALUES>
__device__ __forceinline__ uint2 quant8(const float (&v)[8], float sc) {
  Divider d(sc);
  uint2 out;
  if (d.fast) {
    float t[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) t[i] = BF16_VALUES ? d.div(v[i]) : v[i] / sc;
    out.x = e4m3x4(t[0], t[1], t[2], t[3]);
    out.y = e4m3x4(t[4], t[5], t[6], t[7]);
  } else {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = e4m3_nonfinite_scale(v[i], sc);
    out.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    out.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
  }
  return out;
}

// bf16 chunk (8 values) -> f32
__device__ __forceinline__ void unpack8(const uint4& a, float (&v)[8]) {
  v[0] = bf16lo(a.x); v[1] = bf16hi(a.x); v[2] = bf16lo(a.y); v[3] = bf16hi(a.y);
  v[4] = bf16lo(a.z); v[5] = bf16hi(a.z); v[6] = bf16lo(a.w); v[7] = bf16hi(a.w);
}

// v <- bf16(relu(v)^2): relu exact, the square rounded once.  IEEE maximum
// keeps NaN (jnp.maximum / torch relu propagate it).
__device__ __forceinline__ void relu2_bf16(float (&v)[8]) {
#pragma unroll
  for (int i = 0; i < 8; i += 2) {
    const float a = __builtin_elementwise_maximum(v[i], 0.0f);
    const float b = __builtin_elementwise_maximum(v[i + 1], 0.0f);
    const uint32_t w = pack_bf16x2(a * a, b * b);
    v[i] = bf16lo(w);
    v[i + 1] = bf16hi(w);
  }
}

// The statistics of one row of _rms_norm_pure, by one wave64; lane l holds
// the 16-byte chunks l + 64j (j < J) of the row (chunks past the row are zero).
//   var = mean(f32(x)^2)   f32 squares summed in f64, rounded to f32, / D in f32
//   r   = bf16(rsqrt(var + eps))   (f64 1/sqrt, correctly rounded)
// ADD: x is first replaced by the bf16 residual sum x + delta (each sum
// rounded once), returned in xv.  Returns r (the same in every lane).  Every
// lane of the wave must call this (cross-lane sum).
template <int J, bool ADD>
__device__ __forceinline__ float norm_row_rb(uint4 (&xv)[J], const uint4 (&dv)[J], float dimf, float eps) {
  float xf[J][8];
#pragma unroll
  for (int j = 0; j < J; ++j) unpack8(xv[j], xf[j]);
  if (ADD) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t dw[4] = {dv[j].x, dv[j].y, dv[j].z, dv[j].w};
      uint32_t sw[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        sw[e] = pack_bf16x2(xf[j][2 * e] + bf16lo(dw[e]), xf[j][2 * e + 1] + bf16hi(dw[e]));
        xf[j][2 * e] = bf16lo(sw[e]);
        xf[j][2 * e + 1] = bf16hi(sw[e]);
      }
      xv[j] = make_uint4(sw[0], sw[1], sw[2], sw[3]);
    }
  }
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += (double)(xf[j][e] * xf[j][e]);
  acc = wave_sum_f64(acc);
  const float var = (float)acc / dimf;
  const float ve = var + eps;
  return round_bf16((float)(1.0 / __builtin_sqrt((double)ve)));
}

// y = bf16(bf16(x * r) * g) of one 8-element chunk and, with QUANT, its
// e4m3fn bytes q and block scale s (fp8.py:39-47 on the bf16 y).  The 16
// lanes of a DPP row must hold the 16 chunks of one 128-element block, and
// every lane must call this (DPP maximum); `valid` only gates the divide.
template <bool QUANT>
__device__ __forceinline__ void norm_chunk(const uint4& xc, const float (&g)[8], float rb, bool valid,
                                           uint4& y, uint2& q, float& s) {
  float xf[8], yv[8];
  unpack8(xc, xf);
  uint32_t ow[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t tp = pack_bf16x2(xf[2 * e] * rb, xf[2 * e + 1] * rb);
    const uint32_t yp = pack_bf16x2(bf16lo(tp) * g[2 * e], bf16hi(tp) * g[2 * e + 1]);
    ow[e] = yp;
    yv[2 * e] = bf16lo(yp);
    yv[2 * e + 1] = bf16hi(yp);
  }
  y = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  if (QUANT) {
    const float m = amax3(amax3(yv[0], yv[1], yv[2]), amax3(yv[3], yv[4], yv[5]),
                          __builtin_elementwise_maximum(__builtin_fabsf(yv[6]), __builtin_fabsf(yv[7])));
    const uint32_t mb = row16_max_u32(__float_as_uint(m));   // all lanes take part
    const float sc = block_scale_bf16(mb);
    s = sc;
    q = make_uint2(0, 0);
    if (valid) {
      Divider d(sc);
      if (d.fast) {
        q.x = e4m3x4(d.div(yv[0]), d.div(yv[1]), d.div(yv[2]), d.div(yv[3]));
        q.y = e4m3x4(d.div(yv[4]), d.div(yv[5]), d.div(yv[6]), d.div(yv[7]));
      } else {
        uint32_t b[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = e4m3_nonfinite_scale(yv[e], sc);
        q.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        q.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
      }
    }
  }
}

// One row of _rms_norm_pure by one wave64 (norm_row_rb, then norm_chunk for
// each of the lane's chunks); outputs per chunk: yo (bf16 y), qo (e4m3 bytes),
// so (block scale).  FULL: nch == 64 J (no guards).
template <int J, bool QUANT, bool FULL, bool ADD>
__device__ __forceinline__ void norm_row(uint4 (&xv)[J], const uint4 (&dv)[J], const float (&g)[J][8],
                                         int lane, int nch, float dimf, float eps, uint4 (&yo)[J],
                                         uint2 (&qo)[J], float (&so)[J]) {
  const float rb = norm_row_rb<J, ADD>(xv, dv, dimf, eps);
#pragma unroll
  for (int j = 0; j < J; ++j) norm_chunk<QUANT>(xv[j], g[j], rb, FULL || lane + 64 * j < nch, yo[j], qo[j], so[j]);
}

}  // namespace tg
