// Logit cap + cross-entropy over a large vocabulary, forward and backward
// (the head of /root/reference/model.py:96-97 and the loss of
// /root/reference/losses.py:8-12, as the config-4 block step computes them):
//   z    = cap * tanh(l / cap)                 (f32 from the bf16 logits l)
//   lse  = log sum_v exp(z_v)
//   loss = lse - z[t]                          (per row; the caller takes the mean)
//   dl   = g w_r (softmax(z) - onehot(t)) (1 - (z / cap)^2)     (bf16, one rounding)
// One workgroup per row.  The forward reads the row once: each thread keeps
// a log-sum-exp state (running max m, sum s of e^(z - m)) over 32 values at a
// time (four 16-byte loads in flight), and the states merge across the wave
// with shuffles and across waves through LDS in a fixed order.  The backward
// reads the row once more and writes the gradient once.
// tanh runs on the hardware exponential and reciprocal (absolute error ~2e-7,
// so z is within ~3e-6 of cap * tanh(l / cap)).  A target outside [0, vocab)
// gives a NaN loss and no one-hot term in the gradient.
#include "tg_device.h"
#include "tg_host.h"

namespace tg {

constexpr int kXentThreads = 512;
constexpr int kXentUnroll = 4;         // 16-byte loads in flight per thread

// tanh(x) and 1 - tanh(x)^2 from e = e^(-2|x|) and r = 1 / (1 + e):
// tanh = sign(x) (1 - e) r, sech^2 = 4 e r^2 (relatively accurate for every x,
// 0 when e underflows).
__device__ __forceinline__ float tanh_fast(float x, float* sech2 = nullptr) {
  const float e = __expf(-2.0f * __builtin_fabsf(x));
  const float r = __builtin_amdgcn_rcpf(1.0f + e);
  if (sech2) *sech2 = 4.0f * e * r * r;
  return __builtin_copysignf((1.0f - e) * r, x);
}

__device__ __forceinline__ float capped(float l, float cap, float inv_cap) {
  return cap * tanh_fast(l * inv_cap);
}

// (m, s) <- (m, s) merged with (m2, s2); a state stands for s * e^m.
__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
  const float mn = m > m2 ? m : m2;
  if (mn == -__builtin_inff()) return;                 // both empty
  s = s * __expf(m - mn) + s2 * __expf(m2 - mn);
  m = mn;
}

// Merge of every thread's (m, s) in a fixed order; returns log(sum) to all threads.
__device__ __forceinline__ float block_lse(float m, float s) {
  __shared__ float sm[kXentThreads / 64], ss[kXentThreads / 64];
  for (int off = 32; off > 0; off >>= 1) {
    const float m2 = __shfl_xor(m, off, 64), s2 = __shfl_xor(s, off, 64);
    lse_merge(m, s, m2, s2);
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { sm[wave] = m; ss[wave] = s; }
  __syncthreads();
  float M = sm[0], S = ss[0];
  for (int w = 1; w < kXentThreads / 64; ++w) lse_merge(M, S, sm[w], ss[w]);
  return M + __logf(S);
}

// z of the 8 bf16 values of one 16-byte word
__device__ __forceinline__ void capped8(const uint4& w, float cap, float inv_cap, float* z) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    z[2 * e] = capped(bf16lo(ww[e]), cap, inv_cap);
    z[2 * e + 1] = capped(bf16hi(ww[e]), cap, inv_cap);
  }
}

template <int N>
__device__ __forceinline__ void lse_accum(const float* z, float& m, float& s) {
  float zm = z[0];
#pragma unroll
  for (int e = 1; e < N; ++e) zm = z[e] > zm ? z[e] : zm;
  float part = 0.0f;
#pragma unroll
  for (int e = 0; e < N; ++e) part += __expf(z[e] - zm);
  lse_merge(m, s, zm, part);
}

template <bool VEC>
__global__ __launch_bounds__(kXentThreads) void xent_fwd_kernel(const uint16_t* __restrict__ logits,
                                                               const int64_t* __restrict__ tgt,
                                                               int64_t V, float cap, float inv_cap,
                                                               float* __restrict__ row_loss,
                                                               float* __restrict__ row_lse) {
  const int64_t row = blockIdx.x;
  const uint16_t* lr = logits + row * V;
  float m = -__builtin_inff(), s = 0.0f;
  if (VEC) {
    const uint4* p = reinterpret_cast<const uint4*>(lr);
    const int64_t n8 = V / 8;
    int64_t c = threadIdx.x;
    for (; c + (kXentUnroll - 1) * kXentThreads < n8; c += kXentUnroll * kXentThreads) {
      uint4 w[kXentUnroll];
#pragma unroll
      for (int u = 0; u < kXentUnroll; ++u) w[u] = ldg_stream(p + c + u * kXentThreads);
      float z[8 * kXentUnroll];
#pragma unroll
      for (int u = 0; u < kXentUnroll; ++u) capped8(w[u], cap, inv_cap, z + 8 * u);
      lse_accum<8 * kXentUnroll>(z, m, s);
    }
    for (; c < n8; c += kXentThreads) {
      float z[8];
      capped8(ldg_stream(p + c), cap, inv_cap, z);
      lse_accum<8>(z, m, s);
    }
  } else {
    for (int64_t i = threadIdx.x; i < V; i += kXentThreads) {
      const float z = capped(__uint_as_float((uint32_t)lr[i] << 16), cap, inv_cap);
      lse_merge(m, s, z, 1.0f);
    }
  }
  const float lse = block_lse(m, s);
  if (threadIdx.x == 0) {
    const int64_t t = tgt[row];
    float zt = __builtin_nanf("");
    if (t >= 0 && t < V) zt = capped(__uint_as_float((uint32_t)lr[t] << 16), cap, inv_cap);
    row_loss[row] = lse - zt;
    row_lse[row] = lse;
  }
}

template <bool VEC>
__global__ __launch_bounds__(kXentThreads) void xent_bwd_kernel(const uint16_t* __restrict__ logits,
                                                               const int64_t* __restrict__ tgt,
                                                               const float* __restrict__ row_lse,
                                                               const float* __restrict__ gptr,
                                                               float gscale,
                                                               const float* __restrict__ roww,
                                                               int64_t V, float cap,
                                                               float inv_cap,
                                                               uint16_t* __restrict__ dlogits) {
  const int64_t row = blockIdx.x;
  const uint16_t* lr = logits + row * V;
  uint16_t* dr = dlogits + row * V;
  const float lse = row_lse[row];
  const float g = *gptr * gscale * (roww ? roww[row] : 1.0f);
  const int64_t t = tgt[row];
  auto grad = [&](float l, int64_t i) {
    float s2;
    const float th = tanh_fast(l * inv_cap, &s2);
    const float p = __expf(cap * th - lse) - (i == t ? 1.0f : 0.0f);
    return p * s2 * g;
  };
  auto grad8 = [&](const uint4& w, int64_t i0) {
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_bf16x2(grad(bf16lo(ww[e]), i0 + 2 * e), grad(bf16hi(ww[e]), i0 + 2 * e + 1));
    return make_uint4(o[0], o[1], o[2], o[3]);
  };
  if (VEC) {
    const uint4* p = reinterpret_cast<const uint4*>(lr);
    uint4* q = reinterpret_cast<uint4*>(dr);
    const int64_t n8 = V / 8;
    int64_t c = threadIdx.x;
    for (; c + (kXentUnroll - 1) * kXentThreads < n8; c += kXentUnroll * kXentThreads) {
      uint4 w[kXentUnroll];
#pragma unroll
      for (int u = 0; u < kXentUnroll; ++u) w[u] = ldg_stream(p + c + u * kXentThreads);
#pragma unroll
      for (int u = 0; u < kXentUnroll; ++u) {
        const int64_t cu = c + u * kXentThreads;
        stg_stream(q + cu, grad8(w[u], 8 * cu));
      }
    }
    for (; c < n8; c += kXentThreads) stg_stream(q + c, grad8(ldg_stream(p + c), 8 * c));
  } else {
    for (int64_t i = threadIdx.x; i < V; i += kXentThreads) {
      const float d = grad(__uint_as_float((uint32_t)lr[i] << 16), i);
      dr[i] = (uint16_t)(pack_bf16x2(d, 0.0f) & 0xFFFFu);
    }
  }
}

}  // namespace tg

using namespace tg;

static int xent_check(const void* logits, const int64_t* tgt, int64_t rows, int64_t vocab, float cap) {
  if (rows < 0 || vocab <= 0) return einval("logit_cap_xent: rows must be >= 0 and vocab > 0");
  if (rows > 0x7FFFFFFF) return einval("logit_cap_xent: too many rows");
  if (!(cap > 0.0f) || cap == __builtin_inff()) return einval("logit_cap_xent: cap must be finite and > 0");
  if (rows > 0 && (!logits || !tgt)) return einval("logit_cap_xent: null pointer");
  return TG_OK;
}

extern "C" int tg_logit_cap_xent_fwd(const void* logits, const int64_t* targets, int64_t rows,
                                     int64_t vocab, float cap, float* row_loss, float* row_lse,
                                     void* stream) {
  TG_TRY(xent_check(logits, targets, rows, vocab, cap));
  if (rows == 0) return TG_OK;
  if (!row_loss || !row_lse) return einval("logit_cap_xent_fwd: null pointer");
  const bool vec = vocab % 8 == 0 && aligned(logits, 16);
  auto L = reinterpret_cast<const uint16_t*>(logits);
  if (vec)
    hipLaunchKernelGGL(xent_fwd_kernel<true>, dim3((unsigned)rows), dim3(kXentThreads), 0,
                       as_stream(stream), L, targets, vocab, cap, 1.0f / cap, row_loss, row_lse);
  else
    hipLaunchKernelGGL(xent_fwd_kernel<false>, dim3((unsigned)rows), dim3(kXentThreads), 0,
                       as_stream(stream), L, targets, vocab, cap, 1.0f / cap, row_loss, row_lse);
  return check_launch("logit_cap_xent_fwd");
}

extern "C" int tg_logit_cap_xent_bwd(const void* logits, const int64_t* targets,
                                     const float* row_lse, const float* g, float g_scale,
                                     const float* row_weight, int64_t rows, int64_t vocab,
                                     float cap, void* dlogits, void* stream) {
  TG_TRY(xent_check(logits, targets, rows, vocab, cap));
  if (rows == 0) return TG_OK;
  if (!row_lse || !g || !dlogits) return einval("logit_cap_xent_bwd: null pointer");
  const bool vec = vocab % 8 == 0 && aligned(logits, 16) && aligned(dlogits, 16);
  auto L = reinterpret_cast<const uint16_t*>(logits);
  auto D = reinterpret_cast<uint16_t*>(dlogits);
  if (vec)
    hipLaunchKernelGGL(xent_bwd_kernel<true>, dim3((unsigned)rows), dim3(kXentThreads), 0,
                       as_stream(stream), L, targets, row_lse, g, g_scale, row_weight, vocab, cap,
                       1.0f / cap, D);
  else
    hipLaunchKernelGGL(xent_bwd_kernel<false>, dim3((unsigned)rows), dim3(kXentThreads), 0,
                       as_stream(stream), L, targets, row_lse, g, g_scale, row_weight, vocab, cap,
                       1.0f / cap, D);
  return check_launch("logit_cap_xent_bwd");
}
