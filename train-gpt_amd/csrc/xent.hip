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
// Two implementations:
//  * table (0 < cap <= 24): a bf16 logit has one of 65536 values, and for
//    |l| < 2^-24 or |l| >= 256 the needed quantities are constant to within
//    one f32 ulp (exp(l - cap) ~ exp(-cap); tanh(l / cap) rounds to +-1 for
//    |l| / cap > 9.1).  Each workgroup builds, with the accurate tanhf / expf,
//    a table over the 4096 magnitudes in between: exp(z - cap) for l > 0 and
//    l < 0 (and sech^2(l / cap) for the backward), 32 KiB (48 KiB) in LDS, then
//    walks rows: per element a few integer ops, one (two) LDS lookups and an
//    add (two multiplies).  z <= cap, so exp(z - cap) <= 1 needs no running
//    max, and exp(-2 cap) stays a normal f32.  Workgroups loop over rows so the
//    table is built once per workgroup.  A NaN logit makes its row's loss and
//    gradient NaN (tracked by the largest magnitude bit pattern seen).
//  * direct (any other cap): tanh on the hardware exponential and reciprocal
//    (absolute error ~2e-7, so z is within ~3e-6 of cap * tanh(l / cap)) and a
//    running-max log-sum-exp.
// A target outside [0, vocab) gives a NaN loss and no one-hot term in the
// gradient.
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

// ---------------------------------------------------------------------------
// Table implementation
// ---------------------------------------------------------------------------
constexpr int kLutN = 4096;                   // magnitudes 2^-24 .. 256 - ulp
constexpr uint32_t kLutLo = 103u << 7;        // bf16 bits of 2^-24
constexpr float kLutCapMax = 24.0f;
constexpr int kLutGridFwd = 1024, kLutGridBwd = 768;   // 4 (3) workgroups per CU on 256 CUs

// lut[k] = exp(z - cap), lut[kLutN + k] = exp(-z - cap) with z = cap tanh(l / cap)
// for l = bf16 bits kLutLo + k; with S2 also lut[2 kLutN + k] = sech^2(l / cap)
// = 4 e / (1 + e)^2, e = exp(-2 l / cap) (no cancellation near tanh = 1).
template <bool S2>
__device__ __forceinline__ void build_lut(float* lut, float cap) {
  for (int k = threadIdx.x; k < kLutN; k += blockDim.x) {
    const float l = __uint_as_float((kLutLo + (uint32_t)k) << 16);
    const float x = l / cap;
    const float z = cap * tanhf(x);
    lut[k] = expf(z - cap);
    lut[kLutN + k] = expf(-z - cap);
    if (S2) {
      const float e = expf(-2.0f * x);
      const float r = 1.0f + e;
      lut[2 * kLutN + k] = 4.0f * e / (r * r);
    }
  }
  __syncthreads();
}

// Byte offset of the exp(z - cap) entry of the bf16 value in bits 0..15 (HI:
// 16..31) of w; mag gets its magnitude bits.  The sign selects the second
// half of the table (+16 KiB).
template <bool HI>
__device__ __forceinline__ uint32_t lut_off(uint32_t w, uint32_t& mag) {
  mag = HI ? (w >> 16) & 0x7FFFu : w & 0x7FFFu;
  const uint32_t c = min(max(mag, kLutLo), kLutLo + (uint32_t)kLutN - 1u);
  const uint32_t sgn = (HI ? (w >> 17) : (w >> 1)) & 0x4000u;
  return ((c - kLutLo) << 2) | sgn;
}

__device__ __forceinline__ float lut_at(const float* lut, uint32_t off) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(lut) + off);
}

// Sum over the workgroup in a fixed order (wave shuffles, then waves 0..7),
// and the largest magnitude pattern; red holds 2 x 8 words.  Ends with a
// barrier, so red may be reused at once.
__device__ __forceinline__ float block_sum_max(float s, uint32_t& mx, float* red) {
  for (int off = 32; off > 0; off >>= 1) {
    s += __shfl_xor(s, off, 64);
    mx = max(mx, (uint32_t)__shfl_xor((int)mx, off, 64));
  }
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) { red[wave] = s; reinterpret_cast<uint32_t*>(red)[8 + wave] = mx; }
  __syncthreads();
  float t = red[0];
  uint32_t m = reinterpret_cast<uint32_t*>(red)[8];
  for (int w = 1; w < kXentThreads / 64; ++w) {
    t += red[w];
    m = max(m, reinterpret_cast<uint32_t*>(red)[8 + w]);
  }
  mx = m;
  __syncthreads();
  return t;
}

template <bool VEC>
__global__ __launch_bounds__(kXentThreads) __attribute__((amdgpu_waves_per_eu(8))) void xent_fwd_lut_kernel(const uint16_t* __restrict__ logits,
                                                                   const int64_t* __restrict__ tgt,
                                                                   int64_t rows, int64_t V, float cap,
                                                                   float* __restrict__ row_loss,
                                                                   float* __restrict__ row_lse) {
  __shared__ float lut[2 * kLutN];
  __shared__ float red[16];
  build_lut<false>(lut, cap);
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const uint16_t* lr = logits + row * V;
    float s = 0.0f;
    uint32_t mx = 0;
    auto add_word = [&](uint32_t w) {
      uint32_t m0, m1;
      const uint32_t o0 = lut_off<false>(w, m0), o1 = lut_off<true>(w, m1);
      s += lut_at(lut, o0) + lut_at(lut, o1);
      mx = max(mx, max(m0, m1));
    };
    if (VEC) {
      const uint4* p = reinterpret_cast<const uint4*>(lr);
      const int64_t n8 = V / 8;
      int64_t c = threadIdx.x;
      for (; c + (kXentUnroll - 1) * kXentThreads < n8; c += kXentUnroll * kXentThreads) {
        uint4 w[kXentUnroll];
#pragma unroll
        for (int u = 0; u < kXentUnroll; ++u) w[u] = ldg_stream(p + c + u * kXentThreads);
#pragma unroll
        for (int u = 0; u < kXentUnroll; ++u) {
          add_word(w[u].x); add_word(w[u].y); add_word(w[u].z); add_word(w[u].w);
        }
      }
      for (; c < n8; c += kXentThreads) {
        const uint4 w = ldg_stream(p + c);
        add_word(w.x); add_word(w.y); add_word(w.z); add_word(w.w);
      }
    } else {
      for (int64_t i = threadIdx.x; i < V; i += kXentThreads) {
        uint32_t m;
        s += lut_at(lut, lut_off<false>((uint32_t)lr[i], m));
        mx = max(mx, m);
      }
    }
    const float S = block_sum_max(s, mx, red);
    if (threadIdx.x == 0) {
      const int64_t t = tgt[row];
      const float lse = mx > 0x7F80u ? __builtin_nanf("") : cap + logf(S);
      float zt = __builtin_nanf("");
      if (t >= 0 && t < V) zt = cap * tanhf(__uint_as_float((uint32_t)lr[t] << 16) / cap);
      row_loss[row] = lse - zt;
      row_lse[row] = lse;
    }
  }
}

template <bool VEC>
__global__ __launch_bounds__(kXentThreads) __attribute__((amdgpu_waves_per_eu(6))) void xent_bwd_lut_kernel(const uint16_t* __restrict__ logits,
                                                                   const int64_t* __restrict__ tgt,
                                                                   const float* __restrict__ row_lse,
                                                                   const float* __restrict__ gptr,
                                                                   float gscale,
                                                                   const float* __restrict__ roww,
                                                                   int64_t rows, int64_t V, float cap,
                                                                   uint16_t* __restrict__ dlogits) {
  __shared__ float lut[3 * kLutN];
  build_lut<true>(lut, cap);
  const float g0 = *gptr * gscale;
  for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
    const uint16_t* lr = logits + row * V;
    uint16_t* dr = dlogits + row * V;
    const float g = g0 * (roww ? roww[row] : 1.0f);
    // softmax = exp(z - lse) = exp(z - cap) * exp(cap - lse)
    const float cg = expf(cap - row_lse[row]) * g;
    const int64_t t = tgt[row];
    // d = g (p - onehot) sech^2 with p = E * exp(cap - lse)
    auto grad = [&](uint32_t off, int64_t i) {
      const float e = lut_at(lut, off);
      const float s2 = lut_at(lut + 2 * kLutN, off & 0x3FFFu);
      const float d = e * cg * s2;
      return i == t ? d - g * s2 : d;
    };
    auto grad_fast = [&](uint32_t off) {
      return lut_at(lut, off) * cg * lut_at(lut + 2 * kLutN, off & 0x3FFFu);
    };
    if (VEC) {
      const uint4* p = reinterpret_cast<const uint4*>(lr);
      uint4* q = reinterpret_cast<uint4*>(dr);
      const int64_t n8 = V / 8;
      auto grad8 = [&](const uint4& w, int64_t c) {
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
        uint32_t o[4];
        uint32_t m;
        if ((uint64_t)(t - 8 * c) < 8u) {            // the target is in this chunk
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = pack_bf16x2(grad(lut_off<false>(ww[e], m), 8 * c + 2 * e),
                               grad(lut_off<true>(ww[e], m), 8 * c + 2 * e + 1));
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            o[e] = pack_bf16x2(grad_fast(lut_off<false>(ww[e], m)), grad_fast(lut_off<true>(ww[e], m)));
        }
        return make_uint4(o[0], o[1], o[2], o[3]);
      };
      int64_t c = threadIdx.x;
      for (; c + (kXentUnroll - 1) * kXentThreads < n8; c += kXentUnroll * kXentThreads) {
        uint4 w[kXentUnroll];
#pragma unroll
        for (int u = 0; u < kXentUnroll; ++u) w[u] = ldg_stream(p + c + u * kXentThreads);
#pragma unroll
        for (int u = 0; u < kXentUnroll; ++u) {
          const int64_t cu = c + u * kXentThreads;
          stg_stream(q + cu, grad8(w[u], cu));
        }
      }
      for (; c < n8; c += kXentThreads) stg_stream(q + c, grad8(ldg_stream(p + c), c));
    } else {
      for (int64_t i = threadIdx.x; i < V; i += kXentThreads) {
        uint32_t m;
        const float d = grad(lut_off<false>((uint32_t)lr[i], m), i);
        dr[i] = (uint16_t)(pack_bf16x2(d, 0.0f) & 0xFFFFu);
      }
    }
  }
}

// z = cap * tanh(l * inv_cap), f32, from bf16 logits l: model.py:97 on the
// decode step's unembedding rows, with torch's arithmetic for
// `cap * torch.tanh(l.float() / cap)` (a division by a scalar is a multiply by
// its f32 reciprocal, then the device tanhf and one f32 multiply), so the
// same bits in one launch instead of four
__global__ __launch_bounds__(256) void logit_cap_kernel(const uint16_t* __restrict__ l, float* __restrict__ z,
                                                        int64_t n, float cap, float inv_cap) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) z[i] = cap * tanhf(bf16lo(l[i]) * inv_cap);
}

}  // namespace tg

using namespace tg;

extern "C" int tg_logit_cap(const void* logits, float* out, int64_t n, float cap, void* stream) {
  if (n < 0) return einval("logit_cap: n must be >= 0");
  if (!(cap > 0.0f) || cap == __builtin_inff()) return einval("logit_cap: cap must be finite and > 0");
  if (n == 0) return TG_OK;
  if (!logits || !out) return einval("logit_cap: null pointer");
  if ((n + 255) / 256 > 0x7FFFFFFF) return einval("logit_cap: n too large");
  const float inv_cap = 1.0f / cap;   // the f32 reciprocal torch multiplies by
  hipLaunchKernelGGL(logit_cap_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint16_t*>(logits), out, n, cap, inv_cap);
  return check_launch("logit_cap");
}

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
  if (cap <= kLutCapMax) {
    const dim3 grid((unsigned)(rows < kLutGridFwd ? rows : kLutGridFwd));
    if (vec)
      hipLaunchKernelGGL(xent_fwd_lut_kernel<true>, grid, dim3(kXentThreads), 0, as_stream(stream), L,
                         targets, rows, vocab, cap, row_loss, row_lse);
    else
      hipLaunchKernelGGL(xent_fwd_lut_kernel<false>, grid, dim3(kXentThreads), 0, as_stream(stream), L,
                         targets, rows, vocab, cap, row_loss, row_lse);
    return check_launch("logit_cap_xent_fwd");
  }
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
  if (cap <= kLutCapMax) {
    const dim3 grid((unsigned)(rows < kLutGridBwd ? rows : kLutGridBwd));
    if (vec)
      hipLaunchKernelGGL(xent_bwd_lut_kernel<true>, grid, dim3(kXentThreads), 0, as_stream(stream), L,
                         targets, row_lse, g, g_scale, row_weight, rows, vocab, cap, D);
    else
      hipLaunchKernelGGL(xent_bwd_lut_kernel<false>, grid, dim3(kXentThreads), 0, as_stream(stream), L,
                         targets, row_lse, g, g_scale, row_weight, rows, vocab, cap, D);
    return check_launch("logit_cap_xent_bwd");
  }
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
