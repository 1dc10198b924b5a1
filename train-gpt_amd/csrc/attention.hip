// Decode attention over a KV cache, fused with the cache append and with the
// FP8 quantization of its output (the input of the output projection).
//
// One decode step of /root/reference/model.py:59-68 for one new token per
// sequence at position t (read from device memory, so a captured HIP graph
// replays the step for every position):
//   K[b, h, t] = k, V[b, h, t] = v                      (cache append)
//   o[b, h]    = softmax(q . K[b, h, 0..t]^T / sqrt(Dh)) V[b, h, 0..t]
//   o_bf16     = bf16(o);  (o_q, o_s) = _quantize_to_fp8(o_bf16)   fp8.py:39-47
// Dh is 128: one head is exactly one 128-wide scale block, so the quantization
// of o is local to the workgroup that computes the head.
//
// One workgroup per (sequence, head), 4 waves.  Lane l works on dims
// 8 (l % 16) .. +7 of key (l / 16) of a group of four keys per wave, so a
// K or V row slice is one 16-byte load and the dot product is reduced over a
// 16-lane DPP row.  Each lane row keeps an online softmax (running max, sum
// and 8 weighted-V accumulators, f32) over its keys; the 16 partial states
// are merged through LDS.  The new key is taken from the projection output,
// not read back from the cache.
#include "tg_device.h"
#include "tg_host.h"
#include "gemm_tile.h"

namespace tg {

constexpr int kAttnDh = 128;
constexpr int kAttnWaves = 4;
constexpr int kAttnUnroll = 4;        // key groups in flight per wave

__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // half mirror
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));  // mirror
  return v;
}

// One group of kAttnUnroll key slices per lane: keys (i0 + u) * 16 + 4 wave + kr.
// Rows at or past S fall outside the buffer and read zero (they are never used).
struct KvGroup {
  uint4 k[kAttnUnroll], v[kAttnUnroll];
};

__device__ __forceinline__ void kv_load(KvGroup& G, const __amdgpu_buffer_rsrc_t& rk,
                                        const __amdgpu_buffer_rsrc_t& rv, int64_t i0, int wave, int kr,
                                        int dl) {
#pragma unroll
  for (int u = 0; u < kAttnUnroll; ++u) {
    const int64_t j = (i0 + u) * (4 * kAttnWaves) + 4 * wave + kr;
    const uint32_t off = (uint32_t)((j * kAttnDh + dl * 8) * 2);   // S <= 2^23 keeps this below 2^32
    const u32x4_t a = __builtin_amdgcn_raw_buffer_load_b128(rk, off, 0, 0);
    const u32x4_t b = __builtin_amdgcn_raw_buffer_load_b128(rv, off, 0, 0);
    G.k[u] = make_uint4(a.x, a.y, a.z, a.w);
    G.v[u] = make_uint4(b.x, b.y, b.z, b.w);
  }
}

// online-softmax update of a lane row with the keys of group G; keys past t
// are skipped, key t is the new (k, v) from the projection output
__device__ __forceinline__ void kv_step(const KvGroup& G, int64_t i0, int64_t t, int wave, int kr,
                                        const float (&qf)[8], const uint4& knew, const uint4& vnew, float scale,
                                        float& m, float& l, float (&acc)[8]) {
#pragma unroll
  for (int u = 0; u < kAttnUnroll; ++u) {
    const int64_t j = (i0 + u) * (4 * kAttnWaves) + 4 * wave + kr;
    const uint4 k = j < t ? G.k[u] : knew, v = j < t ? G.v[u] : vnew;
    float d = qf[0] * bf16lo(k.x);
    d = __builtin_fmaf(qf[1], bf16hi(k.x), d);
    d = __builtin_fmaf(qf[2], bf16lo(k.y), d);
    d = __builtin_fmaf(qf[3], bf16hi(k.y), d);
    d = __builtin_fmaf(qf[4], bf16lo(k.z), d);
    d = __builtin_fmaf(qf[5], bf16hi(k.z), d);
    d = __builtin_fmaf(qf[6], bf16lo(k.w), d);
    d = __builtin_fmaf(qf[7], bf16hi(k.w), d);
    const float sc = row16_sum(d) * scale;
    if (j <= t) {                                        // uniform over the 16-lane row
      const float mn = sc > m ? sc : m;
      const float corr = __expf(m - mn), p = __expf(sc - mn);
      l = l * corr + p;
      acc[0] = __builtin_fmaf(p, bf16lo(v.x), acc[0] * corr);
      acc[1] = __builtin_fmaf(p, bf16hi(v.x), acc[1] * corr);
      acc[2] = __builtin_fmaf(p, bf16lo(v.y), acc[2] * corr);
      acc[3] = __builtin_fmaf(p, bf16hi(v.y), acc[3] * corr);
      acc[4] = __builtin_fmaf(p, bf16lo(v.z), acc[4] * corr);
      acc[5] = __builtin_fmaf(p, bf16hi(v.z), acc[5] * corr);
      acc[6] = __builtin_fmaf(p, bf16lo(v.w), acc[6] * corr);
      acc[7] = __builtin_fmaf(p, bf16hi(v.w), acc[7] * corr);
      m = mn;
    }
  }
}

__global__ __launch_bounds__(kAttnWaves * 64) void decode_attention_kernel(
    const uint16_t* __restrict__ qkv, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
    const int64_t* __restrict__ tpos, uint8_t* __restrict__ oq, float* __restrict__ os,
    uint16_t* __restrict__ ob, int H, int S, float scale) {
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh - b * H;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int dl = lane & 15, kr = lane >> 4;            // dims 8 dl .. +7 of key row kr
  const int hd = H * kAttnDh;
  const uint16_t* row = qkv + (int64_t)b * 3 * hd;
  const int64_t cbase = ((int64_t)b * H + h) * S * kAttnDh;   // (b, h, 0, 0) of the caches
  // the first key group's loads do not wait for t: rows past t are read and
  // not used, rows past S read zero (the buffers span this head's S rows)
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kc + cbase, (uint32_t)S * kAttnDh * 2u);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vc + cbase, (uint32_t)S * kAttnDh * 2u);
  // this head's q, k, v are read before t (they do not depend on it): the
  // first key group's arithmetic then waits for one round trip, not for t's
  // and then q's
  KvGroup A, B;
  kv_load(A, rk, rv, 0, wave, kr, dl);
  const uint4 qw = *reinterpret_cast<const uint4*>(row + h * kAttnDh + dl * 8);
  const uint4 knew = *reinterpret_cast<const uint4*>(row + hd + h * kAttnDh + dl * 8);
  const uint4 vnew = *reinterpret_cast<const uint4*>(row + 2 * hd + h * kAttnDh + dl * 8);
  const int64_t t = *tpos;
  if (t < 0 || t >= S) {                   // position outside the cache: touch nothing
    if (threadIdx.x == 0) os[(int64_t)b * H + h] = __builtin_nanf("");
    return;
  }

  float qf[8];
  qf[0] = bf16lo(qw.x); qf[1] = bf16hi(qw.x); qf[2] = bf16lo(qw.y); qf[3] = bf16hi(qw.y);
  qf[4] = bf16lo(qw.z); qf[5] = bf16hi(qw.z); qf[6] = bf16lo(qw.w); qf[7] = bf16hi(qw.w);
  if (wave == 0 && kr == 0) {                           // append k, v at position t
    *reinterpret_cast<uint4*>(kc + cbase + t * kAttnDh + dl * 8) = knew;
    *reinterpret_cast<uint4*>(vc + cbase + t * kAttnDh + dl * 8) = vnew;
  }

  // online softmax over keys j = 16 i + 4 wave + kr (i = 0, 1, ...), j <= t;
  // two key groups in flight: the next group's loads go out before the
  // current group's arithmetic (whole pairs in the loop, no exit inside it)
  float m = -__builtin_inff(), l = 0.0f, acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
  const int64_t nk = t + 1;
  const int64_t ngroups = (nk + 4 * kAttnWaves - 1) / (4 * kAttnWaves);
  const int64_t nit = (ngroups + kAttnUnroll - 1) / kAttnUnroll;   // >= 1
  int64_t i0 = 0;
  for (int64_t p = 0; p + 1 < nit; p += 2) {
    kv_load(B, rk, rv, i0 + kAttnUnroll, wave, kr, dl);
    kv_step(A, i0, t, wave, kr, qf, knew, vnew, scale, m, l, acc);
    kv_load(A, rk, rv, i0 + 2 * kAttnUnroll, wave, kr, dl);
    kv_step(B, i0 + kAttnUnroll, t, wave, kr, qf, knew, vnew, scale, m, l, acc);
    i0 += 2 * kAttnUnroll;
  }
  if (nit & 1) kv_step(A, i0, t, wave, kr, qf, knew, vnew, scale, m, l, acc);

  // merge the 16 partial states (4 key rows x 4 waves) in a fixed order
  __shared__ float sm[16], sl[16];
  __shared__ float sacc[16][kAttnDh];
  const int part = wave * 4 + kr;
  if (dl == 0) { sm[part] = m; sl[part] = l; }
#pragma unroll
  for (int e = 0; e < 8; ++e) sacc[part][dl * 8 + e] = acc[e];
  __syncthreads();
  if (wave != 0 || kr != 0) return;
  float M = sm[0];
  for (int p = 1; p < 16; ++p) M = sm[p] > M ? sm[p] : M;
  float L = 0.0f, o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = 0.0f;
  for (int p = 0; p < 16; ++p) {
    const float w = sl[p] > 0.0f ? __expf(sm[p] - M) : 0.0f;   // empty parts carry nothing
    L = __builtin_fmaf(sl[p], w, L);
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = __builtin_fmaf(sacc[p][dl * 8 + e], w, o[e]);
  }
  const float inv = 1.0f / L;
  uint32_t ow[4];
  float yv[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    ow[e] = pack_bf16x2(o[2 * e] * inv, o[2 * e + 1] * inv);
    yv[2 * e] = bf16lo(ow[e]);
    yv[2 * e + 1] = bf16hi(ow[e]);
  }
  const int64_t oi = (int64_t)b * hd + h * kAttnDh + dl * 8;
  if (ob) *reinterpret_cast<uint4*>(ob + oi) = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  // quantize the bf16 head (one 128-wide block over the 16 lanes of this row)
  uint32_t amb = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) amb = max(amb, __float_as_uint(yv[e]) & 0x7FFFFFFFu);
  amb = row16_max_u32(amb);
  const float sc = block_scale_bf16(amb);
  uint2 qo;
  Divider dv(sc);
  if (dv.fast) {
    qo.x = e4m3x4(dv.div(yv[0]), dv.div(yv[1]), dv.div(yv[2]), dv.div(yv[3]));
    qo.y = e4m3x4(dv.div(yv[4]), dv.div(yv[5]), dv.div(yv[6]), dv.div(yv[7]));
  } else {
    uint32_t bq[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) bq[e] = e4m3_nonfinite_scale(yv[e], sc);
    qo.x = bq[0] | (bq[1] << 8) | (bq[2] << 16) | (bq[3] << 24);
    qo.y = bq[4] | (bq[5] << 8) | (bq[6] << 16) | (bq[7] << 24);
  }
  *reinterpret_cast<uint2*>(oq + oi) = qo;
  if (dl == 0) os[(int64_t)b * H + h] = sc;
}

// The decode step's input rows (model.py:89-90 for one token per sequence):
// out[b] = bf16(embed[tok[b]] + pos[t]), the f32 sum of the two bf16 values
// rounded once (torch's bf16 add).  The rows are read through buffer
// descriptors of the two tables, so a token or position outside them reads a
// zero row and touches no other memory.  One workgroup per sequence, 16-byte
// chunks (d % 8 == 0).
__global__ __launch_bounds__(256) void decode_embed_kernel(const uint16_t* __restrict__ embed,
                                                           const uint16_t* __restrict__ pos,
                                                           const int64_t* __restrict__ tok,
                                                           const int64_t* __restrict__ tpos,
                                                           uint16_t* __restrict__ out, int64_t V, int64_t P, int d) {
  const int b = blockIdx.x;
  const int64_t tk = tok[b], t = *tpos;
  const uint32_t rowb = (uint32_t)d * 2u;
  const __amdgpu_buffer_rsrc_t re = make_rsrc(embed, (uint32_t)V * rowb);
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(pos, (uint32_t)P * rowb);
  const uint32_t eo = tk >= 0 && tk < V ? (uint32_t)tk * rowb : (uint32_t)V * rowb;   // past the end: zeros
  const uint32_t po = t >= 0 && t < P ? (uint32_t)t * rowb : (uint32_t)P * rowb;
  for (int c = threadIdx.x; c < d / 8; c += 256) {
    const u32x4_t e = __builtin_amdgcn_raw_buffer_load_b128(re, eo + (uint32_t)c * 16u, 0, 0);
    const u32x4_t q = __builtin_amdgcn_raw_buffer_load_b128(rp, po + (uint32_t)c * 16u, 0, 0);
    const uint32_t ew[4] = {e.x, e.y, e.z, e.w}, pw[4] = {q.x, q.y, q.z, q.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = pack_bf16x2(bf16lo(ew[i]) + bf16lo(pw[i]), bf16hi(ew[i]) + bf16hi(pw[i]));
    *reinterpret_cast<uint4*>(out + (int64_t)b * d + c * 8) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

}  // namespace tg

using namespace tg;

extern "C" int tg_decode_embed(const void* embed, const void* pos, const int64_t* tok, const int64_t* t,
                               void* out, int64_t B, int64_t V, int64_t P, int64_t d, void* stream) {
  if (B < 0 || V <= 0 || P <= 0 || d <= 0 || d % 8) return einval("decode_embed: bad shape (d a multiple of 8)");
  if (B == 0) return TG_OK;
  if (B > 0x7FFFFFFF || (uint64_t)V * (uint64_t)d * 2u >= (1ull << 32) ||
      (uint64_t)P * (uint64_t)d * 2u >= (1ull << 32))
    return einval("decode_embed: tables too large for 32-bit buffer offsets");
  if (!embed || !pos || !tok || !t || !out) return einval("decode_embed: null pointer");
  if (!aligned(embed, 16) || !aligned(pos, 16) || !aligned(out, 16))
    return einval("decode_embed: embed, pos and out must be 16-byte aligned");
  hipLaunchKernelGGL(decode_embed_kernel, dim3((unsigned)B), dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint16_t*>(embed), reinterpret_cast<const uint16_t*>(pos), tok, t,
                     reinterpret_cast<uint16_t*>(out), V, P, (int)d);
  return check_launch("decode_embed");
}

extern "C" int tg_decode_attention(const void* qkv, void* k_cache, void* v_cache, const int64_t* t,
                                   uint8_t* o_q, float* o_s, void* o, int64_t B, int64_t H,
                                   int64_t S, int64_t head_dim, float scale, void* stream) {
  if (head_dim != kAttnDh) return einval("decode_attention: head_dim must be 128 (one scale block)");
  if (B < 0 || H <= 0 || S <= 0) return einval("decode_attention: bad shape");
  if (B == 0) return TG_OK;
  if (B * H > 0x7FFFFFFF || S > (1 << 23)) return einval("decode_attention: shape too large (S <= 2^23)");
  if (!qkv || !k_cache || !v_cache || !t || !o_q || !o_s) return einval("decode_attention: null pointer");
  if (!aligned(qkv, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16) || !aligned(o_q, 8) ||
      (o && !aligned(o, 16)))
    return einval("decode_attention: qkv and caches must be 16-byte aligned, o_q 8-byte");
  hipLaunchKernelGGL(decode_attention_kernel, dim3((unsigned)(B * H)), dim3(kAttnWaves * 64), 0,
                     as_stream(stream), reinterpret_cast<const uint16_t*>(qkv),
                     reinterpret_cast<uint16_t*>(k_cache), reinterpret_cast<uint16_t*>(v_cache), t,
                     o_q, o_s, reinterpret_cast<uint16_t*>(o), (int)H, (int)S, scale);
  return check_launch("decode_attention");
}
