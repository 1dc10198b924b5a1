// Device helpers shared by the gfx950 kernels of the FP8 hot path.
//
// Numeric contract (restating /root/reference/fp8.py:39-47 and
// /root/reference/kernels.py:30-33 bit for bit):
//   * e4m3fn: OCP E4M3 (bias 7, max 448 = 0x7E, 0x7F/0xFF NaN, no inf),
//     round-to-nearest-even, non-saturating.
//   * x / s is an IEEE f32 divide.  For bf16 inputs it is evaluated as
//     y = 1/s, q0 = x*y, nr = fma(q0, s, -x), q = fma(-nr, y, q0).
//     Over every bf16 amax a (s = max(a/448, 1e-30))
//     and every bf16 x with |x| <= a this gives the same e4m3fn byte as the
//     IEEE quotient, and the same f32 quotient whenever |x/s| > 2^-10 (below
//     that both encode to +-0); the residual only underflows when s is the
//     1e-30 floor and |x| is near the f32 subnormal range.  Checked
//     exhaustively on the host (tests/csrc/div_identity.c) and on the GPU
//     (tg_selftest_divide).
//   * bf16 rounding is RNE (v_cvt_pk_bf16_f32).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tg {

constexpr float kE4M3Max = 448.0f;
constexpr float kScaleFloor = 1e-30f;   // fp8.py:44; f32 bits 0x0DA24260

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte streaming load (data read once: non-temporal hint).
__device__ __forceinline__ uint4 ldg_stream(const void* p) {
  u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// Streaming stores (written once, not re-read by this kernel).
__device__ __forceinline__ void stg_stream(uint4* p, const uint4& v) {
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x4_t*>(p));
}
__device__ __forceinline__ void stg_stream(uint2* p, const uint2& v) {
  const u32x2_t w = {v.x, v.y};
  __builtin_nontemporal_store(w, reinterpret_cast<u32x2_t*>(p));
}

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Two f32 -> packed bf16 (lo in bits 0..15), round-to-nearest-even: one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const f32x2_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

// f32 -> bf16 -> f32 (the value a bf16 tensor would hold).
__device__ __forceinline__ float round_bf16(float x) {
  return __uint_as_float(((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)x)) << 16);
}

// Software e4m3fn encoder (integer RNE on the f32 bits).  Used for the
// non-finite-scale path and as the check of the hardware convert.
__device__ __forceinline__ uint32_t e4m3_sw(float v) {
  uint32_t bits = __float_as_uint(v);
  uint32_t sign = (bits >> 24) & 0x80u;
  uint32_t a = bits & 0x7FFFFFFFu;
  int code_n = (int)((a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - (120 << 3);
  // 2^14 has f32 ulp 2^-9 (the e4m3 subnormal step): the adder rounds |v| (RNE)
  float t = __uint_as_float(a) + 16384.0f;
  int code_s = (int)__float_as_uint(t) - 0x46800000;
  int code = a < 0x3C800000u ? code_s : code_n;
  if (code > 0x7E || a >= 0x7F800000u) code = 0x7F;
  return sign | (uint32_t)code;
}

// Four f32 -> four e4m3fn bytes packed little-endian (a = byte 0).
// TG_FP8_SW_CVT selects the integer encoder; the default is the gfx950
// v_cvt_pk_fp8_f32 convert (OCP e4m3fn, RNE), whose agreement with e4m3_sw is
// checked over every f32 bit pattern by tg_selftest_fp8_cvt.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
#ifdef TG_FP8_SW_CVT
  return e4m3_sw(a) | (e4m3_sw(b) << 8) | (e4m3_sw(c) << 16) | (e4m3_sw(d) << 24);
#else
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
#endif
}

__device__ __forceinline__ uint32_t e4m3x4_sw(float a, float b, float c, float d) {
  return e4m3_sw(a) | (e4m3_sw(b) << 8) | (e4m3_sw(c) << 16) | (e4m3_sw(d) << 24);
}

// Scale of one block from the NaN-propagating amax (carried as |x| bits:
// integer max over abs bit patterns is the IEEE max with NaN winning).
__device__ __forceinline__ float block_scale(uint32_t amax_bits) {
  float amax = __uint_as_float(amax_bits);
  float s = amax / kE4M3Max;                       // IEEE f32 divide
  return (s < kScaleFloor) ? kScaleFloor : s;      // jnp.maximum; NaN stays NaN
}

// The same scale for a bf16-valued amax: fl32(amax / 448) by one refinement
// of amax * fl32(1/448) (three VALU instead of the IEEE divide sequence; equal
// to the IEEE quotient for every bf16 amax, checked by tg_selftest_divide and
// tests/csrc/div_identity.c).  The refinement turns +inf into NaN, so +inf is
// restored explicitly; NaN propagates.
__device__ __forceinline__ float block_scale_bf16(uint32_t amax_bits) {
  const float amax = __uint_as_float(amax_bits);
  constexpr float c = 1.0f / 448.0f;
  const float q0 = amax * c;
  const float r = __builtin_fmaf(-q0, kE4M3Max, amax);
  float s = __builtin_fmaf(r, c, q0);
  if (amax_bits == 0x7F800000u) s = __builtin_inff();
  return (s < kScaleFloor) ? kScaleFloor : s;
}

// |x| bits (as f32 bits) of the larger-magnitude of the two bf16 values in w.
__device__ __forceinline__ uint32_t bf16_amax2(uint32_t w) {
  return max((w << 16) & 0x7FFFFFFFu, w & 0x7FFF0000u);
}

struct Divider {
  float s, y;
  bool fast;
  // y = fl32(1/s): v_rcp_f32 plus one Newton step (equal to the IEEE
  // reciprocal for every scale a bf16 amax can produce, checked by
  // tg_selftest_divide).  A finite scale is >= 1e-30, so s and 1/s are normal.
  __device__ __forceinline__ explicit Divider(float scale) : s(scale) {
    const float y0 = __builtin_amdgcn_rcpf(scale);
    y = __builtin_fmaf(__builtin_fmaf(-scale, y0, 1.0f), y0, y0);
    fast = (__float_as_uint(scale) & 0x7F800000u) != 0x7F800000u;
  }
  // x / s for bf16-valued x and finite s (see header comment):
  // q0 = x*y, nr = q0*s - x (exact), q = q0 - nr*y.  The residual is formed
  // negated so that x = -0 yields -0.
  __device__ __forceinline__ float div(float x) const {
    const float q0 = x * y;
    const float nr = __builtin_fmaf(q0, s, -x);
    return __builtin_fmaf(-nr, y, q0);
  }
};

// Slow path for a non-finite scale, matching the x86 IEEE quotient the
// reference's CPU path produces: s NaN -> x's NaN if x is NaN else s's (+)NaN;
// s = +inf -> +-0 for finite x, and inf/inf -> the default (negative) NaN.
__device__ __forceinline__ uint32_t e4m3_nonfinite_scale(float x, float s) {
  uint32_t xb = __float_as_uint(x);
  bool xnan = (xb & 0x7FFFFFFFu) > 0x7F800000u;
  if ((__float_as_uint(s) & 0x7FFFFFFFu) > 0x7F800000u)
    return xnan ? (((xb >> 24) & 0x80u) | 0x7Fu) : 0x7Fu;
  if ((xb & 0x7FFFFFFFu) == 0x7F800000u) return 0xFFu;
  return (xb >> 24) & 0x80u;
}

// ---- cross-lane reductions (wave64) -------------------------------------
// DPP row operations act within rows of 16 lanes.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}
// max over the 16 lanes of a DPP row (all lanes receive the result)
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));    // quad_perm [1,0,3,2]
  v = max(v, dpp_u32<0x4E>(v));    // quad_perm [2,3,0,1]
  v = max(v, dpp_u32<0x141>(v));   // row_half_mirror
  v = max(v, dpp_u32<0x140>(v));   // row_mirror
  return v;
}
// max over the 4 lanes of a quad
__device__ __forceinline__ uint32_t quad_max_u32(uint32_t v) {
  v = max(v, dpp_u32<0xB1>(v));
  v = max(v, dpp_u32<0x4E>(v));
  return v;
}

__device__ __forceinline__ double shfl_xor_f64(double v, int m) {
  int lo = __double2loint(v), hi = __double2hiint(v);
  lo = __shfl_xor(lo, m, 64);
  hi = __shfl_xor(hi, m, 64);
  return __hiloint2double(hi, lo);
}

template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xF, 0xF, false);
  return __hiloint2double(hi, lo);
}

// Sum over the 64 lanes, every lane getting the same value, in VALU only:
// four DPP steps inside each 16-lane row (pairs, quads, half rows, rows),
// then the gfx950 row swaps (v_permlane16_swap: rows 0<->1 and 2<->3,
// v_permlane32_swap: the two halves).  Each step adds a lane's value to its
// partner's, and both partners form the same sum (IEEE addition commutes),
// so the result is identical in all lanes.
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<0xB1>(v);     // quad_perm [1,0,3,2]
  v += dpp_f64<0x4E>(v);     // quad_perm [2,3,0,1]
  v += dpp_f64<0x141>(v);    // row_half_mirror
  v += dpp_f64<0x140>(v);    // row_mirror
  {
    const int lo = __double2loint(v), hi = __double2hiint(v);
    const auto l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    v = __hiloint2double((int)h[0], (int)l[0]) + __hiloint2double((int)h[1], (int)l[1]);
  }
  {
    const int lo = __double2loint(v), hi = __double2hiint(v);
    const auto l = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto h = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    v = __hiloint2double((int)h[0], (int)l[0]) + __hiloint2double((int)h[1], (int)l[1]);
  }
  return v;
}

}  // namespace tg
