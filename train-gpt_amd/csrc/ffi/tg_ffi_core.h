// The logic of the XLA FFI handlers (tg_xla_ffi.cc) over plain pointers and
// shapes: argument checks, dtype dispatch, workspace requests and the calls
// into the C ABI of include/tg_fp8.h.  tg_xla_ffi.cc only turns XLA's buffers,
// attributes and scratch allocator into the types below and a Status back into
// an ffi::Error, so everything here also builds without jaxlib:
// tg_ffi_core_shim.cc exports it over a C ABI (libtg_ffi_core.so) for the
// tests, which run it on the GPU against the library's direct entry points.
//
// Reference interfaces replaced (via the handlers): jax.nn.scaled_matmul
// (/root/reference/fp8.py:70-76) inside _fp8_forward (fp8.py:50-78), the
// quantizer (fp8.py:39-47), both backward rules (fp8.py:85-98), and the
// RMSNorm forward / backward (/root/reference/kernels.py:30-33, 87-97,
// 104-118).
#pragma once
#include <cstddef>
#include <cstdint>

#include "tg_fp8.h"

namespace tgffi {

// Element types as the handlers see them: the C ABI's codes, plus e4m3fn for
// FP8 operands and kOther for anything else XLA may pass.
enum Dtype : int {
  kBF16 = TG_DTYPE_BF16,
  kF32 = TG_DTYPE_F32,
  kF16 = TG_DTYPE_F16,
  kE4M3 = 16,
  kOther = -1,
};

// One operand: device pointer, element type, row-major shape.
struct View {
  void* data;
  int dtype;
  const int64_t* dims;
  int rank;
};

inline int64_t count(const View& v) {
  int64_t n = 1;
  for (int i = 0; i < v.rank; ++i) n *= v.dims[i];
  return n;
}
inline int64_t last_dim(const View& v) { return v.rank == 0 ? 1 : v.dims[v.rank - 1]; }
inline int64_t rows_of(int64_t cnt, int64_t last) { return last == 0 ? 0 : cnt / last; }

// XLA's scratch allocator behind a callback: alloc returns nullptr when it
// cannot serve the request.
struct Scratch {
  void* (*alloc)(void* ctx, size_t bytes, size_t align);
  void* ctx;
};

// kInvalid -> kInvalidArgument, kExhausted -> kResourceExhausted, kInternal
// (a HIP launch failure) -> kInternal.
enum Code : int { kOk = TG_OK, kInvalid = TG_EINVAL, kInternal = TG_EHIP, kExhausted = 100 };
struct Status {
  int code;
  const char* msg;
};

inline Status ok() { return {kOk, ""}; }
inline Status invalid(const char* msg) { return {kInvalid, msg}; }
inline Status from_rc(int rc) {
  if (rc == TG_OK) return ok();
  return {rc == TG_EINVAL ? kInvalid : kInternal, tg_last_error()};
}

inline bool is_float(int d) { return d == kBF16 || d == kF32; }
inline bool is_norm_float(int d) { return is_float(d) || d == kF16; }

// bytes of scratch (256-byte aligned), or nullptr with *st set when the
// allocator refuses; zero bytes need no allocation.
inline void* take(const Scratch& s, size_t bytes, Status* st) {
  if (bytes == 0) return nullptr;
  void* p = s.alloc(s.ctx, bytes, 256);
  if (!p) *st = {kExhausted, "tg_xla_ffi: scratch allocation failed"};
  return p;
}

// _quantize_to_fp8 (fp8.py:39-47) along the last axis: x (..., K) bf16 or f32
// -> q (..., K) e4m3fn, scales (..., K / block_k) f32.
inline Status quantize_rows(void* stream, const View& x, void* q, float* s, int64_t block_k) {
  if (!is_float(x.dtype)) return invalid("tg_quantize_rows: x must be bf16 or f32");
  const int64_t K = last_dim(x);
  return from_rc(tg_quantize_rows(x.data, x.dtype, rows_of(count(x), K), K, (int)block_k,
                                  static_cast<uint8_t*>(q), s, stream));
}

// _quantize_to_fp8 of x.T (fp8.py:68 on b.T): x (R, C) -> q_t (C, R), scales_t (C, R / block_k).
inline Status quantize_cols(void* stream, const View& x, void* q_t, float* s_t, int64_t block_k) {
  if (!is_float(x.dtype) || x.rank != 2) return invalid("tg_quantize_cols: x must be 2-D bf16 or f32");
  return from_rc(tg_quantize_cols(x.data, x.dtype, x.dims[0], x.dims[1], (int)block_k,
                                  static_cast<uint8_t*>(q_t), s_t, stream));
}

// _fp8_forward (fp8.py:50-78): a (..., K) and b (K, N), bf16 or f32 (fp8.py:66,68
// quantize their f32 values) -> out (..., N) bf16.  bf16 operands take the
// composite entry point; any f32 operand the quantizers + GEMM on the same
// scratch, laid out as tg_block_scaled_matmul lays out its workspace.
inline Status block_scaled_matmul(void* stream, const Scratch& scratch, const View& a, const View& b,
                                  void* out, int64_t block_k) {
  if (!is_float(a.dtype) || !is_float(b.dtype) || b.rank != 2)
    return invalid("block_scaled_matmul: a and b must be bf16 or f32, b 2-D");
  const int64_t K = last_dim(a), M = rows_of(count(a), K);
  const int64_t N = b.dims[1];
  Status st = ok();
  const size_t ws_bytes = tg_block_scaled_matmul_workspace(M, N, K, (int)block_k);
  void* ws = take(scratch, ws_bytes, &st);
  if (ws_bytes && !ws) return st;
  if (a.dtype == kBF16 && b.dtype == kBF16)
    return from_rc(tg_block_scaled_matmul(a.data, b.data, out, M, N, K, (int)block_k, ws, ws_bytes, stream));
  if (block_k <= 0 || K % block_k) return invalid("block_scaled_matmul: block_k must be positive and divide K");
  // qa (M, K), sa (M, K / block_k), qb (N, K), sb (N, K / block_k), each
  // 256-byte aligned; the composite's workspace is at least this large for
  // every block_k (it holds K / 128 scales per row for multiples of 128, and
  // K x 128 / block_k bytes per row below 128)
  auto a256 = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t nkb = (size_t)(K / block_k);
  if (ws_bytes < a256((size_t)M * K) + a256((size_t)M * nkb * 4) + a256((size_t)N * K) + (size_t)N * nkb * 4)
    return invalid("block_scaled_matmul: workspace smaller than its operands' FP8 copies");
  uint8_t* p = static_cast<uint8_t*>(ws);
  uint8_t* qa = p;                          p += a256((size_t)M * K);
  float* sa = reinterpret_cast<float*>(p);  p += a256((size_t)M * nkb * 4);
  uint8_t* qb = p;                          p += a256((size_t)N * K);
  float* sb = reinterpret_cast<float*>(p);
  int rc = tg_quantize_rows(a.data, a.dtype, M, K, (int)block_k, qa, sa, stream);
  if (rc == TG_OK) rc = tg_quantize_cols(b.data, b.dtype, K, N, (int)block_k, qb, sb, stream);
  if (rc == TG_OK)
    rc = tg_gemm_fp8_nt(qa, sa, qb, sb, 1, out, TG_DTYPE_BF16, M, N, K, (int)block_k, stream);
  return from_rc(rc);
}

// The FP8 backward rule (the forward's quantize -> scaled GEMM for both
// gradients): a (M, K), b (K, N), g (M, N) bf16 -> da (M, K), db (K, N) bf16.
inline Status block_scaled_matmul_bwd_fp8(void* stream, const Scratch& scratch, const View& a, const View& b,
                                          const View& g, void* da, void* db, int64_t block_k) {
  if (a.dtype != kBF16 || b.dtype != kBF16 || g.dtype != kBF16 || b.rank != 2)
    return invalid("block_scaled_matmul FP8 backward: a, b, g must be bf16, b 2-D");
  const int64_t K = last_dim(a), M = rows_of(count(a), K);
  const int64_t N = b.dims[1];
  Status st = ok();
  const size_t ws_bytes = tg_block_scaled_matmul_bwd_workspace(M, N, K, (int)block_k);
  void* ws = take(scratch, ws_bytes, &st);
  if (ws_bytes && !ws) return st;
  return from_rc(tg_block_scaled_matmul_bwd_fp8(a.data, b.data, g.data, da, db, M, N, K, (int)block_k, ws,
                                                ws_bytes, stream));
}

// _fp8_backward (fp8.py:85-98), the straight-through bf16 rule: a, b, g bf16 or
// f32 -> da, db bf16 (the Python side widens to a.dtype / b.dtype, fp8.py:95-96).
inline Status block_scaled_matmul_bwd_bf16(void* stream, const Scratch& scratch, const View& a, const View& b,
                                           const View& g, void* da, void* db) {
  if (!is_float(a.dtype) || !is_float(b.dtype) || !is_float(g.dtype) || b.rank != 2)
    return invalid("block_scaled_matmul backward: operands must be bf16 or f32, b 2-D");
  const int64_t K = last_dim(a), M = rows_of(count(a), K);
  const int64_t N = b.dims[1];
  Status st = ok();
  const size_t ws_bytes = tg_block_scaled_matmul_bwd_bf16_workspace(M, N, K);
  void* ws = take(scratch, ws_bytes, &st);
  if (ws_bytes && !ws) return st;
  return from_rc(tg_block_scaled_matmul_bwd_bf16(a.data, a.dtype, b.data, b.dtype, g.data, g.dtype, da, db,
                                                 M, N, K, ws, ws_bytes, stream));
}

// _rms_norm_pure (kernels.py:30-33): x (..., D), scale (D,), each bf16, f16 or
// f32 -> y (..., D) in their promoted dtype (the common one, else f32).
inline Status rms_norm(void* stream, const View& x, const View& scale, const View& y, float eps) {
  if (!is_norm_float(x.dtype) || !is_norm_float(scale.dtype) || !is_norm_float(y.dtype) ||
      y.dtype != (x.dtype == scale.dtype ? x.dtype : kF32))
    return invalid("rms_norm: x, scale bf16, f16 or f32; y in their promoted dtype");
  const int64_t D = last_dim(x);
  return from_rc(tg_rms_norm_ex(x.data, x.dtype, scale.data, scale.dtype, y.data, rows_of(count(x), D), D, eps,
                                stream));
}

// The norm fused with the quantization that feeds the next matmul:
// x (..., D), scale (D,) bf16 -> y (..., D) bf16, q (..., D) e4m3fn,
// s (..., D / block_k) f32.
inline Status rms_norm_fp8(void* stream, const View& x, const View& scale, void* y, void* q, float* s,
                           float eps, int64_t block_k) {
  if (x.dtype != kBF16 || scale.dtype != kBF16) return invalid("rms_norm_fp8: x and scale must be bf16");
  const int64_t D = last_dim(x);
  return from_rc(tg_rms_norm_fp8(x.data, scale.data, y, static_cast<uint8_t*>(q), s, rows_of(count(x), D), D,
                                 eps, (int)block_k, stream));
}

// The norm's _bwd (kernels.py:104-118): x, scale, dy bf16, f16 or f32 -> dx
// in x's dtype, dscale in scale's.
inline Status rms_norm_bwd(void* stream, const Scratch& scratch, const View& x, const View& scale,
                           const View& dy, const View& dx, const View& dscale, float eps) {
  if (!is_norm_float(x.dtype) || !is_norm_float(scale.dtype) || !is_norm_float(dy.dtype) ||
      dx.dtype != x.dtype || dscale.dtype != scale.dtype)
    return invalid("rms_norm backward: bf16 / f16 / f32 operands; dx in x's dtype, dscale in scale's");
  const int64_t D = last_dim(x), rows = rows_of(count(x), D);
  Status st = ok();
  const size_t ws_bytes = tg_rms_norm_bwd_workspace(rows, D);
  void* ws = take(scratch, ws_bytes, &st);
  if (ws_bytes && !ws) return st;
  return from_rc(tg_rms_norm_bwd_ex(x.data, x.dtype, scale.data, scale.dtype, dy.data, dy.dtype, dx.data,
                                    dscale.data, rows, D, eps, ws, ws_bytes, stream));
}

// The scaled GEMM alone on pre-quantized operands (a kept weight's bytes and
// scales, fp8.py:68 done once): a_q (M, K), a_s (M, K/128), b_q (N, K),
// b_s (N or ceil(N/128), K/128) -> c (M, N) bf16.
inline Status gemm_fp8_nt(void* stream, const View& a_q, const float* a_s, const View& b_q, const float* b_s,
                          void* c, int64_t b_scale_bn) {
  if (a_q.dtype != kE4M3 || b_q.dtype != kE4M3 || b_q.rank != 2)
    return invalid("gemm_fp8_nt: a_q and b_q must be e4m3fn, b_q 2-D");
  const int64_t K = last_dim(a_q), M = rows_of(count(a_q), K);
  const int64_t N = b_q.dims[0];
  return from_rc(tg_gemm_fp8_nt(static_cast<const uint8_t*>(a_q.data), a_s, static_cast<const uint8_t*>(b_q.data),
                                b_s, (int)b_scale_bn, c, TG_DTYPE_BF16, M, N, K, 128, stream));
}

}  // namespace tgffi
