// XLA FFI handlers over the C ABI of include/tg_fp8.h: what a JAX caller of
// the reference registers with jax.ffi.register_ffi_target(..., platform="ROCM")
// in place of jax.nn.scaled_matmul (/root/reference/fp8.py:70-76) and the
// Pallas RMSNorm (/root/reference/kernels.py:87-97, selected at :124-127).
//
// Built only where jaxlib is installed (it provides xla/ffi/api/ffi.h through
// jax.ffi.include_dir()); train-gpt_amd/build.py skips it otherwise.
//
// Ownership and threading: XLA owns every operand and result buffer and hands
// the stream; workspaces come from XLA's scratch allocator.  The handlers keep
// no state, enqueue only on XLA's stream, never synchronise and never allocate
// device memory themselves, so they are safe to call concurrently from XLA's
// thread pool (the library's one-time per-device setup is std::call_once) and
// can be declared command-buffer compatible.  Shape and dtype checks that must
// raise the reference's ValueError texts (fp8.py:53-56) stay in Python, before
// ffi_call; the library's own checks come back as kInvalidArgument, HIP
// launch failures as kInternal.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "tg_fp8.h"
#include "xla/ffi/api/ffi.h"

namespace ffi = xla::ffi;

namespace {

ffi::Error status(int rc) {
  if (rc == TG_OK) return ffi::Error::Success();
  return ffi::Error(rc == TG_EINVAL ? ffi::ErrorCode::kInvalidArgument : ffi::ErrorCode::kInternal,
                    tg_last_error());
}

// bf16 / f32 operands map onto the C ABI's dtype codes; anything else is refused.
bool dtype_code(ffi::DataType t, int* code) {
  if (t == ffi::DataType::BF16) { *code = TG_DTYPE_BF16; return true; }
  if (t == ffi::DataType::F32) { *code = TG_DTYPE_F32; return true; }
  return false;
}

// The norm entry points also take f16.
bool norm_dtype_code(ffi::DataType t, int* code) {
  if (t == ffi::DataType::F16) { *code = TG_DTYPE_F16; return true; }
  return dtype_code(t, code);
}

template <typename Dims>
int64_t last_dim(const Dims& d) { return d.empty() ? 1 : d.back(); }
int64_t rows_of(int64_t count, int64_t last) { return last == 0 ? 0 : count / last; }

void* take(ffi::ScratchAllocator& scratch, size_t bytes, ffi::Error* err) {
  if (bytes == 0) return nullptr;
  auto p = scratch.Allocate(bytes, 256);
  if (!p.has_value()) {
    *err = ffi::Error(ffi::ErrorCode::kResourceExhausted, "tg_xla_ffi: scratch allocation failed");
    return nullptr;
  }
  return *p;
}

// _quantize_to_fp8 (fp8.py:39-47) along the last axis: x (..., K) bf16 or f32
// -> q (..., K) e4m3fn, scales (..., K / block_k) f32.
ffi::Error QuantizeRows(hipStream_t stream, ffi::AnyBuffer x, ffi::ResultBuffer<ffi::F8E4M3FN> q,
                        ffi::ResultBuffer<ffi::F32> s, int64_t block_k) {
  int code;
  if (!dtype_code(x.element_type(), &code))
    return ffi::Error(ffi::ErrorCode::kInvalidArgument, "tg_quantize_rows: x must be bf16 or f32");
  const int64_t K = last_dim(x.dimensions());
  return status(tg_quantize_rows(x.untyped_data(), code, rows_of(x.element_count(), K), K,
                                 (int)block_k, static_cast<uint8_t*>(q->untyped_data()),
                                 s->typed_data(), stream));
}

// _quantize_to_fp8 of x.T (fp8.py:68 on b.T): x (R, C) -> q_t (C, R), scales_t (C, R / block_k).
ffi::Error QuantizeCols(hipStream_t stream, ffi::AnyBuffer x, ffi::ResultBuffer<ffi::F8E4M3FN> q_t,
                        ffi::ResultBuffer<ffi::F32> s_t, int64_t block_k) {
  int code;
  if (!dtype_code(x.element_type(), &code) || x.dimensions().size() != 2)
    return ffi::Error(ffi::ErrorCode::kInvalidArgument, "tg_quantize_cols: x must be 2-D bf16 or f32");
  return status(tg_quantize_cols(x.untyped_data(), code, x.dimensions()[0], x.dimensions()[1],
                                 (int)block_k, static_cast<uint8_t*>(q_t->untyped_data()),
                                 s_t->typed_data(), stream));
}

// _fp8_forward (fp8.py:50-78): a (..., K) and b (K, N), bf16 or f32 (fp8.py:66,68
// quantize their f32 values) -> out (..., N) bf16.  bf16 operands take the
// composite entry point; f32 operands the quantizers + GEMM on the same scratch.
ffi::Error BlockScaledMatmul(hipStream_t stream, ffi::ScratchAllocator scratch, ffi::AnyBuffer a,
                             ffi::AnyBuffer b, ffi::ResultBuffer<ffi::BF16> out, int64_t block_k) {
  int ca, cb;
  if (!dtype_code(a.element_type(), &ca) || !dtype_code(b.element_type(), &cb) ||
      b.dimensions().size() != 2)
    return ffi::Error(ffi::ErrorCode::kInvalidArgument,
                      "block_scaled_matmul: a and b must be bf16 or f32, b 2-D");
  const int64_t K = last_dim(a.dimensions()), M = rows_of(a.element_count(), K);
  const int64_t N = b.dimensions()[1];
  ffi::Error err = ffi::Error::Success();
  const size_t ws_bytes = tg_block_scaled_matmul_workspace(M, N, K, (int)block_k);
  void* ws = take(scratch, ws_bytes, &err);
  if (ws_bytes && !ws) return err;
  if (ca == TG_DTYPE_BF16 && cb == TG_DTYPE_BF16)
    return status(tg_block_scaled_matmul(a.untyped_data(), b.untyped_data(), out->untyped_data(),
                                         M, N, K, (int)block_k, ws, ws_bytes, stream));
  // the workspace layout of tg_block_scaled_matmul: qa, sa, qb (N, K), sb, each 256-B aligned
  auto a256 = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t nkb = (size_t)(K / block_k);
  uint8_t* p = static_cast<uint8_t*>(ws);
  uint8_t* qa = p;                               p += a256((size_t)M * K);
  float* sa = reinterpret_cast<float*>(p);       p += a256((size_t)M * nkb * 4);
  uint8_t* qb = p;                               p += a256((size_t)N * K);
  float* sb = reinterpret_cast<float*>(p);
  int rc = tg_quantize_rows(a.untyped_data(), ca, M, K, (int)block_k, qa, sa, stream);
  if (rc == TG_OK) rc = tg_quantize_cols(b.untyped_data(), cb, K, N, (int)block_k, qb, sb, stream);
  if (rc == TG_OK)
    rc = tg_gemm_fp8_nt(qa, sa, qb, sb, 1, out->untyped_data(), TG_DTYPE_BF16, M, N, K, (int)block_k,
                        stream);
  return status(rc);
}

// The FP8 backward rule (the forward's quantize -> scaled GEMM for both
// gradients): a (M, K), b (K, N), g (M, N) bf16 -> da (M, K), db (K, N) bf16.
ffi::Error BlockScaledMatmulBwdFp8(hipStream_t stream, ffi::ScratchAllocator scratch,
                                   ffi::Buffer<ffi::BF16> a, ffi::Buffer<ffi::BF16> b,
                                   ffi::Buffer<ffi::BF16> g, ffi::ResultBuffer<ffi::BF16> da,
                                   ffi::ResultBuffer<ffi::BF16> db, int64_t block_k) {
  const int64_t K = a.dimensions().back(), M = rows_of(a.element_count(), K);
  const int64_t N = b.dimensions()[1];
  ffi::Error err = ffi::Error::Success();
  const size_t ws_bytes = tg_block_scaled_matmul_bwd_workspace(M, N, K, (int)block_k);
  void* ws = take(scratch, ws_bytes, &err);
  if (ws_bytes && !ws) return err;
  return status(tg_block_scaled_matmul_bwd_fp8(a.untyped_data(), b.untyped_data(), g.untyped_data(),
                                               da->untyped_data(), db->untyped_data(), M, N, K,
                                               (int)block_k, ws, ws_bytes, stream));
}

// _fp8_backward (fp8.py:85-98), the straight-through bf16 rule: a, b, g bf16 or
// f32 -> da, db bf16 (the Python side widens to a.dtype / b.dtype, fp8.py:95-96).
ffi::Error BlockScaledMatmulBwdBf16(hipStream_t stream, ffi::ScratchAllocator scratch,
                                    ffi::AnyBuffer a, ffi::AnyBuffer b, ffi::AnyBuffer g,
                                    ffi::ResultBuffer<ffi::BF16> da, ffi::ResultBuffer<ffi::BF16> db) {
  int ca, cb, cg;
  if (!dtype_code(a.element_type(), &ca) || !dtype_code(b.element_type(), &cb) ||
      !dtype_code(g.element_type(), &cg) || b.dimensions().size() != 2)
    return ffi::Error(ffi::ErrorCode::kInvalidArgument,
                      "block_scaled_matmul backward: operands must be bf16 or f32, b 2-D");
  const int64_t K = last_dim(a.dimensions()), M = rows_of(a.element_count(), K);
  const int64_t N = b.dimensions()[1];
  ffi::Error err = ffi::Error::Success();
  const size_t ws_bytes = tg_block_scaled_matmul_bwd_bf16_workspace(M, N, K);
  void* ws = take(scratch, ws_bytes, &err);
  if (ws_bytes && !ws) return err;
  return status(tg_block_scaled_matmul_bwd_bf16(a.untyped_data(), ca, b.untyped_data(), cb,
                                                g.untyped_data(), cg, da->untyped_data(),
                                                db->untyped_data(), M, N, K, ws, ws_bytes, stream));
}

// _rms_norm_pure (kernels.py:30-33): x (..., D), scale (D,), each bf16, f16 or
// f32 -> y (..., D) in their promoted dtype (the common one, else f32).
ffi::Error RmsNorm(hipStream_t stream, ffi::AnyBuffer x, ffi::AnyBuffer scale,
                   ffi::Result<ffi::AnyBuffer> y, float eps) {
  int cx, cs, cy;
  if (!norm_dtype_code(x.element_type(), &cx) || !norm_dtype_code(scale.element_type(), &cs) ||
      !norm_dtype_code(y->element_type(), &cy) || cy != (cx == cs ? cx : TG_DTYPE_F32))
    return ffi::Error(ffi::ErrorCode::kInvalidArgument,
                      "rms_norm: x, scale bf16, f16 or f32; y in their promoted dtype");
  const int64_t D = last_dim(x.dimensions());
  return status(tg_rms_norm_ex(x.untyped_data(), cx, scale.untyped_data(), cs, y->untyped_data(),
                               rows_of(x.element_count(), D), D, eps, stream));
}

// The norm fused with the quantization that feeds the next matmul:
// y (..., D) bf16, q (..., D) e4m3fn, s (..., D / block_k) f32.
ffi::Error RmsNormFp8(hipStream_t stream, ffi::Buffer<ffi::BF16> x, ffi::Buffer<ffi::BF16> scale,
                      ffi::ResultBuffer<ffi::BF16> y, ffi::ResultBuffer<ffi::F8E4M3FN> q,
                      ffi::ResultBuffer<ffi::F32> s, float eps, int64_t block_k) {
  const int64_t D = x.dimensions().back();
  return status(tg_rms_norm_fp8(x.untyped_data(), scale.untyped_data(), y->untyped_data(),
                                static_cast<uint8_t*>(q->untyped_data()), s->typed_data(),
                                rows_of(x.element_count(), D), D, eps, (int)block_k, stream));
}

// The norm's _bwd (kernels.py:104-118): x, scale, dy bf16, f16 or f32 -> dx
// in x's dtype, dscale in scale's.
ffi::Error RmsNormBwd(hipStream_t stream, ffi::ScratchAllocator scratch, ffi::AnyBuffer x,
                      ffi::AnyBuffer scale, ffi::AnyBuffer dy, ffi::Result<ffi::AnyBuffer> dx,
                      ffi::Result<ffi::AnyBuffer> dscale, float eps) {
  int cx, cs, cd, cdx, cds;
  if (!norm_dtype_code(x.element_type(), &cx) || !norm_dtype_code(scale.element_type(), &cs) ||
      !norm_dtype_code(dy.element_type(), &cd) || !norm_dtype_code(dx->element_type(), &cdx) ||
      !norm_dtype_code(dscale->element_type(), &cds) || cdx != cx || cds != cs)
    return ffi::Error(ffi::ErrorCode::kInvalidArgument,
                      "rms_norm backward: bf16 / f16 / f32 operands; dx in x's dtype, dscale in scale's");
  const int64_t D = last_dim(x.dimensions()), rows = rows_of(x.element_count(), D);
  ffi::Error err = ffi::Error::Success();
  const size_t ws_bytes = tg_rms_norm_bwd_workspace(rows, D);
  void* ws = take(scratch, ws_bytes, &err);
  if (ws_bytes && !ws) return err;
  return status(tg_rms_norm_bwd_ex(x.untyped_data(), cx, scale.untyped_data(), cs, dy.untyped_data(), cd,
                                   dx->untyped_data(), dscale->untyped_data(), rows, D, eps, ws,
                                   ws_bytes, stream));
}

// The scaled GEMM alone on pre-quantized operands (a kept weight's bytes and
// scales, fp8.py:68 done once): a_q (M, K), a_s (M, K/128), b_q (N, K),
// b_s (N or ceil(N/128), K/128) -> c (M, N) bf16.
ffi::Error GemmFp8Nt(hipStream_t stream, ffi::Buffer<ffi::F8E4M3FN> a_q, ffi::Buffer<ffi::F32> a_s,
                     ffi::Buffer<ffi::F8E4M3FN> b_q, ffi::Buffer<ffi::F32> b_s,
                     ffi::ResultBuffer<ffi::BF16> c, int64_t b_scale_bn) {
  const int64_t K = a_q.dimensions().back(), M = rows_of(a_q.element_count(), K);
  const int64_t N = b_q.dimensions()[0];
  return status(tg_gemm_fp8_nt(static_cast<const uint8_t*>(a_q.untyped_data()), a_s.typed_data(),
                               static_cast<const uint8_t*>(b_q.untyped_data()), b_s.typed_data(),
                               (int)b_scale_bn, c->untyped_data(), TG_DTYPE_BF16, M, N, K, 128, stream));
}

}  // namespace

// Exported handler symbols (C linkage); the registration names are
// HANDLERS in train-gpt_amd/xla_ffi.py.
XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_quantize_rows, QuantizeRows,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::F8E4M3FN>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("block_k"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_quantize_cols, QuantizeCols,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::F8E4M3FN>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Attr<int64_t>("block_k"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_block_scaled_matmul, BlockScaledMatmul,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Ctx<ffi::ScratchAllocator>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Attr<int64_t>("block_k"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_block_scaled_matmul_bwd_fp8, BlockScaledMatmulBwdFp8,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Ctx<ffi::ScratchAllocator>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Attr<int64_t>("block_k"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_block_scaled_matmul_bwd_bf16, BlockScaledMatmulBwdBf16,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Ctx<ffi::ScratchAllocator>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>());

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_rms_norm, RmsNorm,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Attr<float>("eps"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_rms_norm_fp8, RmsNormFp8,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Arg<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Ret<ffi::Buffer<ffi::F8E4M3FN>>()
                                  .Ret<ffi::Buffer<ffi::F32>>()
                                  .Attr<float>("eps")
                                  .Attr<int64_t>("block_k"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_rms_norm_bwd, RmsNormBwd,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Ctx<ffi::ScratchAllocator>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Arg<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Ret<ffi::AnyBuffer>()
                                  .Attr<float>("eps"));

XLA_FFI_DEFINE_HANDLER_SYMBOL(tg_ffi_gemm_fp8_nt, GemmFp8Nt,
                              ffi::Ffi::Bind()
                                  .Ctx<ffi::PlatformStream<hipStream_t>>()
                                  .Arg<ffi::Buffer<ffi::F8E4M3FN>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Arg<ffi::Buffer<ffi::F8E4M3FN>>()
                                  .Arg<ffi::Buffer<ffi::F32>>()
                                  .Ret<ffi::Buffer<ffi::BF16>>()
                                  .Attr<int64_t>("b_scale_bn"));
