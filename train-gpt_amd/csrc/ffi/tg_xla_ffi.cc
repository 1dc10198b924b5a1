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
//
// Each handler only converts: XLA buffers -> tgffi::View (pointer, dtype,
// shape), the scratch allocator -> tgffi::Scratch, and tgffi::Status ->
// ffi::Error.  The checks, dispatch and C-ABI calls are tg_ffi_core.h, which
// the tests run on the GPU without jaxlib (libtg_ffi_core.so).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "tg_ffi_core.h"
#include "tg_fp8.h"
#include "xla/ffi/api/ffi.h"

namespace ffi = xla::ffi;

namespace {

ffi::Error to_error(const tgffi::Status& st) {
  switch (st.code) {
    case tgffi::kOk: return ffi::Error::Success();
    case tgffi::kInvalid: return ffi::Error(ffi::ErrorCode::kInvalidArgument, st.msg);
    case tgffi::kExhausted: return ffi::Error(ffi::ErrorCode::kResourceExhausted, st.msg);
    default: return ffi::Error(ffi::ErrorCode::kInternal, st.msg);
  }
}

int dtype_of(ffi::DataType t) {
  switch (t) {
    case ffi::DataType::BF16: return tgffi::kBF16;
    case ffi::DataType::F32: return tgffi::kF32;
    case ffi::DataType::F16: return tgffi::kF16;
    case ffi::DataType::F8E4M3FN: return tgffi::kE4M3;
    default: return tgffi::kOther;
  }
}

// A buffer as a View; typed buffers pass their (fixed) element type.
template <typename B>
tgffi::View view(B& b, int dtype) {
  auto d = b.dimensions();
  return {b.untyped_data(), dtype, d.size() ? &d[0] : nullptr, (int)d.size()};
}
tgffi::View view(ffi::AnyBuffer& b) { return view(b, dtype_of(b.element_type())); }

void* scratch_alloc(void* ctx, size_t bytes, size_t align) {
  auto p = static_cast<ffi::ScratchAllocator*>(ctx)->Allocate(bytes, align);
  return p.has_value() ? *p : nullptr;
}
tgffi::Scratch scratch_of(ffi::ScratchAllocator& s) { return {scratch_alloc, &s}; }

ffi::Error QuantizeRows(hipStream_t stream, ffi::AnyBuffer x, ffi::ResultBuffer<ffi::F8E4M3FN> q,
                        ffi::ResultBuffer<ffi::F32> s, int64_t block_k) {
  return to_error(tgffi::quantize_rows(stream, view(x), q->untyped_data(), s->typed_data(), block_k));
}

ffi::Error QuantizeCols(hipStream_t stream, ffi::AnyBuffer x, ffi::ResultBuffer<ffi::F8E4M3FN> q_t,
                        ffi::ResultBuffer<ffi::F32> s_t, int64_t block_k) {
  return to_error(tgffi::quantize_cols(stream, view(x), q_t->untyped_data(), s_t->typed_data(), block_k));
}

ffi::Error BlockScaledMatmul(hipStream_t stream, ffi::ScratchAllocator scratch, ffi::AnyBuffer a,
                             ffi::AnyBuffer b, ffi::ResultBuffer<ffi::BF16> out, int64_t block_k) {
  return to_error(tgffi::block_scaled_matmul(stream, scratch_of(scratch), view(a), view(b), out->untyped_data(),
                                             block_k));
}

ffi::Error BlockScaledMatmulBwdFp8(hipStream_t stream, ffi::ScratchAllocator scratch,
                                   ffi::Buffer<ffi::BF16> a, ffi::Buffer<ffi::BF16> b,
                                   ffi::Buffer<ffi::BF16> g, ffi::ResultBuffer<ffi::BF16> da,
                                   ffi::ResultBuffer<ffi::BF16> db, int64_t block_k) {
  return to_error(tgffi::block_scaled_matmul_bwd_fp8(stream, scratch_of(scratch), view(a, tgffi::kBF16),
                                                     view(b, tgffi::kBF16), view(g, tgffi::kBF16),
                                                     da->untyped_data(), db->untyped_data(), block_k));
}

ffi::Error BlockScaledMatmulBwdBf16(hipStream_t stream, ffi::ScratchAllocator scratch,
                                    ffi::AnyBuffer a, ffi::AnyBuffer b, ffi::AnyBuffer g,
                                    ffi::ResultBuffer<ffi::BF16> da, ffi::ResultBuffer<ffi::BF16> db) {
  return to_error(tgffi::block_scaled_matmul_bwd_bf16(stream, scratch_of(scratch), view(a), view(b), view(g),
                                                      da->untyped_data(), db->untyped_data()));
}

ffi::Error RmsNorm(hipStream_t stream, ffi::AnyBuffer x, ffi::AnyBuffer scale,
                   ffi::Result<ffi::AnyBuffer> y, float eps) {
  return to_error(tgffi::rms_norm(stream, view(x), view(scale), view(*y), eps));
}

ffi::Error RmsNormFp8(hipStream_t stream, ffi::Buffer<ffi::BF16> x, ffi::Buffer<ffi::BF16> scale,
                      ffi::ResultBuffer<ffi::BF16> y, ffi::ResultBuffer<ffi::F8E4M3FN> q,
                      ffi::ResultBuffer<ffi::F32> s, float eps, int64_t block_k) {
  return to_error(tgffi::rms_norm_fp8(stream, view(x, tgffi::kBF16), view(scale, tgffi::kBF16),
                                      y->untyped_data(), q->untyped_data(), s->typed_data(), eps, block_k));
}

ffi::Error RmsNormBwd(hipStream_t stream, ffi::ScratchAllocator scratch, ffi::AnyBuffer x,
                      ffi::AnyBuffer scale, ffi::AnyBuffer dy, ffi::Result<ffi::AnyBuffer> dx,
                      ffi::Result<ffi::AnyBuffer> dscale, float eps) {
  return to_error(tgffi::rms_norm_bwd(stream, scratch_of(scratch), view(x), view(scale), view(dy), view(*dx),
                                      view(*dscale), eps));
}

ffi::Error GemmFp8Nt(hipStream_t stream, ffi::Buffer<ffi::F8E4M3FN> a_q, ffi::Buffer<ffi::F32> a_s,
                     ffi::Buffer<ffi::F8E4M3FN> b_q, ffi::Buffer<ffi::F32> b_s,
                     ffi::ResultBuffer<ffi::BF16> c, int64_t b_scale_bn) {
  return to_error(tgffi::gemm_fp8_nt(stream, view(a_q, tgffi::kE4M3), a_s.typed_data(), view(b_q, tgffi::kE4M3),
                                     b_s.typed_data(), c->untyped_data(), b_scale_bn));
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
