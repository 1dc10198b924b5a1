// libtg_ffi_core.so: the XLA FFI handlers' logic (tg_ffi_core.h) over a C ABI,
// so that tests can run it on the GPU where jaxlib (and with it the XLA FFI
// header the handlers themselves need) is not installed.  Test tooling:
// nothing in the package loads it.
//
// Every entry point returns the tgffi::Code of the call (0 = success,
// TG_EINVAL, TG_EHIP, 100 = scratch exhausted) and copies its message into
// msg[0 .. msg_len).  The scratch allocator XLA would hand a handler is a
// bump allocator over the caller's buffer: `used` comes back as the bytes the
// handler took, and a buffer too small makes the allocation fail as XLA's
// would.
#include <cstring>

#include "tg_ffi_core.h"

namespace {

struct Bump {
  void* base;
  size_t cap;
  size_t used;
};

void* bump_alloc(void* ctx, size_t bytes, size_t align) {
  Bump* b = static_cast<Bump*>(ctx);
  const uintptr_t base = reinterpret_cast<uintptr_t>(b->base);
  const uintptr_t at = (base + b->used + align - 1) & ~(uintptr_t)(align - 1);
  if (!b->base || at + bytes > base + b->cap) return nullptr;
  b->used = at + bytes - base;
  return reinterpret_cast<void*>(at);
}

int done(const tgffi::Status& st, char* msg, size_t msg_len) {
  if (msg && msg_len) {
    std::strncpy(msg, st.msg ? st.msg : "", msg_len - 1);
    msg[msg_len - 1] = '\0';
  }
  return st.code;
}

}  // namespace

extern "C" {

int tg_ffi_core_quantize_rows(void* stream, const tgffi::View* x, void* q, float* s, int64_t block_k, char* msg,
                              size_t msg_len) {
  return done(tgffi::quantize_rows(stream, *x, q, s, block_k), msg, msg_len);
}

int tg_ffi_core_quantize_cols(void* stream, const tgffi::View* x, void* q_t, float* s_t, int64_t block_k,
                              char* msg, size_t msg_len) {
  return done(tgffi::quantize_cols(stream, *x, q_t, s_t, block_k), msg, msg_len);
}

int tg_ffi_core_block_scaled_matmul(void* stream, Bump* scratch, const tgffi::View* a, const tgffi::View* b,
                                    void* out, int64_t block_k, char* msg, size_t msg_len) {
  const tgffi::Scratch s{bump_alloc, scratch};
  return done(tgffi::block_scaled_matmul(stream, s, *a, *b, out, block_k), msg, msg_len);
}

int tg_ffi_core_block_scaled_matmul_bwd_fp8(void* stream, Bump* scratch, const tgffi::View* a,
                                            const tgffi::View* b, const tgffi::View* g, void* da, void* db,
                                            int64_t block_k, char* msg, size_t msg_len) {
  const tgffi::Scratch s{bump_alloc, scratch};
  return done(tgffi::block_scaled_matmul_bwd_fp8(stream, s, *a, *b, *g, da, db, block_k), msg, msg_len);
}

int tg_ffi_core_block_scaled_matmul_bwd_bf16(void* stream, Bump* scratch, const tgffi::View* a,
                                             const tgffi::View* b, const tgffi::View* g, void* da, void* db,
                                             char* msg, size_t msg_len) {
  const tgffi::Scratch s{bump_alloc, scratch};
  return done(tgffi::block_scaled_matmul_bwd_bf16(stream, s, *a, *b, *g, da, db), msg, msg_len);
}

int tg_ffi_core_rms_norm(void* stream, const tgffi::View* x, const tgffi::View* scale, const tgffi::View* y,
                         float eps, char* msg, size_t msg_len) {
  return done(tgffi::rms_norm(stream, *x, *scale, *y, eps), msg, msg_len);
}

int tg_ffi_core_rms_norm_fp8(void* stream, const tgffi::View* x, const tgffi::View* scale, void* y, void* q,
                             float* s, float eps, int64_t block_k, char* msg, size_t msg_len) {
  return done(tgffi::rms_norm_fp8(stream, *x, *scale, y, q, s, eps, block_k), msg, msg_len);
}

int tg_ffi_core_rms_norm_bwd(void* stream, Bump* scratch, const tgffi::View* x, const tgffi::View* scale,
                             const tgffi::View* dy, const tgffi::View* dx, const tgffi::View* dscale, float eps,
                             char* msg, size_t msg_len) {
  const tgffi::Scratch s{bump_alloc, scratch};
  return done(tgffi::rms_norm_bwd(stream, s, *x, *scale, *dy, *dx, *dscale, eps), msg, msg_len);
}

int tg_ffi_core_gemm_fp8_nt(void* stream, const tgffi::View* a_q, const float* a_s, const tgffi::View* b_q,
                            const float* b_s, void* c, int64_t b_scale_bn, char* msg, size_t msg_len) {
  return done(tgffi::gemm_fp8_nt(stream, *a_q, a_s, *b_q, b_s, c, b_scale_bn), msg, msg_len);
}

}  // extern "C"
