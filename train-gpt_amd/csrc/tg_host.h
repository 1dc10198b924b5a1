// Host-side helpers of the C ABI: argument checks and thread-local errors.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "../../include/tg_fp8.h"

namespace tg {

void set_error(const char* fmt, ...);

inline int einval(const char* what) {
  set_error("invalid argument: %s", what);
  return TG_EINVAL;
}

inline int check_launch(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", kernel, hipGetErrorString(e));
    return TG_EHIP;
  }
  return TG_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Compute units of the current device, queried once per device id.  Entry
// points may be called concurrently from several host threads (an XLA FFI
// handler runs on XLA's thread pool), so the one-time query is guarded by a
// per-device std::call_once (one instance program-wide: an inline function's
// statics are shared by every translation unit).
inline int device_cus() {
  constexpr int kMaxDev = 64;
  static std::once_flag once[kMaxDev];
  static int cached[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) dev = 0;
  std::call_once(once[dev], [dev] {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
      v = 256;
    cached[dev] = v;
  });
  return cached[dev];
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Kernel launchers shared between translation units.
// skm: scales stored K-block-major ((cols / 128, rows) for a row quantization,
// (rows / 128, cols) for the transposed one) instead of the reference's
// row-major (rows, cols / 128); the GEMM's *_km entry points read that layout.
int launch_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, uint8_t* q,
                      float* s, hipStream_t st, bool skm = false);
int launch_quant_rows_relu2(const void* x, int64_t rows, int64_t cols, uint8_t* q, float* s,
                            hipStream_t st);
int launch_quant_cols(const void* x, int64_t rows, int64_t cols, uint8_t* q_t, float* s_t,
                      hipStream_t st, bool skm = false);
int launch_quant_dual(const void* x, int64_t rows, int64_t cols, uint8_t* q, float* s, uint8_t* q_t,
                      float* s_t, hipStream_t st, bool skm = false);
int launch_quant_rows_cols(const void* a, int64_t M, int64_t K, uint8_t* qa, float* sa, const void* b,
                           int64_t N, uint8_t* qbt, float* sbt, hipStream_t st, bool skm);
int launch_quant_dual_pair(const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0, float* s0,
                           uint8_t* qt0, float* st0, const void* x1, int64_t rows1, int64_t cols1,
                           uint8_t* q1, float* s1, uint8_t* qt1, float* st1, hipStream_t st, bool skm = false);
int launch_gemm_fp8(const uint8_t* a_q, const float* a_s, const uint8_t* b_q, const float* b_s,
                    int b_scale_bn, void* c, int c_dtype, int64_t M, int64_t N, int64_t K,
                    hipStream_t st, bool skm = false);
// The general path for block_k != 128 (block_generic.hip): row-major scales
// (K-block-major with skm), any block_k >= 1 dividing the contracted extent.
// For the tuned GEMM: srep = bk / 128 writes each block's scale srep times;
// pf = 128 / bk puts each block at the start of a zero-filled 128-byte slot
// (q rows of cols * pf bytes).
// skm: scales K-block-major ((block, slot) x rows, the _km GEMMs' layout).
int launch_quant_rows_gb(const void* x, int x_dtype, int64_t rows, int64_t cols, int bk, uint8_t* q, float* s,
                         hipStream_t st, int srep = 1, int pf = 1, bool skm = false);
int launch_quant_cols_gb(const void* x, bool x_f32, int64_t rows, int64_t cols, int bk, uint8_t* q_t,
                         float* s_t, hipStream_t st, int srep = 1, int pf = 1, bool skm = false);
int launch_gemm_gb(const uint8_t* a_q, const float* a_s, const uint8_t* b_q, const float* b_s, int bn, void* c,
                   int c_dtype, int64_t M, int64_t N, int64_t K, int bk, hipStream_t st);
// n bf16 zeros at p by a fill kernel (no hipMemsetAsync: the callers may be
// captured into a graph); n == 0 launches nothing (gemm_bf16.hip).
int launch_fill_zero_bf16(void* p, int64_t n, hipStream_t st);
// The GEMM entry points' shape and block checks (gemm_fp8.hip); any_block:
// the entry has the general path for block_k != 128.
int check_gemm_args(const char* who, int64_t M, int64_t N, int64_t K, int block_k, int bns,
                    bool any_block = false);
// tg_block_scaled_matmul's kernels (the two quantizers, then the GEMM) on a
// workspace of tg_block_scaled_matmul_workspace(M, N, K, 128) bytes the caller
// has checked (gemm_fp8.hip).
int block_scaled_matmul_on(const void* a, const void* b, void* out, int64_t M, int64_t N, int64_t K,
                           void* workspace, hipStream_t st);

}  // namespace tg

#define TG_TRY(expr)              \
  do {                            \
    int _rc = (expr);             \
    if (_rc != TG_OK) return _rc; \
  } while (0)
