// tg_block_scaled_matmul_noalloc: the forward composite (tg_block_scaled_matmul's
// quantizers and GEMM) on a static device workspace, for callers that cannot
// allocate (no reference counterpart).
//
// The array lives in this translation unit on its own: its code object holds
// no kernel, so the HIP runtime loads it onto a device (and reserves the
// array there) only when this entry point first resolves the array's address
// on that device, not when a process first runs any of the library's other
// kernels.  Every device that ran this entry point keeps its copy until the
// process ends.  The array's name is a host-side handle, not a device
// address: host code only uses the per-device address hipGetSymbolAddress
// returns.
#include <mutex>

#include "tg_host.h"

using namespace tg;

constexpr size_t kScratchBytes = TG_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// scratch's address on the current device, resolved once per device (with
// that device current) and kept; null with the error set if it fails.
static uint8_t* scratch_on_current_device() {
  constexpr int kMaxDev = 64;
  static std::once_flag once[kMaxDev];
  static uint8_t* addr[kMaxDev];
  static hipError_t rc[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    set_error("block_scaled_matmul_noalloc: no usable current device");
    return nullptr;
  }
  std::call_once(once[dev], [dev] {
    void* p = nullptr;
    rc[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    addr[dev] = rc[dev] == hipSuccess ? reinterpret_cast<uint8_t*>(p) : nullptr;
  });
  if (rc[dev] != hipSuccess || !addr[dev]) {
    set_error("block_scaled_matmul_noalloc: hipGetSymbolAddress(scratch) failed: %s",
              hipGetErrorString(rc[dev]));
    return nullptr;
  }
  return addr[dev];
}

extern "C" int tg_block_scaled_matmul_noalloc(const void* a, const void* b, void* out, int64_t M,
                                              int64_t N, int64_t K, int block_k, void* stream) {
  TG_TRY(check_gemm_args("block_scaled_matmul_noalloc", M, N, K, block_k, 1));
  if (M == 0 || N == 0) return TG_OK;
  if (!a || !b || !out) return einval("block_scaled_matmul_noalloc: null pointer");
  if (!aligned(a, 16) || !aligned(b, 16))
    return einval("block_scaled_matmul_noalloc: a, b must be 16-byte aligned");
  const size_t need = tg_block_scaled_matmul_workspace(M, N, K, block_k);
  if (need > kScratchBytes) {
    set_error("invalid argument: block_scaled_matmul_noalloc: M=%lld N=%lld K=%lld needs %zu bytes of "
              "workspace, more than the %zu-byte static scratch (use tg_block_scaled_matmul with a "
              "caller workspace)",
              (long long)M, (long long)N, (long long)K, need, kScratchBytes);
    return TG_EINVAL;
  }
  uint8_t* ws = scratch_on_current_device();
  if (!ws) return TG_EHIP;
  // every byte the GEMM reads is written by the two quantizers first, so the
  // previous call's contents never leak into this one
  return block_scaled_matmul_on(a, b, out, M, N, K, ws, as_stream(stream));
}
