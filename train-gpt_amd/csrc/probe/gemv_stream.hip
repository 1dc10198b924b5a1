// Measurement probe (not part of the product library): the weight and x
// traffic of the direct decode GEMV (gemv_direct_kernel in gemm_fp8.hip) with
// its arithmetic taken out, so that bench.py can time the streaming floor of
// that access pattern on the same launch shape.
//
// Access pattern, as in the direct GEMV: a workgroup of 8 waves walks 16-row
// blocks b, b + grid, ...; wave w takes the contiguous K blocks
// [w kpw, (w + 1) kpw) of a block, kpw = ceil(K / 1024); lane (r, g) loads
// bytes 16 g and 64 + 16 g of row r's 128-byte piece of each of those K
// blocks (64 bytes of 16 rows per load instruction), all of a row block's
// loads at once.  Before them every workgroup reads the x_bytes of x (chunk
// tid + 512 j, XC chunks per thread as the GEMV takes them: 4 up to 32 KiB,
// else 16), as the GEMV copies its x rows.  The loaded words are folded
// into one u32 per thread (written to sink) so that the loads stay live.
// cached = 0 gives the loads the non-temporal hint.
#include "../tg_device.h"
#include "../tg_host.h"
#include "../gemm_tile.h"

namespace tg {

template <int KPW, int AUX, int XC>
__global__ __launch_bounds__(512) void gemv_stream_kernel(const uint8_t* __restrict__ w, const uint8_t* __restrict__ x,
                                                          uint32_t* __restrict__ sink, int N, int K,
                                                          uint32_t x_bytes) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int nkb = K >> 7, kpw = (nkb + 7) / 8, nrb = (N + 15) >> 4;
  const uint32_t wbytes = (uint32_t)N * (uint32_t)K;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, wbytes);
  u32x4_t acc = {0u, 0u, 0u, 0u};
  if (x_bytes) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, x_bytes);
    u32x4_t xv[XC];
#pragma unroll
    for (int j = 0; j < XC; ++j)   // past x_bytes: out of range, reads zero
      xv[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(tid + 512 * j) * 16u, 0, 0);
#pragma unroll
    for (int j = 0; j < XC; ++j) acc ^= xv[j];
  }
  for (int rb = blockIdx.x; rb < nrb; rb += gridDim.x) {
    const uint32_t row = (uint32_t)(rb * 16 + fr);
    u32x4_t v[KPW][2];
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kb = wave * kpw + i;
      const bool ok = i < kpw && kb < nkb && (int)row < N;
      const uint32_t off = ok ? row * (uint32_t)K + (uint32_t)kb * 128u + (uint32_t)fg * 16u : wbytes;
      v[i][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, AUX);
      v[i][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? off + 64u : wbytes, 0, AUX);
    }
#pragma unroll
    for (int i = 0; i < KPW; ++i) acc ^= v[i][0] ^ v[i][1];
  }
  sink[(int64_t)blockIdx.x * 512 + tid] = acc.x ^ acc.y ^ acc.z ^ acc.w;
}

template <int KPW, int XC>
static void launch_gemv_stream_x(const uint8_t* w, const uint8_t* x, uint32_t* sink, int N, int K,
                                 uint32_t x_bytes, int grid, bool cached, hipStream_t st) {
  if (cached)
    hipLaunchKernelGGL((gemv_stream_kernel<KPW, 0, XC>), dim3(grid), dim3(512), 0, st, w, x, sink, N, K, x_bytes);
  else
    hipLaunchKernelGGL((gemv_stream_kernel<KPW, 2, XC>), dim3(grid), dim3(512), 0, st, w, x, sink, N, K, x_bytes);
}

template <int KPW>
static void launch_gemv_stream(const uint8_t* w, const uint8_t* x, uint32_t* sink, int N, int K, uint32_t x_bytes,
                               int grid, bool cached, hipStream_t st) {
  if (x_bytes <= 4u * 512u * 16u) launch_gemv_stream_x<KPW, 4>(w, x, sink, N, K, x_bytes, grid, cached, st);
  else launch_gemv_stream_x<KPW, 16>(w, x, sink, N, K, x_bytes, grid, cached, st);
}

}  // namespace tg

// w: (N, K) bytes; x: x_bytes bytes (<= 131072) read by every workgroup; sink:
// grid * 512 u32.  K % 128 == 0, K <= 12288, 1 <= grid <= ceil(N / 16).
extern "C" int tg_probe_gemv_stream(const void* w, int64_t N, int64_t K, const void* x, int64_t x_bytes,
                                    uint32_t* sink, int grid, int cached, void* stream) {
  using namespace tg;
  if (!w || !sink || N <= 0 || K <= 0 || K % 128 || K > 12288 || x_bytes < 0 || x_bytes > 131072 ||
      (x_bytes && !x) || (uint64_t)N * (uint64_t)K >= (1ull << 32))
    return einval("tg_probe_gemv_stream: bad arguments");
  const int64_t nrb = (N + 15) / 16;
  if (grid < 1 || grid > nrb) return einval("tg_probe_gemv_stream: grid must be 1 .. ceil(N / 16)");
  auto st = static_cast<hipStream_t>(stream);
  auto W = reinterpret_cast<const uint8_t*>(w);
  auto X = reinterpret_cast<const uint8_t*>(x);
  const int kpw = (int)((K / 128 + 7) / 8);
  const int n = (int)N, k = (int)K;
  const uint32_t xb = (uint32_t)x_bytes;
  if (kpw <= 3) launch_gemv_stream<3>(W, X, sink, n, k, xb, grid, cached != 0, st);
  else if (kpw <= 9) launch_gemv_stream<9>(W, X, sink, n, k, xb, grid, cached != 0, st);
  else launch_gemv_stream<12>(W, X, sink, n, k, xb, grid, cached != 0, st);
  return check_launch("gemv_stream");
}
