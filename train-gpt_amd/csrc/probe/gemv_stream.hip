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

// The staged GEMV's weight stream (gemv_fp8_kernel in gemm_fp8.hip, the
// kernel tg_gemv_fp8 runs on C5's 14336 x 4096 weight), with its MFMAs, x
// fragments and cross-wave reduction taken out: workgroup b takes the
// balanced share of the 8-row groups [b G / grid, (b + 1) G / grid), walks K
// in 4 KiB chunks, and within a chunk moves stages of 8 rows -- wave w loads
// row w of a stage as four 1 KiB pieces plus the row's 32 scales --
// registers -> LDS (row pitch 4112 B), three stages in flight, one barrier per
// stage, every load issued unconditionally (past the end: out of range, reads
// zero).  With x_bytes > 0 every workgroup first copies x_bytes of x into LDS
// with whole-row loads, as the GEMV does for up to 8 activation rows.
namespace tg {

constexpr int kStagedPitch = 4112;
constexpr int kStagedStage = 8 * kStagedPitch + 8 * 64 * 4;
__shared__ __attribute__((aligned(16))) uint8_t staged_lds0[kStagedStage];
__shared__ __attribute__((aligned(16))) uint8_t staged_lds1[kStagedStage];
__shared__ __attribute__((aligned(16))) uint8_t staged_lds2[kStagedStage];
template <int S> __device__ __forceinline__ uint8_t* staged_buf() {
  return S == 0 ? staged_lds0 : S == 1 ? staged_lds1 : staged_lds2;
}

template <int BNS>
__global__ __launch_bounds__(512) void gemv_staged_kernel(const uint8_t* __restrict__ w, const float* __restrict__ ws,
                                                          uint32_t* __restrict__ sink, int N, int K,
                                                          const uint8_t* __restrict__ x, uint32_t x_bytes) {
  constexpr int NS = 3;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = K >> 7, nchunk = (nkb + 31) >> 5;
  const int64_t gtot = (N + 7) >> 3;
  const int g_lo = (int)(((int64_t)blockIdx.x * gtot) / gridDim.x);
  const int g_hi = (int)(((int64_t)(blockIdx.x + 1) * gtot) / gridDim.x);
  const int n0 = 8 * g_lo, rows = min(8 * g_hi, N) - n0, ngroups = g_hi - g_lo;
  const uint32_t wbytes = (uint32_t)rows * (uint32_t)K;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + (int64_t)n0 * K, wbytes);
  const int srows = BNS == 1 ? N : (N + BNS - 1) / BNS;
  const uint32_t sbytes = (uint32_t)srows * (uint32_t)nkb * 4u;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(ws, sbytes);
  extern __shared__ __attribute__((aligned(16))) uint8_t staged_x[];
  u32x4_t wr[NS][4];
  float wsr[NS];
  auto load_w = [&](auto slot, int c, int g) {
    constexpr int SL = decltype(slot)::value;
    const int r = 8 * g + wave;
    const bool rv = g < ngroups && r < rows;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t k = (uint32_t)c * 4096u + p * 1024u + lane * 16u;
      const uint32_t off = (rv && k < (uint32_t)K) ? (uint32_t)r * (uint32_t)K + k : wbytes;
      wr[SL][p] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kAuxNT);
    }
    const int b = c * 32 + lane;
    const int srow = BNS == 1 ? n0 + r : (n0 + r) / BNS;
    const uint32_t soff = (rv && lane < 32 && b < nkb) ? ((uint32_t)srow * (uint32_t)nkb + (uint32_t)b) * 4u : sbytes;
    wsr[SL] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, soff, 0, 0));
  };
  auto stage = [&](auto slot, auto grp, int c) {
    constexpr int SL = decltype(slot)::value;
    constexpr int G = decltype(grp)::value;
    uint8_t* buf = staged_buf<G % 3>();
    float* ssw = reinterpret_cast<float*>(buf + 8 * kStagedPitch);
#pragma unroll
    for (int p = 0; p < 4; ++p)
      *reinterpret_cast<u32x4_t*>(buf + wave * kStagedPitch + p * 1024 + lane * 16) = wr[SL][p];
    ssw[wave * 64 + lane] = wsr[SL];
    load_w(slot, c, G + NS);
    __syncthreads();
  };
  // x rows into LDS with whole-row loads (their loads before the first stage's)
  constexpr int XU = 4;   // up to 32 KiB: 4 16-byte chunks per thread
  u32x4_t xv[XU];
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x, x_bytes);
  if (x_bytes) {
#pragma unroll
    for (int u = 0; u < XU; ++u) xv[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(tid + 512 * u) * 16u, 0, 0);
  }
  for (int c = 0; c < nchunk; ++c) {
    load_w(std::integral_constant<int, 0>{}, c, 0);
    load_w(std::integral_constant<int, 1>{}, c, 1);
    load_w(std::integral_constant<int, 2>{}, c, 2);
    if (x_bytes && c == 0) {
#pragma unroll
      for (int u = 0; u < XU; ++u)
        if ((uint32_t)(tid + 512 * u) * 16u < x_bytes)
          *reinterpret_cast<u32x4_t*>(staged_x + (tid + 512 * u) * 16) = xv[u];
      __syncthreads();
    }
    do {
      stage(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, c);
      if (ngroups <= 1) break;
      stage(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, c);
      if (ngroups <= 2) break;
      stage(std::integral_constant<int, 2>{}, std::integral_constant<int, 2>{}, c);
      if (ngroups <= 3) break;
      stage(std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{}, c);
      if (ngroups <= 4) break;
      stage(std::integral_constant<int, 1>{}, std::integral_constant<int, 4>{}, c);
      if (ngroups <= 5) break;
      stage(std::integral_constant<int, 2>{}, std::integral_constant<int, 5>{}, c);
      if (ngroups <= 6) break;
      stage(std::integral_constant<int, 0>{}, std::integral_constant<int, 6>{}, c);
      if (ngroups <= 7) break;
      stage(std::integral_constant<int, 1>{}, std::integral_constant<int, 7>{}, c);
    } while (false);
    __syncthreads();
  }
  // keep the staged bytes live: one word of the last stage buffers and of x
  uint32_t acc = *reinterpret_cast<const uint32_t*>(staged_lds0 + tid * 4) ^
                 *reinterpret_cast<const uint32_t*>(staged_lds1 + tid * 4) ^
                 *reinterpret_cast<const uint32_t*>(staged_lds2 + tid * 4);
  if (x_bytes && (uint32_t)tid * 4u < x_bytes) acc ^= *reinterpret_cast<const uint32_t*>(staged_x + tid * 4);
  sink[(int64_t)blockIdx.x * 512 + tid] = acc;
}

}  // namespace tg

// w: (N, K) e4m3 bytes, ws: its scales (N or ceil(N / 128) rows of K / 128;
// bn 1 or 128); x: x_bytes (<= 32 KiB) copied into LDS by every workgroup;
// sink: grid * 512 u32.  K % 128 == 0; grid workgroups of 8-row groups, at
// most 8 groups each.
extern "C" int tg_probe_gemv_staged(const void* w, const float* ws, int bn, int64_t N, int64_t K, const void* x,
                                    int64_t x_bytes, uint32_t* sink, int grid, void* stream) {
  using namespace tg;
  if (!w || !ws || !sink || N <= 0 || K <= 0 || K % 128 || (bn != 1 && bn != 128) || x_bytes < 0 ||
      x_bytes > 32768 || (x_bytes && !x) || (uint64_t)N * (uint64_t)K >= (1ull << 32))
    return einval("tg_probe_gemv_staged: bad arguments");
  const int64_t groups = (N + 7) / 8;
  if (grid < 1 || grid > groups || (groups + grid - 1) / grid > 8)
    return einval("tg_probe_gemv_staged: grid must give every workgroup 1 .. 8 groups of 8 rows");
  auto st = static_cast<hipStream_t>(stream);
  auto W = reinterpret_cast<const uint8_t*>(w);
  auto X = reinterpret_cast<const uint8_t*>(x);
  const size_t lds = (size_t)x_bytes;
  if (bn == 1)
    hipLaunchKernelGGL(gemv_staged_kernel<1>, dim3(grid), dim3(512), lds, st, W, ws, sink, (int)N, (int)K, X,
                       (uint32_t)x_bytes);
  else
    hipLaunchKernelGGL(gemv_staged_kernel<128>, dim3(grid), dim3(512), lds, st, W, ws, sink, (int)N, (int)K, X,
                       (uint32_t)x_bytes);
  return check_launch("gemv_staged");
}

