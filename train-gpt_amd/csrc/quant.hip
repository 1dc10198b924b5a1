// FP8 e4m3fn quantization kernels for gfx950 (HBM-bound byte work).
//
//   quant_rows_kernel   _quantize_to_fp8 along the last axis (fp8.py:39-47)
//   quant_cols_kernel   _quantize_to_fp8 of x.T (fp8.py:68) for unaligned rows
//   quant_dual_kernel   rows and / or x.T from one read, transposed through LDS
//   quant_w128_kernel   128x128-tile weight quantization for the GEMV format
//   selftest_cvt_kernel hardware e4m3fn convert vs the integer encoder
//
// Layout: a 128-element scale block is 16 lanes x 8 elements (one 16-byte
// load per lane), i.e. exactly one DPP row, so the block amax is four DPP
// max steps with no LDS traffic.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "quant_dual.h"
#include "row_ops.h"
#include "tg_device.h"
#include "tg_host.h"

namespace tg {

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

// ---------------------------------------------------------------------------
// Row quantization.  A "chunk" is 8 consecutive elements; chunks 16c..16c+15
// form scale block c.  Each thread handles UNROLL chunks spaced 256 apart so
// that UNROLL independent 16-byte loads are in flight per lane.
// ---------------------------------------------------------------------------
template <bool F32_IN>
__device__ __forceinline__ void load_chunk(const void* __restrict__ x, int64_t c, bool ok,
                                           float (&v)[8]) {
  if (F32_IN) {
    const uint4* p = reinterpret_cast<const uint4*>(x) + 2 * c;
    uint4 a = ok ? ldg_stream(p) : make_uint4(0, 0, 0, 0);
    uint4 b = ok ? ldg_stream(p + 1) : make_uint4(0, 0, 0, 0);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
    v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(b.x); v[5] = __uint_as_float(b.y);
    v[6] = __uint_as_float(b.z); v[7] = __uint_as_float(b.w);
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(x) + c;
    uint4 a = ok ? ldg_stream(p) : make_uint4(0, 0, 0, 0);
    v[0] = bf16lo(a.x); v[1] = bf16hi(a.x); v[2] = bf16lo(a.y); v[3] = bf16hi(a.y);
    v[4] = bf16lo(a.z); v[5] = bf16hi(a.z); v[6] = bf16lo(a.w); v[7] = bf16hi(a.w);
  }
}

// RELU2: the values quantized are bf16(relu(x)^2) (model.py:72's activation
// as bf16 tensor ops: relu exact, the square rounded once), for bf16 x.
// skm_rows > 0: scales stored K-block-major, s[kb * skm_rows + row] (nkb
// blocks per row), instead of the reference's (rows, nkb) row-major layout.
template <bool F32_IN, int UNROLL, bool RELU2 = false>
__global__ __launch_bounds__(256) void quant_rows_kernel(const void* __restrict__ x,
                                                         uint2* __restrict__ q,
                                                         float* __restrict__ s,
                                                         int64_t nchunks, int64_t skm_rows = 0,
                                                         int nkb = 1) {
  const int64_t base = (int64_t)blockIdx.x * (256 * UNROLL) + threadIdx.x;
  float v[UNROLL][8];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    int64_t c = base + u * 256;
    load_chunk<F32_IN>(x, c, c < nchunks, v[u]);
    if (RELU2) relu2_bf16(v[u]);
  }
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    int64_t c = base + u * 256;
    uint32_t m = row16_max_u32(absmax8(v[u]));   // uniform control flow for DPP
    float sc = F32_IN ? block_scale(m) : block_scale_bf16(m);
    if (c < nchunks) {
      q[c] = quant8<!F32_IN>(v[u], sc);
      if ((threadIdx.x & 15) == 0) {
        const int64_t b = c >> 4;
        s[skm_rows > 0 ? (b % nkb) * skm_rows + b / nkb : b] = sc;
      }
    }
  }
}

int launch_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, uint8_t* q,
                      float* s, hipStream_t st, bool skm) {
  const int64_t nchunks = rows * cols / 8;
  if (nchunks == 0) return TG_OK;
  constexpr int UNROLL = 4;
  const int64_t grid = (nchunks + 256 * UNROLL - 1) / (256 * UNROLL);
  const int64_t skm_rows = skm ? rows : 0;
  const int nkb = (int)(cols / 128);
  if (x_dtype == TG_DTYPE_F32)
    hipLaunchKernelGGL((quant_rows_kernel<true, UNROLL>), dim3((unsigned)grid), dim3(256), 0, st, x,
                       reinterpret_cast<uint2*>(q), s, nchunks, skm_rows, nkb);
  else
    hipLaunchKernelGGL((quant_rows_kernel<false, UNROLL>), dim3((unsigned)grid), dim3(256), 0, st,
                       x, reinterpret_cast<uint2*>(q), s, nchunks, skm_rows, nkb);
  return check_launch("quant_rows");
}

int launch_quant_rows_relu2(const void* x, int64_t rows, int64_t cols, uint8_t* q, float* s,
                            hipStream_t st) {
  const int64_t nchunks = rows * cols / 8;
  if (nchunks == 0) return TG_OK;
  constexpr int UNROLL = 4;
  const int64_t grid = (nchunks + 256 * UNROLL - 1) / (256 * UNROLL);
  hipLaunchKernelGGL((quant_rows_kernel<false, UNROLL, true>), dim3((unsigned)grid), dim3(256), 0,
                     st, x, reinterpret_cast<uint2*>(q), s, nchunks);
  return check_launch("quant_rows_relu2");
}

// ---------------------------------------------------------------------------
// Column quantization with transpose for rows that are not 16-byte aligned
// (cols % 8 != 0; element loads, VEC = false).  Aligned rows take
// quant_dual_kernel<false, ...> below.  Tile = 128 rows (one scale block of the
// output) x 64 columns.  Load coalesced rows into LDS (row pitch 136 B), let
// 4 lanes share each column (rows 16i + 4j + r for lane j, so a DPP quad holds
// the block), stage the e4m3 bytes in a second LDS tile (pitch 144 B) and
// store 32 contiguous bytes per lane.  Both pitches keep the column reads and
// the 16-byte reads bank-conflict free for 32- and 64-bank LDS.
// ---------------------------------------------------------------------------
template <bool VEC>
__global__ __launch_bounds__(256) void quant_cols_kernel(const uint16_t* __restrict__ x,
                                                         int64_t rows, int64_t cols,
                                                         uint8_t* __restrict__ qt,
                                                         float* __restrict__ st, bool skm = false) {
  __shared__ uint32_t tile[128 * 34];
  __shared__ uint32_t tq[64 * 36];
  const int tid = threadIdx.x;
  const int64_t c0 = (int64_t)blockIdx.x * 64;
  const int64_t r0 = (int64_t)blockIdx.y * 128;

#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int id = tid + 256 * u;
    const int row = id >> 3, ch = id & 7;
    const int64_t col = c0 + ch * 8;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (VEC) {
      if (col < cols) v = ldg_stream(x + (r0 + row) * cols + col);
    } else {
      // rows are not 16-byte aligned when cols % 8 != 0: element loads
      uint32_t e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = (col + k < cols) ? x[(r0 + row) * cols + col + k] : 0u;
      v = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
    }
    uint2* p = reinterpret_cast<uint2*>(&tile[row * 34 + ch * 4]);
    p[0] = make_uint2(v.x, v.y);
    p[1] = make_uint2(v.z, v.w);
  }
  __syncthreads();

  const int n = tid >> 2, j = tid & 3;
  const uint16_t* t16 = reinterpret_cast<const uint16_t*>(tile);
  float f[32];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r)
      f[i * 4 + r] = __uint_as_float(((uint32_t)t16[(16 * i + 4 * j + r) * 68 + n]) << 16);
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) m = max(m, __float_as_uint(f[i]) & 0x7FFFFFFFu);
  m = quad_max_u32(m);
  const float sc = block_scale_bf16(m);
  Divider d(sc);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    uint32_t w;
    if (d.fast) {
      w = e4m3x4(d.div(f[4 * i]), d.div(f[4 * i + 1]), d.div(f[4 * i + 2]), d.div(f[4 * i + 3]));
    } else {
      w = e4m3_nonfinite_scale(f[4 * i], sc) | (e4m3_nonfinite_scale(f[4 * i + 1], sc) << 8) |
          (e4m3_nonfinite_scale(f[4 * i + 2], sc) << 16) |
          (e4m3_nonfinite_scale(f[4 * i + 3], sc) << 24);
    }
    tq[n * 36 + 4 * i + j] = w;
  }
  const bool col_ok = (c0 + n) < cols;
  if (j == 0 && col_ok) st[skm ? (int64_t)blockIdx.y * cols + c0 + n : (c0 + n) * (rows >> 7) + blockIdx.y] = sc;
  __syncthreads();
  if (col_ok) {
    const uint4* src = reinterpret_cast<const uint4*>(&tq[n * 36 + 8 * j]);
    uint4* dst = reinterpret_cast<uint4*>(qt + (c0 + n) * rows + r0 + 32 * j);
    dst[0] = src[0];
    dst[1] = src[1];
  }
}


// The dual kernel (rows and / or x.T from one read) lives in quant_dual.h,
// shared with the I/O-floor probe csrc/probe/quant_floor.hip.

int launch_quant_cols(const void* x, int64_t rows, int64_t cols, uint8_t* q_t, float* s_t,
                      hipStream_t st, bool skm) {
  if (rows == 0 || cols == 0) return TG_OK;
  if (rows / 128 > 65535) return einval("quantize_cols: rows / 128 must be <= 65535");
  if (cols % 8 == 0 && aligned(x, 16)) {
    // 128 x 128 tiles: column pairs per LDS read, 64-byte contiguous stores
    DualJobs jobs{};
    TG_TRY(dual_job(jobs.job[0], "quantize_cols", x, rows, cols, nullptr, nullptr, q_t, s_t, false, skm));
    jobs.nblk0 = jobs.job[0].gx * jobs.job[0].gy;
    const dim3 grid((unsigned)jobs.nblk0);
    if (cols % 128 == 0)
      hipLaunchKernelGGL((quant_dual_kernel<false, false>), grid, dim3(kDualThreads), 0, st, jobs);
    else
      hipLaunchKernelGGL((quant_dual_kernel<false, true>), grid, dim3(kDualThreads), 0, st, jobs);
    return check_launch("quant_cols");
  }
  // rows not 16-byte aligned: the element-load kernel
  const dim3 grid((unsigned)((cols + 63) / 64), (unsigned)(rows / 128));
  hipLaunchKernelGGL(quant_cols_kernel<false>, grid, dim3(256), 0, st,
                     reinterpret_cast<const uint16_t*>(x), rows, cols, q_t, s_t, skm);
  return check_launch("quant_cols");
}

int launch_quant_dual(const void* x, int64_t rows, int64_t cols, uint8_t* q, float* s, uint8_t* q_t,
                      float* s_t, hipStream_t st, bool skm) {
  if (rows == 0 || cols == 0) return TG_OK;
  if (rows % 128 || cols % 128) return einval("quantize_dual: rows and cols must be multiples of 128");
  DualJobs jobs{};
  TG_TRY(dual_job(jobs.job[0], "quantize_dual", x, rows, cols, q, s, q_t, s_t, true, skm));
  jobs.nblk0 = jobs.job[0].gx * jobs.job[0].gy;
  hipLaunchKernelGGL((quant_dual_kernel<true, false>), dim3((unsigned)jobs.nblk0), dim3(kDualThreads), 0,
                     st, jobs);
  return check_launch("quant_dual");
}

int launch_quant_dual_pair(const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0, float* s0,
                           uint8_t* qt0, float* st0, const void* x1, int64_t rows1, int64_t cols1,
                           uint8_t* q1, float* s1, uint8_t* qt1, float* st1, hipStream_t st, bool skm) {
  const bool e0 = rows0 == 0 || cols0 == 0, e1 = rows1 == 0 || cols1 == 0;
  if (e0 && e1) return TG_OK;
  if (e0) return launch_quant_dual(x1, rows1, cols1, q1, s1, qt1, st1, st, skm);
  if (e1) return launch_quant_dual(x0, rows0, cols0, q0, s0, qt0, st0, st, skm);
  if (rows0 % 128 || cols0 % 128 || rows1 % 128 || cols1 % 128)
    return einval("quantize_dual_pair: rows and cols must be multiples of 128");
  DualJobs jobs{};
  TG_TRY(dual_job(jobs.job[0], "quantize_dual_pair", x0, rows0, cols0, q0, s0, qt0, st0, true, skm));
  jobs.nblk0 = jobs.job[0].gx * jobs.job[0].gy;
  TG_TRY(dual_job(jobs.job[1], "quantize_dual_pair", x1, rows1, cols1, q1, s1, qt1, st1,
                  jobs.nblk0 % 8 == 0, skm));
  const int64_t total = (int64_t)jobs.nblk0 + (int64_t)jobs.job[1].gx * jobs.job[1].gy;
  if (total > kDualMaxTiles) return einval("quantize_dual_pair: too many 128 x 128 tiles");
  hipLaunchKernelGGL((quant_dual_kernel<true, false>), dim3((unsigned)total), dim3(kDualThreads), 0, st, jobs);
  return check_launch("quant_dual_pair");
}

// The forward's two quantizations in one launch: a (M, K) along its rows
// (fp8.py:66) and b (K, N) as b.T along K (fp8.py:68), the bytes and scales of
// launch_quant_rows and launch_quant_cols.  Every extent a multiple of 128.
int launch_quant_rows_cols(const void* a, int64_t M, int64_t K, uint8_t* qa, float* sa, const void* b,
                           int64_t N, uint8_t* qbt, float* sbt, hipStream_t st, bool skm) {
  if (M % 128 || K % 128 || N % 128) return einval("quantize_rows_cols: M, K and N must be multiples of 128");
  if (M == 0 || K == 0 || N == 0) return TG_OK;
  DualJobs jobs{};
  TG_TRY(dual_job(jobs.job[0], "quantize_rows_cols", a, M, K, qa, sa, nullptr, nullptr, true, skm));
  jobs.job[0].part = 1;
  jobs.nblk0 = jobs.job[0].gx * jobs.job[0].gy;
  TG_TRY(dual_job(jobs.job[1], "quantize_rows_cols", b, K, N, nullptr, nullptr, qbt, sbt, jobs.nblk0 % 8 == 0,
                  skm));
  jobs.job[1].part = 2;
  const int64_t total = (int64_t)jobs.nblk0 + (int64_t)jobs.job[1].gx * jobs.job[1].gy;
  if (total > kDualMaxTiles) return einval("quantize_rows_cols: too many 128 x 128 tiles");
  hipLaunchKernelGGL((quant_dual_kernel<true, false>), dim3((unsigned)total), dim3(kDualThreads), 0, st, jobs);
  return check_launch("quant_rows_cols");
}

// ---------------------------------------------------------------------------
// 128x128-tile weight quantization (offline weight preparation for the GEMV).
// One workgroup per tile: the tile (128 rows of K x 128 columns of N, bf16)
// is copied to LDS with 16-byte loads while each thread keeps its maximum;
// the tile amax gives the scale; then thread (column c, half h) quantizes
// rows 64h .. 64h+63 of column c from LDS (a wave reads 64 consecutive
// columns of one row, 128 B) and stores them as 4 x 16 bytes of w.T's row c.
// ---------------------------------------------------------------------------
constexpr int kW128Pitch = 128 * 2 + 16;
__global__ __launch_bounds__(256) void quant_w128_kernel(const uint16_t* __restrict__ w, int64_t K,
                                                         int64_t N, uint8_t* __restrict__ wq,
                                                         float* __restrict__ ws, int vec) {
  __shared__ __attribute__((aligned(16))) uint8_t tile[128 * kW128Pitch];
  __shared__ uint32_t red[4];
  const int tid = threadIdx.x;
  const int64_t k0 = (int64_t)blockIdx.y * 128, n0 = (int64_t)blockIdx.x * 128;
  const int ch = tid & 15, rr = tid >> 4;          // 16-byte chunk of a row, first row
  const int64_t nc = n0 + ch * 8;
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = rr + 16 * i;
    const uint16_t* src = w + (k0 + r) * N + nc;
    uint4 v;
    if (vec && nc + 8 <= N) {
      v = *reinterpret_cast<const uint4*>(src);
    } else {                                       // N % 8 != 0, unaligned w, or the tile's ragged edge
      uint32_t e[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) e[j] = nc + j < N ? (uint32_t)src[j] : 0u;
      v = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
    }
    *reinterpret_cast<uint4*>(tile + r * kW128Pitch + ch * 16) = v;
    m = max(m, max(max(bf16_amax2(v.x), bf16_amax2(v.y)), max(bf16_amax2(v.z), bf16_amax2(v.w))));
  }
  for (int o = 32; o >= 1; o >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, o, 64));
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  m = max(max(red[0], red[1]), max(red[2], red[3]));
  const float sc = block_scale_bf16(m);
  if (tid == 0) ws[blockIdx.x * (K >> 7) + blockIdx.y] = sc;
  Divider d(sc);
  const int c = tid & 127, half = tid >> 7;
  const int64_t n = n0 + c;
  if (n >= N) return;
  uint32_t out[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    float f[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      f[r] = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(
                                 tile + (half * 64 + 4 * i + r) * kW128Pitch + c * 2) << 16);
    if (d.fast)
      out[i] = e4m3x4(d.div(f[0]), d.div(f[1]), d.div(f[2]), d.div(f[3]));
    else
      out[i] = e4m3_nonfinite_scale(f[0], sc) | (e4m3_nonfinite_scale(f[1], sc) << 8) |
               (e4m3_nonfinite_scale(f[2], sc) << 16) | (e4m3_nonfinite_scale(f[3], sc) << 24);
  }
  uint4* dst = reinterpret_cast<uint4*>(wq + n * K + k0 + half * 64);
#pragma unroll
  for (int i = 0; i < 4; ++i)
    dst[i] = make_uint4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
}

// ---------------------------------------------------------------------------
// Self-test of the hardware convert over all 2^32 f32 bit patterns.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void selftest_cvt_kernel(unsigned long long* counts) {
  unsigned long long c0 = 0, c1 = 0, c2 = 0;
  const uint64_t stride = (uint64_t)gridDim.x * 256 * 4;
  for (uint64_t base = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4; base < (1ull << 32);
       base += stride) {
    float f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float((uint32_t)(base + i));
    int hw = __builtin_amdgcn_cvt_pk_fp8_f32(f[0], f[1], 0, false);
    hw = __builtin_amdgcn_cvt_pk_fp8_f32(f[2], f[3], hw, true);
    const uint32_t sw = e4m3x4_sw(f[0], f[1], f[2], f[3]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t hb = ((uint32_t)hw >> (8 * i)) & 0xFF, sb = (sw >> (8 * i)) & 0xFF;
      if (hb != sb) {
        const uint32_t a = __float_as_uint(f[i]) & 0x7FFFFFFFu;
        if (a >= 0x7F800000u) ++c2;
        else if (a <= 0x43E00E00u) ++c0;   // 448 * (1 + 2^-12)
        else ++c1;
      }
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    c0 += __shfl_xor(c0, o, 64);
    c1 += __shfl_xor(c1, o, 64);
    c2 += __shfl_xor(c2, o, 64);
  }
  if ((threadIdx.x & 63) == 0) {
    atomicAdd(&counts[0], c0);
    atomicAdd(&counts[1], c1);
    atomicAdd(&counts[2], c2);
  }
}

// Self-test of the bf16 quantizer arithmetic against the device's IEEE
// operations, over every bf16 amax (one workgroup each) and every bf16 x
// with |x| <= amax, both signs.  counts[0]: e4m3fn byte mismatches of
// Divider::div; counts[1]: f32 quotient mismatches with |x/s| > 2^-10;
// counts[2]: quotient mismatches at or below 2^-10; counts[3]:
// block_scale_bf16 != IEEE scale; counts[4]: Divider's reciprocal != IEEE 1/s.
__global__ __launch_bounds__(256) void selftest_divide_kernel(unsigned long long* counts) {
  const uint32_t ab = blockIdx.x;                       // bf16 pattern of amax
  const float a = __uint_as_float(ab << 16);
  const float sc = block_scale_bf16(__float_as_uint(a));
  const float sc_ieee = block_scale(__float_as_uint(a));
  const Divider d(sc);
  if (threadIdx.x == 0) {
    if (__float_as_uint(sc) != __float_as_uint(sc_ieee)) atomicAdd(&counts[3], 1ull);
    if (d.fast && __float_as_uint(d.y) != __float_as_uint(1.0f / sc)) atomicAdd(&counts[4], 1ull);
  }
  unsigned long long c0 = 0, c1 = 0, c2 = 0;
  for (uint32_t i = threadIdx.x; i <= 2 * ab + 1; i += 256) {
    const float x = __uint_as_float(((i >> 1) << 16) | ((i & 1u) << 31));
    const float q = d.div(x);
    const float ref = x / sc;
    if (e4m3_sw(q) != e4m3_sw(ref)) ++c0;
    if (__float_as_uint(q) != __float_as_uint(ref)) {
      if (__builtin_fabsf(ref) > 0x1p-10f) ++c1; else ++c2;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    c0 += __shfl_xor(c0, o, 64);
    c1 += __shfl_xor(c1, o, 64);
    c2 += __shfl_xor(c2, o, 64);
  }
  if ((threadIdx.x & 63) == 0 && (c0 | c1 | c2)) {
    atomicAdd(&counts[0], c0);
    atomicAdd(&counts[1], c1);
    atomicAdd(&counts[2], c2);
  }
}

__global__ void zero_kernel(unsigned long long* c, int n) {
  if ((int)threadIdx.x < n) c[threadIdx.x] = 0;
}

}  // namespace tg

using namespace tg;

extern "C" const char* tg_last_error(void) { return g_err; }

extern "C" int tg_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                int block_k, uint8_t* q, float* scales, void* stream) {
  if (block_k <= 0) return einval("quantize_rows: block_k must be positive");
  if (rows < 0 || cols < 0) return einval("quantize_rows: negative shape");
  if (cols % block_k) return einval("quantize_rows: cols not divisible by block_k");
  if (x_dtype != TG_DTYPE_BF16 && x_dtype != TG_DTYPE_F32)
    return einval("quantize_rows: x_dtype must be TG_DTYPE_BF16 or TG_DTYPE_F32");
  if (rows * cols == 0) return TG_OK;
  if (!x || !q || !scales) return einval("quantize_rows: null pointer");
  if (block_k != 128) {   // the general path: any block size, element-aligned pointers
    if (!aligned(x, x_dtype == TG_DTYPE_F32 ? 4 : 2) || !aligned(scales, 4))
      return einval("quantize_rows: x and scales must be aligned to their element size");
    return launch_quant_rows_gb(x, x_dtype, rows, cols, block_k, q, scales, as_stream(stream));
  }
  if (!aligned(x, 16) || !aligned(q, 8) || !aligned(scales, 4))
    return einval("quantize_rows: x must be 16-byte and q 8-byte aligned");
  return launch_quant_rows(x, x_dtype, rows, cols, q, scales, as_stream(stream));
}

extern "C" int tg_quantize_rows_relu2(const void* x, int64_t rows, int64_t cols, int block_k,
                                      uint8_t* q, float* scales, void* stream) {
  if (block_k != 128) return einval("quantize_rows_relu2: block_k must be 128");
  if (rows < 0 || cols < 0) return einval("quantize_rows_relu2: bad shape");
  if (cols % block_k) return einval("quantize_rows_relu2: cols not divisible by block_k");
  if (rows == 0 || cols == 0) return TG_OK;
  if (!x || !q || !scales) return einval("quantize_rows_relu2: null pointer");
  if (!aligned(x, 16) || !aligned(q, 8)) return einval("quantize_rows_relu2: x must be 16-byte and q 8-byte aligned");
  return launch_quant_rows_relu2(x, rows, cols, q, scales, as_stream(stream));
}

extern "C" int tg_quantize_cols(const void* x, int x_dtype, int64_t rows, int64_t cols,
                                int block_k, uint8_t* q_t, float* scales_t, void* stream) {
  if (block_k <= 0) return einval("quantize_cols: block_k must be positive");
  if (x_dtype != TG_DTYPE_BF16 && x_dtype != TG_DTYPE_F32)
    return einval("quantize_cols: x_dtype must be TG_DTYPE_BF16 or TG_DTYPE_F32");
  if (rows < 0 || cols < 0) return einval("quantize_cols: negative shape");
  if (rows % block_k) return einval("quantize_cols: rows not divisible by block_k");
  if (rows * cols == 0) return TG_OK;
  if (!x || !q_t || !scales_t) return einval("quantize_cols: null pointer");
  // f32 input (any block_k) and block_k != 128 take the general kernel
  if (block_k != 128 || x_dtype == TG_DTYPE_F32) {
    if (!aligned(x, x_dtype == TG_DTYPE_F32 ? 4 : 2) || !aligned(scales_t, 4))
      return einval("quantize_cols: x and scales_t must be aligned");
    return launch_quant_cols_gb(x, x_dtype == TG_DTYPE_F32, rows, cols, block_k, q_t, scales_t,
                                as_stream(stream));
  }
  if (!aligned(x, 2) || !aligned(q_t, 16)) return einval("quantize_cols: q_t must be 16-byte aligned");
  return launch_quant_cols(x, rows, cols, q_t, scales_t, as_stream(stream));
}

extern "C" int tg_quantize_weight_128x128(const void* w, int64_t K, int64_t N, uint8_t* w_q,
                                          float* w_s, void* stream) {
  if (K <= 0 || K % 128) return einval("quantize_weight_128x128: K must be a positive multiple of 128");
  if (N < 0) return einval("quantize_weight_128x128: bad shape");
  if (K / 128 > 65535) return einval("quantize_weight_128x128: K too large");
  if (N == 0) return TG_OK;
  if (!w || !w_q || !w_s) return einval("quantize_weight_128x128: null pointer");
  if (!aligned(w_q, 16)) return einval("quantize_weight_128x128: w_q must be 16-byte aligned");
  dim3 grid((unsigned)((N + 127) / 128), (unsigned)(K / 128));
  const int vec = N % 8 == 0 && aligned(w, 16);
  hipLaunchKernelGGL(quant_w128_kernel, grid, dim3(256), 0, as_stream(stream),
                     reinterpret_cast<const uint16_t*>(w), K, N, w_q, w_s, vec);
  return check_launch("quant_w128");
}

extern "C" int tg_selftest_fp8_cvt(uint64_t* counts, void* stream) {
  if (!counts) return einval("selftest_fp8_cvt: null pointer");
  auto* c = reinterpret_cast<unsigned long long*>(counts);
  hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(64), 0, as_stream(stream), c, 3);
  TG_TRY(check_launch("zero"));
  hipLaunchKernelGGL(selftest_cvt_kernel, dim3(4096), dim3(256), 0, as_stream(stream), c);
  return check_launch("selftest_cvt");
}

extern "C" int tg_selftest_divide(uint64_t* counts, void* stream) {
  if (!counts) return einval("selftest_divide: null pointer");
  auto* c = reinterpret_cast<unsigned long long*>(counts);
  hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(64), 0, as_stream(stream), c, 5);
  TG_TRY(check_launch("zero"));
  hipLaunchKernelGGL(selftest_divide_kernel, dim3(0x7F80), dim3(256), 0, as_stream(stream), c);
  return check_launch("selftest_divide");
}

static int quantize_dual_entry(const void* x, int64_t rows, int64_t cols, int block_k, uint8_t* q,
                               float* s, uint8_t* q_t, float* s_t, void* stream, bool skm) {
  if (block_k != 128) return einval("quantize_dual: block_k must be 128");
  if (rows < 0 || cols < 0) return einval("quantize_dual: bad shape");
  if (rows == 0 || cols == 0) return TG_OK;
  if (!x || !q || !s || !q_t || !s_t) return einval("quantize_dual: null pointer");
  if (!aligned(x, 16) || !aligned(q, 8) || !aligned(q_t, 16))
    return einval("quantize_dual: x and q_t must be 16-byte, q 8-byte aligned");
  return launch_quant_dual(x, rows, cols, q, s, q_t, s_t, as_stream(stream), skm);
}
extern "C" int tg_quantize_dual(const void* x, int64_t rows, int64_t cols, int block_k, uint8_t* q,
                                float* s, uint8_t* q_t, float* s_t, void* stream) {
  return quantize_dual_entry(x, rows, cols, block_k, q, s, q_t, s_t, stream, false);
}
extern "C" int tg_quantize_dual_km(const void* x, int64_t rows, int64_t cols, int block_k, uint8_t* q,
                                   float* s_km, uint8_t* q_t, float* s_t_km, void* stream) {
  return quantize_dual_entry(x, rows, cols, block_k, q, s_km, q_t, s_t_km, stream, true);
}

static int quantize_dual_pair_entry(const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0,
                                    float* s0, uint8_t* q_t0, float* s_t0, const void* x1,
                                    int64_t rows1, int64_t cols1, uint8_t* q1, float* s1,
                                    uint8_t* q_t1, float* s_t1, int block_k, void* stream, bool skm) {
  if (block_k != 128) return einval("quantize_dual_pair: block_k must be 128");
  if (rows0 < 0 || cols0 < 0 || rows1 < 0 || cols1 < 0) return einval("quantize_dual_pair: bad shape");
  const bool u0 = rows0 > 0 && cols0 > 0, u1 = rows1 > 0 && cols1 > 0;
  if ((u0 && (!x0 || !q0 || !s0 || !q_t0 || !s_t0)) || (u1 && (!x1 || !q1 || !s1 || !q_t1 || !s_t1)))
    return einval("quantize_dual_pair: null pointer");
  if ((u0 && (!aligned(x0, 16) || !aligned(q0, 8) || !aligned(q_t0, 16))) ||
      (u1 && (!aligned(x1, 16) || !aligned(q1, 8) || !aligned(q_t1, 16))))
    return einval("quantize_dual_pair: x and q_t must be 16-byte, q 8-byte aligned");
  return launch_quant_dual_pair(x0, rows0, cols0, q0, s0, q_t0, s_t0, x1, rows1, cols1, q1, s1, q_t1,
                                s_t1, as_stream(stream), skm);
}
extern "C" int tg_quantize_dual_pair(const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0,
                                     float* s0, uint8_t* q_t0, float* s_t0, const void* x1,
                                     int64_t rows1, int64_t cols1, uint8_t* q1, float* s1,
                                     uint8_t* q_t1, float* s_t1, int block_k, void* stream) {
  return quantize_dual_pair_entry(x0, rows0, cols0, q0, s0, q_t0, s_t0, x1, rows1, cols1, q1, s1, q_t1,
                                  s_t1, block_k, stream, false);
}
extern "C" int tg_quantize_dual_pair_km(const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0,
                                        float* s0_km, uint8_t* q_t0, float* s_t0_km, const void* x1,
                                        int64_t rows1, int64_t cols1, uint8_t* q1, float* s1_km,
                                        uint8_t* q_t1, float* s_t1_km, int block_k, void* stream) {
  return quantize_dual_pair_entry(x0, rows0, cols0, q0, s0_km, q_t0, s_t0_km, x1, rows1, cols1, q1, s1_km,
                                  q_t1, s_t1_km, block_k, stream, true);
}
