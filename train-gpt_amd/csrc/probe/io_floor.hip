// Measurement probe (not part of the product library): the HBM traffic of the
// fused RMSNorm -> FP8 kernel (rmsnorm_kernel<4, true, true> in rmsnorm.hip)
// with its arithmetic taken out, so that bench.py can time the I/O floor of
// config 2's exact read / write mix on the same launch shape.
//
// Access pattern, as in the norm kernel at dim 2048: one wave64 per row, lane
// l owns the 16-byte chunks l + 64 j (j < 4) of its row, rows walked with a
// grid stride, the next row's x loaded (non-temporal) before the current one
// is stored; y as 16-byte and q as 8-byte non-temporal stores per chunk, one
// f32 scale per 128-element block from the first lane of each 16-lane group.
//
// mode 0: read x only (one f32 per row is written so the loads stay live)
// mode 1: read x, write y                      (a bf16 copy)
// mode 2: read x, write y, q and the scales    (config 2's mix)
// mode 3: write y, q and the scales, read nothing
#include <type_traits>

#include "../gemm_tile.h"
#include "../tg_device.h"
#include "../tg_host.h"

namespace tg {

template <int MODE>
__global__ __launch_bounds__(256) void io_floor_kernel(const uint4* __restrict__ x, uint4* __restrict__ y,
                                                       uint2* __restrict__ q, float* __restrict__ s,
                                                       int64_t rows) {
  constexpr int J = 4, NCH = 256;
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * 4;
  auto load_row = [&](int64_t row, uint4 (&v)[J]) {
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if (MODE == 3) v[j] = make_uint4((uint32_t)row, (uint32_t)lane, (uint32_t)j, 0u);
      else v[j] = ldg_stream(x + row * NCH + lane + 64 * j);
    }
  };
  uint4 nxt[J];
  if (wave0 < rows) load_row(wave0, nxt);
  for (int64_t row = wave0; row < rows; row += wstride) {
    uint4 cur[J];
#pragma unroll
    for (int j = 0; j < J; ++j) cur[j] = nxt[j];
    if (row + wstride < rows) load_row(row + wstride, nxt);
    if (MODE == 0) {
      uint32_t acc = 0;
#pragma unroll
      for (int j = 0; j < J; ++j) acc ^= cur[j].x ^ cur[j].y ^ cur[j].z ^ cur[j].w;
      if (lane == 0) s[row] = __uint_as_float(acc);
      continue;
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      stg_stream(&y[row * NCH + c], cur[j]);
      if (MODE >= 2) {
        stg_stream(&q[row * NCH + c], make_uint2(cur[j].x ^ cur[j].z, cur[j].y ^ cur[j].w));
        if ((lane & 15) == 0) s[row * (NCH >> 4) + (c >> 4)] = __uint_as_float(cur[j].x);
      }
    }
  }
}

}  // namespace tg

// rows x 2048 bf16 input; the grid is sized like the norm kernel's for the
// given rows per wave (at least 512 workgroups, at most 16384).
extern "C" int tg_probe_io_floor(int mode, const void* x, void* y, void* q, float* s, int64_t rows,
                                 int rows_per_wave, void* stream) {
  using namespace tg;
  if (mode < 0 || mode > 3 || rows <= 0 || rows_per_wave <= 0) return einval("tg_probe_io_floor: bad arguments");
  if ((mode != 3 && !x) || (mode != 0 && !y) || (mode >= 2 && !q) || !s)
    return einval("tg_probe_io_floor: null pointer");
  int64_t grid = (rows + 4 * rows_per_wave - 1) / (4 * rows_per_wave);
  if (grid < 512) grid = (rows + 3) / 4 < 512 ? (rows + 3) / 4 : 512;
  if (grid > 16384) grid = 16384;
  auto st = static_cast<hipStream_t>(stream);
  auto X = reinterpret_cast<const uint4*>(x);
  auto Y = reinterpret_cast<uint4*>(y);
  auto Q = reinterpret_cast<uint2*>(q);
  const dim3 g((unsigned)grid), b(256);
  switch (mode) {
    case 0: hipLaunchKernelGGL(io_floor_kernel<0>, g, b, 0, st, X, Y, Q, s, rows); break;
    case 1: hipLaunchKernelGGL(io_floor_kernel<1>, g, b, 0, st, X, Y, Q, s, rows); break;
    case 2: hipLaunchKernelGGL(io_floor_kernel<2>, g, b, 0, st, X, Y, Q, s, rows); break;
    default: hipLaunchKernelGGL(io_floor_kernel<3>, g, b, 0, st, X, Y, Q, s, rows); break;
  }
  return check_launch("io_floor");
}

// The same rows, pipelined: each wave keeps two rows' loads in flight and
// stores a row's y / q / scales one row later, after the wait for the next
// row's loads; every access is an unconditional raw buffer access over the
// row's own bytes (a row past the end, and a lane that stores no scale, touch
// no memory), so the compiler's waits are for the loads consumed, never for
// stores issued in the same step.  (io_floor_kernel's prefetch and stores sit
// behind branches, and its wait for the prefetched row also waits for the
// current row's stores: VMEM operations retire from vmcnt in issue order.)
namespace tg {

template <int MODE>
__global__ __launch_bounds__(256) void io_pipe_kernel(const uint4* __restrict__ x, uint4* __restrict__ y,
                                                      uint2* __restrict__ q, float* __restrict__ s,
                                                      int64_t rows) {
  constexpr int J = 4, NCH = 256;
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * 4;
  auto rsrc_of = [&](const void* base, int64_t row, uint32_t row_bytes) {
    const bool in = row < rows;
    return make_rsrc(static_cast<const uint8_t*>(base) + (in ? row : 0) * row_bytes, in ? row_bytes : 0u);
  };
  u32x4_t buf[2][J], pend[J];
  int64_t pend_row = rows;   // none yet: its stores are dropped
#pragma unroll
  for (int j = 0; j < J; ++j) pend[j] = u32x4_t{0u, 0u, 0u, 0u};
  auto load_slot = [&](auto slot, int64_t row) {
    constexpr int S = decltype(slot)::value;
    const __amdgpu_buffer_rsrc_t rx = rsrc_of(x, row, NCH * 16);
#pragma unroll
    for (int j = 0; j < J; ++j)
      buf[S][j] = MODE == 3 ? u32x4_t{(uint32_t)row, (uint32_t)lane, (uint32_t)j, 0u}
                            : __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(lane + 64 * j) * 16u, 0, kAuxNT);
  };
  auto store_pend = [&]() {
    if (MODE == 0) {
      uint32_t acc = 0;
#pragma unroll
      for (int j = 0; j < J; ++j) acc ^= pend[j].x ^ pend[j].y ^ pend[j].z ^ pend[j].w;
      const __amdgpu_buffer_rsrc_t rs = rsrc_of(s, pend_row, 4);
      __builtin_amdgcn_raw_buffer_store_b32(acc, rs, lane == 0 ? 0u : 0x80000000u, 0, 0);
      return;
    }
    const __amdgpu_buffer_rsrc_t ry = rsrc_of(y, pend_row, NCH * 16);
    const __amdgpu_buffer_rsrc_t rq = rsrc_of(q, pend_row, NCH * 8);
    const __amdgpu_buffer_rsrc_t rs = rsrc_of(s, pend_row, NCH / 16 * 4);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t c = (uint32_t)(lane + 64 * j);
      __builtin_amdgcn_raw_buffer_store_b128(pend[j], ry, c * 16u, 0, kAuxNT);
      if (MODE >= 2) {
        const u32x2_t qv = {pend[j].x ^ pend[j].z, pend[j].y ^ pend[j].w};
        __builtin_amdgcn_raw_buffer_store_b64(qv, rq, c * 8u, 0, kAuxNT);
        __builtin_amdgcn_raw_buffer_store_b32(pend[j].x, rs, (lane & 15) == 0 ? (c >> 4) * 4u : 0x80000000u, 0, 0);
      }
    }
  };
  auto step = [&](auto slot, int64_t row) {
    constexpr int S = decltype(slot)::value;
    u32x4_t cur[J];
#pragma unroll
    for (int j = 0; j < J; ++j) cur[j] = buf[S][j];
    store_pend();
    load_slot(slot, row + 2 * wstride);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < J; ++j) pend[j] = cur[j];
    pend_row = row;
  };
  load_slot(std::integral_constant<int, 0>{}, wave0);
  __builtin_amdgcn_sched_barrier(0);
  load_slot(std::integral_constant<int, 1>{}, wave0 + wstride);
  __builtin_amdgcn_sched_barrier(0);
  for (int64_t row = wave0; row < rows; row += 2 * wstride) {
    step(std::integral_constant<int, 0>{}, row);
    step(std::integral_constant<int, 1>{}, row + wstride);
  }
  store_pend();
}

}  // namespace tg

// io_floor_kernel's modes and grid, on io_pipe_kernel.
extern "C" int tg_probe_io_pipe(int mode, const void* x, void* y, void* q, float* s, int64_t rows,
                                int rows_per_wave, void* stream) {
  using namespace tg;
  if (mode < 0 || mode > 3 || rows <= 0 || rows_per_wave <= 0) return einval("tg_probe_io_pipe: bad arguments");
  if ((mode != 3 && !x) || (mode != 0 && !y) || (mode >= 2 && !q) || !s)
    return einval("tg_probe_io_pipe: null pointer");
  int64_t grid = (rows + 4 * rows_per_wave - 1) / (4 * rows_per_wave);
  if (grid < 512) grid = (rows + 3) / 4 < 512 ? (rows + 3) / 4 : 512;
  if (grid > 16384) grid = 16384;
  auto st = static_cast<hipStream_t>(stream);
  auto X = reinterpret_cast<const uint4*>(x);
  auto Y = reinterpret_cast<uint4*>(y);
  auto Q = reinterpret_cast<uint2*>(q);
  const dim3 g((unsigned)grid), b(256);
  switch (mode) {
    case 0: hipLaunchKernelGGL(io_pipe_kernel<0>, g, b, 0, st, X, Y, Q, s, rows); break;
    case 1: hipLaunchKernelGGL(io_pipe_kernel<1>, g, b, 0, st, X, Y, Q, s, rows); break;
    case 2: hipLaunchKernelGGL(io_pipe_kernel<2>, g, b, 0, st, X, Y, Q, s, rows); break;
    default: hipLaunchKernelGGL(io_pipe_kernel<3>, g, b, 0, st, X, Y, Q, s, rows); break;
  }
  return check_launch("io_pipe");
}

// The norm backward's traffic (rmsnorm_bwd_kernel<4, true> at dim 2048, the
// kernel behind tg_rms_norm_bwd): x and dy rows read, dx rows written, with
// that kernel's pipelined row walk (two rows' loads in flight per wave, each
// row's dx stored one row later, unconditional raw buffer accesses) and one
// 2048-float partial row per workgroup at the end; dx is a bit mix of x and
// dy, no arithmetic.  bench.py --only norm_bwd times it on the product's grid
// (one workgroup per CU) and on larger ones, and with 3 or 4 rows in flight.
namespace tg {

template <int PD>
__global__ __launch_bounds__(256) void io_bwd_kernel(const uint4* __restrict__ x, const uint4* __restrict__ dy,
                                                     uint4* __restrict__ dx, float* __restrict__ partial,
                                                     int64_t rows) {
  constexpr int J = 4, NCH = 256;
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * 4;
  auto rsrc_of = [&](const uint4* base, int64_t row) {
    const bool in = row < rows;
    return make_rsrc(base + (in ? row : 0) * NCH, in ? (uint32_t)NCH * 16u : 0u);
  };
  u32x4_t bx[PD][J], bd[PD][J], pend[J];
  int64_t pend_row = rows;   // none yet: its stores are dropped
#pragma unroll
  for (int j = 0; j < J; ++j) pend[j] = u32x4_t{0u, 0u, 0u, 0u};
  uint32_t mix = 0;
  auto load_slot = [&](auto slot, int64_t row) {
    constexpr int S = decltype(slot)::value;
    const __amdgpu_buffer_rsrc_t rx = rsrc_of(x, row), rd = rsrc_of(dy, row);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const uint32_t off = (uint32_t)(lane + 64 * j) * 16u;
      bx[S][j] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, kAuxNT);
      bd[S][j] = __builtin_amdgcn_raw_buffer_load_b128(rd, off, 0, kAuxNT);
    }
  };
  auto store_pend = [&]() {
    const __amdgpu_buffer_rsrc_t ro = rsrc_of(dx, pend_row);
#pragma unroll
    for (int j = 0; j < J; ++j)
      __builtin_amdgcn_raw_buffer_store_b128(pend[j], ro, (uint32_t)(lane + 64 * j) * 16u, 0, kAuxNT);
  };
  auto step = [&](auto slot, int64_t row) {
    constexpr int S = decltype(slot)::value;
    u32x4_t cur[J];
#pragma unroll
    for (int j = 0; j < J; ++j) cur[j] = bx[S][j] ^ bd[S][j];
    store_pend();
    load_slot(slot, row + PD * wstride);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      pend[j] = cur[j];
      mix ^= cur[j].x;
    }
    pend_row = row;
  };
  load_slot(std::integral_constant<int, 0>{}, wave0);
  __builtin_amdgcn_sched_barrier(0);
  load_slot(std::integral_constant<int, 1>{}, wave0 + wstride);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (PD > 2) {
    load_slot(std::integral_constant<int, 2 % PD>{}, wave0 + 2 * wstride);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (PD > 3) {
    load_slot(std::integral_constant<int, 3 % PD>{}, wave0 + 3 * wstride);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int64_t row = wave0; row < rows; row += PD * wstride) {
    step(std::integral_constant<int, 0>{}, row);
    step(std::integral_constant<int, 1>{}, row + wstride);
    if constexpr (PD > 2) step(std::integral_constant<int, 2 % PD>{}, row + 2 * wstride);
    if constexpr (PD > 3) step(std::integral_constant<int, 3 % PD>{}, row + 3 * wstride);
  }
  store_pend();
  // the workgroup's partial row (2048 floats, as the product writes its dscale partials)
  for (int i = threadIdx.x; i < NCH * 8; i += 256)
    partial[(int64_t)blockIdx.x * NCH * 8 + i] = __uint_as_float(mix ^ (uint32_t)i);
}

}  // namespace tg

// rows x 2048 bf16 x and dy, dx written; partial holds grid x 2048 floats;
// depth 2, 3 or 4 rows' loads in flight per wave (the product keeps 2).
extern "C" int tg_probe_io_bwd(const void* x, const void* dy, void* dx, float* partial, int64_t rows, int grid,
                               int depth, void* stream) {
  using namespace tg;
  if (rows <= 0 || grid <= 0 || grid > 65535 || depth < 2 || depth > 4)
    return einval("tg_probe_io_bwd: bad arguments");
  if (!x || !dy || !dx || !partial) return einval("tg_probe_io_bwd: null pointer");
  auto st = static_cast<hipStream_t>(stream);
  auto X = reinterpret_cast<const uint4*>(x);
  auto DY = reinterpret_cast<const uint4*>(dy);
  auto DX = reinterpret_cast<uint4*>(dx);
  const dim3 g((unsigned)grid), b(256);
  if (depth == 2) hipLaunchKernelGGL(io_bwd_kernel<2>, g, b, 0, st, X, DY, DX, partial, rows);
  else if (depth == 3) hipLaunchKernelGGL(io_bwd_kernel<3>, g, b, 0, st, X, DY, DX, partial, rows);
  else hipLaunchKernelGGL(io_bwd_kernel<4>, g, b, 0, st, X, DY, DX, partial, rows);
  return check_launch("io_bwd");
}

// A different access pattern for the same bytes: no rows at all.  x is a
// stream of 16-byte units (8 bf16); unit i is read once (non-temporal) and
// gives a 16-byte y store, an 8-byte q store and, every 16th unit, one 4-byte
// scale -- config 2's byte mix (2 B read, 2 + 1 + 4/128 B written per element)
// in address order.  Thread t of a grid of G workgroups x 256 threads takes
// units t, t + 256 G, ... with U of them loaded before the first is stored,
// so U x 16 B per lane are in flight; G and U are swept by bench.py.
namespace tg {

template <int U>
__global__ __launch_bounds__(256) void io_stream_kernel(const uint4* __restrict__ x, uint4* __restrict__ y,
                                                        uint2* __restrict__ q, float* __restrict__ s,
                                                        int64_t units) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t base = (int64_t)blockIdx.x * 256 + threadIdx.x; base < units; base += stride * U) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * stride;
      v[u] = i < units ? ldg_stream(x + i) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + u * stride;
      if (i < units) {
        stg_stream(&y[i], v[u]);
        stg_stream(&q[i], make_uint2(v[u].x ^ v[u].z, v[u].y ^ v[u].w));
        if ((i & 15) == 0) s[i >> 4] = __uint_as_float(v[u].x);
      }
    }
  }
}

}  // namespace tg

// units 16-byte units of x (units % 16 == 0), grid workgroups of 256 threads,
// unroll 2, 4 or 8 units in flight per thread.
extern "C" int tg_probe_io_stream(const void* x, void* y, void* q, float* s, int64_t units, int grid,
                                  int unroll, void* stream) {
  using namespace tg;
  if (units <= 0 || units % 16 || grid <= 0 || (unroll != 2 && unroll != 4 && unroll != 8))
    return einval("tg_probe_io_stream: bad arguments");
  if (!x || !y || !q || !s) return einval("tg_probe_io_stream: null pointer");
  auto st = static_cast<hipStream_t>(stream);
  auto X = reinterpret_cast<const uint4*>(x);
  auto Y = reinterpret_cast<uint4*>(y);
  auto Q = reinterpret_cast<uint2*>(q);
  const dim3 g((unsigned)grid), b(256);
  if (unroll == 2) hipLaunchKernelGGL(io_stream_kernel<2>, g, b, 0, st, X, Y, Q, s, units);
  else if (unroll == 4) hipLaunchKernelGGL(io_stream_kernel<4>, g, b, 0, st, X, Y, Q, s, units);
  else hipLaunchKernelGGL(io_stream_kernel<8>, g, b, 0, st, X, Y, Q, s, units);
  return check_launch("io_stream");
}
