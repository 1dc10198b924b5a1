// Pieces shared by the 256 x 256 MFMA GEMM kernels (FP8 and bf16): tile
// order, raw buffer descriptors and the LDS row swizzle.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tg {

typedef float v4f __attribute__((ext_vector_type(4)));

// XCD-aware, grouped tile order.  Consecutive workgroup ids land on
// different XCDs, so ids are remapped to give each XCD a contiguous range of
// tiles; within that range tiles are walked in groups of 8 tile-rows so the
// concurrently running tiles of one XCD share B panels in its L2.
// Returns the (tile_m, tile_n) of workgroup bid.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int ntiles = tiles_m * tiles_n;
  const int xcd = bid & 7, slot = bid >> 3;
  const int q = ntiles >> 3, rem = ntiles & 7;
  const int t = xcd * q + min(xcd, rem) + slot;
  constexpr int GROUP = 8;
  const int per_group = GROUP * tiles_n;
  const int g = t / per_group;
  const int first_m = g * GROUP;
  const int gsize = min(tiles_m - first_m, GROUP);
  const int in_g = t - g * per_group;
  tm = first_m + in_g % gsize;
  tn = in_g / gsize;
}

constexpr int kBufferWord3 = 0x00020000;   // gfx9 raw buffer: 32-bit data format
// Cache-policy operand of the raw buffer loads: nt (streaming, read once).
constexpr int kAuxNT = 2;

// LDS row swizzle of the 256-tile kernels: 16-byte chunk c of row r is stored
// at chunk position c ^ swz(r).  (r >> 1) & 7 spreads the 16 rows one
// fragment read touches over all 64 banks (two rows per 256-byte bank line).
__host__ __device__ constexpr int g256_swz(int r) { return (r >> 1) & 7; }

// Raw buffer descriptor over [p, p + bytes): loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, kBufferWord3);
}

}  // namespace tg
