// Block-scaled FP8 GEMM ("NT": both operands K-contiguous) for gfx950.
//
// Computes what jax.nn.scaled_matmul does at /root/reference/fp8.py:70-78:
//   c[m, n] = bf16( sum_kb sa[m, kb] * sb[n, kb] * sum_{k in kb} qa[m, k] * qb[n, k] )
// with e4m3fn operands and one fp32 scale per 128-wide K block.
//
// Two kernels: gemm_fp8_nt_256_kernel (256 x 256 tiles on 32 x 32 x 64
// MFMAs, persistent; used once a launch has >= 128 tiles, see its own
// comment) and gemm_fp8_nt_kernel below (128 x 128 tiles) for smaller shapes.
//
// Design of the 128 x 128 kernel (gfx950, wave64):
//   * v_mfma_f32_16x16x128_f8f6f4: one MFMA consumes exactly one 128-wide
//     scale block, so its 16x16 fp32 result P is promoted immediately:
//     acc = fma(P, sa[m] * sb[n], acc).  The promotion is VALU work that
//     overlaps the MFMA pipe of the other wave on the SIMD.
//   * Workgroup tile BM x BN x 128 (2 x 2 waves, each TM x TN MFMA tiles),
//     staged through LDS with two buffers: while the waves run the MFMAs of
//     K block kb from one buffer, the next block's bytes and scales travel
//     HBM -> registers and are written to the other buffer; one barrier per
//     K block.  16-byte chunks are XOR-swizzled by row so the fragment reads
//     (16 rows x 32 B per 16 lanes) spread over all LDS banks.
//   * Tile order: consecutive workgroup ids go to different XCDs, so ids are
//     remapped to give each XCD a contiguous range of tiles, and within that
//     range tiles are walked in groups of 8 tile-rows for L2 reuse of B.
#include <mutex>
#include <type_traits>

#include "row_ops.h"
#include "tg_device.h"
#include "tg_host.h"
#include "gemm_tile.h"

namespace tg {

typedef int v8i __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_f8_16x16x128(const v8i& a, const v8i& b, const v4f& c) {
  // Format codes 0/0 = FP8 E4M3 for A and B; zero scale operands select the
  // unscaled v_mfma_f32_16x16x128_f8f6f4.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ v8i as_v8i(const uint4& lo, const uint4& hi) {
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}
__device__ __forceinline__ v8i as_v8i(const u32x4_t& lo, const u32x4_t& hi) {
  v8i r;
  r[0] = (int)lo.x; r[1] = (int)lo.y; r[2] = (int)lo.z; r[3] = (int)lo.w;
  r[4] = (int)hi.x; r[5] = (int)hi.y; r[6] = (int)hi.z; r[7] = (int)hi.w;
  return r;
}


// SKM: scales K-block-major (see gemm_fp8_nt_256_kernel).
template <int TM, int TN, int BNS, bool OUT_F32, bool SKM>
__global__ __launch_bounds__(256, 2) void gemm_fp8_nt_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ SA, const uint8_t* __restrict__ B,
    const float* __restrict__ SB, void* __restrict__ C, int M, int N, int K, int tiles_m,
    int tiles_n) {
  constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
  constexpr int LA = BM / 32, LB = BN / 32;          // 16-byte chunks per thread per K block
  constexpr int STAGE = (BM + BN) * 8;               // uint4 per stage (128 B per row)
  static_assert(BM + BN <= 256, "one scale per thread per K block");
  extern __shared__ uint4 smem[];
  float* sscale = reinterpret_cast<float*>(smem + 2 * STAGE);   // [2][BM + BN]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  int tmi, tni;
  tile_of(blockIdx.x, tiles_m, tiles_n, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int nkb = K >> 7;

  // ---- global -> register staging of one K block ----
  uint4 ra[LA], rb[LB];
  float rs = 0.0f;
  auto gload = [&](int kb) {
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      const int id = tid + 256 * u, row = id >> 3, ch = id & 7;
      const int m = m0 + row;
      ra[u] = m < M ? *reinterpret_cast<const uint4*>(A + (int64_t)m * K + kb * 128 + ch * 16)
                    : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int id = tid + 256 * u, row = id >> 3, ch = id & 7;
      const int n = n0 + row;
      rb[u] = n < N ? *reinterpret_cast<const uint4*>(B + (int64_t)n * K + kb * 128 + ch * 16)
                    : make_uint4(0, 0, 0, 0);
    }
    if (tid < BM) {
      const int m = m0 + tid;
      rs = m < M ? SA[SKM ? (int64_t)kb * M + m : (int64_t)m * nkb + kb] : 0.0f;
    } else if (tid < BM + BN) {
      const int n = n0 + tid - BM;
      const int64_t nsb = BNS == 1 ? N : (N + BNS - 1) / BNS;
      rs = n < N ? SB[SKM ? (int64_t)kb * nsb + n / BNS : (int64_t)(n / BNS) * nkb + kb] : 0.0f;
    }
  };
  auto lstore = [&](int stage) {
    uint4* sa = smem + stage * STAGE;
    uint4* sb = sa + BM * 8;
#pragma unroll
    for (int u = 0; u < LA; ++u) {
      const int id = tid + 256 * u, row = id >> 3, ch = id & 7;
      sa[row * 8 + (ch ^ (row & 7))] = ra[u];
    }
#pragma unroll
    for (int u = 0; u < LB; ++u) {
      const int id = tid + 256 * u, row = id >> 3, ch = id & 7;
      sb[row * 8 + (ch ^ (row & 7))] = rb[u];
    }
    if (tid < BM + BN) sscale[stage * (BM + BN) + tid] = rs;
  };

  v4f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  gload(0);
  lstore(0);
  __syncthreads();

  const int fr = lane & 15, fg = lane >> 4;     // fragment row, 32-byte K group
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) gload(kb + 1);

    const uint4* sa = smem + cur * STAGE;
    const uint4* sb = sa + BM * 8;
    const float* ssa = sscale + cur * (BM + BN);
    const float* ssb = ssa + BM;

    v8i bf[TN];
    float sbv[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int r = wn * TN * 16 + j * 16 + fr;
      bf[j] = as_v8i(sb[r * 8 + ((2 * fg) ^ (r & 7))], sb[r * 8 + ((2 * fg + 1) ^ (r & 7))]);
      sbv[j] = ssb[r];
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = wm * TM * 16 + i * 16 + fr;
      const v8i af = as_v8i(sa[r * 8 + ((2 * fg) ^ (r & 7))], sa[r * 8 + ((2 * fg + 1) ^ (r & 7))]);
      const float4 sav = *reinterpret_cast<const float4*>(ssa + wm * TM * 16 + i * 16 + 4 * fg);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const v4f p = mfma_f8_16x16x128(af, bf[j], zero);
        acc[i][j][0] = __builtin_fmaf(p[0], sav.x * sbv[j], acc[i][j][0]);
        acc[i][j][1] = __builtin_fmaf(p[1], sav.y * sbv[j], acc[i][j][1]);
        acc[i][j][2] = __builtin_fmaf(p[2], sav.z * sbv[j], acc[i][j][2]);
        acc[i][j][3] = __builtin_fmaf(p[3], sav.w * sbv[j], acc[i][j][3]);
      }
    }
    if (kb + 1 < nkb) lstore(cur ^ 1);
    __syncthreads();
  }

  // ---- epilogue: lane holds rows 4*fg + r, column fr of each 16x16 tile ----
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * TN * 16 + j * 16 + fr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * TM * 16 + i * 16 + 4 * fg + r;
        if (m < M && n < N) {
          if (OUT_F32)
            reinterpret_cast<float*>(C)[(int64_t)m * N + n] = acc[i][j][r];
          else
            reinterpret_cast<__bf16*>(C)[(int64_t)m * N + n] = (__bf16)acc[i][j][r];
        }
      }
    }
}

template <int V> using IntC = std::integral_constant<int, V>;

// ---------------------------------------------------------------------------
// Short-K kernel for launches of fewer than 128 tiles of 256 x 256 (C1's
// 2048 x 3072 x 768 and the decode prefill's GEMMs).  With a few K blocks per
// tile (6 at K = 768) the time a block's bytes take to arrive, not the MFMAs,
// is what one block in flight leaves exposed; here NST stages of one K block
// each ring through LDS, so NST - 1 blocks are in flight while one is computed.
//   * Workgroup tile 128 x BN (BN = 32 * TN), 2 x WN waves, wave tile
//     64 x BN / WN on v_mfma_f32_16x16x128_f8f6f4: the same fragments, MFMA
//     operand order and promotion as gemm_fp8_nt_kernel, so the same bits.
//   * Copies: HBM -> LDS with buffer_load ... lds (no VGPR staging).  A stage
//     is 128 + BN rows of 128 B plus the block's scales; the W waves split the
//     A rows and the B rows evenly, 8 rows (1 KiB) per instruction, and the
//     64-float scale copies (padded to a multiple of W with copies that read
//     nothing).  16-byte chunk c of row r sits at c ^ g256_swz(r): the 16 rows
//     one fragment read touches (two per 256-byte bank line) fall on all 64
//     banks.  The swizzle is applied to the global offset a lane fetches.  Rows past M / N and blocks past the last fall outside the
//     buffer range and read as zero; every wave issues the same count per
//     block, so one vmcnt immediate says "block kb has landed".
//   * Step kb (stage kb % NST): wait for this wave's copies of block kb, bare
//     s_barrier (block kb complete; every wave done reading block kb - 1),
//     issue block kb + NST - 1 into block kb - 1's stage, compute block kb.
//     The stages are distinct __shared__ objects and the loop is unrolled by
//     NST, so the compiler tells the copies in flight from the reads.
//   * bf16 output with N % 8 == 0: each wave stages its result in a private
//     LDS region and stores whole 16-byte pieces of rows; otherwise element
//     stores.
// ---------------------------------------------------------------------------
template <int TN, int WN> struct LatCfg {
  static constexpr int TM = 4, BM = 128, BN = 32 * TN, W = 2 * WN;
  static constexpr int TNW = 2 * TN / WN;                     // 16-column tiles per wave
  static constexpr int APW = 16 / W, BPW = 4 * TN / W;        // 1 KiB copies per wave: A, B
  static constexpr int SAC = BM / 64, SBC = (BN + 63) / 64;   // 64-float scale copies of A / B
  static constexpr int SCW = (SAC + SBC + W - 1) / W;         // scale copies per wave (padded)
  static constexpr int SREG = W * SCW * 64;                   // scale floats per stage
  static constexpr int STAGE = (BM + BN) * 128 + SREG * 4;    // bytes per stage
  static constexpr int NST = 163840 / STAGE > 6 ? 6 : 163840 / STAGE;
  static constexpr int IPW = APW + BPW + SCW;                 // copy instructions per wave per block
  static constexpr int RP = 32 * TNW + 16;                    // epilogue row pitch (bytes)
  static constexpr int RPS = (W + NST - 1) / NST;             // epilogue regions per stage
  static_assert(16 % W == 0 && (4 * TN) % W == 0 && (2 * TN) % WN == 0, "even split over the waves");
  static_assert(APW <= 4 && BPW <= 6 && SCW <= 2, "within LatLoad's arrays");
};

typedef __attribute__((address_space(3))) uint8_t lds_u8;
__device__ __forceinline__ u32x4_t lat_ld16(const lds_u8* p) {
  return *(const __attribute__((address_space(3))) u32x4_t*)p;
}
__device__ __forceinline__ float lat_ldf(const lds_u8* p) {
  return *(const __attribute__((address_space(3))) float*)p;
}

// Loader state of one wave: buffer descriptors and per-lane offsets of its
// operand and scale copies.
constexpr int kLatMaxAPW = 4, kLatMaxBPW = 6, kLatMaxSCW = 2;
struct LatLoad {
  __amdgpu_buffer_rsrc_t ra, rb, rsa, rsb;
  uint32_t voa[kLatMaxAPW], vob[kLatMaxBPW], vos[kLatMaxSCW], skb[kLatMaxSCW];
  bool sb[kLatMaxSCW];        // scale copy u reads B scales (else A scales)
  int wave, nkb;
};

// The LDS destination of an LDS-DMA copy, cast explicitly: in a template,
// the implicit generic -> LDS conversion fails the host pass's instantiation,
// and a kernel whose host instantiation fails gets no launch stub (the build
// checks the library for undefined stubs).
#define TG_LAT_LDS(p) ((__attribute__((address_space(3))) void*)(p))

// Block kb into the stage at l.  Blocks past the last read zero, at offset
// 2^31: beyond any buffer here (32-bit sizes), and voa + 2^31 < 2^32.
template <class Cfg>
__device__ __forceinline__ void lat_issue(const LatLoad& c, uint8_t* l, int kb) {
  const bool in = kb < c.nkb;
  const uint32_t k0 = in ? (uint32_t)kb * 128u : 0x80000000u;
#pragma unroll
  for (int p = 0; p < Cfg::APW; ++p)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.ra, TG_LAT_LDS(l + (8 * Cfg::APW * c.wave + 8 * p) * 128), 16, c.voa[p],
                                             k0, 0, 0);
#pragma unroll
  for (int p = 0; p < Cfg::BPW; ++p)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rb, TG_LAT_LDS(l + (Cfg::BM + 8 * Cfg::BPW * c.wave + 8 * p) * 128), 16,
                                             c.vob[p], k0, 0, 0);
#pragma unroll
  for (int u = 0; u < Cfg::SCW; ++u)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.sb[u] ? c.rsb : c.rsa,
                                             TG_LAT_LDS(l + (Cfg::BM + Cfg::BN) * 128 + (c.wave + Cfg::W * u) * 256), 4,
                                             c.vos[u], in ? (uint32_t)kb * c.skb[u] : 0x80000000u, 0, 0);
}

// LDS byte offsets (within a stage) of this lane's fragment chunks and scales
// for m-tile 0 / n-tile 0.
struct LatFrag {
  uint32_t fa0, fa1, fb0, fb1, fsa, fsb;
};

// Step of block kb: wait for this wave's copies of it, barrier, refill the
// stage block kb - 1 used with block kb_refill, compute block kb from cur.
template <class Cfg>
__device__ __forceinline__ void lat_step(const LatLoad& ld, const LatFrag& f,
                                         v4f (&acc)[Cfg::TM][Cfg::TNW], const uint8_t* cur, uint8_t* refill,
                                         int kb_refill) {
  constexpr int TM = Cfg::TM, TNW = Cfg::TNW;
  constexpr int kWait = (Cfg::NST - 2) * Cfg::IPW;
  // s_waitcnt vmcnt(kWait) in the gfx9 encoding (vmcnt low bits 3:0, high
  // bits 15:14; expcnt and lgkmcnt not waited)
  constexpr int kWaitImm = (kWait & 15) | ((kWait >> 4) << 14) | (0x7 << 4) | (0xF << 8);
  __builtin_amdgcn_s_waitcnt(kWaitImm);
  __builtin_amdgcn_s_barrier();
  lat_issue<Cfg>(ld, refill, kb_refill);
  const lds_u8* l = (const lds_u8*)cur;
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  v8i bf[TNW];
  float sbv[TNW];
#pragma unroll
  for (int j = 0; j < TNW; ++j) {
    bf[j] = as_v8i(lat_ld16(l + f.fb0 + j * 2048), lat_ld16(l + f.fb1 + j * 2048));
    sbv[j] = lat_ldf(l + f.fsb + j * 64);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const v8i af = as_v8i(lat_ld16(l + f.fa0 + i * 2048), lat_ld16(l + f.fa1 + i * 2048));
    const u32x4_t sv = lat_ld16(l + f.fsa + i * 64);
    const float4 sav = make_float4(__uint_as_float(sv.x), __uint_as_float(sv.y), __uint_as_float(sv.z),
                                   __uint_as_float(sv.w));
    // the m-tile's MFMAs first, then their promotions: the VALU work of tile
    // j runs while the MFMAs after it are in the matrix pipe
    v4f p[TNW];
#pragma unroll
    for (int j = 0; j < TNW; ++j) p[j] = mfma_f8_16x16x128(af, bf[j], zero);
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
      acc[i][j][0] = __builtin_fmaf(p[j][0], sav.x * sbv[j], acc[i][j][0]);
      acc[i][j][1] = __builtin_fmaf(p[j][1], sav.y * sbv[j], acc[i][j][1]);
      acc[i][j][2] = __builtin_fmaf(p[j][2], sav.z * sbv[j], acc[i][j][2]);
      acc[i][j][3] = __builtin_fmaf(p[j][3], sav.w * sbv[j], acc[i][j][3]);
    }
  }
}

template <int S>
__device__ __forceinline__ uint8_t* lat_pick(uint8_t* s0, uint8_t* s1, uint8_t* s2, uint8_t* s3, uint8_t* s4,
                                             uint8_t* s5) {
  return S == 0 ? s0 : S == 1 ? s1 : S == 2 ? s2 : S == 3 ? s3 : S == 4 ? s4 : s5;
}

// (At one workgroup per CU the compiler would put the MFMA results in AGPRs,
// each element then copied out for the promotion; this file is built with
// -amdgpu-mfma-vgpr-form, which keeps them in VGPRs and changes no other
// kernel here.)
template <int TN, int WN, int BNS, bool OUT_F32, bool SKM>
__global__ __launch_bounds__(128 * WN, 1) void gemm_fp8_lat_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ SA, const uint8_t* __restrict__ B,
    const float* __restrict__ SB, void* __restrict__ C, int M, int N, int K, int tiles_m, int tiles_n,
    int vec_out) {
  using Cfg = LatCfg<TN, WN>;
  constexpr int TM = Cfg::TM, BM = Cfg::BM, BN = Cfg::BN, NST = Cfg::NST, STAGE = Cfg::STAGE;
  constexpr int TNW = Cfg::TNW, W = Cfg::W;
  static_assert(NST >= 3, "at least two blocks in flight");
  static_assert((NST - 2) * Cfg::IPW <= 63, "vmcnt immediate");
  static_assert(Cfg::RPS * 64 * Cfg::RP <= STAGE, "epilogue regions fit the stages");
  __shared__ __attribute__((aligned(16))) uint8_t st0[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st1[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st2[STAGE];
  __shared__ __attribute__((aligned(16))) uint8_t st3[NST > 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(16))) uint8_t st4[NST > 4 ? STAGE : 16];
  __shared__ __attribute__((aligned(16))) uint8_t st5[NST > 5 ? STAGE : 16];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  int tmi, tni;
  tile_of(blockIdx.x, tiles_m, tiles_n, tmi, tni);
  const int m0 = tmi * BM, n0 = tni * BN;
  const int nkb = K >> 7;
  const uint32_t uK = (uint32_t)K;

  // ---- loader state ----
  LatLoad ld;
  ld.wave = wave;
  ld.nkb = nkb;
  ld.ra = make_rsrc(A, (uint32_t)M * uK);
  ld.rb = make_rsrc(B, (uint32_t)N * uK);
  // the lane's slot in copy p holds logical chunk (lane & 7) ^ g256_swz(row),
  // row = 8 * g + lane / 8 for the copy's 8-row group g: g256_swz(row) =
  // 4 * (g & 1) + lane / 16
#pragma unroll
  for (int p = 0; p < Cfg::APW; ++p) {
    const int g = Cfg::APW * wave + p;
    ld.voa[p] = (uint32_t)(m0 + 8 * g + (lane >> 3)) * uK + (uint32_t)((lane & 7) ^ (4 * (g & 1) + (lane >> 4))) * 16u;
  }
#pragma unroll
  for (int p = 0; p < Cfg::BPW; ++p) {
    const int g = Cfg::BPW * wave + p;
    ld.vob[p] = (uint32_t)(n0 + 8 * g + (lane >> 3)) * uK + (uint32_t)((lane & 7) ^ (4 * (g & 1) + (lane >> 4))) * 16u;
  }
  const int nsb = BNS == 1 ? N : (N + BNS - 1) / BNS;
  ld.rsa = make_rsrc(SA, (uint32_t)M * (uint32_t)nkb * 4u);
  ld.rsb = make_rsrc(SB, (uint32_t)nsb * (uint32_t)nkb * 4u);
#pragma unroll
  for (int u = 0; u < Cfg::SCW; ++u) {
    const int c = wave + W * u;                       // scale copy c: floats 64c .. 64c+63 of the region
    if (c < Cfg::SAC) {
      const uint32_t m = (uint32_t)(m0 + 64 * c + lane);
      ld.sb[u] = false;
      ld.vos[u] = SKM ? m * 4u : m * (uint32_t)nkb * 4u;
      ld.skb[u] = SKM ? (uint32_t)M * 4u : 4u;
    } else if (c < Cfg::SAC + Cfg::SBC) {
      const uint32_t sn = (uint32_t)((n0 + 64 * (c - Cfg::SAC) + lane) / BNS);
      ld.sb[u] = true;
      ld.vos[u] = SKM ? sn * 4u : sn * (uint32_t)nkb * 4u;
      ld.skb[u] = SKM ? (uint32_t)nsb * 4u : 4u;
    } else {                                          // padding copy: out of range, reads zero
      ld.sb[u] = false;
      ld.vos[u] = 0x80000000u;
      ld.skb[u] = 0u;
    }
  }

  // ---- compute state: lane (fr, fg) reads logical chunks 2fg, 2fg + 1 ----
  const int fr = lane & 15, fg = lane >> 4;
  const int ra0 = wm * 16 * TM + fr, rb0 = wn * 16 * TNW + fr;      // fragment rows of tile 0
  // (g256_swz(row + 16 i) == g256_swz(row))
  LatFrag f;
  f.fa0 = (uint32_t)ra0 * 128u + (uint32_t)(((2 * fg) ^ g256_swz(ra0)) * 16);
  f.fa1 = (uint32_t)ra0 * 128u + (uint32_t)(((2 * fg + 1) ^ g256_swz(ra0)) * 16);
  f.fb0 = (uint32_t)(BM + rb0) * 128u + (uint32_t)(((2 * fg) ^ g256_swz(rb0)) * 16);
  f.fb1 = (uint32_t)(BM + rb0) * 128u + (uint32_t)(((2 * fg + 1) ^ g256_swz(rb0)) * 16);
  f.fsa = (uint32_t)(BM + BN) * 128u + (uint32_t)(wm * 16 * TM + 4 * fg) * 4u;
  f.fsb = (uint32_t)(BM + BN) * 128u + (uint32_t)(Cfg::SAC * 64 + rb0) * 4u;

  v4f acc[TM][TNW];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

#define TG_LAT_STEP(S, KB)                                                                                 \
  lat_step<Cfg>(ld, f, acc, lat_pick<S>(st0, st1, st2, st3, st4, st5),                                  \
                lat_pick<((S) + NST - 1) % NST>(st0, st1, st2, st3, st4, st5), (KB) + NST - 1)
  lat_issue<Cfg>(ld, st0, 0);
  lat_issue<Cfg>(ld, st1, 1);
  if constexpr (NST > 3) lat_issue<Cfg>(ld, st2, 2);
  if constexpr (NST > 4) lat_issue<Cfg>(ld, st3, 3);
  if constexpr (NST > 5) lat_issue<Cfg>(ld, st4, 4);
  int kb = 0;
  for (; kb + NST <= nkb; kb += NST) {
    TG_LAT_STEP(0, kb);
    TG_LAT_STEP(1, kb + 1);
    TG_LAT_STEP(2, kb + 2);
    if constexpr (NST > 3) TG_LAT_STEP(3, kb + 3);
    if constexpr (NST > 4) TG_LAT_STEP(4, kb + 4);
    if constexpr (NST > 5) TG_LAT_STEP(5, kb + 5);
  }
  if (kb < nkb) {
    TG_LAT_STEP(0, kb);
    if (kb + 1 < nkb) {
      TG_LAT_STEP(1, kb + 1);
      if constexpr (NST > 3) if (kb + 2 < nkb) {
        TG_LAT_STEP(2, kb + 2);
        if constexpr (NST > 4) if (kb + 3 < nkb) {
          TG_LAT_STEP(3, kb + 3);
          if constexpr (NST > 5) if (kb + 4 < nkb) TG_LAT_STEP(4, kb + 4);
        }
      }
    }
  }
#undef TG_LAT_STEP

  // ---- epilogue: lane holds rows 4 * fg + r, column fr of each 16 x 16 tile ----
  const int mw = m0 + wm * 16 * TM, nw = n0 + wn * 16 * TNW;
  if (!OUT_F32 && vec_out) {
    // every copy has landed (the last ones read zero) and every wave is done
    // with the stages before they hold results
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0F00);    // vmcnt(0)
    __builtin_amdgcn_s_barrier();
    const int so = wave % NST;
    uint8_t* wb = (so == 0 ? st0 : so == 1 ? st1 : so == 2 ? st2 : so == 3 ? st3 : so == 4 ? st4 : st5) +
                  (wave / NST) * 64 * Cfg::RP;
    lds_u8* wl = (lds_u8*)wb;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TNW; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          *(__attribute__((address_space(3))) __bf16*)(wl + (16 * i + 4 * fg + r) * Cfg::RP + (16 * j + fr) * 2) =
              (__bf16)acc[i][j][r];
    // a wave reads back only what it wrote; LDS completes a wave's accesses in order
    constexpr int CPR = 2 * TNW;                    // 16-byte pieces per row
#pragma unroll
    for (int u = 0; u < CPR; ++u) {
      const int idx = lane + 64 * u, row = idx / CPR, ch = idx % CPR;
      const u32x4_t v = lat_ld16(wl + row * Cfg::RP + ch * 16);
      const int m = mw + row, n = nw + ch * 8;
      if (m < M && n < N)
        *reinterpret_cast<u32x4_t*>(reinterpret_cast<__bf16*>(C) + (int64_t)m * N + n) = v;
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TNW; ++j) {
      const int n = nw + j * 16 + fr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mw + i * 16 + 4 * fg + r;
        if (m < M && n < N) {
          if (OUT_F32)
            reinterpret_cast<float*>(C)[(int64_t)m * N + n] = acc[i][j][r];
          else
            reinterpret_cast<__bf16*>(C)[(int64_t)m * N + n] = (__bf16)acc[i][j][r];
        }
      }
    }
}

// ---------------------------------------------------------------------------
// Large-tile kernel: workgroup tile 256 x 256 x 128, 8 waves (4 along M x 2
// along N), wave tile 64 x 128.  Operands travel HBM -> LDS with
// buffer_load_dwordx4 ... lds (no VGPR staging): each lane's 16-byte chunk
// lands at LDS offset lane * 16 of its wave's 1 KiB slot, so the XOR swizzle
// is applied to the global offset a lane fetches.  Rows past M / N fall
// outside the buffer's range and read as zero.  Per-lane state is one 32-bit
// offset per operand; the row step and the K-block step ride in SGPR offsets.
// The two stages are distinct __shared__ objects and the K loop is unrolled
// by two, so the compiler's per-object alias scopes tell the prefetch into
// one stage from the fragment reads of the other and it puts no wait
// between them.
// ---------------------------------------------------------------------------
// The compiler lays out LDS objects by size, then by name.  A DS read's
// immediate offset is 16 bits, so reads of an object past 64 KiB cost an
// address add each; the B stages, read twice as often as the A stages, sort
// first (the A stages' names start with z so that they sort last).
__shared__ __attribute__((aligned(16))) uint8_t g256_b0[256 * 128];
__shared__ __attribute__((aligned(16))) uint8_t g256_b1[256 * 128];
__shared__ __attribute__((aligned(16))) uint8_t g256_za0[256 * 128];
__shared__ __attribute__((aligned(16))) uint8_t g256_za1[256 * 128];
__shared__ __attribute__((aligned(16))) float g256_s0[512];
__shared__ __attribute__((aligned(16))) float g256_s1[512];

template <int S> __device__ __forceinline__ uint8_t* g256_a() { return S ? g256_za1 : g256_za0; }
template <int S> __device__ __forceinline__ uint8_t* g256_b() { return S ? g256_b1 : g256_b0; }
template <int S> __device__ __forceinline__ float* g256_s() { return S ? g256_s1 : g256_s0; }

// ---------------------------------------------------------------------------
// 256 x 256 x 128 workgroup tile on v_mfma_f32_32x32x64_f8f6f4.
//
// The block-scale promotion costs two VALU per output and K block (the scale
// product and the fma), which is as many VALU cycles as the matrix pipe
// needs for the block's MFMAs.  A 32 x 32 x 64 MFMA pair covers a 32 x 32
// tile's 128-wide block with half as many MFMA issues as four 16 x 16 x 128
// MFMAs, and measured on gfx950 the MFMA + promotion mix runs ~20% faster on
// it (two waves per SIMD, each overlapping its own MFMAs with the promotion
// of its previous tile).
//
// Layout (8 waves, two per SIMD): wave w owns rows wm * 64 .. +63 (wm = w/2)
// and columns wn * 128 .. +127 (wn = w%2) of the tile: 2 x 4 tiles of
// 32 x 32.  Each tile is computed as B.A^T (B fragment in the MFMA's A slot),
// so lane (c = lane % 32, g = lane / 32) holds output row m = c and the 16
// columns n = 8q + 4g + t (register 4q + t) of the tile: one A-row scale per
// tile and 16 B-column scales.  The column scales are spread over the lane's
// quad: quad lane k keeps the four values n = 8q + 4g + k (q = 0..3) and the
// promotion's multiply reads lane t's value through a quad_perm DPP source,
// so 4 registers per tile hold what 16 would.  The LDS copy of the B scales
// is permuted (within each group of 32 rows, float (4g + k) * 4 + q holds row
// 8q + 4g + k) so that those four values are one 16-byte read.
//
// Steps: tile t = (i, j) = (t % 2, t / 2) for t = 0..7 per K block.  Step t
// issues the MFMA pair of tile t and, between and after the two MFMAs, the
// promotion of the previous tile (the previous K block's tile 7 in step 0),
// so the promotion always runs in the shadow of the wave's own MFMAs.  The
// fragment chunks a lane feeds (16-byte logical chunks 4h + 2g and
// 4h + 2g + 1 of its row for K half h) pair the same K positions in A and B.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ v16f mfma_f8_32x32x64(const v8i& a, const v8i& b, const v16f& c) {
  // format codes 0/0 = FP8 E4M3 for A and B; zero scale operands select the
  // unscaled v_mfma_f32_32x32x64_f8f6f4
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// v broadcast from quad lane T to the four lanes of each quad (folded into
// the consuming VALU op as a DPP source).
template <int T>
__device__ __forceinline__ float quad_bcast(float v) {
  constexpr int ctrl = T | (T << 2) | (T << 4) | (T << 6);
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
}

// acc[4q + t] += p[4q + t] * (sa * sb[n = 8q + 4g + t]) for q = 2h, 2h + 1;
// sbl[q] holds the column scale of n = 8q + 4g + (lane % 4).
__device__ __forceinline__ void w32_promote_half(v16f& acc, const v16f& p, float sa, const float4& sbl,
                                                 int h) {
  const float s0 = h == 0 ? sbl.x : sbl.z, s1 = h == 0 ? sbl.y : sbl.w;
  float t[8] = {quad_bcast<0>(s0) * sa, quad_bcast<1>(s0) * sa, quad_bcast<2>(s0) * sa,
                quad_bcast<3>(s0) * sa, quad_bcast<0>(s1) * sa, quad_bcast<1>(s1) * sa,
                quad_bcast<2>(s1) * sa, quad_bcast<3>(s1) * sa};
  // all eight products first, then the eight fmas: a DPP multiply's result
  // read by the next instruction, or its destination (the value disabled
  // lanes keep) written by the previous one, costs a wait state
  asm volatile("" : "+v"(t[0]), "+v"(t[1]), "+v"(t[2]), "+v"(t[3]));
  asm volatile("" : "+v"(t[4]), "+v"(t[5]), "+v"(t[6]), "+v"(t[7]));
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[8 * h + k] = __builtin_fmaf(p[8 * h + k], t[k], acc[8 * h + k]);
}

struct W32Ctx {
  __amdgpu_buffer_rsrc_t ra, rb, rsa, rsb;
  uint32_t voa[2], vob[2];    // per-lane byte offsets (kb = 0) for even / odd u
  uint32_t vosa, vosb;
  uint32_t skb_a, skb_b;      // bytes from one K block's scales to the next (4, or rows x 4 K-block-major)
  uint32_t row8;              // 8 rows of A / B in bytes (8 * K)
  int wave, nkb;
  // LDS byte addresses of this lane's fragment chunks [K half][chunk] and
  // scales (lds_addr of the object included): B in stage 0 (stage 1 is within
  // the 16-bit DS offset of it); A and the scales per stage [S], since their
  // stage-1 objects lie past 64 KiB and an address add per read would cost
  // VALU issue slots
  uint32_t fa[2][2][2], fb[2][2];
  uint32_t fsa[2];               // A-row scale of m-tile 0
  uint32_t fsb[2];               // B-column scales (this lane's quad share) of n-tile 0
};

// The carried promotion state: the MFMA result of the previous tile and the
// scales it is promoted with.
struct W32Prev {
  v16f p;
  float sa;
  float4 sb;
};

typedef __attribute__((address_space(3))) const uint8_t lds_cu8;

// 32-bit LDS address of a __shared__ object (a link-time constant).
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
  return (uint32_t)(size_t)(lds_cu8*)p;   // C-style cast: generic -> LDS address space
}
// The stage-S copy of stage-0 LDS address a0 inside object objS: the pointer
// derives from objS itself, so the compiler's per-object alias scopes still
// tell these reads apart from the copies landing in the other stage (a read
// based on the stage-0 object would wait for every copy in flight), while
// the address stays one register plus an immediate offset.  w32_at(o, o, a)
// is address a of object o, as a pointer derived from o.
template <typename T>
__device__ __forceinline__ lds_cu8* w32_at(const T* obj0, const T* objS, uint32_t a0) {
  return (lds_cu8*)objS + (a0 - lds_addr(obj0));
}
__device__ __forceinline__ u32x4_t lds_ld16(lds_cu8* p) {
  return *(const __attribute__((address_space(3))) u32x4_t*)p;
}
template <int S>
__device__ __forceinline__ v8i w32_frag_a(const W32Ctx& c, int i, int h) {
  return as_v8i(lds_ld16(w32_at(g256_a<S>(), g256_a<S>(), c.fa[S][h][0]) + i * 4096),
                lds_ld16(w32_at(g256_a<S>(), g256_a<S>(), c.fa[S][h][1]) + i * 4096));
}
template <int S>
__device__ __forceinline__ v8i w32_frag_b(const W32Ctx& c, int j, int h) {
  return as_v8i(lds_ld16(w32_at(g256_b0, g256_b<S>(), c.fb[h][0]) + j * 4096),
                lds_ld16(w32_at(g256_b0, g256_b<S>(), c.fb[h][1]) + j * 4096));
}
template <int S>
__device__ __forceinline__ float4 w32_sb(const W32Ctx& c, int j) {
  const u32x4_t v = lds_ld16(w32_at(g256_s<S>(), g256_s<S>(), c.fsb[S]) + j * 128);
  return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
}
template <int S>
__device__ __forceinline__ float w32_sa(const W32Ctx& c, int i) {
  return __uint_as_float(*(const __attribute__((address_space(3))) uint32_t*)(w32_at(g256_s<S>(), g256_s<S>(), c.fsa[S]) + i * 128));
}

__device__ __forceinline__ void w32_issue_part(const W32Ctx& c, uint8_t* la, uint8_t* lb, float* ls,
                                               int kb, int part) {
  const uint32_t kofs = (uint32_t)kb * 128u;
  const int slot = c.wave + ((part >> 2) & 1) * 4;
  const int u = part & 3;
  const uint32_t sofs = kofs + u * c.row8 + ((part >> 2) & 1) * 16u * c.row8;   // slot w+4: +128 rows
  if (part < 8)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.ra, la + slot * 4096 + u * 1024, 16, c.voa[u & 1],
                                             sofs, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rb, lb + slot * 4096 + u * 1024, 16, c.vob[u & 1],
                                             sofs, 0, 0);
  if (part == 0) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rsa, ls + c.wave * 64, 4, c.vosa, (uint32_t)kb * c.skb_a, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(c.rsb, ls + 256 + c.wave * 64, 4, c.vosb, (uint32_t)kb * c.skb_b, 0, 0);
  }
}

// The fragment and scale registers of one K block.  bf holds the current
// n-tile's two K halves; each half is replaced by the next n-tile's as soon
// as the last MFMA that reads it has issued, so one MFMA pair plus one
// promotion covers every LDS read's latency with 16 registers in use.
struct W32Regs {
  v8i af[2][2];     // A fragments [m-tile][K half]
  v8i bf[2];        // B fragment of the current n-tile [K half]
  float4 sb;        // column scales of the current n-tile (this lane's quad share)
  float sa[2];      // A-row scales [m-tile]
};

// Step T of a K block from stage S: the MFMA pair of tile (i, j) = (T % 2,
// T / 2) and the promotion of prev (the previous tile) into acc_prev.  On
// odd steps the B registers move on to n-tile j + 1 (step 7: to the next K
// block's n-tile 0 and A fragments of m-tile 1, from stage S ^ 1).
template <int S, int T, typename F>
__device__ __forceinline__ void w32_step(const W32Ctx& c, v16f& acc_prev, W32Prev& prev, W32Regs& r,
                                         bool more, F&& copies) {
  constexpr int i = T & 1, j = T >> 1;
  constexpr bool next_n = i == 1 && j < 3;           // B registers move to n-tile j + 1
  constexpr bool next_blk = T == 7;                  // ... to the next block's n-tile 0
  const v16f zero = {};
  // register fence: the promotion of the previous tile stays in this step
  asm volatile("" : "+v"(acc_prev));
  v16f t = mfma_f8_32x32x64(r.bf[0], r.af[i][0], zero);
  // the loader waves' copies go out behind the first MFMA, whose 64 cycles
  // hide the issue stall of the DMA instructions
  copies();
  if (next_n) r.bf[0] = w32_frag_b<S>(c, j + 1, 0);
  if (next_blk && more) r.bf[0] = w32_frag_b<S ^ 1>(c, 0, 0);
  w32_promote_half(acc_prev, prev.p, prev.sa, prev.sb, 0);
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA K half 0
  if (next_n || next_blk) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // its B half's successor
  __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);    // promotion, first half
  const v16f pn = mfma_f8_32x32x64(r.bf[1], r.af[i][1], t);
  const float sa_cur = r.sa[i];
  const float4 sb_cur = r.sb;
  if (next_n) {
    r.bf[1] = w32_frag_b<S>(c, j + 1, 1);
    r.sb = w32_sb<S>(c, j + 1);
  }
  if (next_blk && more) {
    r.bf[1] = w32_frag_b<S ^ 1>(c, 0, 1);
    r.sb = w32_sb<S ^ 1>(c, 0);
    r.af[1][0] = w32_frag_a<S ^ 1>(c, 1, 0);
    r.af[1][1] = w32_frag_a<S ^ 1>(c, 1, 1);
    r.sa[0] = w32_sa<S ^ 1>(c, 0);
    r.sa[1] = w32_sa<S ^ 1>(c, 1);
  }
  w32_promote_half(acc_prev, prev.p, prev.sa, prev.sb, 1);
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // MFMA K half 1
  if (next_n) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
  if (next_blk) __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
  __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);    // promotion, second half
  asm volatile("" : "+v"(acc_prev) : "v"(pn));
  prev.p = pn;
  prev.sa = sa_cur;
  prev.sb = sb_cur;
}

// One K block from stage S.  r holds this block's A fragments, n-tile 0's B
// fragment and column scales and the A-row scales (read by the previous
// block); on return the next block's (when `more`).  The loader waves (0-3)
// issue the copies of K block kb_next of the tile the loader offsets point at
// into stage S ^ 1 during steps 0-6; the barrier before step 7 is where every
// copy has landed and every wave is done reading stage S ^ 1's previous
// block.  m-tile 0's A fragments are dead after step 6's MFMAs and take the
// next block's right after the barrier.
template <int S>
__device__ __forceinline__ void w32_block(const W32Ctx& c, v16f (&acc)[2][4], W32Prev& prev, W32Regs& r,
                                          int kb_next, bool more) {
  const bool pf = more && c.wave < 4;                // loader waves (more: wave-uniform)
  auto issue = [&](int p) {
    w32_issue_part(c, g256_a<S ^ 1>(), g256_b<S ^ 1>(), g256_s<S ^ 1>(), kb_next, p);
  };
  auto dma = [&](int t) {
    if (pf) {
      if (t == 0) {
#pragma unroll
        for (int p = 0; p < 4; ++p) issue(p);
      } else {
        issue(2 * t + 2);
        issue(2 * t + 3);
      }
    }
  };
  w32_step<S, 0>(c, acc[1][3], prev, r, more, [&] { dma(0); });
  w32_step<S, 1>(c, acc[0][0], prev, r, more, [&] { dma(1); });
  w32_step<S, 2>(c, acc[1][0], prev, r, more, [&] { dma(2); });
  w32_step<S, 3>(c, acc[0][1], prev, r, more, [&] { dma(3); });
  w32_step<S, 4>(c, acc[1][1], prev, r, more, [&] { dma(4); });
  w32_step<S, 5>(c, acc[0][2], prev, r, more, [&] { dma(5); });
  w32_step<S, 6>(c, acc[1][2], prev, r, more, [&] { dma(6); });
  // every copy of block kb+1 was issued by step 6: wait for this wave's, then
  // for everybody's (and for every wave to be done with stage S ^ 1)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (more) {
    r.af[0][0] = w32_frag_a<S ^ 1>(c, 0, 0);
    r.af[0][1] = w32_frag_a<S ^ 1>(c, 0, 1);
  }
  w32_step<S, 7>(c, acc[0][3], prev, r, more, [] {});
}

// The 64 x 128 result tile of one wave (rows m0w.., columns n0w..).  bf16
// with N % 8 == 0: through LDS stage S (free once the tile's last K block has
// passed its barrier), 8 KiB per wave, one 32-row m-tile at a time: lane
// (c, g) writes the 8-byte pieces p = 8j + 2q + g of row c at slot p ^ c
// (distinct banks for the 32 rows one write instruction touches), then 16
// lanes per row read the row's 256 bytes back (pieces 2k, 2k + 1 sit in one
// 16-byte slot, swapped when the row is odd) and store them whole.  A wave
// reads back only what it wrote and LDS completes a wave's accesses in
// order, so waiting for its own writes is enough.
template <int S, bool OUT_F32>
__device__ __forceinline__ void w32_store_tile(const v16f (&acc)[2][4], void* __restrict__ C, int M, int N,
                                               int m0w, int n0w, int wave, int lane_in) {
  // an opaque copy of the lane index: the store addresses derive from it, so
  // the compiler cannot hoist them out of the tile loop (where they would
  // stay live across the K loop)
  int lane = lane_in;
  asm volatile("" : "+v"(lane));
  const int cl = lane & 31, g = lane >> 5;
  if (!OUT_F32 && (N % 8) == 0) {
    uint8_t* wbuf = (wave < 4 ? g256_a<S>() : g256_b<S>()) + (wave & 3) * 8192;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int p = 8 * j + 2 * q + g;
          const v16f& v = acc[i][j];
          *reinterpret_cast<uint2*>(wbuf + cl * 256 + (p ^ cl) * 8) =
              make_uint2(pack_bf16x2(v[4 * q], v[4 * q + 1]), pack_bf16x2(v[4 * q + 2], v[4 * q + 3]));
        }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      const int k = lane & 15;
#pragma unroll
      for (int qq = 0; qq < 8; ++qq) {
        const int r = qq * 4 + (lane >> 4);
        uint4 v = *reinterpret_cast<const uint4*>(wbuf + r * 256 + ((2 * k) ^ (r & 30)) * 8);
        if (r & 1) v = make_uint4(v.z, v.w, v.x, v.y);
        const int m = m0w + 32 * i + r;
        const int n = n0w + k * 8;
        if (m < M && n < N)
          *reinterpret_cast<uint4*>(reinterpret_cast<__bf16*>(C) + (int64_t)m * N + n) = v;
      }
    }
    return;
  }
  // f32 output, or N not a multiple of 8: straight from registers; lane
  // (c, g) holds row c and the four consecutive columns 8q + 4g .. +3 of
  // every n-tile
  const bool vec_ok = (N % 4) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int m = m0w + 32 * i + cl;
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int n = n0w + 32 * j + 8 * q + 4 * g;
        const v16f& v = acc[i][j];
        if (OUT_F32) {
          float* dst = reinterpret_cast<float*>(C) + (int64_t)m * N + n;
          if (vec_ok && n + 4 <= N) {
            *reinterpret_cast<float4*>(dst) = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (n + t < N) dst[t] = v[4 * q + t];
          }
        } else {
          __bf16* dst = reinterpret_cast<__bf16*>(C) + (int64_t)m * N + n;
          if (vec_ok && n + 4 <= N) {
            *reinterpret_cast<uint2*>(dst) =
                make_uint2(pack_bf16x2(v[4 * q], v[4 * q + 1]), pack_bf16x2(v[4 * q + 2], v[4 * q + 3]));
          } else {
#pragma unroll
            for (int t = 0; t < 4; ++t)
              if (n + t < N) dst[t] = (__bf16)v[4 * q + t];
          }
        }
      }
  }
}

// Persistent over tiles: workgroup b takes launch
// slots b, b + G, ... (G a multiple of 8, so its slots stay on its XCD) and
// walks the K blocks of all its tiles as one stream; a tile's last K block
// copies the next tile's block 0 into the other stage.
//
// SKM: scales stored K-block-major, SA[kb * M + m] and SB[kb * nsb + n / BNS]
// (the transpose of the reference's (rows, K/128) layout).  A K block's 64
// row scales per loader lane group are then 256 contiguous bytes instead of
// 64 rows K/32 bytes apart, which takes the scale copies from 64 cache lines
// per instruction to two.
template <int BNS, bool OUT_F32, bool SKM>
__global__ __launch_bounds__(512, 1) void gemm_fp8_nt_256_kernel(
    const uint8_t* __restrict__ A, const float* __restrict__ SA, const uint8_t* __restrict__ B,
    const float* __restrict__ SB, void* __restrict__ C, int M, int N, int K, int tiles_m,
    int tiles_n) {
  W32Ctx c;
  const int tid = threadIdx.x, lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform: keeps descriptors in SGPRs
  c.nkb = K >> 7;
  const int wm = c.wave >> 1, wn = c.wave & 1;
  const int ntiles = tiles_m * tiles_n;

  const int nsb = BNS == 1 ? N : (N + 127) / 128;
  c.ra = make_rsrc(A, (uint32_t)M * (uint32_t)K);
  c.rb = make_rsrc(B, (uint32_t)N * (uint32_t)K);
  c.row8 = 8u * (uint32_t)K;
  // loader slot: LDS row wave*32 + u*8 + lane/8, physical chunk lane%8 holds
  // logical chunk (lane%8) ^ swz(row); swz(row) only depends on lane/8 and
  // on the parity of u (wave*32 + u*8 with u even / odd)
  const int lrow = c.wave * 32 + (lane >> 3);
  int slot = blockIdx.x;
  int tm_cur, tn_cur;
  tile_of(slot, tiles_m, tiles_n, tm_cur, tn_cur);
  uint32_t lm0 = (uint32_t)tm_cur * 256u, ln0 = (uint32_t)tn_cur * 256u;   // the loader's tile
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int lch = (lane & 7) ^ g256_swz(lrow + par * 8);
    c.voa[par] = (lm0 + lrow) * (uint32_t)K + lch * 16;
    c.vob[par] = (ln0 + lrow) * (uint32_t)K + lch * 16;
  }
  // scales: LDS float (wave & 3) * 64 + lane of each scale region; the A rows
  // in order, the B rows permuted within groups of 32 (see the layout note)
  const int mu = lane & 31;
  const int sidx_a = (c.wave & 3) * 64 + lane;
  const int sidx_b = (c.wave & 3) * 64 + (lane & 32) + 8 * (mu & 3) + 4 * (mu >> 4) + ((mu >> 2) & 3);
  const uint32_t srow_a = SKM ? 4u : c.nkb * 4u, srow_b = SKM ? 4u : c.nkb * 4u;   // bytes per scale row
  c.skb_a = SKM ? (uint32_t)M * 4u : 4u;
  c.skb_b = SKM ? (uint32_t)nsb * 4u : 4u;
  c.rsa = make_rsrc(SA, (uint32_t)M * c.nkb * 4u);
  c.vosa = (lm0 + sidx_a) * srow_a;
  c.rsb = make_rsrc(SB, (uint32_t)nsb * c.nkb * 4u);
  c.vosb = ((ln0 + sidx_b) / BNS) * srow_b;
  // move the loader to the tile of launch slot `s`: every per-lane offset is
  // (tile origin + lane part) * stride, so the move adds a workgroup-uniform
  // difference (mod 2^32).  Rows past M / N keep landing past the buffer's
  // end and read as zero.  With BNS = 128, (n0 + sidx_b) / 128 = n0 / 128 +
  // sidx_b / 128 (n0 % 256 == 0, sidx_b < 256).
  auto point_loader = [&](int s) {
    int tm, tn;
    tile_of(s, tiles_m, tiles_n, tm, tn);
    const uint32_t m0 = (uint32_t)tm * 256u, n0 = (uint32_t)tn * 256u;
    const uint32_t da = (m0 - lm0) * (uint32_t)K, db = (n0 - ln0) * (uint32_t)K;
#pragma unroll
    for (int par = 0; par < 2; ++par) {
      c.voa[par] += da;
      c.vob[par] += db;
    }
    c.vosa += (m0 - lm0) * srow_a;
    c.vosb += (n0 / BNS - ln0 / BNS) * srow_b;   // divide first: n0 - ln0 may wrap
    lm0 = m0;
    ln0 = n0;
  };
  // fragment chunks: lane (cl, g) feeds logical chunks 4h + 2g and 4h + 2g + 1
  // of row (tile row) + cl for K half h, at physical chunk (logical) ^ swz(row)
  // with swz(row) == swz(cl) (the tile rows are multiples of 32)
  const int cl = lane & 31, g = lane >> 5;
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t pat = (uint32_t)cl * 128u + (uint32_t)(((4 * h + 2 * g + e) ^ g256_swz(cl)) * 16);
      c.fa[0][h][e] = lds_addr(g256_za0) + (uint32_t)(wm * 64) * 128u + pat;
      c.fa[1][h][e] = lds_addr(g256_za1) + (uint32_t)(wm * 64) * 128u + pat;
      c.fb[h][e] = lds_addr(g256_b0) + (uint32_t)(wn * 128) * 128u + pat;
    }
  const uint32_t sa_ofs = (uint32_t)(wm * 64 + cl) * 4u;                                 // A-row scale of row cl
  const uint32_t sb_ofs = (uint32_t)(256 + wn * 128 + (g * 4 + (lane & 3)) * 4) * 4u;       // B-column scales
  c.fsa[0] = lds_addr(g256_s0) + sa_ofs;
  c.fsa[1] = lds_addr(g256_s1) + sa_ofs;
  c.fsb[0] = lds_addr(g256_s0) + sb_ofs;
  c.fsb[1] = lds_addr(g256_s1) + sb_ofs;
  // opaque from here on: the compiler would otherwise cancel the stage-0 base
  // against w32_at's subtraction and re-add the (large) object address per read
  asm volatile("" : "+v"(c.fa[0][0][0]), "+v"(c.fa[0][0][1]), "+v"(c.fa[0][1][0]), "+v"(c.fa[0][1][1]));
  asm volatile("" : "+v"(c.fa[1][0][0]), "+v"(c.fa[1][0][1]), "+v"(c.fa[1][1][0]), "+v"(c.fa[1][1][1]));
  asm volatile("" : "+v"(c.fb[0][0]), "+v"(c.fb[0][1]), "+v"(c.fb[1][0]), "+v"(c.fb[1][1]));
  asm volatile("" : "+v"(c.fsa[0]), "+v"(c.fsb[0]), "+v"(c.fsa[1]), "+v"(c.fsb[1]));

  v16f acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};

  // this workgroup's tiles, and the K blocks of all of them as one stream
  const int my_tiles = (ntiles - slot + (int)gridDim.x - 1) / (int)gridDim.x;
  const int nsteps = my_tiles * c.nkb;

  if (c.wave < 4) {
#pragma unroll
    for (int p = 0; p < 16; ++p) w32_issue_part(c, g256_za0, g256_b0, g256_s0, 0, p);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  W32Regs r;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int h = 0; h < 2; ++h) r.af[i][h] = w32_frag_a<0>(c, i, h);
  r.bf[0] = w32_frag_b<0>(c, 0, 0);
  r.bf[1] = w32_frag_b<0>(c, 0, 1);
  r.sb = w32_sb<0>(c, 0);
  r.sa[0] = w32_sa<0>(c, 0);
  r.sa[1] = w32_sa<0>(c, 1);
  // nothing to promote before the first tile: a zero product with zero
  // scales into acc[1][3], which stays zero
  W32Prev prev;
  prev.p = v16f{};
  prev.sa = 0.0f;
  prev.sb = make_float4(0.f, 0.f, 0.f, 0.f);

  int kb = 0, step = 0;
  auto one_step = [&](auto stage) {
    constexpr int S = decltype(stage)::value;
    const bool last = kb + 1 == c.nkb;
    const bool more = step + 1 < nsteps;
    if (last && more) point_loader(slot + (int)gridDim.x);
    w32_block<S>(c, acc, prev, r, last ? 0 : kb + 1, more);
    ++step;
    if (!last) {
      ++kb;
      return;
    }
    // the tile's last step promoted tile 6; tile 7's promotion has no MFMA of
    // this tile left to hide behind
    w32_promote_half(acc[1][3], prev.p, prev.sa, prev.sb, 0);
    w32_promote_half(acc[1][3], prev.p, prev.sa, prev.sb, 1);
    prev.p = v16f{};
    prev.sa = 0.0f;
    prev.sb = make_float4(0.f, 0.f, 0.f, 0.f);
    w32_store_tile<S, OUT_F32>(acc, C, M, N, tm_cur * 256 + wm * 64, tn_cur * 256 + wn * 128, c.wave,
                               lane);
    if (more) {
      // every wave is done with stage S before the next block's copies land there
      __syncthreads();
      slot += gridDim.x;
      tile_of(slot, tiles_m, tiles_n, tm_cur, tn_cur);
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v16f{};
    }
    kb = 0;
  };
  while (step + 1 < nsteps) {
    one_step(IntC<0>{});
    one_step(IntC<1>{});
  }
  if (step < nsteps) one_step(IntC<0>{});
}

template <int BNS, bool OUT_F32, bool SKM>
static int launch_gemm_256(const uint8_t* a_q, const float* a_s, const uint8_t* b_q,
                           const float* b_s, void* c, int M, int N, int K, hipStream_t st) {
  const int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
  // one workgroup per CU (135 KiB of LDS each), looping over its tiles; the
  // grid stays a multiple of 8 so that a workgroup's slots share its XCD
  const int ntiles = tiles_m * tiles_n;
  const int slots = device_cus() & ~7;
  const int grid = ntiles <= slots || slots == 0 ? ntiles : slots;
  hipLaunchKernelGGL((gemm_fp8_nt_256_kernel<BNS, OUT_F32, SKM>), dim3((unsigned)grid), dim3(512), 0, st,
                     a_q, a_s, b_q, b_s, c, M, N, K, tiles_m, tiles_n);
  return check_launch("gemm_fp8_nt_256");
}

template <int TM, int TN, int BNS, bool OUT_F32, bool SKM>
static int launch_gemm_cfg(const uint8_t* a_q, const float* a_s, const uint8_t* b_q,
                           const float* b_s, void* c, int M, int N, int K, hipStream_t st) {
  constexpr int BM = 2 * TM * 16, BN = 2 * TN * 16;
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const size_t lds = (size_t)2 * (BM + BN) * 128 + (size_t)2 * (BM + BN) * 4;
  auto kern = gemm_fp8_nt_kernel<TM, TN, BNS, OUT_F32, SKM>;
  // the dynamic-LDS limit is a per-device function attribute: set once per
  // device (thread-safe, see device_cus)
  constexpr int kMaxDev = 64;
  static std::once_flag once[kMaxDev];
  static hipError_t attr_rc[kMaxDev];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) dev = 0;
  std::call_once(once[dev], [&] {
    attr_rc[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  });
  if (attr_rc[dev] != hipSuccess) {
    set_error("gemm_fp8 (set LDS size): %s", hipGetErrorString(attr_rc[dev]));
    return TG_EHIP;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)(tiles_m * tiles_n)), dim3(256), lds, st, a_q, a_s, b_q,
                     b_s, c, M, N, K, tiles_m, tiles_n);
  return check_launch("gemm_fp8_nt");
}

#ifndef TG_LAT_WN
#define TG_LAT_WN 4
#endif
template <int TN, bool SKM>
static int launch_gemm_lat(const uint8_t* a_q, const float* a_s, const uint8_t* b_q, const float* b_s,
                           int b_scale_bn, void* c, bool f32, int M, int N, int K, hipStream_t st) {
  constexpr int BM = 128, BN = 32 * TN, WN = TG_LAT_WN;
  if constexpr ((2 * TN) % WN != 0) {
    return einval("gemm_fp8_lat: tile width not split over the waves");
  } else {
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int vec = !f32 && N % 8 == 0 && aligned(c, 16);
  const dim3 grid((unsigned)(tiles_m * tiles_n));
#define TG_LAT(BNS, F32)                                                                                    \
  hipLaunchKernelGGL((gemm_fp8_lat_kernel<TN, WN, BNS, F32, SKM>), grid, dim3(128 * WN), 0, st, a_q, a_s, b_q, \
                     b_s, c, M, N, K, tiles_m, tiles_n, vec)
  if (b_scale_bn == 1) {
    if (f32) TG_LAT(1, true); else TG_LAT(1, false);
  } else {
    if (f32) TG_LAT(128, true); else TG_LAT(128, false);
  }
#undef TG_LAT
  return check_launch("gemm_fp8_lat");
  }
}

// Build-time choice of the short-K kernel (0: the VGPR-staged 128-row kernel
// for every launch below 128 tiles of 256).
#ifndef TG_GEMM_LAT
#define TG_GEMM_LAT 1
#endif
static bool lat_kernel_enabled() { return TG_GEMM_LAT != 0; }

// The short-K kernel's tile width: 192, 128, 96 or 64 columns, whichever
// leaves the busiest CU the least work, counted as workgroups per CU (one
// fits a CU) times (columns + 48), the 48 standing for a tile's fixed cost
// (pipeline fill, epilogue).  C1's 2048 x 3072: 256 tiles of 192, one per CU.
static int lat_tile_n(int m, int n) {
  const int64_t cus = device_cus() > 0 ? device_cus() : 1;
  int best = 6;
  int64_t best_cost = -1;
  for (int tn : {6, 4, 3, 2}) {
    if ((2 * tn) % TG_LAT_WN) continue;               // the wave split needs whole 16-column tiles
    const int64_t tiles = (int64_t)((m + 127) / 128) * ((n + 32 * tn - 1) / (32 * tn));
    const int64_t cost = (tiles + cus - 1) / cus * (32 * tn + 48);
    if (best_cost < 0 || cost < best_cost) {
      best = tn;
      best_cost = cost;
    }
  }
  return best;
}

template <bool SKM>
static int launch_gemm_fp8_layout(const uint8_t* a_q, const float* a_s, const uint8_t* b_q,
                                  const float* b_s, int b_scale_bn, void* c, bool f32, int m, int n,
                                  int k, bool big, bool lat, hipStream_t st) {
  if (lat) {
    switch (lat_tile_n(m, n)) {
      case 6: return launch_gemm_lat<6, SKM>(a_q, a_s, b_q, b_s, b_scale_bn, c, f32, m, n, k, st);
      case 4: return launch_gemm_lat<4, SKM>(a_q, a_s, b_q, b_s, b_scale_bn, c, f32, m, n, k, st);
      case 3: return launch_gemm_lat<3, SKM>(a_q, a_s, b_q, b_s, b_scale_bn, c, f32, m, n, k, st);
      default: return launch_gemm_lat<2, SKM>(a_q, a_s, b_q, b_s, b_scale_bn, c, f32, m, n, k, st);
    }
  }
  if (big) {
    if (b_scale_bn == 1)
      return f32 ? launch_gemm_256<1, true, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st)
                 : launch_gemm_256<1, false, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st);
    return f32 ? launch_gemm_256<128, true, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st)
               : launch_gemm_256<128, false, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st);
  }
  // 128 x 128 or 128 x 96 tiles, whichever leaves the busiest CU the fewer
  // outputs (tiles per CU, rounded up, times the tile's columns): C1's 2048 x
  // 3072 is 384 tiles of 128 (two on half the CUs) or 512 of 96 (two on
  // every CU), 10% faster
  const int64_t cus = device_cus() > 0 ? device_cus() : 1;
  const int64_t tm = (m + 127) / 128;
  const int64_t load128 = (tm * ((n + 127) / 128) + cus - 1) / cus * 128;
  const int64_t load96 = (tm * ((n + 95) / 96) + cus - 1) / cus * 96;
  if (load96 < load128) {
    if (b_scale_bn == 1)
      return f32 ? launch_gemm_cfg<4, 3, 1, true, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st)
                 : launch_gemm_cfg<4, 3, 1, false, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st);
    return f32 ? launch_gemm_cfg<4, 3, 128, true, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st)
               : launch_gemm_cfg<4, 3, 128, false, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st);
  }
  if (b_scale_bn == 1)
    return f32 ? launch_gemm_cfg<4, 4, 1, true, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st)
               : launch_gemm_cfg<4, 4, 1, false, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st);
  return f32 ? launch_gemm_cfg<4, 4, 128, true, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st)
             : launch_gemm_cfg<4, 4, 128, false, SKM>(a_q, a_s, b_q, b_s, c, m, n, k, st);
}

int launch_gemm_fp8(const uint8_t* a_q, const float* a_s, const uint8_t* b_q, const float* b_s,
                    int b_scale_bn, void* c, int c_dtype, int64_t M, int64_t N, int64_t K,
                    hipStream_t st, bool skm) {
  if (M == 0 || N == 0) return TG_OK;
  const int m = (int)M, n = (int)N, k = (int)K;
  const bool f32 = c_dtype == TG_DTYPE_F32;
  // 256 x 256 tiles once they fill the chip (>= 128 workgroups), else 128 x 128
  const bool fits32 = (uint64_t)M * (uint64_t)K < (1ull << 31) && (uint64_t)N * (uint64_t)K < (1ull << 31);
  const bool big = fits32 && ((M + 255) / 256) * ((N + 255) / 256) >= 128;
  // below that, the short-K ring kernel (32-bit buffer offsets, as the 256 kernel)
  const bool lat = fits32 && !big && lat_kernel_enabled();
  return skm ? launch_gemm_fp8_layout<true>(a_q, a_s, b_q, b_s, b_scale_bn, c, f32, m, n, k, big, lat, st)
             : launch_gemm_fp8_layout<false>(a_q, a_s, b_q, b_s, b_scale_bn, c, f32, m, n, k, big, lat, st);
}

// ---------------------------------------------------------------------------
// Decode-shape GEMM (M <= 16 * MT) on a pre-quantized weight; HBM-bound on W.
//
// Every workgroup owns R <= 64 consecutive weight rows (chosen on the host so
// that each CU streams the same number of W bytes: 56 rows of the 14336-row C5
// weight on 256 CUs).  K is walked in chunks of 32 blocks (4 KiB of a row);
// within a chunk the rows are walked in stages of 8, and wave w loads row w of
// a stage as four contiguous 1 KiB pieces.  Reading the workgroup's rows in
// address order keeps each DRAM page to one visit: stages of 1 KiB from every
// row (K-major) measured ~30% slower on the C5 weight.  Stages travel through
// registers into LDS (row pitch 4112 B, so the 8 rows of a fragment read
// spread over the banks) together with their W scales; three stages are in
// flight, so the loads of stage G + 3 start as soon as stage G has landed,
// whatever the compute of stage G costs.  Wave w computes blocks 4w .. 4w+3 of each stage: the MFMA takes the 8 rows
// as its A operand (rows 8..15 repeat them and are discarded) and 16 x rows as
// B; x fragments of the chunk stay in registers.  Every load is issued
// unconditionally (masked lanes read zero through the buffer range check), so
// the compiler counts the loads of each stage exactly.  The partial sums of
// the 8 waves are added in wave order through LDS (deterministic).
constexpr int kGemvPitch = 4112;                 // LDS bytes per W row of a stage
constexpr int kGemvGroups = 8;                   // stages of 8 rows per chunk, at most
constexpr int kGemvStage = 8 * kGemvPitch + 8 * 64 * 4;   // W rows + scales (64 per row)
__shared__ __attribute__((aligned(16))) uint8_t gemv_lds0[kGemvStage];
__shared__ __attribute__((aligned(16))) uint8_t gemv_lds1[kGemvStage];
__shared__ __attribute__((aligned(16))) uint8_t gemv_lds2[kGemvStage];
template <int S> __device__ __forceinline__ uint8_t* gemv_stage() {
  return S == 0 ? gemv_lds0 : S == 1 ? gemv_lds1 : gemv_lds2;
}


// Where a GEMV's activation rows come from (the GEMVs below): PRO_X already
// quantized x_q / x_s; PRO_NORM / PRO_NORM_ADD rmsnorm of x (after the
// residual add x + delta) -> FP8 rows, computed by the GEMV's workgroup;
// PRO_RELU2 bf16(relu(u)^2) -> FP8 rows.
// PRO_XCOPY: x_q / x_s already quantized, at most 8 rows, copied into LDS by
// the workgroup with whole-row loads before the K loop (the fragment loads
// from x_q would each touch 16 rows' 64-byte pieces; see gemv_fp8_kernel).
enum { PRO_X = 0, PRO_NORM = 1, PRO_NORM_ADD = 2, PRO_RELU2 = 3, PRO_XCOPY = 4 };

// The norm prologue's inputs (PRO_NORM*): x, delta (M, K) bf16, gamma (K,)
// bf16; with PRO_NORM_ADD workgroup 0 stores the residual sum bf16(x + delta)
// to xout (M, K).
struct GemvNormIn {
  const uint4* x;
  const uint4* delta;
  const uint4* gamma;
  uint4* xout;
  float eps;
};

// NS: stages in flight (three per workgroup, one workgroup per CU; or two, and
// two workgroups per CU).  Workgroup b takes the balanced share of the 8-row
// groups: groups [b G / grid, (b + 1) G / grid), at most kGemvGroups.
//
// PRO_NORM*: before the K loop each workgroup computes the FP8 rows of
// rms_norm(x [+ delta]) itself -- wave w takes rows w and w + 8, one row per
// wave as in the norm kernel and with its routine (norm_row: the same bytes
// and scales as tg_rms_norm_fp8 / tg_add_rms_norm_fp8) -- into dynamic LDS
// (row pitch K + 16 bytes, so the 16 rows of a fragment read fall on distinct
// banks), and the x fragments are read from there instead of from HBM.  One
// launch replaces the norm kernel + the GEMV of a decode step for 3..16 rows;
// every workgroup repeats the rows' arithmetic (M x K elements, against its
// W rows' 56 x K bytes of HBM traffic).  J: 16-byte chunks per lane of a row.
template <int MT, int BNS, int NS, int PRO = PRO_X, int J = 1>
__global__ __launch_bounds__(512) void gemv_fp8_kernel(const uint8_t* __restrict__ XQ,
                                                       const float* __restrict__ XS,
                                                       const uint8_t* __restrict__ WQ,
                                                       const float* __restrict__ WS,
                                                       __bf16* __restrict__ out, int M, int N,
                                                       int K, GemvNormIn nin) {
  constexpr int NW = 8;
  constexpr bool XLDS = PRO == PRO_NORM || PRO == PRO_NORM_ADD || PRO == PRO_XCOPY;
  static_assert(PRO == PRO_X || (XLDS && MT == 1), "the norm prologue takes at most 16 rows");
  // rows of x held in LDS: 16 for the norm prologue, 8 for the copy
  constexpr int XROWS = PRO == PRO_XCOPY ? 8 : 16;
  // 17..32 rows from x_q: x loaded as whole K-block rows and permuted into
  // fragments in the wave (half the cache lines per load; at 9..16 rows, one
  // x tile per K block, it measured no faster)
  constexpr bool XROW8 = PRO == PRO_X && MT == 2;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int nkb = K >> 7;
  const int nchunk = (nkb + 31) >> 5;
  const int64_t gtot = (N + 7) >> 3;
  const int g_lo = (int)(((int64_t)blockIdx.x * gtot) / gridDim.x);
  const int g_hi = (int)(((int64_t)(blockIdx.x + 1) * gtot) / gridDim.x);
  const int n0 = 8 * g_lo;
  const int rows = min(8 * g_hi, N) - n0;
  const int ngroups = g_hi - g_lo;

  const uint32_t wbytes = (uint32_t)rows * (uint32_t)K;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(WQ + (int64_t)n0 * K, wbytes);
  const int srows = BNS == 1 ? N : (N + BNS - 1) / BNS;
  const uint32_t sbytes = (uint32_t)srows * (uint32_t)nkb * 4u;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(WS, sbytes);
  const uint32_t xbytes = (uint32_t)M * (uint32_t)K;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(XQ, xbytes);
  const uint32_t xsbytes = (uint32_t)M * (uint32_t)nkb * 4u;
  const __amdgpu_buffer_rsrc_t rxs = make_rsrc(XS, xsbytes);

  u32x4_t wr[NS][4];              // this wave's row of the NS stages in flight (4 x 1 KiB)
  float wsr[NS];                  // its 32 scales (lanes 0..31; lanes 32..63 read zero)
  u32x4_t xr[4][MT][2];           // x fragments of blocks 4w .. 4w+3 of the chunk
  float sxr[4][MT];
  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  // acc[P]: the pair of 8-row groups 2P (MFMA rows 0..7, lanes fg < 2) and
  // 2P + 1 (rows 8..15, lanes fg >= 2)
  v4f acc[kGemvGroups / 2][MT];
#pragma unroll
  for (int g = 0; g < kGemvGroups / 2; ++g)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[g][mt] = zero;

  // row 8g + w of chunk c (and its 32 scales) into register slot SL
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
    const uint32_t soff = (rv && lane < 32 && b < nkb) ? ((uint32_t)srow * (uint32_t)nkb + (uint32_t)b) * 4u
                                                       : sbytes;
    wsr[SL] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, soff, 0, 0));
  };

  // XROW8: the x rows of a chunk -> MFMA fragments, within the wave (the
  // loads below take whole 128-byte K-block rows, 8 rows per load): lane
  // (fr, fg) takes chunks fg and 4 + fg of row fr, held by lane (fr % 8) * 8 +
  // chunk of the load of rows 0..7 (fr < 8) or of rows 8..15.  Run once the
  // chunk's first stages' loads are issued, so their round trip covers it.
  auto x_fragments = [&]() {
    const int s0 = ((fr & 7) * 8 + fg) * 4, s1 = s0 + 16;
    const bool lo = fr < 8;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4_t a = xr[i][mt][0], b = xr[i][mt][1];
        u32x4_t x0, x1;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const uint32_t a0 = (uint32_t)__builtin_amdgcn_ds_bpermute(s0, (int)a[d]);
          const uint32_t b0 = (uint32_t)__builtin_amdgcn_ds_bpermute(s0, (int)b[d]);
          const uint32_t a1 = (uint32_t)__builtin_amdgcn_ds_bpermute(s1, (int)a[d]);
          const uint32_t b1 = (uint32_t)__builtin_amdgcn_ds_bpermute(s1, (int)b[d]);
          x0[d] = lo ? a0 : b0;
          x1[d] = lo ? a1 : b1;
        }
        xr[i][mt][0] = x0;
        xr[i][mt][1] = x1;
      }
  };

  // stage (c, G): registers -> LDS buffer SL = G % NS, start the loads of stage
  // G + NS into the same registers, barrier; then, on odd G, blocks 4w .. 4w+3
  // of the 16 rows of stages G - 1 (MFMA rows 0..7) and G (rows 8..15), both
  // still in LDS (stage G - 1's buffer is rewritten only after the next
  // barrier); on the last stage when it is even, its 8 rows alone (rows 8..15
  // repeat them and are never stored).  One MFMA per pair of stages instead of
  // one per stage with half its rows repeated.
  auto stage = [&](auto slot, auto grp, int c) {
    constexpr int SL = decltype(slot)::value;
    constexpr int G = decltype(grp)::value;
    uint8_t* buf = gemv_stage<SL>();
    float* ssw = reinterpret_cast<float*>(buf + 8 * kGemvPitch);
#pragma unroll
    for (int p = 0; p < 4; ++p)
      *reinterpret_cast<u32x4_t*>(buf + wave * kGemvPitch + p * 1024 + lane * 16) = wr[SL][p];
    ssw[wave * 64 + lane] = wsr[SL];      // every lane stores: no load sunk into a branch
    load_w(slot, c, G + NS);
    __syncthreads();
    if (G % 2 == 0 && ngroups != G + 1) return;     // paired with stage G + 1
    constexpr int SLP = (G + NS - 1) % NS;           // stage G - 1's buffer (odd G)
    uint8_t* bprev = gemv_stage<SLP>();
    const uint8_t* ba = G % 2 == 1 && fr < 8 ? bprev : buf;      // this lane's A-fragment row
    const float* bs = reinterpret_cast<const float*>((G % 2 == 1 && fg < 2 ? bprev : buf) + 8 * kGemvPitch);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kb = c * 32 + 4 * wave + i;
      if (kb < nkb) {
        const uint8_t* pa = ba + (fr & 7) * kGemvPitch + (4 * wave + i) * 128 + fg * 16;
        const v8i wa = as_v8i(*reinterpret_cast<const uint4*>(pa),
                              *reinterpret_cast<const uint4*>(pa + 64));
        float sw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) sw[r] = bs[((4 * fg + r) & 7) * 64 + 4 * wave + i];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const v4f pr = mfma_f8_16x16x128(wa, as_v8i(xr[i][mt][0], xr[i][mt][1]), zero);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[G / 2][mt][r] = __builtin_fmaf(pr[r], sw[r] * sxr[i][mt], acc[G / 2][mt][r]);
        }
      }
    }
  };

  // PRO_NORM*: the FP8 rows of the norm in LDS (x bytes at pitch K + 16 for
  // 16 rows, then their scales), from the norm row routine; rows >= M are
  // never read (their fragments are zero).  The rows' loads go out first, then
  // the first chunk's weight stages, so the norm's arithmetic runs while the
  // weight stream is already in flight.
  extern __shared__ __attribute__((aligned(16))) uint8_t gemv_xl[];
  const int xpitch = K + 16;
  float* gemv_xs = reinterpret_cast<float*>(gemv_xl + XROWS * xpitch);
  if constexpr (PRO == PRO_XCOPY) {
    // x rows (M <= 8) into LDS at pitch K + 16: 16-byte loads, consecutive
    // threads on consecutive bytes of a row (whole lines), then the scales;
    // the loads go out before the first chunk's weight stages, whose loads
    // then overlap this copy's round trip
    const int nch = K >> 4;                        // 16-byte chunks per row
    const int tot = M * nch;
    constexpr int XU = 8;                          // chunks per thread in flight (8 rows x 4 KiB / 512 threads)
    u32x4_t xv[XU];
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int e = tid + u * 512;
      const uint32_t off = e < tot ? (uint32_t)(e / nch) * (uint32_t)K + (uint32_t)(e % nch) * 16u : xbytes;
      xv[u] = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
    }
    const int nsc = M * nkb;
    const float sv = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(rxs, tid < nsc ? (uint32_t)tid * 4u : xsbytes, 0, 0));
    load_w(IntC<0>{}, 0, 0);
    load_w(IntC<1>{}, 0, 1);
    if constexpr (NS > 2) load_w(IntC<2 % NS>{}, 0, 2);
#pragma unroll
    for (int u = 0; u < XU; ++u) {
      const int e = tid + u * 512;
      if (e < tot) *reinterpret_cast<u32x4_t*>(gemv_xl + (e / nch) * xpitch + (e % nch) * 16) = xv[u];
    }
    // rows beyond K / 16 * XU chunks per thread: a tail loop (K > 4096)
    for (int e = tid + XU * 512; e < tot; e += 512)
      *reinterpret_cast<u32x4_t*>(gemv_xl + (e / nch) * xpitch + (e % nch) * 16) =
          __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(e / nch) * (uint32_t)K + (uint32_t)(e % nch) * 16u, 0, 0);
    if (tid < nsc) gemv_xs[tid] = sv;
    for (int e = tid + 512; e < nsc; e += 512)
      gemv_xs[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxs, (uint32_t)e * 4u, 0, 0));
    __syncthreads();
  }
  if constexpr (PRO == PRO_NORM || PRO == PRO_NORM_ADD) {
    constexpr bool ADD = PRO == PRO_NORM_ADD;
    const int nch = K >> 3;
    // both of a wave's rows are loaded ahead for J <= 5; with J = 8 the
    // second row's loads wait for the first row's registers (no spills)
    constexpr int RR = J <= 5 ? 2 : 1;
    uint4 xv[RR][J], dv[RR][J], gq[J];
    auto load_row = [&](int rr, int slot) {
      const int m = wave + NW * rr;
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = lane + 64 * j;
        const bool ok = m < M && c < nch;
        xv[slot][j] = ok ? nin.x[(int64_t)m * nch + c] : make_uint4(0, 0, 0, 0);
        dv[slot][j] = ADD && ok ? nin.delta[(int64_t)m * nch + c] : make_uint4(0, 0, 0, 0);
      }
    };
#pragma unroll
    for (int rr = 0; rr < RR; ++rr) load_row(rr, rr);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      gq[j] = c < nch ? nin.gamma[c] : make_uint4(0, 0, 0, 0);
    }
    load_w(IntC<0>{}, 0, 0);
    load_w(IntC<1>{}, 0, 1);
    if constexpr (NS > 2) load_w(IntC<2 % NS>{}, 0, 2);
    float g[J][8];
#pragma unroll
    for (int j = 0; j < J; ++j) unpack8(gq[j], g[j]);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int m = wave + NW * rr;
      const int slot = RR == 2 ? rr : 0;
      if (RR == 1 && rr == 1) load_row(1, 0);
      if (m < M) {                                 // wave-uniform: the DPP reductions see every lane
        uint4 yo[J];
        uint2 qo[J];
        float so[J];
        norm_row<J, true, false, ADD>(xv[slot], dv[slot], g, lane, nch, (float)K, nin.eps, yo, qo, so);
#pragma unroll
        for (int j = 0; j < J; ++j) {
          const int c = lane + 64 * j;
          if (c < nch) {
            *reinterpret_cast<uint2*>(gemv_xl + m * xpitch + c * 8) = qo[j];
            if ((c & 15) == 0) gemv_xs[m * nkb + (c >> 4)] = so[j];
            if (ADD && blockIdx.x == 0) nin.xout[(int64_t)m * nch + c] = xv[slot][j];
          }
        }
      }
    }
    __syncthreads();
  }

  for (int c = 0; c < nchunk; ++c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int kb = c * 32 + 4 * wave + i;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + fr;
        const bool ok = m < M && kb < nkb;
        if constexpr (XLDS) {
          const uint8_t* px = gemv_xl + m * xpitch + kb * 128 + fg * 16;
          const u32x4_t z = {0u, 0u, 0u, 0u};
          xr[i][mt][0] = ok ? *reinterpret_cast<const u32x4_t*>(px) : z;
          xr[i][mt][1] = ok ? *reinterpret_cast<const u32x4_t*>(px + 64) : z;
          sxr[i][mt] = ok ? gemv_xs[m * nkb + kb] : 0.0f;
        } else {
          if constexpr (XROW8) {
            // whole 128-byte K-block rows, 8 rows per load (one cache line
            // each, against 16 rows' 64-byte halves for a fragment-shaped
            // load): lane (r8, c8) takes 16-byte chunk c8 of rows mt*16 + r8
            // and mt*16 + 8 + r8; x_fragments moves them into the fragment
            // layout
            const int r8 = lane >> 3, c8 = lane & 7;
            const int m1 = mt * 16 + r8, m2 = m1 + 8;
            const uint32_t kofs = (uint32_t)kb * 128u + c8 * 16u;
            xr[i][mt][0] = __builtin_amdgcn_raw_buffer_load_b128(
                rx, m1 < M && kb < nkb ? (uint32_t)m1 * (uint32_t)K + kofs : xbytes, 0, 0);
            xr[i][mt][1] = __builtin_amdgcn_raw_buffer_load_b128(
                rx, m2 < M && kb < nkb ? (uint32_t)m2 * (uint32_t)K + kofs : xbytes, 0, 0);
          } else {
            const uint32_t xo = ok ? (uint32_t)m * (uint32_t)K + (uint32_t)kb * 128u + fg * 16u : xbytes;
            xr[i][mt][0] = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
            xr[i][mt][1] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? xo + 64u : xbytes, 0, 0);
          }
          const uint32_t so = ok ? ((uint32_t)m * (uint32_t)nkb + (uint32_t)kb) * 4u : xsbytes;
          sxr[i][mt] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxs, so, 0, 0));
        }
      }
    }
    if (!XLDS || c > 0) {                  // XLDS: chunk 0's stages went out before the norm
      load_w(IntC<0>{}, c, 0);
      load_w(IntC<1>{}, c, 1);
      if constexpr (NS > 2) load_w(IntC<2 % NS>{}, c, 2);
    }
    if constexpr (XROW8) x_fragments();
    // every path to stage G runs stages 0 .. G-1 first (early exits only), so
    // the compiler's count of the loads in flight at stage G is exact
    do {
      stage(IntC<0 % NS>{}, IntC<0>{}, c);
      if (ngroups <= 1) break;
      stage(IntC<1 % NS>{}, IntC<1>{}, c);
      if (ngroups <= 2) break;
      stage(IntC<2 % NS>{}, IntC<2>{}, c);
      if (ngroups <= 3) break;
      stage(IntC<3 % NS>{}, IntC<3>{}, c);
      if (ngroups <= 4) break;
      stage(IntC<4 % NS>{}, IntC<4>{}, c);
      if (ngroups <= 5) break;
      stage(IntC<5 % NS>{}, IntC<5>{}, c);
      if (ngroups <= 6) break;
      stage(IntC<6 % NS>{}, IntC<6>{}, c);
      if (ngroups <= 7) break;
      stage(IntC<7 % NS>{}, IntC<7>{}, c);
    } while (false);
    __syncthreads();                      // the next chunk rewrites the stage buffers
  }

  // wave-ordered sum of the partial tiles through LDS (stage memory reused):
  // lane (fr, fg) of pair tile P holds rows 8(2P + fg / 2) + 4(fg % 2) .. +3,
  // so each wave stores its 4 pair tiles of every x-row tile (32 KiB per tile
  // for the workgroup, tile mt in stage buffer mt), and after one barrier wave
  // g adds group g's partials of the 8 waves in wave order
  static_assert(MT <= 2 && NW * (kGemvGroups / 2) * 64 * sizeof(v4f) <= kGemvStage, "partials fit a stage buffer");
  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    v4f* red = reinterpret_cast<v4f*>(mt == 0 ? gemv_lds0 : gemv_lds1);   // [NW][4][64]
#pragma unroll
    for (int pp = 0; pp < kGemvGroups / 2; ++pp) red[(wave * (kGemvGroups / 2) + pp) * 64 + lane] = acc[pp][mt];
  }
  __syncthreads();
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const v4f* red = reinterpret_cast<const v4f*>(mt == 0 ? gemv_lds0 : gemv_lds1);
    const int g = wave;
    const int m = mt * 16 + fr, lr = 8 * g + 4 * fg;
    const int src = (g & 1) * 32 + lane;  // the lane of pair tile g / 2 holding these rows
    if (fg < 2 && g < ngroups && m < M && lr < rows) {
      v4f s = red[(g >> 1) * 64 + src];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) {
        const v4f o = red[(w2 * (kGemvGroups / 2) + (g >> 1)) * 64 + src];
        s[0] += o[0]; s[1] += o[1]; s[2] += o[2]; s[3] += o[3];
      }
      __bf16* o = out + (int64_t)m * N + n0 + lr;
      if (vec && lr + 3 < rows) {
        *reinterpret_cast<uint2*>(o) = make_uint2(pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3]));
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (lr + r < rows) o[r] = (__bf16)s[r];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Decode GEMV, direct form (M <= 16 MT rows): the weight's MFMA fragments go
// from HBM straight into registers.
//   * A row block is 16 weight rows, the MFMA's A operand.  Workgroup b takes
//     row blocks b, b + grid, ...; its 8 waves split K: wave w takes the
//     contiguous K blocks [w kpw, (w + 1) kpw).  Lane (r, g) loads row r's
//     16-byte pieces g and 4 + g of each of its K blocks (each load
//     instruction reads 64 contiguous bytes of 16 rows), all of a row block
//     at once: one memory round trip per row block, and the next row block's
//     loads go out before this one's reduction.
//   * The x rows (bytes and scales) sit in LDS at pitch K + 16 (the 16 rows of
//     a fragment read fall on distinct banks): copied from x_q / x_s (PRO_X,
//     their loads issued before the weight's) or computed by the norm
//     prologue (PRO_NORM*, M <= 8: wave w normalises row w with the norm
//     kernel's row routine; the rows' loads, then the weight's, then the
//     norm's arithmetic).
//   * acc = fma(P, w_s * x_s, acc) per K block; the 8 waves' partial tiles are
//     added in wave order through LDS, so the result is deterministic and the
//     same for every prologue.
// Against the staged kernel above (4 KiB-contiguous reads through LDS, K walked
// in 4 KiB chunks) this has no staging and no serial chunk walk: on the
// reference decode weights (5-21 MB) the staged kernel's fixed cost and its
// chunk walk over the 9 KiB w_down rows dominated.
// KPW: K blocks per wave (at least ceil(K / 1024)); XC: 16-byte x chunks per
// thread of the PRO_X copy; J: 16-byte chunks per lane of a norm row.
// ---------------------------------------------------------------------------
template <int MT, int BNS, int KPW, int PRO, int XC, int J>
__global__ __launch_bounds__(512) void gemv_direct_kernel(const uint8_t* __restrict__ XQ,
                                                          const float* __restrict__ XS,
                                                          const uint8_t* __restrict__ WQ,
                                                          const float* __restrict__ WS,
                                                          __bf16* __restrict__ out, int M, int N, int K,
                                                          GemvNormIn nin) {
  constexpr int NW = 8;
  constexpr bool XNORM = PRO == PRO_NORM || PRO == PRO_NORM_ADD;
  static_assert(PRO == PRO_X || (XNORM && MT == 1), "the norm prologue takes at most 8 rows");
  extern __shared__ __attribute__((aligned(16))) uint8_t gdx[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fg = lane >> 4;
  const int nkb = K >> 7;
  const int xpitch = K + 16;
  float* xsl = reinterpret_cast<float*>(gdx + M * xpitch);                            // (M, nkb)
  v4f* red = reinterpret_cast<v4f*>(gdx + ((M * xpitch + M * nkb * 4 + 15) & ~15));   // [NW][MT][64]
  const int nrb = (N + 15) >> 4;
  const int kpw = (nkb + NW - 1) / NW;        // <= KPW (host)
  const int kb0 = wave * kpw;

  // ---- x rows: loads first (PRO_X into registers; PRO_NORM* the norm rows) ----
  u32x4_t xc[PRO == PRO_X ? XC : 1];
  float xsc[2] = {0.0f, 0.0f};
  const int xchunks = M * (K >> 4);
  uint4 nxv[XNORM ? J : 1], ndv[XNORM ? J : 1], ngq[XNORM ? J : 1];
  const int nch = K >> 3;
  if constexpr (PRO == PRO_X) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(XQ, (uint32_t)M * (uint32_t)K);
    const __amdgpu_buffer_rsrc_t rxs = make_rsrc(XS, (uint32_t)M * (uint32_t)nkb * 4u);
#pragma unroll
    for (int j = 0; j < XC; ++j)           // chunk tid + 512 j of the (M, K) bytes; past them: zero
      xc[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(tid + 512 * j) * 16u, 0, 0);
    // M * nkb <= 1024 (the host keeps M * K <= 131072): two scales per thread, no drain before the barrier
#pragma unroll
    for (int j = 0; j < 2; ++j)
      xsc[j] = __builtin_bit_cast(float,
                                  __builtin_amdgcn_raw_buffer_load_b32(rxs, (uint32_t)(tid + 512 * j) * 4u, 0, 0));
  } else {
    constexpr bool ADD = PRO == PRO_NORM_ADD;
    const int m = wave;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      const bool ok = m < M && c < nch;
      nxv[j] = ok ? nin.x[(int64_t)m * nch + c] : make_uint4(0, 0, 0, 0);
      ndv[j] = ADD && ok ? nin.delta[(int64_t)m * nch + c] : make_uint4(0, 0, 0, 0);
      ngq[j] = c < nch ? nin.gamma[c] : make_uint4(0, 0, 0, 0);
    }
  }

  // ---- the first row block's weight fragments and scales ----
  const uint32_t wbytes = (uint32_t)N * (uint32_t)K;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(WQ, wbytes);
  const int srows = BNS == 1 ? N : (N + BNS - 1) / BNS;
  const uint32_t sbytes = (uint32_t)srows * (uint32_t)nkb * 4u;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(WS, sbytes);
  constexpr int NSC = BNS == 1 ? 4 : 1;      // W scales per lane and K block
  struct Frag {
    u32x4_t w[KPW][2];
    float s[KPW][NSC];
  };
  auto load_rb = [&](Frag& F, int rb) {
    const int row = rb * 16 + fr;
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kb = kb0 + i;
      const bool kok = i < kpw && kb < nkb;
      const bool ok = kok && row < N;
      const uint32_t off = ok ? (uint32_t)row * (uint32_t)K + (uint32_t)kb * 128u + fg * 16u : wbytes;
      // cached loads: the two 64-byte halves of a weight line come from two instructions, and the
      // second one hits in L2 (non-temporal, each half was fetched on its own: 10-13% slower)
      F.w[i][0] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
      F.w[i][1] = __builtin_amdgcn_raw_buffer_load_b128(rw, ok ? off + 64u : wbytes, 0, 0);
#pragma unroll
      for (int r = 0; r < NSC; ++r) {
        const int srow = BNS == 1 ? rb * 16 + 4 * fg + r : (rb * 16) / BNS;
        const bool sok = kok && srow < srows;
        const uint32_t so = sok ? ((uint32_t)srow * (uint32_t)nkb + (uint32_t)kb) * 4u : sbytes;
        F.s[i][r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, so, 0, 0));
      }
    }
  };
  // one register set, refilled with the next row block's fragments before each
  // reduction (a second set, to keep two row blocks in flight, measured slower:
  // the registers cost a workgroup per CU)
  Frag FA;
  const int G = (int)gridDim.x;
  load_rb(FA, blockIdx.x);                    // the host launches at most nrb workgroups

  // ---- x rows into LDS ----
  if constexpr (PRO == PRO_X) {
    const int kc = K >> 4;                    // 16-byte chunks per row
#pragma unroll
    for (int j = 0; j < XC; ++j) {
      const int c = tid + 512 * j;
      if (c < xchunks) {
        const int m = c / kc, k16 = c - m * kc;
        *reinterpret_cast<u32x4_t*>(gdx + m * xpitch + k16 * 16) = xc[j];
      }
    }
    if (tid < M * nkb) xsl[tid] = xsc[0];
    if (tid + 512 < M * nkb) xsl[tid + 512] = xsc[1];
  } else {
    constexpr bool ADD = PRO == PRO_NORM_ADD;
    const int m = wave;
    if (m < M) {                              // wave-uniform: the DPP reductions see every lane
      float g[J][8];
#pragma unroll
      for (int j = 0; j < J; ++j) unpack8(ngq[j], g[j]);
      uint4 yo[J];
      uint2 qo[J];
      float so[J];
      norm_row<J, true, false, ADD>(nxv, ndv, g, lane, nch, (float)K, nin.eps, yo, qo, so);
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = lane + 64 * j;
        if (c < nch) {
          *reinterpret_cast<uint2*>(gdx + m * xpitch + c * 8) = qo[j];
          if ((c & 15) == 0) xsl[m * nkb + (c >> 4)] = so[j];
          if (ADD && blockIdx.x == 0) nin.xout[(int64_t)m * nch + c] = nxv[j];
        }
      }
    }
  }
  __syncthreads();

  const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 7) == 0;
  // one row block from register set F: MFMAs, then (refill) the 8 waves'
  // partial tiles added in wave order through LDS and stored
  auto process = [&](Frag& F, int rb, int refill_rb) {
    v4f acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < KPW; ++i) {
      const int kb = kb0 + i;
      if (i < kpw && kb < nkb) {              // wave-uniform
        const v8i a = as_v8i(F.w[i][0], F.w[i][1]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = mt * 16 + fr;
          const bool mok = m < M;
          const int mc = mok ? m : M - 1;     // rows past M read row M - 1 and are zeroed
          const uint8_t* px = gdx + mc * xpitch + kb * 128 + fg * 16;
          u32x4_t b0 = *reinterpret_cast<const u32x4_t*>(px);
          u32x4_t b1 = *reinterpret_cast<const u32x4_t*>(px + 64);
          const u32x4_t z = {0u, 0u, 0u, 0u};
          b0 = mok ? b0 : z;
          b1 = mok ? b1 : z;
          const float sx = mok ? xsl[mc * nkb + kb] : 0.0f;
          const v4f pr = mfma_f8_16x16x128(a, as_v8i(b0, b1), v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[mt][r] = __builtin_fmaf(pr[r], F.s[i][BNS == 1 ? r : 0] * sx, acc[mt][r]);
        }
      }
    }
    if (refill_rb < nrb) load_rb(F, refill_rb);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[(wave * MT + mt) * 64 + lane] = acc[mt];
    __syncthreads();
    if (wave < MT) {
      const int mt = wave;
      v4f sm = red[mt * 64 + lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) {
        const v4f o = red[(w2 * MT + mt) * 64 + lane];
        sm[0] += o[0]; sm[1] += o[1]; sm[2] += o[2]; sm[3] += o[3];
      }
      const int m = mt * 16 + fr, n = rb * 16 + 4 * fg;
      if (m < M && n < N) {
        __bf16* o = out + (int64_t)m * N + n;
        if (vec) {
          *reinterpret_cast<uint2*>(o) = make_uint2(pack_bf16x2(sm[0], sm[1]), pack_bf16x2(sm[2], sm[3]));
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) o[r] = (__bf16)sm[r];
        }
      }
    }
    __syncthreads();                          // red is rewritten by the next row block
  };
  for (int rb = blockIdx.x; rb < nrb; rb += G) process(FA, rb, rb + G);
}

// ---------------------------------------------------------------------------
// GEMV for one or two activation rows on the VALU (no MFMA, no LDS staging of
// W).  With M <= 2 the MFMA kernel above spends its time moving each weight
// row through LDS so that 8 rows can feed one 16-row MFMA fragment; here each
// wave streams whole weight rows and takes the dot products itself.
//   * A unit is NQ KiB of one weight row: NQ 1 KiB loads (16 bytes per lane)
//     and the NQ W scales of those lanes; NQ = 3 when the row is a multiple of
//     3 KiB or shorter (the decode widths 2304 and 9216: 2.25 of 4 KiB-unit
//     pieces, or a last unit of 1 KiB, would be loaded and computed for
//     nothing), else 4.  A wave owns rows gw, gw + nw, ... (nw = waves in the
//     grid), walked unit by unit with two units in flight.
//   * Per 16-byte piece: 16 e4m3 x 16 e4m3 products (v_cvt_pk_f32_fp8, f32
//     fma chain) into the block partial, scaled by w_s * x_s of its 128-wide
//     block; at a row's end a 64-lane butterfly, and the row's sum is parked
//     in lane (row index & 63) until 64 rows (or the wave's last row) are
//     stored together.
//   * x bytes and scales sit in LDS.  The prologue that fills them is one of:
//       PRO_X      copy of already-quantized x_q / x_s
//       PRO_NORM   rmsnorm of x (optionally after the residual add x + delta,
//                  which workgroup 0 also stores) -> FP8 rows, by the same
//                  row routine as the norm kernel (same bits)
//       PRO_RELU2  bf16(relu(u)^2) -> FP8 rows, as quant_rows_kernel<RELU2>
//     Its loads are issued first, then the first unit's weight loads, so the
//     prologue's arithmetic overlaps the first HBM round trip.
//   * Every load is a buffer load at an offset inside its matrix (lanes past
//     a row re-read the row's first piece and are masked out of the sum); the
//     loop runs whole pairs of units with no exit inside it, so the compiler's
//     wait counts stay exact.
// The block sums are f32 fma chains, not the MFMA's arithmetic, so outputs
// agree with tg_gemv_fp8 / tg_gemm_fp8_nt to rounding, not bit for bit.
// ---------------------------------------------------------------------------
typedef float v2f __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot16_e4m3(const u32x4_t& w, const uint4& x) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w}, xx[4] = {x.x, x.y, x.z, x.w};
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const v2f w0 = __builtin_amdgcn_cvt_pk_f32_fp8(ww[e], false);
    const v2f w1 = __builtin_amdgcn_cvt_pk_f32_fp8(ww[e], true);
    const v2f x0 = __builtin_amdgcn_cvt_pk_f32_fp8(xx[e], false);
    const v2f x1 = __builtin_amdgcn_cvt_pk_f32_fp8(xx[e], true);
    s = __builtin_fmaf(w0.x, x0.x, s);
    s = __builtin_fmaf(w0.y, x0.y, s);
    s = __builtin_fmaf(w1.x, x1.x, s);
    s = __builtin_fmaf(w1.y, x1.y, s);
  }
  return s;
}

constexpr int kRowdotMaxK = 16384;   // x of two rows (32 KiB) + scales in LDS
constexpr int kRowdotProWaves = 8;  // waves per workgroup of the norm / relu^2 prologue variants
constexpr int kRowdotNormMaxK = 4096;

struct RowdotIn {
  const uint8_t* xq;      // PRO_X: (M, K) e4m3 bytes
  const float* xs;        // PRO_X: (M, K/128) scales
  const uint4* x;         // PRO_NORM*: (M, K) bf16 rows; PRO_RELU2: u (M, K) bf16
  const uint4* delta;     // PRO_NORM_ADD: (M, K) bf16
  const uint4* gamma;     // PRO_NORM*: (K,) bf16
  uint4* xout;            // PRO_NORM_ADD: (M, K) bf16 residual sum (workgroup 0 stores it)
  const __bf16* resid;    // RES: (M, N) bf16 residual; out = bf16(resid + bf16(dot))
  float eps;
};

struct RowdotUnit {
  u32x4_t w[4];
  float s[4];
};

// unit (row, g): 1 KiB pieces 4g .. 4g+3 of weight row `row`
template <int NQ>
__device__ __forceinline__ void rowdot_load(RowdotUnit& U, const __amdgpu_buffer_rsrc_t& rw,
                                            const __amdgpu_buffer_rsrc_t& rs, int row, int g, int K,
                                            int nkb, int bns, int lane) {
  const uint32_t rbase = (uint32_t)row * (uint32_t)K;
  const uint32_t sbase = (uint32_t)(bns == 1 ? row : row >> 7) * (uint32_t)nkb;
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const uint32_t k = (uint32_t)(g * NQ + q) * 1024u + lane * 16u;
    const bool ok = k < (uint32_t)K;
    U.w[q] = __builtin_amdgcn_raw_buffer_load_b128(rw, rbase + (ok ? k : 0u), 0, kAuxNT);
    U.s[q] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           rs, (sbase + (ok ? (k >> 7) : 0u)) * 4u, 0, 0));
  }
}

template <int NX, int NQ>
__device__ __forceinline__ void rowdot_compute(const RowdotUnit& U, const uint8_t* xl, const float* sxs,
                                               int g, int K, int nkb, int lane, float (&acc)[NX]) {
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const uint32_t k = (uint32_t)(g * NQ + q) * 1024u + lane * 16u;
    const bool ok = k < (uint32_t)K;
    const uint32_t kk = ok ? k : 0u;
#pragma unroll
    for (int m = 0; m < NX; ++m) {
      const uint4 xv = *reinterpret_cast<const uint4*>(xl + m * K + kk);
      const float t = __builtin_fmaf(dot16_e4m3(U.w[q], xv), U.s[q] * sxs[m * nkb + (kk >> 7)], acc[m]);
      acc[m] = ok ? t : acc[m];
    }
  }
}

// XL: 4 KiB pieces of x staged by PRO_X (NX * K <= 4096 * XL), or 16-byte
// chunks of u per thread for PRO_RELU2 (NX * K <= 8 * 64 * WPG * XL); J:
// chunks per lane of the norm row (K <= 512 * J); WPG: waves per workgroup
// (4 for PRO_X; 8 for the computing prologues, whose bf16 row loads every
// workgroup repeats: 8 waves measured best of 4, 8 and 16 at the decode
// shapes).
template <int NX, int PRO, int XL, int J, int WPG, bool RES, int NQ>
__global__ __launch_bounds__(64 * WPG) void gemv_rowdot_kernel(RowdotIn in, const uint8_t* __restrict__ WQ,
                                                          const float* __restrict__ WS, int bns,
                                                          __bf16* __restrict__ out, int N, int K,
                                                          int sx_off) {
  static_assert(PRO != PRO_X || WPG == 4, "the x copy is laid out for 256 threads");
  constexpr int NT = 64 * WPG;
  extern __shared__ __attribute__((aligned(16))) uint8_t rowdot_lds[];   // x bytes, then x scales
  uint8_t* xl = rowdot_lds;
  float* sxs = reinterpret_cast<float*>(rowdot_lds + sx_off);
  // the wave index through readfirstlane: the row loop is uniform control flow to the compiler
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = K >> 7, nch = K >> 3;
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(WQ, (uint32_t)N * (uint32_t)K);
  const int srows = bns == 1 ? N : (N + 127) >> 7;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(WS, (uint32_t)srows * (uint32_t)nkb * 4u);
  const int nw = gridDim.x * WPG, gw = blockIdx.x * WPG + wave;
  const int G = (K + NQ * 1024 - 1) / (NQ * 1024);     // units per row
  const int nrows = gw < N ? (N - 1 - gw) / nw + 1 : 0;
  const int nu = nrows * G;

  // ---- prologue loads ----
  u32x4_t xr[PRO == PRO_X ? XL : 1];
  float xsr = 0.f;
  uint4 nx[J], nd[J];
  constexpr int CI = PRO == PRO_NORM || PRO == PRO_NORM_ADD ? (NX * J * 64 + NT - 1) / NT : 1;   // chunks per thread
  uint4 ng[CI];
  uint4 rv[PRO == PRO_RELU2 ? XL : 1];
  if (PRO == PRO_X) {
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(in.xq, (uint32_t)(NX * K));
    const __amdgpu_buffer_rsrc_t rxs = make_rsrc(in.xs, (uint32_t)(NX * nkb) * 4u);
#pragma unroll
    for (int j = 0; j < XL; ++j)   // past NX * K: out of range, reads zero
      xr[j] = __builtin_amdgcn_raw_buffer_load_b128(rx, (uint32_t)(j * 4096 + tid * 16), 0, 0);
    xsr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rxs, (uint32_t)tid * 4u, 0, 0));
  } else if (PRO == PRO_NORM || PRO == PRO_NORM_ADD) {
    // unconditional buffer loads: chunks past the row and the rows of waves
    // >= NX fall outside the buffers and read zero
    const uint32_t rbytes = (uint32_t)(NX * K) * 2u;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(in.x, rbytes);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(PRO == PRO_NORM_ADD ? (const void*)in.delta : (const void*)in.x, rbytes);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(in.gamma, (uint32_t)K * 2u);
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = lane + 64 * j;
      const uint32_t xo = c < nch ? (uint32_t)(wave * nch + c) * 16u : rbytes;
      const u32x4_t vx = __builtin_amdgcn_raw_buffer_load_b128(rx, xo, 0, 0);
      nx[j] = make_uint4(vx.x, vx.y, vx.z, vx.w);
      if (PRO == PRO_NORM_ADD) {
        const u32x4_t vd = __builtin_amdgcn_raw_buffer_load_b128(rd, xo, 0, 0);
        nd[j] = make_uint4(vd.x, vd.y, vd.z, vd.w);
      } else {
        nd[j] = make_uint4(0, 0, 0, 0);
      }
    }
    // gamma for this thread's chunks of the second phase (chunk c of the
    // flattened (NX, K) rows uses gamma chunk c mod nch)
#pragma unroll
    for (int i = 0; i < CI; ++i) {
      const int c = tid + NT * i;
      const uint32_t go = c < NX * nch ? (uint32_t)(c % nch) * 16u : (uint32_t)K * 2u;
      const u32x4_t vg = __builtin_amdgcn_raw_buffer_load_b128(rg, go, 0, 0);
      ng[i] = make_uint4(vg.x, vg.y, vg.z, vg.w);
    }
  } else {
    const __amdgpu_buffer_rsrc_t ru = make_rsrc(in.x, (uint32_t)(NX * K) * 2u);
#pragma unroll
    for (int r = 0; r < XL; ++r) {   // past NX * K: out of range, reads zero
      const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(ru, (uint32_t)(tid + NT * r) * 16u, 0, 0);
      rv[r] = make_uint4(v.x, v.y, v.z, v.w);
    }
  }

  // ---- first unit's weight loads, after the prologue's (loads complete in
  // order, so the prologue's arithmetic can start before these arrive) ----
  __builtin_amdgcn_sched_barrier(0);
  RowdotUnit A, B;
  rowdot_load<NQ>(A, rw, rs, gw < N ? gw : N - 1, 0, K, nkb, bns, lane);
  __builtin_amdgcn_sched_barrier(0);

  // ---- prologue arithmetic -> LDS ----
  if (PRO == PRO_X) {
    // unconditional writes: a skipped write would leave its load outstanding
    // to the compiler, which then waits for every load at the loop header
#pragma unroll
    for (int j = 0; j < XL; ++j) *reinterpret_cast<u32x4_t*>(xl + j * 4096 + tid * 16) = xr[j];
    sxs[tid] = xsr;
  } else if (PRO == PRO_NORM || PRO == PRO_NORM_ADD) {
    // phase 1: wave m < NX takes row m's statistics (the norm kernel's own
    // routine and lane layout, so the same f64 sum) and parks the residual
    // sums (bf16) and r in LDS; phase 2: all threads norm and quantize
    // 8-element chunks, 16 consecutive chunks (one scale block) per DPP row
    uint4* sums = reinterpret_cast<uint4*>(rowdot_lds + ((sx_off + NX * nkb * 4 + 15) & ~15));
    float* rbs = reinterpret_cast<float*>(sums + NX * nch);
    if (wave < NX) {
      const float rb = norm_row_rb<J, PRO == PRO_NORM_ADD>(nx, nd, (float)K, in.eps);
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int c = lane + 64 * j;
        if (c < nch) {
          sums[wave * nch + c] = nx[j];
          if (PRO == PRO_NORM_ADD && blockIdx.x == 0) in.xout[wave * nch + c] = nx[j];
        }
      }
      if (lane == 0) rbs[wave] = rb;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CI; ++i) {
      const int c = tid + NT * i;
      const bool valid = c < NX * nch;
      const int m = valid ? c / nch : 0;
      const uint4 xc = valid ? sums[c] : make_uint4(0, 0, 0, 0);
      float g[8];
      unpack8(ng[i], g);
      uint4 y;
      uint2 q;
      float sc;
      norm_chunk<true>(xc, g, rbs[m], valid, y, q, sc);
      if (valid) {
        *reinterpret_cast<uint2*>(xl + c * 8) = q;
        if ((lane & 15) == 0) sxs[c >> 4] = sc;
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < XL; ++r) {
      const int c = tid + NT * r;   // chunk of the flattened (NX, K) rows; 16 chunks = one block
      float v[8];
      unpack8(rv[r], v);
      relu2_bf16(v);
      const float sc = block_scale_bf16(row16_max_u32(absmax8(v)));   // uniform: DPP
      if (c < NX * nch) {
        *reinterpret_cast<uint2*>(xl + c * 8) = quant8<true>(v, sc);
        if ((lane & 15) == 0) sxs[c >> 4] = sc;
      }
    }
  }
  __syncthreads();
  if (nu == 0) return;

  float acc[NX], res[NX];
#pragma unroll
  for (int m = 0; m < NX; ++m) acc[m] = res[m] = 0.f;
  auto finish = [&](int jr) {            // row jr of this wave is complete
#pragma unroll
    for (int m = 0; m < NX; ++m) {
      float v = acc[m];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
      res[m] = lane == (jr & 63) ? v : res[m];
      acc[m] = 0.f;
    }
    if ((jr & 63) == 63 || jr == nrows - 1) {   // store rows (jr & ~63) .. jr
      const int r = gw + ((jr & ~63) + lane) * nw;
      if (lane <= (jr & 63)) {
#pragma unroll
        for (int m = 0; m < NX; ++m) {
          const int64_t o = (int64_t)m * N + r;
          if constexpr (RES) {   // the bf16 tensor add: f32 sum of the two bf16 values, rounded once
            const float sum = (float)in.resid[o] + (float)(__bf16)res[m];
            out[o] = __builtin_bit_cast(__bf16, (uint16_t)(pack_bf16x2(sum, 0.0f) & 0xFFFFu));
          } else {
            out[o] = (__bf16)res[m];
          }
        }
      }
    }
  };
  auto next = [&](int& r, int& g, int& j) {
    if (++g == G) {
      g = 0;
      r += nw;
      ++j;
    }
  };
  int row = gw, g = 0, j = 0;   // unit = (row j of this wave, 4 KiB group g)
  const int pairs = (nu - 1) >> 1;
  for (int it = 0; it < pairs; ++it) {
    int row1 = row, g1 = g, j1 = j;
    next(row1, g1, j1);
    rowdot_load<NQ>(B, rw, rs, row1, g1, K, nkb, bns, lane);
    rowdot_compute<NX, NQ>(A, xl, sxs, g, K, nkb, lane, acc);
    if (g == G - 1) finish(j);
    int row2 = row1, g2 = g1, j2 = j1;
    next(row2, g2, j2);
    rowdot_load<NQ>(A, rw, rs, row2, g2, K, nkb, bns, lane);
    rowdot_compute<NX, NQ>(B, xl, sxs, g1, K, nkb, lane, acc);
    if (g1 == G - 1) finish(j1);
    row = row2;
    g = g2;
    j = j2;
  }
  if ((nu & 1) == 0) {
    int row1 = row, g1 = g, j1 = j;
    next(row1, g1, j1);
    rowdot_load<NQ>(B, rw, rs, row1, g1, K, nkb, bns, lane);
    rowdot_compute<NX, NQ>(A, xl, sxs, g, K, nkb, lane, acc);
    if (g == G - 1) finish(j);
    rowdot_compute<NX, NQ>(B, xl, sxs, g1, K, nkb, lane, acc);
    finish(j1);
  } else {
    rowdot_compute<NX, NQ>(A, xl, sxs, g, K, nkb, lane, acc);
    finish(j);
  }
}

}  // namespace tg

using namespace tg;

// any_block: the entry has the general path for block_k != 128 (block_generic.hip)
int tg::check_gemm_args(const char* who, int64_t M, int64_t N, int64_t K, int block_k, int bns,
                        bool any_block) {
  if (any_block ? block_k <= 0 : block_k != 128)
    return einval(any_block ? "block_k must be positive" : "block_k must be 128");
  if (M < 0 || N < 0 || K <= 0) return einval("bad GEMM shape");
  if (K % block_k) return einval("K not divisible by block_k");
  if (M > 0x7FFFFFFF || N > 0x7FFFFFFF || K > 0x7FFFFFFF) return einval("GEMM dimension too large");
  if (bns != 1 && bns != 128) return einval("scale block along N must be 1 or 128");
  (void)who;
  return TG_OK;
}

static int gemm_fp8_nt_entry(const char* who, const uint8_t* a_q, const float* a_s, const uint8_t* b_q,
                             const float* b_s, int b_scale_bn, void* c, int c_dtype, int64_t M,
                             int64_t N, int64_t K, int block_k, void* stream, bool skm) {
  TG_TRY(check_gemm_args(who, M, N, K, block_k, b_scale_bn, !skm));
  if (c_dtype != TG_DTYPE_BF16 && c_dtype != TG_DTYPE_F32) return einval("gemm_fp8_nt: bad c_dtype");
  if (M == 0 || N == 0) return TG_OK;
  if (!a_q || !a_s || !b_q || !b_s || !c) return einval("gemm_fp8_nt: null pointer");
  if (block_k != 128)
    return launch_gemm_gb(a_q, a_s, b_q, b_s, b_scale_bn, c, c_dtype, M, N, K, block_k, as_stream(stream));
  if (!aligned(a_q, 16) || !aligned(b_q, 16)) return einval("gemm_fp8_nt: operands must be 16-byte aligned");
  return launch_gemm_fp8(a_q, a_s, b_q, b_s, b_scale_bn, c, c_dtype, M, N, K, as_stream(stream), skm);
}

extern "C" int tg_gemm_fp8_nt(const uint8_t* a_q, const float* a_s, const uint8_t* b_q,
                              const float* b_s, int b_scale_bn, void* c, int c_dtype, int64_t M,
                              int64_t N, int64_t K, int block_k, void* stream) {
  return gemm_fp8_nt_entry("gemm_fp8_nt", a_q, a_s, b_q, b_s, b_scale_bn, c, c_dtype, M, N, K, block_k,
                           stream, false);
}

extern "C" int tg_gemm_fp8_nt_km(const uint8_t* a_q, const float* a_s_km, const uint8_t* b_q,
                                 const float* b_s_km, int b_scale_bn, void* c, int c_dtype, int64_t M,
                                 int64_t N, int64_t K, int block_k, void* stream) {
  return gemm_fp8_nt_entry("gemm_fp8_nt_km", a_q, a_s_km, b_q, b_s_km, b_scale_bn, c, c_dtype, M, N, K,
                           block_k, stream, true);
}

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// How the composites feed a block_k != 128 to the tuned GEMM (128-wide scale
// blocks): a multiple of 128 repeats each block's scale per 128 columns
// (srep); a divisor of 128 down to 16 puts each block in a zero-filled
// 128-byte slot (pf, the contraction grows pf-fold); other sizes run the
// general GEMM.
static inline int gb_srep(int block_k) { return block_k % 128 == 0 ? block_k / 128 : 1; }
static inline int gb_pf(int block_k) { return block_k < 128 && block_k >= 16 && 128 % block_k == 0 ? 128 / block_k : 1; }
static inline bool gb_tuned(int block_k) { return gb_srep(block_k) > 1 || gb_pf(block_k) > 1; }
// scale entries per row for a contraction of `extent`
static inline size_t scale_cols(int64_t extent, int block_k) {
  return (size_t)(block_k % 128 == 0 ? extent / 128 : extent / block_k);
}

extern "C" size_t tg_block_scaled_matmul_workspace(int64_t M, int64_t N, int64_t K, int block_k) {
  if (block_k <= 0 || M < 0 || N < 0 || K < 0) return 0;
  const size_t nkb = scale_cols(K, block_k), kq = (size_t)K * (size_t)gb_pf(block_k);
  return align256((size_t)M * kq) + align256((size_t)M * nkb * 4) + align256((size_t)N * kq) +
         align256((size_t)N * nkb * 4);
}

// The forward composite's kernels on a workspace the caller has checked.
int tg::block_scaled_matmul_on(const void* a, const void* b, void* out, int64_t M, int64_t N,
                               int64_t K, void* workspace, hipStream_t st) {
  const int64_t nkb = K / 128;
  uint8_t* p = reinterpret_cast<uint8_t*>(workspace);
  uint8_t* qa = p;                 p += align256((size_t)M * K);
  float* sa = reinterpret_cast<float*>(p);   p += align256((size_t)M * nkb * 4);
  uint8_t* qb = p;                 p += align256((size_t)N * K);
  float* sb = reinterpret_cast<float*>(p);
  // the composite's own workspace: scales K-block-major (the GEMM's cheaper scale reads)
  if (M % 128 == 0 && N % 128 == 0) {
    // both quantizations in one launch (fp8.py:66, 68): one kernel's fixed
    // cost instead of two's, which is most of the time at small shapes
    TG_TRY(launch_quant_rows_cols(a, M, K, qa, sa, b, N, qb, sb, st, true));
  } else {
    TG_TRY(launch_quant_rows(a, TG_DTYPE_BF16, M, K, qa, sa, st, true));     // fp8.py:66
    TG_TRY(launch_quant_cols(b, K, N, qb, sb, st, true));                     // fp8.py:68
  }
  return launch_gemm_fp8(qa, sa, qb, sb, 1, out, TG_DTYPE_BF16, M, N, K, st, true);   // fp8.py:70-78
}

// The forward composite for block_k != 128: row-major scales, the general
// quantizers; a multiple of 128 then runs the tuned GEMM on its scales
// repeated per 128-wide sub-block.  The bytes and scales are the block's; the
// f32 sum is the same in exact arithmetic but rounds differently: the tuned
// GEMM folds acc = fma(P_128, sa * sb, acc) once per 128-wide sub-block,
// where tg_gemm_fp8_nt at the same block_k (the general GEMM) forms one P per
// block and folds it once, so the two agree to f32 rounding, not bit for bit.
// Any other block size runs the general GEMM.
static int block_scaled_matmul_gb(const void* a, const void* b, void* out, int64_t M, int64_t N, int64_t K,
                                  int bk, void* workspace, hipStream_t st) {
  const int64_t nkb = (int64_t)scale_cols(K, bk);
  // the tuned GEMM takes a 32-bit contraction extent: a zero-slot layout that
  // would grow K past it runs the general kernels instead
  const bool tuned = gb_tuned(bk) && K * gb_pf(bk) <= 0x7FFFFFFF;
  const int srep = tuned ? gb_srep(bk) : 1, pf = tuned ? gb_pf(bk) : 1;
  const int64_t kq = K * pf;
  uint8_t* p = reinterpret_cast<uint8_t*>(workspace);
  uint8_t* qa = p;                 p += align256((size_t)M * kq);
  float* sa = reinterpret_cast<float*>(p);   p += align256((size_t)M * nkb * 4);
  uint8_t* qb = p;                 p += align256((size_t)N * kq);
  float* sb = reinterpret_cast<float*>(p);
  // the tuned GEMM reads the scales K-block-major (the _km layout: one column
  // of scales per K block), the general one row-major
  TG_TRY(launch_quant_rows_gb(a, TG_DTYPE_BF16, M, K, bk, qa, sa, st, srep, pf, tuned));     // fp8.py:66
  TG_TRY(launch_quant_cols_gb(b, false, K, N, bk, qb, sb, st, srep, pf, tuned));             // fp8.py:68
  if (tuned) return launch_gemm_fp8(qa, sa, qb, sb, 1, out, TG_DTYPE_BF16, M, N, kq, st, true);
  return launch_gemm_gb(qa, sa, qb, sb, 1, out, TG_DTYPE_BF16, M, N, K, bk, st);   // fp8.py:70-78
}

extern "C" int tg_block_scaled_matmul(const void* a, const void* b, void* out, int64_t M,
                                      int64_t N, int64_t K, int block_k, void* workspace,
                                      size_t workspace_bytes, void* stream) {
  TG_TRY(check_gemm_args("block_scaled_matmul", M, N, K, block_k, 1, true));
  if (M == 0 || N == 0) return TG_OK;
  if (!a || !b || !out || !workspace) return einval("block_scaled_matmul: null pointer");
  if (workspace_bytes < tg_block_scaled_matmul_workspace(M, N, K, block_k))
    return einval("block_scaled_matmul: workspace too small");
  if (block_k != 128) {
    if (!aligned(workspace, 256) || !aligned(a, 2) || !aligned(b, 2))
      return einval("block_scaled_matmul: a, b must be 2-byte and workspace 256-byte aligned");
    return block_scaled_matmul_gb(a, b, out, M, N, K, block_k, workspace, as_stream(stream));
  }
  if (!aligned(workspace, 256) || !aligned(a, 16) || !aligned(b, 16))
    return einval("block_scaled_matmul: a, b must be 16-byte and workspace 256-byte aligned");
  return block_scaled_matmul_on(a, b, out, M, N, K, workspace, as_stream(stream));
}

extern "C" size_t tg_block_scaled_matmul_bwd_workspace(int64_t M, int64_t N, int64_t K, int block_k) {
  if (block_k <= 0 || M < 0 || N < 0 || K < 0) return 0;
  const size_t mkb = scale_cols(M, block_k), nkb = scale_cols(N, block_k), pf = (size_t)gb_pf(block_k);
  return align256((size_t)M * N * pf) + align256((size_t)M * nkb * 4) +   // g along N
         align256((size_t)K * N * pf) + align256((size_t)K * nkb * 4) +   // b along N
         align256((size_t)K * M * pf) + align256((size_t)K * mkb * 4) +   // a.T along M
         align256((size_t)N * M * pf) + align256((size_t)N * mkb * 4);    // g.T along M
}

extern "C" int tg_block_scaled_matmul_bwd_fp8(const void* a, const void* b, const void* g,
                                              void* da, void* db, int64_t M, int64_t N, int64_t K,
                                              int block_k, void* workspace,
                                              size_t workspace_bytes, void* stream) {
  TG_TRY(check_gemm_args("block_scaled_matmul_bwd_fp8", M, N, K, block_k, 1, true));
  if (M % block_k || N % block_k)
    return einval("block_scaled_matmul_bwd_fp8: M and N must be multiples of block_k");
  if (M == 0 || N == 0) {
    // an empty M or N: the gradient that sums over it is zero (db = a.T @ g
    // over M = 0, da = g @ b.T over N = 0), the other one is empty
    if ((M * K && !da) || (K * N && !db)) return einval("block_scaled_matmul_bwd_fp8: null pointer");
    TG_TRY(launch_fill_zero_bf16(da, M * K, as_stream(stream)));
    return launch_fill_zero_bf16(db, K * N, as_stream(stream));
  }
  if (!a || !b || !g || !da || !db || !workspace) return einval("block_scaled_matmul_bwd_fp8: null pointer");
  if (workspace_bytes < tg_block_scaled_matmul_bwd_workspace(M, N, K, block_k))
    return einval("block_scaled_matmul_bwd_fp8: workspace too small");
  if (block_k != 128) {
    // the general kernels, row-major scales: g along N, b along N, a.T along M, g.T along M
    if (!aligned(workspace, 256) || !aligned(a, 2) || !aligned(b, 2) || !aligned(g, 2))
      return einval("block_scaled_matmul_bwd_fp8: inputs must be 2-byte and workspace 256-byte aligned");
    hipStream_t st = as_stream(stream);
    const int bk = block_k;
    const int64_t mkb = (int64_t)scale_cols(M, bk), nkb = (int64_t)scale_cols(N, bk);
    // the tuned GEMM's layouts (see block_scaled_matmul_gb), while the grown
    // contraction extents (N * pf for dX, M * pf for dW) stay 32-bit
    const bool tuned = gb_tuned(bk) && N * gb_pf(bk) <= 0x7FFFFFFF && M * gb_pf(bk) <= 0x7FFFFFFF;
    const int srep = tuned ? gb_srep(bk) : 1, pf = tuned ? gb_pf(bk) : 1;
    const int64_t nq = N * pf, mq = M * pf;
    uint8_t* p = reinterpret_cast<uint8_t*>(workspace);
    uint8_t* qg = p;    p += align256((size_t)M * nq);
    float* sg = reinterpret_cast<float*>(p);    p += align256((size_t)M * nkb * 4);
    uint8_t* qb = p;    p += align256((size_t)K * nq);
    float* sb = reinterpret_cast<float*>(p);    p += align256((size_t)K * nkb * 4);
    uint8_t* qat = p;   p += align256((size_t)K * mq);
    float* sat = reinterpret_cast<float*>(p);   p += align256((size_t)K * mkb * 4);
    uint8_t* qgt = p;   p += align256((size_t)N * mq);
    float* sgt = reinterpret_cast<float*>(p);
    TG_TRY(launch_quant_rows_gb(g, TG_DTYPE_BF16, M, N, bk, qg, sg, st, srep, pf, tuned));
    TG_TRY(launch_quant_rows_gb(b, TG_DTYPE_BF16, K, N, bk, qb, sb, st, srep, pf, tuned));
    if (tuned) TG_TRY(launch_gemm_fp8(qg, sg, qb, sb, 1, da, TG_DTYPE_BF16, M, K, nq, st, true));
    else TG_TRY(launch_gemm_gb(qg, sg, qb, sb, 1, da, TG_DTYPE_BF16, M, K, N, bk, st));      // dX = g . b.T
    TG_TRY(launch_quant_cols_gb(a, false, M, K, bk, qat, sat, st, srep, pf, tuned));
    TG_TRY(launch_quant_cols_gb(g, false, M, N, bk, qgt, sgt, st, srep, pf, tuned));
    if (tuned) return launch_gemm_fp8(qat, sat, qgt, sgt, 1, db, TG_DTYPE_BF16, K, N, mq, st, true);
    return launch_gemm_gb(qat, sat, qgt, sgt, 1, db, TG_DTYPE_BF16, K, N, M, bk, st);   // dW = a.T . g
  }
  if (!aligned(workspace, 256) || !aligned(a, 16) || !aligned(b, 16) || !aligned(g, 16))
    return einval("block_scaled_matmul_bwd_fp8: inputs must be 16-byte and workspace 256-byte aligned");
  hipStream_t st = as_stream(stream);
  const int64_t mkb = M / 128, nkb = N / 128;
  uint8_t* p = reinterpret_cast<uint8_t*>(workspace);
  uint8_t* qg = p;    p += align256((size_t)M * N);
  float* sg = reinterpret_cast<float*>(p);    p += align256((size_t)M * nkb * 4);
  uint8_t* qb = p;    p += align256((size_t)K * N);
  float* sb = reinterpret_cast<float*>(p);    p += align256((size_t)K * nkb * 4);
  uint8_t* qat = p;   p += align256((size_t)K * M);
  float* sat = reinterpret_cast<float*>(p);   p += align256((size_t)K * mkb * 4);
  uint8_t* qgt = p;   p += align256((size_t)N * M);
  float* sgt = reinterpret_cast<float*>(p);
  // g along N and g.T along M from one read of g; every scale array of the
  // workspace K-block-major
  TG_TRY(launch_quant_dual(g, M, N, qg, sg, qgt, sgt, st, true));
  TG_TRY(launch_quant_rows(b, TG_DTYPE_BF16, K, N, qb, sb, st, true));
  TG_TRY(launch_gemm_fp8(qg, sg, qb, sb, 1, da, TG_DTYPE_BF16, M, K, N, st, true));    // dX = g . b.T
  TG_TRY(launch_quant_cols(a, M, K, qat, sat, st, true));
  return launch_gemm_fp8(qat, sat, qgt, sgt, 1, db, TG_DTYPE_BF16, K, N, M, st, true);  // dW = a.T . g
}


// Rows per workgroup: equal rows per CU, a multiple of 8, at most 64.
// Stages in flight per workgroup of the MFMA GEMV (see gemv_fp8_kernel).
constexpr int kGemvNS = 3;

template <int MT>
static int launch_gemv(const uint8_t* x_q, const float* x_s, const uint8_t* w_q, const float* w_s,
                       int bn, __bf16* out, int M, int N, int K, hipStream_t st) {
  constexpr int NS = kGemvNS;
  // as many workgroups as fit at once (one per CU with three stages in flight,
  // two with two), each with a balanced share of the 8-row groups (at most
  // kGemvGroups: more workgroups than fit when N is large)
  const int64_t groups = ((int64_t)N + 7) / 8;
  int64_t nwg = (int64_t)device_cus() * (NS == 2 ? 2 : 1);
  if (nwg > groups) nwg = groups;
  const int64_t need = (groups + kGemvGroups - 1) / kGemvGroups;
  if (nwg < need) nwg = need;
  const dim3 grid((unsigned)nwg);
  const GemvNormIn none{};
  // up to 8 rows: x copied into LDS with whole-row loads (PRO_XCOPY), when it
  // fits beside the three weight stages
  const size_t xlds = (size_t)8 * (size_t)(K + 16) + (size_t)8 * (size_t)(K / 128) * 4;
  if (MT == 1 && M <= 8 && xlds <= (size_t)160 * 1024 - (size_t)NS * kGemvStage) {
    if (bn == 1)
      hipLaunchKernelGGL((gemv_fp8_kernel<1, 1, NS, PRO_XCOPY>), grid, dim3(512), xlds, st, x_q, x_s, w_q, w_s,
                         out, M, N, K, none);
    else
      hipLaunchKernelGGL((gemv_fp8_kernel<1, 128, NS, PRO_XCOPY>), grid, dim3(512), xlds, st, x_q, x_s, w_q,
                         w_s, out, M, N, K, none);
    return check_launch("gemv_fp8");
  }
  if (bn == 1)
    hipLaunchKernelGGL((gemv_fp8_kernel<MT, 1, NS>), grid, dim3(512), 0, st, x_q, x_s, w_q, w_s, out, M,
                       N, K, none);
  else
    hipLaunchKernelGGL((gemv_fp8_kernel<MT, 128, NS>), grid, dim3(512), 0, st, x_q, x_s, w_q, w_s, out,
                       M, N, K, none);
  return check_launch("gemv_fp8");
}

// The norm prologue's LDS (x bytes of 16 rows at pitch K + 16, their scales),
// beside the three static weight stages (up to K = 3456 would fit).
static size_t gemv_norm_lds(int64_t K) { return (size_t)16 * (size_t)(K + 16) + (size_t)16 * (size_t)(K / 128) * 4; }
constexpr size_t kGemvNormMaxLds = (size_t)160 * 1024 - (size_t)3 * kGemvStage;

template <int PRO, int J>
static int launch_gemv_norm(const GemvNormIn& nin, const uint8_t* w_q, const float* w_s, int bn, __bf16* out,
                            int M, int N, int K, hipStream_t st) {
  constexpr int NS = kGemvNS;
  const int64_t groups = ((int64_t)N + 7) / 8;
  int64_t nwg = (int64_t)device_cus();
  if (nwg > groups) nwg = groups;
  const int64_t need = (groups + kGemvGroups - 1) / kGemvGroups;
  if (nwg < need) nwg = need;
  const dim3 grid((unsigned)nwg);
  const size_t lds = gemv_norm_lds(K);
  if (bn == 1)
    hipLaunchKernelGGL((gemv_fp8_kernel<1, 1, NS, PRO, J>), grid, dim3(512), lds, st, nullptr, nullptr, w_q,
                       w_s, out, M, N, K, nin);
  else
    hipLaunchKernelGGL((gemv_fp8_kernel<1, 128, NS, PRO, J>), grid, dim3(512), lds, st, nullptr, nullptr,
                       w_q, w_s, out, M, N, K, nin);
  return check_launch("rms_norm_fp8_gemv");
}

// K <= 2560 (at most 5 chunks per lane of a row: a wider row's registers
// spill beside the weight stages')
constexpr int64_t kGemvNormMaxK = 2560;
template <int PRO>
static int launch_gemv_norm_k(const GemvNormIn& nin, const uint8_t* w_q, const float* w_s, int bn,
                              __bf16* out, int M, int N, int K, hipStream_t st) {
  const int jneed = (K / 8 + 63) / 64;   // 16-byte chunks per lane of a row
  if (jneed <= 4) return launch_gemv_norm<PRO, 4>(nin, w_q, w_s, bn, out, M, N, K, st);
  return launch_gemv_norm<PRO, 5>(nin, w_q, w_s, bn, out, M, N, K, st);
}

// ---- the direct GEMV (gemv_direct_kernel) ----
// LDS: x rows at pitch K + 16, their scales, the 8 waves' partial tiles.
static size_t gemv_direct_lds(int64_t M, int64_t K, int mt) {
  const size_t x = (size_t)M * (size_t)(K + 16) + (size_t)M * (size_t)(K / 128) * 4;
  return ((x + 15) & ~(size_t)15) + (size_t)8 * mt * 64 * 16;
}
// Whether the direct kernel takes (M, N, K).  Shape: at most 8 or 17-32 rows
// (9-16 rows stay on the staged kernel, whose norm prologue takes them, so
// that tg_rms_norm_fp8_gemv and tg_gemv_fp8 keep one summation order per
// shape), K blocks of a wave in registers (K <= 12288, and <= 4096 past 16
// rows), the x copy in one round of 16 chunks per thread, and the LDS above
// within a CU's 160 KiB.  Speed (same-box A/B at the reference decode shapes
// and C5): direct wins up to ~2.5 row blocks per CU (<= 640 blocks: the
// decode wo, w_down, q|k|v and w_up weights; w_up 6.9 against 8.0 us at 8
// rows) and past N = 16384 (the 50257-row unembedding, where the staged
// kernel runs several rounds of workgroups); in between (C5's 14336 rows:
// 14.8 against 13.1 us) the staged kernel's 4 KiB-contiguous row reads
// stream better than 64 bytes of 16 rows per load.
static bool gemv_direct_fits(int64_t M, int64_t N, int64_t K) {
  if (M < 1 || M > 32 || (M > 8 && M <= 16)) return false;
  const int64_t nrb = (N + 15) / 16;
  if (nrb > 640 && N <= 16384) return false;
  const int mt = M <= 16 ? 1 : 2;
  const int64_t kpw = (K / 128 + 7) / 8;
  if (kpw > (mt == 1 ? 12 : 4)) return false;
  if ((M * K / 16 + 511) / 512 > 16) return false;
  return gemv_direct_lds(M, K, mt) <= (size_t)160 * 1024;
}

template <int MT, int BNS, int KPW, int PRO, int XC, int J>
static int launch_gemv_direct_t(const uint8_t* x_q, const float* x_s, const GemvNormIn& nin, const uint8_t* w_q,
                                const float* w_s, __bf16* out, int M, int N, int K, hipStream_t st) {
  auto kern = gemv_direct_kernel<MT, BNS, KPW, PRO, XC, J>;
  // workgroups resident at once: registers (once per instantiation), LDS per launch
  static const int occ_regs = [] {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, gemv_direct_kernel<MT, BNS, KPW, PRO, XC, J>, 512, 0) !=
            hipSuccess || v <= 0)
      v = 1;
    return v;
  }();
  const size_t lds = gemv_direct_lds(M, K, MT);
  int per_cu = occ_regs;
  const int by_lds = (int)(((size_t)160 * 1024) / lds);
  if (by_lds < per_cu) per_cu = by_lds < 1 ? 1 : by_lds;
  const int64_t nrb = ((int64_t)N + 15) / 16, cap = (int64_t)per_cu * (device_cus() > 0 ? device_cus() : 1);
  const int grid = (int)(nrb < cap ? nrb : cap);
  if (lds > 64 * 1024) {
    // the dynamic-LDS limit is a per-device function attribute (set once per device)
    constexpr int kMaxDev = 64;
    static std::once_flag once[kMaxDev];
    static hipError_t attr_rc[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) dev = 0;
    std::call_once(once[dev], [&] {
      attr_rc[dev] = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    if (attr_rc[dev] != hipSuccess) {
      set_error("gemv_fp8 (set LDS size): %s", hipGetErrorString(attr_rc[dev]));
      return TG_EHIP;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(512), lds, st, x_q, x_s, w_q, w_s, out, M, N, K, nin);
  return check_launch("gemv_fp8 (direct)");
}

template <int MT, int BNS>
static int launch_gemv_direct_x(const uint8_t* x_q, const float* x_s, const uint8_t* w_q, const float* w_s,
                                __bf16* out, int M, int N, int K, hipStream_t st) {
  const GemvNormIn none{};
  const int kpw = (K / 128 + 7) / 8;
  const int xc = (M * (K / 16) + 511) / 512;
  if constexpr (MT == 2) {
    return launch_gemv_direct_t<2, BNS, 4, PRO_X, 16, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
  } else {
    // K blocks per wave: exact for the decode widths (3 at K = 2304, 9 at 9216), else rounded up
    if (xc <= 4) {
      if (kpw <= 3) return launch_gemv_direct_t<1, BNS, 3, PRO_X, 4, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
      if (kpw <= 4) return launch_gemv_direct_t<1, BNS, 4, PRO_X, 4, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
      if (kpw <= 8) return launch_gemv_direct_t<1, BNS, 8, PRO_X, 4, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
      if (kpw <= 9) return launch_gemv_direct_t<1, BNS, 9, PRO_X, 4, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
      return launch_gemv_direct_t<1, BNS, 12, PRO_X, 4, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
    }
    if (kpw <= 3) return launch_gemv_direct_t<1, BNS, 3, PRO_X, 16, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
    if (kpw <= 4) return launch_gemv_direct_t<1, BNS, 4, PRO_X, 16, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
    if (kpw <= 8) return launch_gemv_direct_t<1, BNS, 8, PRO_X, 16, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
    if (kpw <= 9) return launch_gemv_direct_t<1, BNS, 9, PRO_X, 16, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
    return launch_gemv_direct_t<1, BNS, 12, PRO_X, 16, 1>(x_q, x_s, none, w_q, w_s, out, M, N, K, st);
  }
}

static int launch_gemv_direct(const uint8_t* x_q, const float* x_s, const uint8_t* w_q, const float* w_s, int bn,
                              __bf16* out, int M, int N, int K, hipStream_t st) {
  if (M <= 16)
    return bn == 1 ? launch_gemv_direct_x<1, 1>(x_q, x_s, w_q, w_s, out, M, N, K, st)
                   : launch_gemv_direct_x<1, 128>(x_q, x_s, w_q, w_s, out, M, N, K, st);
  return bn == 1 ? launch_gemv_direct_x<2, 1>(x_q, x_s, w_q, w_s, out, M, N, K, st)
                 : launch_gemv_direct_x<2, 128>(x_q, x_s, w_q, w_s, out, M, N, K, st);
}

// The norm prologue in the direct GEMV: at most 8 rows, K <= 2560 (one K
// block group of <= 4 per wave; 5 chunks per lane of a norm row).
template <int PRO>
static int launch_gemv_direct_norm(const GemvNormIn& nin, const uint8_t* w_q, const float* w_s, int bn,
                                   __bf16* out, int M, int N, int K, hipStream_t st) {
  if ((K / 128 + 7) / 8 <= 3)
    return bn == 1 ? launch_gemv_direct_t<1, 1, 3, PRO, 1, 5>(nullptr, nullptr, nin, w_q, w_s, out, M, N, K, st)
                   : launch_gemv_direct_t<1, 128, 3, PRO, 1, 5>(nullptr, nullptr, nin, w_q, w_s, out, M, N, K, st);
  return bn == 1 ? launch_gemv_direct_t<1, 1, 4, PRO, 1, 5>(nullptr, nullptr, nin, w_q, w_s, out, M, N, K, st)
                 : launch_gemv_direct_t<1, 128, 4, PRO, 1, 5>(nullptr, nullptr, nin, w_q, w_s, out, M, N, K, st);
}

extern "C" int tg_gemv_fp8(const uint8_t* x_q, const float* x_s, const uint8_t* w_q,
                           const float* w_s, int w_scale_bn, void* out, int64_t M, int64_t N,
                           int64_t K, int block_k, void* stream) {
  TG_TRY(check_gemm_args("gemv_fp8", M, N, K, block_k, w_scale_bn));
  if (M > 64) return einval("gemv_fp8: M must be <= 64 (use tg_gemm_fp8_nt)");
  if (M == 0 || N == 0) return TG_OK;
  if (!x_q || !x_s || !w_q || !w_s || !out) return einval("gemv_fp8: null pointer");
  if (!aligned(x_q, 16) || !aligned(w_q, 16)) return einval("gemv_fp8: operands must be 16-byte aligned");
  if ((uint64_t)N * (uint64_t)(K / 128) * 4u >= (1ull << 32) || (uint64_t)M * (uint64_t)K >= (1ull << 32) ||
      (uint64_t)64 * (uint64_t)K >= (1ull << 32))
    return einval("gemv_fp8: operand too large for 32-bit buffer offsets");
  hipStream_t st = as_stream(stream);
  const int m = (int)M, n = (int)N, k = (int)K;
  auto o = reinterpret_cast<__bf16*>(out);
  if (gemv_direct_fits(M, N, K)) return launch_gemv_direct(x_q, x_s, w_q, w_s, w_scale_bn, o, m, n, k, st);
  if (M <= 16) return launch_gemv<1>(x_q, x_s, w_q, w_s, w_scale_bn, o, m, n, k, st);
  if (M <= 32) return launch_gemv<2>(x_q, x_s, w_q, w_s, w_scale_bn, o, m, n, k, st);
  // 33 <= M <= 64: the GEMM (one pass over W on the short-K ring kernel: 20.7
  // against 33.3 us for two 32-row GEMV passes at 64 x 14336 x 4096)
  return launch_gemm_fp8(x_q, x_s, w_q, w_s, w_scale_bn, out, TG_DTYPE_BF16, M, N, K, st, false);
}

template <int NX, int PRO, int XL, int J, int WPG = 4, bool RES = false, int NQ = 4>
static void launch_rowdot_k(const RowdotIn& in, const uint8_t* w_q, const float* w_s, int bns, __bf16* o,
                            int n, int k, int sx_off, size_t lds, hipStream_t st) {
  // persistent waves, one wave per weight row at a time: as many workgroups
  // as fit on the CUs at once (registers: once per instantiation; LDS: 160 KiB
  // per CU), at most 32 waves per CU, so that no workgroup waits for a free
  // slot (a function-local static: its initializer runs once, thread-safely)
  static const int occ_regs = [] {
    int v = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, gemv_rowdot_kernel<NX, PRO, XL, J, WPG, RES, NQ>, 64 * WPG, 0) !=
            hipSuccess || v <= 0)
      v = 16 / WPG;
    return v;
  }();
  constexpr int kMaxPerCu = 32 / WPG;
  int per_cu = occ_regs < kMaxPerCu ? occ_regs : kMaxPerCu;
  const int by_lds = (int)((160 * 1024) / (lds > 0 ? lds : 1));
  if (by_lds < per_cu) per_cu = by_lds < 1 ? 1 : by_lds;
  const int64_t wgs = ((int64_t)n + WPG - 1) / WPG, cap = (int64_t)per_cu * device_cus();
  hipLaunchKernelGGL((gemv_rowdot_kernel<NX, PRO, XL, J, WPG, RES, NQ>), dim3((unsigned)(wgs < cap ? wgs : cap)),
                     dim3(64 * WPG), lds, st, in, w_q, w_s, bns, o, n, k, sx_off);
}

// PRO_X: XL 4 KiB pieces of x; PRO_RELU2: XL 16-byte chunks of u per thread;
// PRO_NORM*: J chunks of the norm row per lane.
template <int NX, int PRO, bool RES, int NQ>
static int launch_rowdot_q(const RowdotIn& in, const uint8_t* w_q, const float* w_s, int bns, __bf16* o,
                         int n, int k, hipStream_t st) {
  if constexpr (PRO == PRO_X) {
    const int need = (NX * k + 4095) / 4096;
    const int sx_off = (need <= 1 ? 1 : need <= 2 ? 2 : need <= 4 ? 4 : 8) * 4096;
    const size_t lds = (size_t)sx_off + 1024;
    if (need <= 1) launch_rowdot_k<NX, PRO, 1, 1, 4, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
    else if (need <= 2) launch_rowdot_k<NX, PRO, 2, 1, 4, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
    else if (need <= 4) launch_rowdot_k<NX, PRO, 4, 1, 4, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
    else launch_rowdot_k<NX, PRO, 8, 1, 4, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
  } else {
    const int sx_off = NX * k;   // a multiple of 128
    // x bytes, x scales; for the norm prologues also the bf16 residual sums and r
    const size_t lds = PRO == PRO_RELU2
                           ? (size_t)sx_off + (size_t)NX * (k / 128) * 4
                           : (((size_t)sx_off + (size_t)NX * (k / 128) * 4 + 15) & ~(size_t)15) +
                                 (size_t)NX * k * 2 + 16;
    constexpr int W = kRowdotProWaves;
    if constexpr (PRO == PRO_RELU2) {
      const int need = (NX * k / 8 + 64 * W - 1) / (64 * W);   // 16-byte chunks of u per thread
      if (need <= 1) launch_rowdot_k<NX, PRO, 1, 1, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else if (need <= 2) launch_rowdot_k<NX, PRO, 2, 1, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else if (need <= 4) launch_rowdot_k<NX, PRO, 4, 1, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else if (need <= 8) launch_rowdot_k<NX, PRO, 8, 1, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else launch_rowdot_k<NX, PRO, 16, 1, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
    } else {
      const int jneed = (k / 8 + 63) / 64;
      if (jneed <= 1) launch_rowdot_k<NX, PRO, 1, 1, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else if (jneed <= 2) launch_rowdot_k<NX, PRO, 1, 2, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else if (jneed <= 4) launch_rowdot_k<NX, PRO, 1, 4, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else if (jneed <= 5) launch_rowdot_k<NX, PRO, 1, 5, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
      else launch_rowdot_k<NX, PRO, 1, 8, W, RES, NQ>(in, w_q, w_s, bns, o, n, k, sx_off, lds, st);
    }
  }
  return TG_OK;
}

// Units of 3 KiB when the rows are a multiple of 3 KiB or shorter, else 4 KiB.
template <int NX, int PRO, bool RES = false>
static int launch_rowdot(const RowdotIn& in, const uint8_t* w_q, const float* w_s, int bns, __bf16* o,
                         int n, int k, hipStream_t st) {
  if (k % 3072 == 0 || k <= 3072) return launch_rowdot_q<NX, PRO, RES, 3>(in, w_q, w_s, bns, o, n, k, st);
  return launch_rowdot_q<NX, PRO, RES, 4>(in, w_q, w_s, bns, o, n, k, st);
}

static int rowdot_common_checks(const char* who, int64_t M, int64_t N, int64_t K, int w_scale_bn,
                                const uint8_t* w_q, const float* w_s, const void* out, int64_t kmax) {
  TG_TRY(check_gemm_args(who, M, N, K, 128, w_scale_bn));
  char msg[160];
  const char* what = nullptr;
  if (M > 2) what = "M must be <= 2 (use tg_gemv_fp8)";
  else if (K > kmax) what = kmax == kRowdotMaxK ? "K must be <= 16384" : "K must be <= 4096";
  else if (M == 0 || N == 0) return TG_OK;
  else if (!w_q || !w_s || !out) what = "null pointer";
  else if (!aligned(w_q, 16)) what = "operands must be 16-byte aligned";
  else if ((uint64_t)N * (uint64_t)K >= (1ull << 32) || (uint64_t)N * (uint64_t)(K / 128) * 4u >= (1ull << 32))
    what = "operand too large for 32-bit buffer offsets";
  if (!what) return TG_OK;
  snprintf(msg, sizeof(msg), "%s: %s", who, what);
  return einval(msg);
}

static bool ranges_overlap(const void* a, const void* b, size_t bytes) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + bytes && y < x + bytes;
}

extern "C" int tg_gemv_fp8_rowdot(const uint8_t* x_q, const float* x_s, const uint8_t* w_q,
                                  const float* w_s, int w_scale_bn, void* out, int64_t M, int64_t N,
                                  int64_t K, int block_k, void* stream) {
  if (block_k != 128) return einval("block_k must be 128");
  TG_TRY(rowdot_common_checks("gemv_fp8_rowdot", M, N, K, w_scale_bn, w_q, w_s, out, kRowdotMaxK));
  if (M == 0 || N == 0) return TG_OK;
  if (!x_q || !x_s) return einval("gemv_fp8_rowdot: null pointer");
  if (!aligned(x_q, 16)) return einval("gemv_fp8_rowdot: operands must be 16-byte aligned");
  RowdotIn in{};
  in.xq = x_q;
  in.xs = x_s;
  auto o = reinterpret_cast<__bf16*>(out);
  hipStream_t st = as_stream(stream);
  if (M == 1) TG_TRY((launch_rowdot<1, PRO_X>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  else TG_TRY((launch_rowdot<2, PRO_X>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  return check_launch("gemv_fp8_rowdot");
}

// 3..16 rows: the MFMA GEMV with the norm prologue (tg_gemv_fp8's arithmetic).
static int gemv_norm_checks(int64_t M, int64_t N, int64_t K, int w_scale_bn, const uint8_t* w_q,
                            const float* w_s, const void* out) {
  TG_TRY(check_gemm_args("rms_norm_fp8_gemv", M, N, K, 128, w_scale_bn));
  const char* what = nullptr;
  char msg[200];
  if (M > 16) {
    what = "M must be <= 16 (the norm prologue holds 16 rows)";
  } else if (K > kGemvNormMaxK || gemv_norm_lds(K) > kGemvNormMaxLds) {
    snprintf(msg, sizeof(msg), "rms_norm_fp8_gemv: K=%lld too large for 3-16 rows (K <= %lld)", (long long)K,
             (long long)kGemvNormMaxK);
    return einval(msg);
  } else if (N == 0) {
    return TG_OK;
  } else if (!w_q || !w_s || !out) {
    what = "null pointer";
  } else if (!aligned(w_q, 16)) {
    what = "operands must be 16-byte aligned";
  } else if ((uint64_t)N * (uint64_t)(K / 128) * 4u >= (1ull << 32) || (uint64_t)64 * (uint64_t)K >= (1ull << 32)) {
    what = "operand too large for 32-bit buffer offsets";
  }
  if (!what) return TG_OK;
  snprintf(msg, sizeof(msg), "rms_norm_fp8_gemv: %s", what);
  return einval(msg);
}

extern "C" int tg_rms_norm_fp8_gemv(const void* x, const void* delta, const void* gamma, float eps,
                                    void* xout, const uint8_t* w_q, const float* w_s, int w_scale_bn,
                                    void* out, int64_t M, int64_t N, int64_t K, void* stream) {
  if (M > 2)
    TG_TRY(gemv_norm_checks(M, N, K, w_scale_bn, w_q, w_s, out));
  else
    TG_TRY(rowdot_common_checks("rms_norm_fp8_gemv", M, N, K, w_scale_bn, w_q, w_s, out, kRowdotNormMaxK));
  if (M == 0 || N == 0) return TG_OK;
  if (!x || !gamma || (delta && !xout)) return einval("rms_norm_fp8_gemv: null pointer");
  if (!aligned(x, 16) || !aligned(gamma, 16) || (delta && (!aligned(delta, 16) || !aligned(xout, 16))))
    return einval("rms_norm_fp8_gemv: x, delta, gamma and xout must be 16-byte aligned");
  const size_t rb = (size_t)M * (size_t)K * 2;
  if (delta && (ranges_overlap(xout, x, rb) || ranges_overlap(xout, delta, rb)))
    return einval("rms_norm_fp8_gemv: xout must not overlap x or delta (other workgroups read them "
                  "while workgroup 0 stores xout)");
  auto o = reinterpret_cast<__bf16*>(out);
  hipStream_t st = as_stream(stream);
  const int n = (int)N, k = (int)K;
  if (M > 2) {
    GemvNormIn gi{};
    gi.x = reinterpret_cast<const uint4*>(x);
    gi.delta = reinterpret_cast<const uint4*>(delta);
    gi.gamma = reinterpret_cast<const uint4*>(gamma);
    gi.xout = reinterpret_cast<uint4*>(xout);
    gi.eps = eps;
    if (M <= 8 && gemv_direct_fits(M, N, K)) {   // the rows tg_gemv_fp8 would take directly
      if (delta) return launch_gemv_direct_norm<PRO_NORM_ADD>(gi, w_q, w_s, w_scale_bn, o, (int)M, n, k, st);
      return launch_gemv_direct_norm<PRO_NORM>(gi, w_q, w_s, w_scale_bn, o, (int)M, n, k, st);
    }
    if (delta) return launch_gemv_norm_k<PRO_NORM_ADD>(gi, w_q, w_s, w_scale_bn, o, (int)M, n, k, st);
    return launch_gemv_norm_k<PRO_NORM>(gi, w_q, w_s, w_scale_bn, o, (int)M, n, k, st);
  }
  RowdotIn in{};
  in.x = reinterpret_cast<const uint4*>(x);
  in.delta = reinterpret_cast<const uint4*>(delta);
  in.gamma = reinterpret_cast<const uint4*>(gamma);
  in.xout = reinterpret_cast<uint4*>(xout);
  in.eps = eps;
  if (delta) {
    if (M == 1) TG_TRY((launch_rowdot<1, PRO_NORM_ADD>(in, w_q, w_s, w_scale_bn, o, n, k, st)));
    else TG_TRY((launch_rowdot<2, PRO_NORM_ADD>(in, w_q, w_s, w_scale_bn, o, n, k, st)));
  } else {
    if (M == 1) TG_TRY((launch_rowdot<1, PRO_NORM>(in, w_q, w_s, w_scale_bn, o, n, k, st)));
    else TG_TRY((launch_rowdot<2, PRO_NORM>(in, w_q, w_s, w_scale_bn, o, n, k, st)));
  }
  return check_launch("rms_norm_fp8_gemv");
}

extern "C" int tg_relu2_fp8_gemv(const void* u, const uint8_t* w_q, const float* w_s, int w_scale_bn,
                                 void* out, int64_t M, int64_t N, int64_t K, void* stream) {
  TG_TRY(rowdot_common_checks("relu2_fp8_gemv", M, N, K, w_scale_bn, w_q, w_s, out, kRowdotMaxK));
  if (M == 0 || N == 0) return TG_OK;
  if (!u) return einval("relu2_fp8_gemv: null pointer");
  if (!aligned(u, 16)) return einval("relu2_fp8_gemv: u must be 16-byte aligned");
  RowdotIn in{};
  in.x = reinterpret_cast<const uint4*>(u);
  auto o = reinterpret_cast<__bf16*>(out);
  hipStream_t st = as_stream(stream);
  if (M == 1) TG_TRY((launch_rowdot<1, PRO_RELU2>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  else TG_TRY((launch_rowdot<2, PRO_RELU2>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  return check_launch("relu2_fp8_gemv");
}

// The residual adds of model.py:75-76 fused into the GEMV that produces their
// term (1-2 rows, the VALU GEMV): out (M, N) = bf16(resid + bf16(x . W^T)),
// the bf16 tensor add of the plain entry point's output.  out may be resid
// itself (each element is read and written by one lane); any other overlap
// is refused.
static int rowdot_add_checks(const char* who, const void* resid, const void* out, int64_t M, int64_t N) {
  char msg[160];
  const char* what = nullptr;
  if (!resid) what = "null pointer";
  else if (!aligned(resid, 2)) what = "resid must be 2-byte aligned";
  else if (out != resid && ranges_overlap(out, resid, (size_t)M * (size_t)N * 2))
    what = "out must be resid itself or not overlap it";
  if (!what) return TG_OK;
  snprintf(msg, sizeof(msg), "%s: %s", who, what);
  return einval(msg);
}

extern "C" int tg_gemv_fp8_rowdot_add(const uint8_t* x_q, const float* x_s, const uint8_t* w_q,
                                      const float* w_s, int w_scale_bn, const void* resid, void* out,
                                      int64_t M, int64_t N, int64_t K, int block_k, void* stream) {
  if (block_k != 128) return einval("block_k must be 128");
  TG_TRY(rowdot_common_checks("gemv_fp8_rowdot_add", M, N, K, w_scale_bn, w_q, w_s, out, kRowdotMaxK));
  if (M == 0 || N == 0) return TG_OK;
  if (!x_q || !x_s) return einval("gemv_fp8_rowdot_add: null pointer");
  if (!aligned(x_q, 16)) return einval("gemv_fp8_rowdot_add: operands must be 16-byte aligned");
  TG_TRY(rowdot_add_checks("gemv_fp8_rowdot_add", resid, out, M, N));
  RowdotIn in{};
  in.xq = x_q;
  in.xs = x_s;
  in.resid = reinterpret_cast<const __bf16*>(resid);
  auto o = reinterpret_cast<__bf16*>(out);
  hipStream_t st = as_stream(stream);
  if (M == 1) TG_TRY((launch_rowdot<1, PRO_X, true>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  else TG_TRY((launch_rowdot<2, PRO_X, true>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  return check_launch("gemv_fp8_rowdot_add");
}

extern "C" int tg_relu2_fp8_gemv_add(const void* u, const uint8_t* w_q, const float* w_s, int w_scale_bn,
                                     const void* resid, void* out, int64_t M, int64_t N, int64_t K,
                                     void* stream) {
  TG_TRY(rowdot_common_checks("relu2_fp8_gemv_add", M, N, K, w_scale_bn, w_q, w_s, out, kRowdotMaxK));
  if (M == 0 || N == 0) return TG_OK;
  if (!u) return einval("relu2_fp8_gemv_add: null pointer");
  if (!aligned(u, 16)) return einval("relu2_fp8_gemv_add: u must be 16-byte aligned");
  TG_TRY(rowdot_add_checks("relu2_fp8_gemv_add", resid, out, M, N));
  RowdotIn in{};
  in.x = reinterpret_cast<const uint4*>(u);
  in.resid = reinterpret_cast<const __bf16*>(resid);
  auto o = reinterpret_cast<__bf16*>(out);
  hipStream_t st = as_stream(stream);
  if (M == 1) TG_TRY((launch_rowdot<1, PRO_RELU2, true>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  else TG_TRY((launch_rowdot<2, PRO_RELU2, true>(in, w_q, w_s, w_scale_bn, o, (int)N, (int)K, st)));
  return check_launch("relu2_fp8_gemv_add");
}
