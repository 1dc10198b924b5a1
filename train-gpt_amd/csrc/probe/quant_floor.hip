// Measurement probe (not part of the product library): the I/O floor of the
// dual quantizer (quant_dual_kernel in ../quant_dual.h, the kernel behind
// tg_quantize_dual_km / tg_quantize_dual_pair_km).  The probe instantiates
// that same kernel with IO = true: every load, LDS access and store at the
// same addresses, widths and order, on the same grid and tile order, with
// the amax reductions, divides and e4m3 converts taken out.  bench.py
// --only quant_floor times it beside the product kernel on config 3's dY
// (8192 x 8192) and x + W pair.
//
// mode 0: the product's I/O including the K-block-major scale stores
// mode 1: the same without the scale stores
#include "../quant_dual.h"

extern "C" int tg_probe_quant_floor(int mode, const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0,
                                    float* s0, uint8_t* qt0, float* st0, const void* x1, int64_t rows1,
                                    int64_t cols1, uint8_t* q1, float* s1, uint8_t* qt1, float* st1,
                                    void* stream) {
  using namespace tg;
  if (mode < 0 || mode > 1) return einval("tg_probe_quant_floor: mode must be 0 or 1");
  if (rows0 <= 0 || cols0 <= 0 || rows0 % 128 || cols0 % 128 || rows1 < 0 || cols1 < 0 || rows1 % 128 ||
      cols1 % 128)
    return einval("tg_probe_quant_floor: extents must be positive multiples of 128 (tensor 1 may be empty)");
  if (!x0 || !q0 || !s0 || !qt0 || !st0) return einval("tg_probe_quant_floor: null pointer");
  DualJobs jobs{};
  TG_TRY(dual_job(jobs.job[0], "tg_probe_quant_floor", x0, rows0, cols0, q0, s0, qt0, st0, true, true));
  jobs.nblk0 = jobs.job[0].gx * jobs.job[0].gy;
  int64_t total = jobs.nblk0;
  if (rows1 > 0 && cols1 > 0) {
    if (!x1 || !q1 || !s1 || !qt1 || !st1) return einval("tg_probe_quant_floor: null pointer");
    TG_TRY(dual_job(jobs.job[1], "tg_probe_quant_floor", x1, rows1, cols1, q1, s1, qt1, st1,
                    jobs.nblk0 % 8 == 0, true));
    total += (int64_t)jobs.job[1].gx * jobs.job[1].gy;
  }
  auto st = static_cast<hipStream_t>(stream);
  if (mode == 0)
    hipLaunchKernelGGL((quant_dual_kernel<true, false, true, true>), dim3((unsigned)total), dim3(kDualThreads), 0,
                       st, jobs);
  else
    hipLaunchKernelGGL((quant_dual_kernel<true, false, true, false>), dim3((unsigned)total), dim3(kDualThreads), 0,
                       st, jobs);
  return check_launch("probe_quant_floor");
}
