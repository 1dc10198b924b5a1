/*
 * tg_fp8.h -- C ABI of the MI355X (gfx950) FP8 hot path of train-gpt.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * passed as void*.  None allocates device memory, none synchronises the
 * host, and all work is enqueued on `stream`, so each is usable from an XLA
 * FFI handler (which receives its buffers and stream from XLA) or from a
 * ctypes/torch caller.  Return value: 0 on success, TG_EINVAL for a bad
 * argument (nothing is launched), TG_EHIP for a HIP launch failure;
 * tg_last_error() returns the calling thread's last message.
 *
 * Layouts are row-major and contiguous.  bf16 is passed as uint16_t bits,
 * e4m3fn bytes as uint8_t (OCP float8_e4m3fn, the gfx950 FP8 format).
 * block_k: the reference's block_scaled_matmul takes any block_k dividing K
 * (fp8.py:30-36, 55-56; DEFAULT_BLOCK_K = 128, fp8.py:27).  tg_quantize_rows,
 * tg_quantize_cols, tg_gemm_fp8_nt, tg_block_scaled_matmul and
 * tg_block_scaled_matmul_bwd_fp8 accept every block_k >= 1 that divides the
 * contracted extent: 128 runs the tuned kernels (two FP8 MFMA K steps per
 * scale block); other sizes quantize with the general kernels (bytes and
 * scales bit for bit those of the 128 path's contract).  The composites
 * (tg_block_scaled_matmul, tg_block_scaled_matmul_bwd_fp8) then run the
 * tuned GEMM for 16, 32, 64 (each block in a zero-filled 128-wide slot) and
 * multiples of 128 (the block's scale repeated per 128-wide sub-block, so the
 * f32 sum is folded once per sub-block and can differ from tg_gemm_fp8_nt at
 * the same block_k in the last bits), and the general GEMM (one P per block,
 * folded once) for every other size.  Every other entry point is a fused
 * kernel of this library and takes block_k == 128 only.
 *
 * Reference citations are /root/reference/<file>:<line>.
 */
#ifndef TG_FP8_H
#define TG_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { TG_OK = 0, TG_EINVAL = 1, TG_EHIP = 2 };
/* Element types of untyped operands.  TG_DTYPE_F16 is taken by tg_rms_norm_ex
 * and tg_rms_norm_bwd_ex only; every other entry point refuses it. */
enum { TG_DTYPE_BF16 = 0, TG_DTYPE_F32 = 1, TG_DTYPE_F16 = 2 };

/* Message for the calling thread's last non-zero return. */
const char* tg_last_error(void);

/* _quantize_to_fp8 (fp8.py:39-47) along the last axis.
 * x: (rows, cols) bf16 or f32; q: (rows, cols) e4m3fn; scales: (rows, cols/block_k) f32.
 * scale = max(amax/448, 1e-30); q = e4m3fn(x / scale).  cols % block_k == 0. */
int tg_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t cols, int block_k,
                     uint8_t* q, float* scales, void* stream);

/* _quantize_to_fp8 (fp8.py:39-47) of bf16(relu(x)^2) along the last axis: the
 * MLP activation of model.py:72 (jax.nn.relu(x @ w_up) ** 2 on bf16, the
 * square rounded once to bf16) fused with the quantization that feeds w_down.
 * x: (rows, cols) bf16; q, scales as tg_quantize_rows.  relu keeps NaN. */
int tg_quantize_rows_relu2(const void* x, int64_t rows, int64_t cols, int block_k, uint8_t* q,
                           float* scales, void* stream);

/* _quantize_to_fp8 of x.T (fp8.py:68 applies it to b.T, whatever b's float
 * dtype, after astype(f32)): quantizes the columns of x (rows, cols) and writes
 * them transposed: q_t: (cols, rows) e4m3fn; scales_t: (cols, rows/block_k)
 * f32.  x_dtype TG_DTYPE_BF16 or TG_DTYPE_F32; rows % block_k == 0; any cols.
 * bf16 with block_k == 128 runs the tuned tile kernel (16-byte loads when
 * cols % 8 == 0 and x is 16-byte aligned); f32 and other block sizes the
 * general one-thread-per-block kernel. */
int tg_quantize_cols(const void* x, int x_dtype, int64_t rows, int64_t cols, int block_k,
                     uint8_t* q_t, float* scales_t, void* stream);

/* Both of the above from one read of x: _quantize_to_fp8 (fp8.py:39-47) of x
 * along its rows and of x.T, the two forms of dY that the FP8 backward feeds to
 * its dX and dW GEMMs.  x (rows, cols) bf16, 16-byte aligned; rows and cols
 * multiples of block_k.  q (rows, cols) + scales (rows, cols/block_k) are
 * bit-identical to tg_quantize_rows, q_t (cols, rows) + scales_t
 * (cols, rows/block_k) to tg_quantize_cols. */
int tg_quantize_dual(const void* x, int64_t rows, int64_t cols, int block_k, uint8_t* q,
                     float* scales, uint8_t* q_t, float* scales_t, void* stream);

/* tg_quantize_dual of two tensors in one launch: the forward of fp8.py:50-78
 * quantizes both operands (fp8.py:66 a along K, fp8.py:68 b.T along K); with
 * the backward's forms kept from the same reads this is x along K + x.T along
 * M and W along N + W.T along K.  Each tensor's outputs are bit-identical to
 * tg_quantize_dual on it alone; a tensor with rows or cols 0 is skipped (its
 * pointers may then be null).  The two tensors' outputs must not overlap. */
int tg_quantize_dual_pair(const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0, float* scales0,
                          uint8_t* q_t0, float* scales_t0, const void* x1, int64_t rows1,
                          int64_t cols1, uint8_t* q1, float* scales1, uint8_t* q_t1,
                          float* scales_t1, int block_k, void* stream);

/* K-block-major scales.  The same quantizations (fp8.py:39-47, the bytes
 * bit-identical) with every scale array stored transposed: scales of x along
 * its rows as (cols/block_k, rows), scales of x.T as (rows/block_k, cols), i.e.
 * scales_km[kb * rows + r] == scales[r * (cols/block_k) + kb].  This is the
 * layout tg_gemm_fp8_nt_km reads (a K block's row scales contiguous), which the
 * composites below use internally; the reference's own layout is the one
 * above. */
int tg_quantize_dual_km(const void* x, int64_t rows, int64_t cols, int block_k, uint8_t* q,
                        float* scales_km, uint8_t* q_t, float* scales_t_km, void* stream);
int tg_quantize_dual_pair_km(const void* x0, int64_t rows0, int64_t cols0, uint8_t* q0,
                             float* scales0_km, uint8_t* q_t0, float* scales_t0_km, const void* x1,
                             int64_t rows1, int64_t cols1, uint8_t* q1, float* scales1_km,
                             uint8_t* q_t1, float* scales_t1_km, int block_k, void* stream);

/* jax.nn.scaled_matmul + bf16 cast as called at fp8.py:70-78 ("NT" layout):
 * c[m, n] = sum_kb a_s[m, kb] * b_s[n / b_scale_bn, kb] * sum_{k in kb} a_q[m, k] * b_q[n, k]
 * a_q: (M, K) e4m3fn, a_s: (M, K/block_k) f32; b_q: (N, K) e4m3fn;
 * b_s: (N, K/block_k) f32 when b_scale_bn == 1 (fp8.py:68's per-column scales)
 *      or (ceil(N/128), K/block_k) when b_scale_bn == 128 (128x128 weight tiles
 *      at block_k 128).
 * c: (M, N) bf16 (RNE, fp8.py:78) or f32 (c_dtype).  f32 accumulation.
 * block_k: any divisor of K (128: the tuned MFMA kernels). */
int tg_gemm_fp8_nt(const uint8_t* a_q, const float* a_s, const uint8_t* b_q, const float* b_s,
                   int b_scale_bn, void* c, int c_dtype, int64_t M, int64_t N, int64_t K,
                   int block_k, void* stream);

/* tg_gemm_fp8_nt (jax.nn.scaled_matmul, fp8.py:70-76) on K-block-major scales:
 * a_s_km (K/128, M) and b_s_km (K/128, N) (or (K/128, ceil(N/128)) when
 * b_scale_bn == 128), the transposes of tg_gemm_fp8_nt's a_s and b_s.  Same
 * kernels, same output bits; a K block's scales are read as contiguous runs. */
int tg_gemm_fp8_nt_km(const uint8_t* a_q, const float* a_s_km, const uint8_t* b_q,
                      const float* b_s_km, int b_scale_bn, void* c, int c_dtype, int64_t M, int64_t N,
                      int64_t K, int block_k, void* stream);

/* Device workspace (bytes) tg_block_scaled_matmul needs for its quantized operands. */
size_t tg_block_scaled_matmul_workspace(int64_t M, int64_t N, int64_t K, int block_k);

/* _fp8_forward (fp8.py:50-78) in one call: quantize a (M, K) and b.T (b is (K, N)),
 * then the scaled GEMM into out (M, N) bf16.  a and b are bf16; block_k any divisor of K.
 * workspace: >= tg_block_scaled_matmul_workspace(M, N, K, block_k) bytes, 256-B aligned. */
int tg_block_scaled_matmul(const void* a, const void* b, void* out, int64_t M, int64_t N,
                           int64_t K, int block_k, void* workspace, size_t workspace_bytes,
                           void* stream);

/* tg_block_scaled_matmul without a caller workspace, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  The quantized
 * operands live in a static device array of TG_NOALLOC_SCRATCH_BYTES (each
 * device this entry point has run on holds it from that first call until the
 * process ends), whose address is resolved once per device; the call
 * allocates nothing.  Shapes whose
 * workspace (tg_block_scaled_matmul_workspace) exceeds it return TG_EINVAL;
 * C3's forward (8192 x 2048 x 8192) needs 34.6 MB.  Output bits equal
 * tg_block_scaled_matmul's.  All calls on one device share the array: calls
 * that overlap on one device (different streams, or host threads) race;
 * serialize them.  a, b 16-byte aligned; block_k 128. */
#define TG_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int tg_block_scaled_matmul_noalloc(const void* a, const void* b, void* out, int64_t M, int64_t N,
                                   int64_t K, int block_k, void* stream);

/* Device workspace (bytes) of tg_block_scaled_matmul_bwd_fp8. */
size_t tg_block_scaled_matmul_bwd_workspace(int64_t M, int64_t N, int64_t K, int block_k);

/* FP8 backward of block_scaled_matmul (the custom_vjp of fp8.py:81-101 with
 * the forward's quantize -> scaled GEMM composition reused for both
 * gradients; fp8.py:85-98 itself is the bf16 straight-through rule):
 *   da (M, K) = fwd(g, b.T):  g row-quantized along N, b row-quantized along N
 *   db (K, N) = fwd(a.T, g):  a.T and g.T quantized along M
 * a: (M, K), b: (K, N), g: (M, N), all bf16; da, db bf16.  block_k any
 * divisor of K; M and N multiples of block_k (a caller pads a ragged last
 * block with zeros, which change neither amax nor any product).  M == 0 or
 * N == 0: the gradient that sums over the empty extent is written as zeros
 * (db with M == 0, da with N == 0); only an empty gradient's pointer may be
 * null, and a, b, g, workspace are not read. */
int tg_block_scaled_matmul_bwd_fp8(const void* a, const void* b, const void* g, void* da,
                                   void* db, int64_t M, int64_t N, int64_t K, int block_k,
                                   void* workspace, size_t workspace_bytes, void* stream);

/* The bf16 dot of the straight-through backward (fp8.py:95-96, `x @ y` on bf16
 * operands): c (M, N) = bf16(sum_k a[m, k] * b[n, k]) with fp32 accumulation.
 * a (M, K), b (N, K), c (M, N), all bf16 row-major; K % 64 == 0; a and b
 * 16-byte aligned and each below 2 GiB. */
int tg_gemm_bf16_nt(const void* a, const void* b, void* c, int64_t M, int64_t N, int64_t K,
                    void* stream);

/* The `.astype(jnp.bfloat16)` operand casts of fp8.py:92-94 (RNE for f32),
 * optionally transposed (the `a_2d.T` of fp8.py:96), into rows padded with
 * zeros to `pitch` elements:
 *   transpose = 0: x (rows, cols) -> y (rows, pitch), pitch >= cols
 *   transpose = 1: x (rows, cols) -> y (cols, pitch), pitch >= rows
 * x_dtype: TG_DTYPE_BF16 or TG_DTYPE_F32; y bf16. */
int tg_pack_bf16(const void* x, int x_dtype, int64_t rows, int64_t cols, int transpose, void* y,
                 int64_t pitch, void* stream);

/* Device workspace (bytes) of tg_block_scaled_matmul_bwd_bf16. */
size_t tg_block_scaled_matmul_bwd_bf16_workspace(int64_t M, int64_t N, int64_t K);

/* _fp8_backward (fp8.py:85-98), the reference's straight-through rule:
 *   da (M, K) = bf16(g) @ bf16(b).T      db (K, N) = bf16(a).T @ bf16(g)
 * a (M, K), b (K, N), g (M, N), each bf16 or f32 (its *_dtype); da, db bf16
 * (the caller widens to a.dtype / b.dtype as fp8.py:95-96 does).  Any M, N, K;
 * an empty contraction writes zero gradients. */
int tg_block_scaled_matmul_bwd_bf16(const void* a, int a_dtype, const void* b, int b_dtype,
                                    const void* g, int g_dtype, void* da, void* db, int64_t M,
                                    int64_t N, int64_t K, void* workspace, size_t workspace_bytes,
                                    void* stream);

/* _rms_norm_pure (kernels.py:30-33) over the last axis of x (rows, dim) bf16,
 * scale (dim,) bf16, y (rows, dim) bf16:
 * r = bf16(rsqrt(mean(x^2) + eps)); y = bf16(bf16(x * r) * scale).
 * Replaces the Pallas rms_norm_gpu forward (kernels.py:41-99) on ROCm. */
int tg_rms_norm(const void* x, const void* scale, void* y, int64_t rows, int64_t dim, float eps,
                void* stream);

/* _rms_norm_pure (kernels.py:30-33) for any float dtypes: x (rows, dim) and
 * scale (dim,) each bf16, f16 or f32 (x_dtype / scale_dtype); y (rows, dim) is
 * in their common dtype when they agree, else f32 (jnp's promotion of
 * x_n * scale: bf16 with f16 gives f32).
 * r = rsqrt(mean(x^2) + eps) rounded to x's dtype, x_n = x * r rounded to
 * x's dtype, y = x_n * scale.  Any dim; bf16/bf16 takes tg_rms_norm's kernel. */
int tg_rms_norm_ex(const void* x, int x_dtype, const void* scale, int scale_dtype, void* y,
                   int64_t rows, int64_t dim, float eps, void* stream);

/* Fused RMSNorm -> FP8 quantize (the composition of kernels.py:30-33 and
 * fp8.py:39-47 on the bf16 norm output, from one read of x):
 * y (rows, dim) bf16, q (rows, dim) e4m3fn, s (rows, dim/block_k) f32. */
int tg_rms_norm_fp8(const void* x, const void* scale, void* y, uint8_t* q, float* s,
                    int64_t rows, int64_t dim, float eps, int block_k, void* stream);

/* The residual add of model.py:75-76 fused with the next norm -> FP8 quantize:
 * x_out = bf16(x + delta) (the bf16 tensor add), then y = _rms_norm_pure(x_out,
 * scale, eps) (kernels.py:30-33) and (q, s) = _quantize_to_fp8(f32(y))
 * (fp8.py:39-47), exactly as tg_rms_norm_fp8 on x_out.  x_out may be x (in
 * place); y may be NULL.  Shapes and alignment as tg_rms_norm_fp8. */
int tg_add_rms_norm_fp8(const void* x, const void* delta, const void* scale, void* x_out, void* y,
                        uint8_t* q, float* s, int64_t rows, int64_t dim, float eps, int block_k,
                        void* stream);

/* Device workspace (bytes) of tg_rms_norm_bwd. */
size_t tg_rms_norm_bwd_workspace(int64_t rows, int64_t dim);

/* rms_norm's backward, the custom VJP _bwd of kernels.py:104-118:
 *   rnorm = rsqrt(mean(x^2) + eps), normed = x * rnorm, gs = dy * scale
 *   dx = bf16(rnorm * (gs - normed * mean(gs * normed)))   (rows, dim)
 *   dscale = bf16(sum over rows of dy * normed)            (dim,)
 * x, dy, dx bf16 (rows, dim); scale, dscale bf16 (dim,); dim % 8 == 0 (widths
 * above 4096 take tg_rms_norm_bwd_ex's general kernels).  dscale is summed in
 * a fixed order (identical on every call); rows == 0 gives dscale = 0. */
int tg_rms_norm_bwd(const void* x, const void* scale, const void* dy, void* dx, void* dscale,
                    int64_t rows, int64_t dim, float eps, void* workspace, size_t workspace_bytes,
                    void* stream);

/* The same backward for any float dtypes: x, scale, dy each bf16, f16 or f32 (their
 * *_dtype codes); dx is written in x's dtype, dscale in scale's (the
 * .astype(x.dtype) / .astype(scale.dtype) of kernels.py:115-117); any dim.
 * Workspace as tg_rms_norm_bwd_workspace. */
int tg_rms_norm_bwd_ex(const void* x, int x_dtype, const void* scale, int scale_dtype, const void* dy,
                       int dy_dtype, void* dx, void* dscale, int64_t rows, int64_t dim, float eps,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Decode-shape GEMM with a pre-quantized weight (no reference function; the
 * reference re-quantizes W every call at fp8.py:68):
 * out[m, n] = sum_kb x_s[m, kb] * w_s[n / w_scale_bn, kb] * sum_k x_q[m, k] * w_q[n, k]
 * x_q (M, K), x_s (M, K/128); w_q (N, K), w_s as b_s of tg_gemm_fp8_nt;
 * out (M, N) bf16.  M <= 64; 33-64 rows run tg_gemm_fp8_nt's kernel (one pass
 * over W instead of two 32-row passes). */
int tg_gemv_fp8(const uint8_t* x_q, const float* x_s, const uint8_t* w_q, const float* w_s,
                int w_scale_bn, void* out, int64_t M, int64_t N, int64_t K, int block_k,
                void* stream);

/* The same product for one or two activation rows (M <= 2, K <= 16384) on the
 * VALU: each 128-wide block's sum is an f32 fma chain instead of the MFMA's
 * arithmetic, so the result agrees with tg_gemv_fp8 to rounding (not bit for
 * bit).  Faster for single-token decode: W streams through registers with no
 * LDS staging.  Arguments as tg_gemv_fp8. */
int tg_gemv_fp8_rowdot(const uint8_t* x_q, const float* x_s, const uint8_t* w_q, const float* w_s,
                       int w_scale_bn, void* out, int64_t M, int64_t N, int64_t K, int block_k,
                       void* stream);

/* Decode-step fusions of the norm / activation that feeds a GEMV (no
 * reference counterpart: generate.py runs model.forward per token; these fuse
 * model.py:61-62 / 71 with the projection that follows, for one or two rows):
 *
 * tg_rms_norm_fp8_gemv: h = the FP8 rows (bytes and 1x128 scales) that
 * tg_rms_norm_fp8 (delta == NULL) or tg_add_rms_norm_fp8 (delta != NULL) would
 * produce from x (M, K) bf16, gamma (K,) bf16 and eps, bit for bit; then
 * out (M, N) = h @ W^T, as tg_gemv_fp8_rowdot for M <= 2 (K <= 4096) and as
 * tg_gemv_fp8 (the MFMA GEMV, the same bits) for 3 <= M <= 16 (K <= 2560).
 * With delta, the residual sum bf16(x + delta) is also stored to xout (M, K),
 * which must not overlap x or delta.  K % 128 == 0; x, delta, gamma, xout
 * 16-byte aligned.  Replaces the norm launch + the GEMV launch of a decode
 * step.
 *
 * tg_relu2_fp8_gemv: h = the FP8 rows tg_quantize_rows_relu2 would produce
 * from u (M, K) bf16 (model.py:72's relu^2), then out = h @ W^T as
 * tg_gemv_fp8_rowdot.  M <= 2, K <= 16384. */
int tg_rms_norm_fp8_gemv(const void* x, const void* delta, const void* gamma, float eps, void* xout,
                         const uint8_t* w_q, const float* w_s, int w_scale_bn, void* out, int64_t M,
                         int64_t N, int64_t K, void* stream);
int tg_relu2_fp8_gemv(const void* u, const uint8_t* w_q, const float* w_s, int w_scale_bn, void* out,
                      int64_t M, int64_t N, int64_t K, void* stream);

/* The residual adds of model.py:75-76 (x = x + attn(...), x = x + mlp(...))
 * fused into the decode GEMV that produces their term (no reference
 * counterpart; one or two rows): out (M, N) = bf16(resid + bf16(h @ W^T)),
 * h from x_q / x_s as tg_gemv_fp8_rowdot or from relu(u)^2 as
 * tg_relu2_fp8_gemv; the same bits as that entry point followed by the bf16
 * tensor add (f32 sum of the two bf16 values, rounded once).  resid (M, N)
 * bf16, 2-byte aligned; out may be resid itself (the residual stream updated
 * in place), any other overlap is refused.  M <= 2, K <= 16384.  The norm that
 * follows then needs no add of its own (tg_rms_norm_fp8_gemv, delta == NULL). */
int tg_gemv_fp8_rowdot_add(const uint8_t* x_q, const float* x_s, const uint8_t* w_q, const float* w_s,
                           int w_scale_bn, const void* resid, void* out, int64_t M, int64_t N, int64_t K,
                           int block_k, void* stream);
int tg_relu2_fp8_gemv_add(const void* u, const uint8_t* w_q, const float* w_s, int w_scale_bn,
                          const void* resid, void* out, int64_t M, int64_t N, int64_t K, void* stream);

/* Quantize W.T into the pre-quantized weight format with one scale per
 * 128x128 tile (w_scale_bn == 128).  w: (K, N) bf16; w_q (N, K); w_s (ceil(N/128), K/128). */
int tg_quantize_weight_128x128(const void* w, int64_t K, int64_t N, uint8_t* w_q, float* w_s,
                               void* stream);

/* Test support: compares the hardware e4m3fn convert with the integer
 * encoder over every f32 bit pattern.  counts[0] = mismatches with
 * |v| <= 448*(1+2^-12) (covering the range quantization produces), counts[1] =
 * mismatches elsewhere (finite), counts[2] = mismatches for NaN/inf inputs.
 * counts must point to 3 device uint64_t (zeroed by the call). */
int tg_selftest_fp8_cvt(uint64_t* counts, void* stream);

/* Test support: compares the quantizers' bf16 arithmetic with IEEE f32
 * operations for every bf16 amax and every bf16 x with |x| <= amax.
 * counts[0] = e4m3fn byte mismatches of the refined divide, counts[1] = f32
 * quotient mismatches with |x/s| > 2^-10, counts[2] = quotient mismatches at
 * or below 2^-10 (which encode to +-0 either way), counts[3] = refined scale
 * amax/448 != IEEE, counts[4] = refined reciprocal != IEEE 1/s.
 * 5 device uint64_t, zeroed by the call. */
int tg_selftest_divide(uint64_t* counts, void* stream);

/* One decode step of the attention of model.py:59-68 over a KV cache, for one
 * new token per sequence at position t = *t_pos (device memory, 0 <= t < S; so a
 * captured graph serves every position), fused with the cache append and the
 * FP8 quantization of the output (the input of the output projection):
 *   k_cache[b, h, t] = k[b, h];  v_cache[b, h, t] = v[b, h]
 *   o[b, h] = softmax(q[b, h] . k_cache[b, h, 0..t]^T * scale) v_cache[b, h, 0..t]
 *   (o_q, o_s) = _quantize_to_fp8(bf16(o))  (fp8.py:39-47; one scale per head)
 * qkv: (B, 3 * H * head_dim) bf16, row b = [q | k | v] (the fused projection);
 * k_cache, v_cache: (B, H, S, head_dim) bf16; o_q: (B, H * head_dim) e4m3fn;
 * o_s: (B, H) f32; o: (B, H * head_dim) bf16 or NULL.  head_dim must be 128.
 * Replaces the per-token full-context recompute of generate.py:166-171 (with
 * cuDNN attention inside model.forward, model.py:67).  A t outside [0, S)
 * touches no memory and writes NaN scales. */
int tg_decode_attention(const void* qkv, void* k_cache, void* v_cache, const int64_t* t_pos,
                        uint8_t* o_q, float* o_s, void* o, int64_t B, int64_t H, int64_t S,
                        int64_t head_dim, float scale, void* stream);

/* The logit cap of model.py:97 on bf16 logits: out (n,) f32 = cap * tanh(l / cap)
 * with torch's arithmetic for `cap * torch.tanh(l.float() / cap)` (l times the
 * f32 reciprocal of cap, the device tanhf, one f32 multiply), the same bits in
 * one launch.  For the decode step's unembedding rows (the reference applies
 * the cap inside model.forward, generate.py:166-171).  cap finite and > 0. */
int tg_logit_cap(const void* logits, float* out, int64_t n, float cap, void* stream);

/* The decode step's input rows, model.py:89-90 for one token per sequence:
 * out[b] (d) bf16 = bf16(embed[tok[b]] + pos[t]) (the f32 sum of the two bf16
 * values, rounded once: torch's bf16 add), with tok (B,) and t (1,) int64 in
 * device memory (a captured graph serves every token).  embed (V, d) and pos
 * (P, d) bf16, d a multiple of 8.  A token or position outside its table
 * reads a zero row (no fault; torch's indexing would assert). */
int tg_decode_embed(const void* embed, const void* pos, const int64_t* tok, const int64_t* t, void* out,
                    int64_t B, int64_t V, int64_t P, int64_t d, void* stream);

/* Logit cap + cross entropy, forward: for each row r of the bf16 logits
 * (rows, vocab) and target t = targets[r],
 *   z = cap * tanh(l / cap)   (f32; model.py:96-97 with config.logit_cap)
 *   row_lse[r]  = log sum_v exp(z_v)
 *   row_loss[r] = row_lse[r] - z_t      (losses.py:8-12 before the mean)
 * Replaces the f32 cast, tanh, log_softmax and take_along_axis passes of
 * losses.py:8-12 over the model output.  A target outside [0, vocab) gives
 * a NaN row loss.  row_loss, row_lse: (rows,) f32. */
int tg_logit_cap_xent_fwd(const void* logits, const int64_t* targets, int64_t rows, int64_t vocab,
                          float cap, float* row_loss, float* row_lse, void* stream);

/* Logit cap + cross entropy, backward (the autodiff of losses.py:8-12, or of
 * the masked mean of losses.py:15-34, through model.py:97): with
 * g_r = *g * g_scale * row_weight[r] (g in device memory, so the upstream
 * gradient needs no host read; row_weight NULL means 1; g_scale = 1 / rows
 * for the mean; row_weight = mask / max(sum mask, 1) for the masked mean),
 *   dlogits = bf16(g_r * (exp(z - row_lse) - onehot(t)) * (1 - (z / cap)^2))
 * dlogits: (rows, vocab) bf16; it may not alias logits. */
int tg_logit_cap_xent_bwd(const void* logits, const int64_t* targets, const float* row_lse,
                          const float* g, float g_scale, const float* row_weight, int64_t rows,
                          int64_t vocab, float cap, void* dlogits, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* TG_FP8_H */
