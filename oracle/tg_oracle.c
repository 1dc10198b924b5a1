/*
 * C restatement of the reference's e4m3fn cast and 1x128 quantizer.
 * TEST INFRASTRUCTURE ONLY: used by tests/ for exhaustive sweeps and by
 * bench.py's cpu_baseline leg; never linked into the product library.
 *
 *   ora_e4m3fn_encode        astype(float8_e4m3fn), fp8.py:46 (OCP e4m3fn, RNE,
 *                            non-saturating: overflow and +-inf -> NaN)
 *   ora_quantize_rows_*      _quantize_to_fp8, fp8.py:39-47
 *   ora_rms_norm_quant_bf16  _rms_norm_pure (kernels.py:30-33) feeding
 *                            _quantize_to_fp8 (fp8.py:66)
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math: every
 * operation here is a single IEEE-754 f32/f64 operation).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint8_t ora_e4m3fn_encode(float v) {
    uint32_t bits = f2u(v);
    uint32_t sign = (bits >> 24) & 0x80u;
    uint32_t a = bits & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint8_t)(sign | 0x7Fu);      /* NaN, +-inf */
    int64_t code;
    if (a < 0x3C800000u) {                                       /* |v| < 2^-6 */
        /* 2^14 has f32 ulp 2^-9: the adder rounds |v| to the subnormal grid (RNE) */
        volatile float t = u2f(a) + 16384.0f;
        code = (int64_t)f2u(t) - (int64_t)f2u(16384.0f);
    } else {
        uint64_t rnd = ((uint64_t)a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20;
        code = (int64_t)rnd - (120 << 3);
    }
    if (code > 0x7E) code = 0x7F;                                /* above 448 after rounding */
    return (uint8_t)(sign | (uint32_t)code);
}

void ora_e4m3fn_encode_range(uint32_t start, uint64_t count, uint8_t* out) {
    for (uint64_t i = 0; i < count; ++i) out[i] = ora_e4m3fn_encode(u2f((uint32_t)(start + i)));
}

void ora_e4m3fn_encode_array(const float* v, int64_t n, uint8_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = ora_e4m3fn_encode(v[i]);
}

static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

static inline uint16_t f32_to_bf16(float f) {
    uint32_t b = f2u(f);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
    return (uint16_t)(((uint64_t)b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

/* amax with NaN propagation (jnp.max semantics) */
static inline float nan_max(float m, float v) {
    if (isnan(m) || isnan(v)) return NAN;
    return v > m ? v : m;
}

static void quantize_block(const float* x, int block, uint8_t* q, float* s) {
    float amax = 0.0f;
    for (int i = 0; i < block; ++i) amax = nan_max(amax, fabsf(x[i]));
    float sc = amax / 448.0f;
    if (!isnan(sc) && sc < 1e-30f) sc = 1e-30f;                  /* jnp.maximum(., 1e-30) */
    *s = sc;
    for (int i = 0; i < block; ++i) q[i] = ora_e4m3fn_encode(x[i] / sc);
}

void ora_quantize_rows_f32(const float* x, int64_t rows, int64_t cols, int block,
                           uint8_t* q, float* s) {
    int64_t nb = cols / block;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b)
            quantize_block(x + r * cols + b * block, block, q + r * cols + b * block, s + r * nb + b);
}

void ora_quantize_rows_bf16(const uint16_t* x, int64_t rows, int64_t cols, int block,
                            uint8_t* q, float* s) {
    float buf[1024];
    int64_t nb = cols / block;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t b = 0; b < nb; ++b) {
            const uint16_t* xs = x + r * cols + b * block;
            for (int i = 0; i < block; ++i) buf[i] = bf16_to_f32(xs[i]);
            quantize_block(buf, block, q + r * cols + b * block, s + r * nb + b);
        }
}

/* Column quantization: x (rows, cols) -> q (cols, rows), s (cols, rows/block):
 * the quantization of x.T along its last axis (fp8.py:68 applied to b). */
void ora_quantize_cols_bf16(const uint16_t* x, int64_t rows, int64_t cols, int block,
                            uint8_t* q, float* s) {
    float buf[1024];
    int64_t nb = rows / block;
    for (int64_t c = 0; c < cols; ++c)
        for (int64_t b = 0; b < nb; ++b) {
            for (int i = 0; i < block; ++i) buf[i] = bf16_to_f32(x[(b * block + i) * cols + c]);
            quantize_block(buf, block, q + c * rows + b * block, s + c * nb + b);
        }
}

/* _rms_norm_pure (kernels.py:30-33) + _quantize_to_fp8 of its bf16 output.
 * Sum of f32 squares accumulated in double (order-free to far below an f32
 * ulp), rounded to f32, divided by D in f32; rsqrt correctly rounded via
 * double.  bf16 rounding after each of rsqrt, x*r and t*gamma. */
void ora_rms_norm_quant_bf16(const uint16_t* x, const uint16_t* gamma, int64_t rows, int64_t D,
                             float eps, int block, uint16_t* y, uint8_t* q, float* s) {
    float buf[16384];
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* xr = x + r * D;
        double acc = 0.0;
        for (int64_t d = 0; d < D; ++d) {
            float v = bf16_to_f32(xr[d]);
            float sq = v * v;
            acc += (double)sq;
        }
        float var = (float)acc / (float)D;
        float ve = var + eps;
        float rs = (float)(1.0 / sqrt((double)ve));
        float rb = bf16_to_f32(f32_to_bf16(rs));
        for (int64_t d = 0; d < D; ++d) {
            float t = bf16_to_f32(f32_to_bf16(bf16_to_f32(xr[d]) * rb));
            uint16_t yb = f32_to_bf16(t * bf16_to_f32(gamma[d]));
            y[r * D + d] = yb;
            buf[d] = bf16_to_f32(yb);
        }
        if (q) {
            int64_t nb = D / block;
            for (int64_t b = 0; b < nb; ++b)
                quantize_block(buf + b * block, block, q + r * D + b * block, s + r * nb + b);
        }
    }
}
