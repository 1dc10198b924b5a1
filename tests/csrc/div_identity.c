/*
 * Exhaustive host check of the arithmetic the gfx950 quantizers use for
 * bf16-valued inputs (train-gpt_amd/csrc/tg_device.h):
 *   scale:  q0 = a*c (c = fl(1/448)); r = fma(-q0, 448, a); s = fma(r, c, q0),
 *           floored at 1e-30                              (block_scale_bf16)
 *   divide: y = fl(1/s); q0 = x*y; nr = fma(q0, s, -x); q = fma(-nr, y, q0)
 *                                                         (Divider::div)
 * against IEEE a/448 and x/s, for every bf16 amax a and every bf16 x (both
 * signs) with |x| <= a -- the only (x, s) pairs the row/column/norm
 * quantizers form.  (The device's reciprocal is checked against IEEE 1/s by
 * tg_selftest_divide.)
 *
 * Printed "pairs enc_mismatch q_mismatch_above q_mismatch_below scale_mismatch":
 *   enc_mismatch        e4m3fn bytes of q and x/s differ       (must be 0)
 *   q_mismatch_above    f32 q != x/s with |x/s| >  2^-10        (must be 0)
 *   q_mismatch_below    f32 q != x/s with |x/s| <= 2^-10        (reported;
 *                       both encode to +-0 there)
 *   scale_mismatch      refined scale != IEEE scale            (must be 0)
 * Compile with -O2 -mfma -ffp-contract=off.  The operands pass through
 * volatile so that the compiler keeps each fma exactly as written: gcc
 * otherwise rewrites -fma(a, b, c) as fnmsub -(a*b) - c, which differs in
 * the sign of a zero result.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* OCP e4m3fn, RNE, non-saturating (same rule as oracle/tg_oracle.c) */
static uint8_t enc(float v) {
    uint32_t bits = f2u(v), sign = (bits >> 24) & 0x80u, a = bits & 0x7FFFFFFFu;
    if (a >= 0x7F800000u) return (uint8_t)(sign | 0x7Fu);
    int64_t code;
    if (a < 0x3C800000u) {
        volatile float t = u2f(a) + 16384.0f;
        code = (int64_t)f2u(t) - (int64_t)f2u(16384.0f);
    } else {
        code = (int64_t)(((uint64_t)a + 0x7FFFFu + ((a >> 20) & 1u)) >> 20) - 960;
    }
    if (code > 0x7E) code = 0x7F;
    return (uint8_t)(sign | (uint32_t)code);
}

static float scale_refined(float a) {
    volatile float c = 1.0f / 448.0f, m = 448.0f;
    const float q0 = a * c;
    const float r = __builtin_fmaf(-q0, m, a);
    float s = __builtin_fmaf(r, c, q0);
    if (isinf(a)) s = a;
    return s < 1e-30f ? 1e-30f : s;
}

int main(int argc, char** argv) {
    uint32_t a_lo = 0, a_hi = 0x7F7F;      /* positive finite bf16 patterns */
    if (argc == 3) { a_lo = (uint32_t)strtoul(argv[1], 0, 0); a_hi = (uint32_t)strtoul(argv[2], 0, 0); }
    unsigned long long pairs = 0, bad_enc = 0, bad_hi = 0, bad_lo = 0, bad_scale = 0;
    for (uint32_t ab = a_lo; ab <= a_hi; ++ab) {
        const float a = u2f(ab << 16);
        float s_ieee = a / 448.0f;
        if (s_ieee < 1e-30f) s_ieee = 1e-30f;
        const float s = scale_refined(a);
        if (f2u(s) != f2u(s_ieee)) ++bad_scale;
        const float y = 1.0f / s;
        for (uint32_t xb = 0; xb <= ab; ++xb) {
            for (uint32_t sign = 0; sign < 2; ++sign) {
                volatile float xv = u2f((xb << 16) | (sign << 31));
                const float x = xv;
                const float q0 = x * y;
                volatile float nx = -x, vs = s;
                volatile float nr = __builtin_fmaf(q0, vs, nx);   /* stored: not fused into its negation */
                const float nnr = -nr;
                volatile float vy = y;
                const float q = __builtin_fmaf(nnr, vy, q0);
                const float ref = x / s;
                ++pairs;
                if (enc(q) != enc(ref)) {
                    if (bad_enc < 5) fprintf(stderr, "byte mismatch a=%08x x=%08x q=%08x ref=%08x\n",
                                             f2u(a), f2u(x), f2u(q), f2u(ref));
                    ++bad_enc;
                }
                if (f2u(q) != f2u(ref)) {
                    if (fabsf(ref) > 0x1p-10f) ++bad_hi; else ++bad_lo;
                }
            }
        }
    }
    printf("%llu %llu %llu %llu %llu\n", pairs, bad_enc, bad_hi, bad_lo, bad_scale);
    return 0;
}
