/* Exhaustive check of the quantizer's division (used by tests/test_divide.py).
 *
 * The HIP quantizers form the int8 code of a 16-bit input x and the row's
 * divisor d = T(s) from q0 = RN(x * r), r = RN(1 / d)
 * (imagine_amd/csrc/w8a8_common.h, code_quotient).  This program compares
 * that, and the one-fma-corrected quotient q = RN(fma(RN(fma(-q0, d, x)), r, q0)),
 * with the IEEE quotient for every pair the quantizer can see:
 * every reachable 16-bit divisor d and every finite 16-bit x with
 * |x| <= 128 * d (a row's elements never exceed amax, and d >= amax/127 up to
 * one 16-bit rounding).  Sign symmetry covers negative x.  Requirements: the
 * final int8 code clamp(rint(T(q))) equals the IEEE one for every pair, and
 * the fp32 quotient itself is identical whenever x and x/d are >= 2^-100 (else the
 * fma remainder or the quotient is subnormal and loses bits; the quotient
 * is then below 2^-70 and both codes are 0).  Also required: the code from the
 * uncorrected product q0 = RN(x * r) alone equals the IEEE code for every pair
 * (the kernels that only need the int8 code use q0).  Prints mismatch counts;
 * exit 0 iff none.
 * Usage: divide_check bf16|f16
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static float bf16_val(uint16_t h) { return u2f((uint32_t)h << 16); }
static float f16_val(uint16_t h) {
    uint32_t exp = (h >> 10) & 0x1f, mant = h & 0x3ff;
    if (exp == 0) return (float)mant * (1.0f / 16777216.0f);
    if (exp == 31) return INFINITY;
    return u2f(((exp - 15 + 127) << 23) | (mant << 13));
}

static float round16(float v, int bf) {
    uint32_t u = f2u(v);
    if (bf) {
        u += 0x7fffu + ((u >> 16) & 1u);
        return u2f(u & 0xffff0000u);
    }
    /* fp16 RNE of a value in the quantizer's range (|v| <= 128): go through
     * the exact half grid with rintf at the right scale */
    float a = fabsf(v);
    if (a < 6.103515625e-05f) { /* subnormal half: unit 2^-24 */
        float r = rintf(a * 16777216.0f) / 16777216.0f;
        return v < 0 ? -r : r;
    }
    int e;
    frexpf(a, &e);                       /* a = m * 2^e, m in [0.5, 1) */
    float unit = ldexpf(1.0f, e - 11);   /* half has 11 significant bits */
    float r = rintf(a / unit) * unit;    /* a / unit exact (power of two) */
    return v < 0 ? -r : r;
}

static int code(float q, int bf) {
    float v = rintf(round16(q, bf));
    if (v < -128.0f) v = -128.0f;
    if (v > 127.0f) v = 127.0f;
    return (int)v;
}

int main(int argc, char** argv) {
    int bf = argc > 1 && strcmp(argv[1], "bf16") == 0;
    long long pairs = 0, bad_code = 0, bad_quot = 0, bad_prod = 0;
    for (uint32_t dh = 1; dh < 0x7f80u; ++dh) {
        float d = bf ? bf16_val((uint16_t)dh) : f16_val((uint16_t)dh);
        if (!bf && dh >= 0x7c00u) break; /* f16 inf/nan */
        if (!(d > 0.0f) || isinf(d)) continue;
        /* reachable divisors: T(s) with 1e-30 <= s <= T_max / 127 (a zero T(s)
         * becomes T's tiny, itself in range) */
        if (bf && (d < bf16_val(0x0da2u) || d > 3.38953139e38f / 127.0f * 1.01f)) continue;
        volatile float r = 1.0f / d;
        float lim = 128.0f * d;
        uint32_t xmax = bf ? 0x7f80u : 0x7c00u;
        for (uint32_t xh = 0; xh < xmax; ++xh) {
            float x = bf ? bf16_val((uint16_t)xh) : f16_val((uint16_t)xh);
            if (x > lim) break; /* positive 16-bit values are ordered by bits */
            float q0 = x * r;
            float e = fmaf(-q0, d, x);
            float q = fmaf(e, r, q0);
            float ref = x / d;
            ++pairs;
            if (code(q, bf) != code(ref, bf)) {
                if (bad_code < 10) printf("code mismatch d=%a x=%a got=%a want=%a\n", d, x, q, ref);
                ++bad_code;
            }
            if (code(q0, bf) != code(ref, bf)) {
                if (bad_prod < 10) printf("product code mismatch d=%a x=%a got=%a want=%a\n", d, x, q0, ref);
                ++bad_prod;
            }
            if (x >= 0x1p-100f && ref >= 0x1p-100f && f2u(q) != f2u(ref)) {
                if (bad_quot < 10) printf("quotient mismatch d=%a x=%a got=%a want=%a\n", d, x, q, ref);
                ++bad_quot;
            }
        }
    }
    printf("%s pairs=%lld code_mismatches=%lld quotient_mismatches=%lld product_code_mismatches=%lld\n",
           bf ? "bf16" : "f16", pairs, bad_code, bad_quot, bad_prod);
    return (bad_code != 0 || bad_quot != 0 || bad_prod != 0);
}
