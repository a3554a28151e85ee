/*
 * w8a8_oracle.c -- CPU restatement of the reference's W8A8 linear family.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels are
 * compared against; nothing in the product library links, loads or calls it.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * Plain C99, no dependencies, compiled with -O2 -ffp-contract=off so that every
 * float operation below is exactly one IEEE-754 binary32 operation in the
 * written order (the restatement must not be re-associated or contracted
 * unless a function says it contracts on purpose).
 *
 * Dtype codes follow the reference's output-code convention
 * (inference/src/cuda_linear.rs:488-497): 0 = fp32, 1 = fp16, 2 = bf16.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   bf16/fp16 rounding   exhaustive against numpy's float16 and a brute-force
 *                        nearest-even search; torch CPU casts.
 *   w8o_quant_rowwise    reference golden vectors (int8 + scale bytes) from
 *                        reference_primitives.py:357-365 and :388-391, and the
 *                        1386 + 504 + 612 + 1728 end-to-end CUDA payloads.
 *   w8o_gemm_i32         brute force in int64 (python ints) and the reference's
 *                        int8_mm golden vectors (reference_int8_linear.py:18-30).
 *   w8o_epilogue_kitchen reference CUDA payloads (GEMM/GEMV/M1 routes, all dtypes).
 *   w8o_epilogue_eager   reference eager_int8_linear CPU payloads.
 *   w8o_gelu_tanh        reference gelu_tanh activation payloads; every bf16 / fp16
 *                        value against ATen (equal outside the saturated tail);
 *                        its tanh against an 80-bit long double evaluation.
 *   w8o_residual         reference CUDA residual payloads (fused, unaligned and
 *                        eager residual modes of the GEMM, GEMV and M=1 routes).
 *   w8o_quant_tensorwise reference tensorwise golden vectors
 *                        (reference_primitives.py:357-365, deterministic cases).
 *   w8o_input_act        every 16-bit input of silu / sigmoid / tanh against ATen;
 *                        the SwiGLU and SiTU op chains against ATen on random
 *                        pairs; rms_norm against ATen within one ulp; the
 *                        reference's swiglu / situ / rms_norm CUDA payloads.
 *   w8o_convrot_quant_act the reference's ConvRot + activation CUDA payloads
 *                        (fast-math exp / tanh there: see the function).
 *   w8o_convrot_*        reference ConvRot CUDA payloads (fused group-256 route
 *                        and rotate-then-quantize route); the stage order against
 *                        a dense float64 Hadamard matmul (H built by Kronecker
 *                        products) and H.H^T = I.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define W8O_F32 0
#define W8O_F16 1
#define W8O_BF16 2

/* ------------------------------------------------------------------------ */
/* Floating-point storage conversions (round to nearest even).             */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

uint16_t w8o_f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float w8o_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t w8o_f32_to_f16(float f) {
    uint32_t u = f2u(f);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {                                    /* below 2^-14: subnormal half */
        /* value = a_float; half subnormal unit is 2^-24. */
        float v = u2f(a);
        /* exact scaling by 2^24 then round-half-even to integer */
        float s = v * 16777216.0f;                               /* exact (power of two) */
        float r = rintf(s);                                      /* default mode: half-even */
        return (uint16_t)(sign | (uint32_t)r);
    }
    uint32_t mant = a & 0x7fffffu;
    uint32_t exp = (a >> 23) - 127 + 15;
    uint32_t h = (exp << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1; /* carries into exponent correctly */
    return (uint16_t)(sign | h);
}

float w8o_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    if (exp == 0) {
        float v = (float)mant * (1.0f / 16777216.0f); /* exact */
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((exp - 15 + 127) << 23) | (mant << 13));
}

/* Load element i of a buffer of the given dtype as float (exact widening). */
static inline float load_as_f32(const void* p, int dtype, int64_t i) {
    switch (dtype) {
        case W8O_F16: return w8o_f16_to_f32(((const uint16_t*)p)[i]);
        case W8O_BF16: return w8o_bf16_to_f32(((const uint16_t*)p)[i]);
        default: return ((const float*)p)[i];
    }
}

/* Round a float to the given dtype and widen back (the value a tensor of that
 * dtype would hold). */
static inline float round_to(float v, int dtype) {
    switch (dtype) {
        case W8O_F16: return w8o_f16_to_f32(w8o_f32_to_f16(v));
        case W8O_BF16: return w8o_bf16_to_f32(w8o_f32_to_bf16(v));
        default: return v;
    }
}

static inline void store_from_f32(void* p, int dtype, int64_t i, float v) {
    switch (dtype) {
        case W8O_F16: ((uint16_t*)p)[i] = w8o_f32_to_f16(v); break;
        case W8O_BF16: ((uint16_t*)p)[i] = w8o_f32_to_bf16(v); break;
        default: ((float*)p)[i] = v; break;
    }
}

float w8o_round_to(float v, int dtype) { return round_to(v, dtype); }

/* ------------------------------------------------------------------------ */
/* GELU, tanh approximation, as ATen's CPU kernel orders it:
 *   0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3)))
 * Applied by the reference as input_act="gelu_tanh"
 * (inference/src/int8_linear.rs:37-41 -> x.gelu("tanh")).  Computed in fp32 for
 * 16-bit dtypes (ATen's opmath), result rounded to the tensor dtype.
 *
 * tanh itself is the correctly rounded fp32 value: the double-precision tanh
 * of the fp32 argument, rounded once to fp32.  A 1-ulp tanhf (glibc's, ATen's
 * vectorised one) rounds the same on nearly every argument; where they differ
 * the reference's own implementations differ from each other too (ATen's
 * vector tanh saturates to -1 a little early, so four bf16 inputs near -5.1
 * give -0 there instead of -1.5e-7).  The correctly rounded form is the one
 * both agree with elsewhere, and it is what this build binds to. */
float w8o_tanh_cr(float u) { return (float)tanh((double)u); }

float w8o_gelu_tanh(float x) {
    const float kBeta = (float)(1.41421356237309504880 * 1.12837916709551257390 * 0.5);
    const float kKappa = 0.044715f;
    float x_cube = x * x * x;
    float inner = kBeta * (x + kKappa * x_cube);
    return 0.5f * x * (1.0f + w8o_tanh_cr(inner));
}

/* ------------------------------------------------------------------------ */
/* Per-token dynamic absmax INT8 quantization.
 *
 * Follows inference/src/eager.rs:159-171 (quantize_int8_rowwise_with_seed, no
 * seed) with int8_scale_for_math (:94-109) and round_int8 (:110-121):
 *   s  = clamp_min(float(amax_k |x_k|) / 127, 1e-30)         IEEE division
 *   sT = dtype(s); if sT == 0: sT = tiny(dtype)
 *   q  = int8(clamp(round_half_even(dtype(float(x) / float(sT))), -128, 127))
 * scale_mode 1 replaces the scale by the Kitchen CUDA form
 * fmaxf(fminf(amax, finite_max) * (1/127f), 1e-30)
 * (native/comfy-port/kitchen/int8_linear.cu:36-39,205-208); the quotient
 * (int8_linear.cu:47-51,214) is the same IEEE form in both modes.
 * act 1 first applies gelu_tanh to x and rounds it to the dtype
 * (inference/src/int8_linear.rs:37-41 then :198-199).
 * x is [M, K] row-major; q is [M, K]; s is [M].  Finite inputs only. */
static float row_scale(float amax, int dtype, int scale_mode) {
    const float finite_max = dtype == W8O_F16 ? 65504.0f
                           : dtype == W8O_BF16 ? 3.38953139e38f : 3.40282347e38f;
    float scale;
    if (scale_mode == 1) {
        float a = amax < finite_max ? amax : finite_max;
        scale = a * (1.0f / 127.0f);
    } else {
        scale = amax / 127.0f;
    }
    if (!(scale >= 1e-30f)) scale = 1e-30f;
    return scale;
}

/* dtype(s), with the eager rule that a scale rounding to zero becomes tiny(dtype). */
static float scale_in_dtype(float scale, int dtype) {
    const float tiny = dtype == W8O_F16 ? 6.103515625e-5f : 1.17549435e-38f;
    float sT = round_to(scale, dtype);
    if (sT == 0.0f) sT = tiny;
    return sT;
}

/* int8(clamp(round_half_even(dtype(v / sT)), -128, 127)); v already in dtype. */
static int8_t quant_value(float v, float sT, int dtype) {
    float quot = round_to(v / sT, dtype);
    float r = rintf(quot); /* half-even in the default rounding mode */
    if (r < -128.0f) r = -128.0f;
    if (r > 127.0f) r = 127.0f;
    return (int8_t)r;
}

void w8o_quant_rowwise(const void* x, int dtype, int64_t M, int64_t K, int scale_mode,
                       int act, int8_t* q, float* s) {
    for (int64_t m = 0; m < M; ++m) {
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float v = load_as_f32(x, dtype, m * K + k);
            if (act == 1) v = round_to(w8o_gelu_tanh(v), dtype);
            float a = fabsf(v);
            if (a > amax) amax = a;
        }
        const float scale = row_scale(amax, dtype, scale_mode);
        s[m] = scale;
        const float sT = scale_in_dtype(scale, dtype);
        for (int64_t k = 0; k < K; ++k) {
            float v = load_as_f32(x, dtype, m * K + k);
            if (act == 1) v = round_to(w8o_gelu_tanh(v), dtype);
            q[m * K + k] = quant_value(v, sT, dtype);
        }
    }
}

/* Tensorwise INT8 quantization (inference/src/eager.rs:134-151; the CUDA
 * backend runs the same eager body, backend_bindings.rs:549-585):
 *   s = given ? *given : max(float(amax |x|) / 127, 1e-30)   (scale_mode 1:
 *       the amax * (1/127) form of w8o_quant_rowwise)
 *   q = int8(clamp(round_half_even(dtype(float(x) / float(sT))), -128, 127)),
 *       sT = dtype(s), a zero sT replaced by tiny(dtype).
 * x has n elements; *s receives the scale. */
void w8o_quant_tensorwise(const void* x, int dtype, int64_t n, const float* given, int scale_mode,
                          int8_t* q, float* s) {
    float scale;
    if (given) {
        scale = *given;
    } else {
        float amax = 0.0f;
        for (int64_t i = 0; i < n; ++i) {
            float a = fabsf(load_as_f32(x, dtype, i));
            if (a > amax) amax = a;
        }
        scale = row_scale(amax, dtype, scale_mode);
    }
    *s = scale;
    const float sT = scale_in_dtype(scale, dtype);
    for (int64_t i = 0; i < n; ++i) q[i] = quant_value(load_as_f32(x, dtype, i), sT, dtype);
}

/* ------------------------------------------------------------------------ */
/* ConvRot: a regular Hadamard rotation of every `group`-wide slice of a row,
 * y = x_g . H_G with H_G = (H4 (x) H4 (x) ... (x) H4) / sqrt(G) and
 * H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] (inference/src/
 * int8_utils.rs:21-58, rotate_activation :97-106).  G is a power of 4.
 *
 * Computed the way the reference's fused CUDA quantizer does it
 * (native/comfy-port/kitchen/int8_linear.cu:881-895 stages, :1270-1289 driver):
 * radix-4 stages at strides 1, 4, 16, ... in fp32, every output
 * 0.5f * (x0 + x1 + x2 - x3) (and the three other sign rows of H4) with the
 * operands added left to right.  The 0.5 of each stage makes up 1/sqrt(G). */
static void fht_group(float* v, int64_t G) {
    for (int64_t S = 1; S < G; S *= 4) {
        for (int64_t blk = 0; blk < G; blk += 4 * S) {
            for (int64_t j = 0; j < S; ++j) {
                float* p = v + blk + j;
                const float x0 = p[0], x1 = p[S], x2 = p[2 * S], x3 = p[3 * S];
                p[0] = 0.5f * (x0 + x1 + x2 - x3);
                p[S] = 0.5f * (x0 + x1 - x2 + x3);
                p[2 * S] = 0.5f * (x0 - x1 + x2 + x3);
                p[3 * S] = 0.5f * (-x0 + x1 + x2 + x3);
            }
        }
    }
}

/* Rotate-then-quantize route, rotation half (convrot.rs:474-484 with
 * int8_utils.rs:97-106): y = dtype(rotation of x), [M, K] -> [M, K] in the
 * same dtype.  `work` holds G floats. */
void w8o_convrot_rotate(const void* x, int dtype, int64_t M, int64_t K, int64_t G, void* y,
                        float* work) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t g = 0; g < K; g += G) {
            for (int64_t i = 0; i < G; ++i) work[i] = load_as_f32(x, dtype, m * K + g + i);
            fht_group(work, G);
            for (int64_t i = 0; i < G; ++i) store_from_f32(y, dtype, m * K + g + i, work[i]);
        }
    }
}

/* Fused rotation + quantization (quantize_int8_rowwise_convrot64_kernel,
 * native/comfy-port/kitchen/int8_linear.cu:1204-1314; G = 256):
 *   y    = rotation of x in fp32, NOT rounded to the dtype
 *   amax = max |y|;  s = scale of amax as in w8o_quant_rowwise (scale_mode)
 *   q    = int8(clamp(round_half_even(dtype(dtype(y) / dtype(s))), -128, 127))
 * (quant_div_float_to_float, int8_linear.cu:53-57).  `work` holds K floats. */
void w8o_convrot_quant(const void* x, int dtype, int64_t M, int64_t K, int64_t G,
                       int scale_mode, int8_t* q, float* s, float* work) {
    for (int64_t m = 0; m < M; ++m) {
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) work[k] = load_as_f32(x, dtype, m * K + k);
        for (int64_t g = 0; g < K; g += G) fht_group(work + g, G);
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(work[k]);
            if (a > amax) amax = a;
        }
        const float scale = row_scale(amax, dtype, scale_mode);
        s[m] = scale;
        const float sT = scale_in_dtype(scale, dtype);
        for (int64_t k = 0; k < K; ++k) q[m * K + k] = quant_value(round_to(work[k], dtype), sT, dtype);
    }
}

/* ------------------------------------------------------------------------ */
/* Input activations of the linear (act codes of Kitchen's input_act_codes.h,
 * SiTU = 4 as the crate passes it, convrot.rs:211-238):
 *   0 none, 1 gelu_tanh, 2 swiglu, 3 rms_norm, 4 situ.
 * SwiGLU and SiTU read a [gate | up] row twice as wide as the K they write.
 * exp and tanh are the correctly rounded fp32 values (double evaluation
 * rounded once); ATen's CPU silu, sigmoid and tanh equal them on every 16-bit
 * input (tests/test_oracle.py). */
static float exp_cr(float v) { return (float)exp((double)v); }
static float tanh_cr(float v) { return (float)tanh((double)v); }

/* Mean of squares of a row: the squares of 16-bit or fp32 values are exact in
 * double and their double sum is exact for rows of ordinary dynamic range, so
 * this is the exact mean rounded once to fp32 (any summation order gives it). */
static float row_mean_sq(const void* x, int dtype, int64_t base, int64_t K) {
    double acc = 0.0;
    for (int64_t k = 0; k < K; ++k) {
        const double v = (double)load_as_f32(x, dtype, base + k);
        acc += v * v;
    }
    return (float)(acc / (double)K);
}

/* The eager form (inference/src/int8_linear.rs:37-97): ATen ops on tensors of
 * the input dtype, each result rounded to it:
 *   gelu_tanh  T(gelu(x))
 *   swiglu     T(T(silu(a)) * b),  silu(a) = a / (1 + exp(-a))
 *   situ       T(T(T(tanh(T(a / 25))) * 25) * T(T(T(tanh(T(b / 4))) * 4) * T(sigmoid(b))))
 *   rms_norm   T(x * rstd * T(w)),  rstd = 1 / sqrt(mean(x^2) + eps)   (ATen's
 *              fused rms_norm: the weight applied in fp32, one rounding)
 * x is [M, K] or [M, 2K]; y is [M, K] in the dtype; weight [K] in the dtype. */
void w8o_input_act(const void* x, int dtype, int64_t M, int64_t K, int act, const void* weight, float eps,
                   void* y) {
    const int64_t in_w = (act == 2 || act == 4) ? 2 * K : K;
    for (int64_t m = 0; m < M; ++m) {
        const int64_t base = m * in_w;
        float rstd = 1.0f;
        if (act == 3) rstd = 1.0f / sqrtf(row_mean_sq(x, dtype, base, K) + eps);
        for (int64_t k = 0; k < K; ++k) {
            const float a = load_as_f32(x, dtype, base + k);
            float v = a;
            if (act == 1) {
                v = round_to(w8o_gelu_tanh(a), dtype);
            } else if (act == 2) {
                const float b = load_as_f32(x, dtype, base + K + k);
                v = round_to(round_to(a / (1.0f + exp_cr(-a)), dtype) * b, dtype);
            } else if (act == 4) {
                const float b = load_as_f32(x, dtype, base + K + k);
                const float t4 = round_to(round_to(tanh_cr(round_to(b / 4.0f, dtype)), dtype) * 4.0f, dtype);
                const float sg = round_to(1.0f / (1.0f + exp_cr(-b)), dtype);
                const float gated = round_to(t4 * sg, dtype);
                const float t25 = round_to(round_to(tanh_cr(round_to(a / 25.0f, dtype)), dtype) * 25.0f, dtype);
                v = round_to(t25 * gated, dtype);
            } else if (act == 3) {
                v = round_to((a * rstd) * load_as_f32(weight, dtype, k), dtype);
            }
            store_from_f32(y, dtype, m * K + k, v);
        }
    }
}

/* The fused form inside the ConvRot quantizer
 * (native/comfy-port/kitchen/int8_linear.cu:1175-1200,1230-1262): the activated
 * value stays in fp32 (no rounding to the dtype) and feeds the rotation:
 *   gelu_tanh  0.5 v (1 + tanh(sqrt(2/pi) (v + ((0.044715 v) v) v)))
 *   swiglu     (g / (1 + exp(-g))) * u
 *   situ       (tanh(a / 25) * 25) * ((tanh(b / 4) * 4) * (1 / (1 + exp(-b))))
 *   rms_norm   (v * rstd) * w,  rstd = 1 / sqrt(mean(v^2) + eps)
 * The reference compiles it with fast-math exp / tanh / rsqrt, which no
 * fixture tells from these correctly rounded ones (parity unpinned there). */
static float fused_act(const void* x, int dtype, int64_t base, int64_t K, int64_t k, int act,
                       const void* weight, float rstd) {
    const float a = load_as_f32(x, dtype, base + k);
    if (act == 1) {
        const float kBeta = (float)(1.41421356237309504880 * 1.12837916709551257390 * 0.5);
        const float inner = kBeta * (a + 0.044715f * a * a * a);
        return 0.5f * a * (1.0f + tanh_cr(inner));
    }
    if (act == 2) {
        const float u = load_as_f32(x, dtype, base + K + k);
        return (a / (1.0f + exp_cr(-a))) * u;
    }
    if (act == 4) {
        const float b = load_as_f32(x, dtype, base + K + k);
        return (tanh_cr(a / 25.0f) * 25.0f) * ((tanh_cr(b / 4.0f) * 4.0f) * (1.0f / (1.0f + exp_cr(-b))));
    }
    if (act == 3) return (a * rstd) * load_as_f32(weight, dtype, k);
    return a;
}

/* w8o_convrot_quant with a fused input activation: x is [M, K] or [M, 2K]. */
void w8o_convrot_quant_act(const void* x, int dtype, int64_t M, int64_t K, int64_t G, int scale_mode, int act,
                           const void* weight, float eps, int8_t* q, float* s, float* work) {
    const int64_t in_w = (act == 2 || act == 4) ? 2 * K : K;
    for (int64_t m = 0; m < M; ++m) {
        const int64_t base = m * in_w;
        float rstd = 1.0f;
        if (act == 3) rstd = 1.0f / sqrtf(row_mean_sq(x, dtype, base, K) + eps);
        for (int64_t k = 0; k < K; ++k) work[k] = fused_act(x, dtype, base, K, k, act, weight, rstd);
        for (int64_t g = 0; g < K; g += G) fht_group(work + g, G);
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) {
            float a = fabsf(work[k]);
            if (a > amax) amax = a;
        }
        const float scale = row_scale(amax, dtype, scale_mode);
        s[m] = scale;
        const float sT = scale_in_dtype(scale, dtype);
        for (int64_t k = 0; k < K; ++k) q[m * K + k] = quant_value(round_to(work[k], dtype), sT, dtype);
    }
}

/* ------------------------------------------------------------------------ */
/* C[m, n] = sum_k A[m, k] * B[n, k] in int32 (exact: |C| <= K * 128 * 127 <
 * 2^31 for K <= 132104).  A is [M, K], B is [N, K] row-major (the reference's
 * weight layout, cutlass_gemm_int8.cu:71-72 "B[N,K] row == [K,N] col"). */
void w8o_gemm_i32(const int8_t* A, const int8_t* B, int64_t M, int64_t N, int64_t K,
                  int32_t* C) {
    for (int64_t m = 0; m < M; ++m) {
        const int8_t* a = A + m * K;
        for (int64_t n = 0; n < N; ++n) {
            const int8_t* b = B + n * K;
            int32_t acc = 0;
            for (int64_t k = 0; k < K; ++k) acc += (int32_t)a[k] * (int32_t)b[k];
            C[m * N + n] = acc;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* The GPU routes' dequant epilogue, single rounding:
 *   out = O( (float(acc) * xs[m]) * ws[n] + float(bias[n]) )
 * CUTLASS EVT Mul0 -> Mul1 -> Add2 (cutlass_gemm_int8.cu:84-95), cuBLAS route
 * dequantize_int8_linear_kernel (int8_linear.cu:517-541) and the GEMV kernels
 * (int8_linear.cu:628-708).  bias is stored in the output dtype (the crate
 * converts it, cuda_linear.rs:694-697) and may be NULL.  ws has ws_size 1
 * (broadcast) or N entries.  contract = 1 evaluates the last multiply-add as
 * one fused multiply-add, fmaf(float(acc) * xs, ws, bias), which is how nvcc's
 * default --fmad=true compiles the reference's expression; contract = 0 rounds
 * the product first.  act 1 appends gelu_tanh on the output-dtype value,
 * out = O(gelu(float(O(lin)))), i.e. the next linear's input_act applied in
 * the output dtype (int8_linear.rs:37-41).  xs has M entries. */
void w8o_epilogue_kitchen(const int32_t* acc, const float* xs, const float* ws, int64_t ws_size,
                          const void* bias, void* out, int out_dtype, int64_t M, int64_t N,
                          int contract, int act) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            float w = ws[ws_size == 1 ? 0 : n];
            float b = bias ? load_as_f32(bias, out_dtype, n) : 0.0f;
            float t = (float)acc[m * N + n] * xs[m];
            float v = contract ? fmaf(t, w, b) : (t * w + b);
            if (act == 1) v = w8o_gelu_tanh(round_to(v, out_dtype));
            store_from_f32(out, out_dtype, m * N + n, v);
        }
    }
}

/* The CPU eager route's epilogue (inference/src/int8_linear.rs:240-269):
 *   chunk = O( float(acc) * (xs[m] * ws[n]) )      scales multiplied first
 *   out   = O( float(chunk) + float(O(bias[n])) )   bias added in the output dtype
 * bias is given as fp32 values (the reference converts whatever dtype it has
 * to the output dtype first, :263-269) and may be NULL. */
void w8o_epilogue_eager(const int32_t* acc, const float* xs, const float* ws, int64_t ws_size,
                        const float* bias, void* out, int out_dtype, int64_t M, int64_t N) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            float scale = xs[m] * ws[ws_size == 1 ? 0 : n];
            float v = round_to((float)acc[m * N + n] * scale, out_dtype);
            if (bias) v = round_to(v + round_to(bias[n], out_dtype), out_dtype);
            store_from_f32(out, out_dtype, m * N + n, v);
        }
    }
}

/* Residual step after the linear's output rounding, in the output dtype:
 *   out[m,n] = O( float(resid[m,n]) + float(out[m,n]) * float(rscale[n]) )
 * contract = 1: one fused multiply-add (a single fp32 rounding before O);
 * contract = 0: the product is rounded to fp32 before the add.
 * The reference's fused CUTLASS form (archived cutlass_gemm_int8.cu:122-188:
 * Add2 rounds the linear to the output type, Mul3 / Add4 in fp32, then O) and
 * its eager apply_residual (inference/src/int8_linear.rs:99-111: residual
 * .to(out).addcmul(out, scale.to(out))).  rscale has rs_size 1 or N entries;
 * resid is [M, N].  All three tensors are in the output dtype. */
void w8o_residual(void* out, const void* resid, const void* rscale, int64_t rs_size, int dtype,
                  int64_t M, int64_t N, int contract) {
    for (int64_t m = 0; m < M; ++m) {
        for (int64_t n = 0; n < N; ++n) {
            float o = load_as_f32(out, dtype, m * N + n);
            float r = load_as_f32(resid, dtype, m * N + n);
            float s = load_as_f32(rscale, dtype, rs_size == 1 ? 0 : n);
            float v = contract ? fmaf(o, s, r) : (r + o * s);
            store_from_f32(out, dtype, m * N + n, v);
        }
    }
}

/* Element-wise gelu_tanh on a tensor of the given dtype, result rounded to it. */
void w8o_gelu_tanh_tensor(const void* x, void* y, int dtype, int64_t count) {
    for (int64_t i = 0; i < count; ++i)
        store_from_f32(y, dtype, i, w8o_gelu_tanh(load_as_f32(x, dtype, i)));
}

/* Bulk dtype conversions for the Python side. */
void w8o_f32_to_bf16_n(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = w8o_f32_to_bf16(x[i]);
}
void w8o_f32_to_f16_n(const float* x, uint16_t* y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = w8o_f32_to_f16(x[i]);
}
