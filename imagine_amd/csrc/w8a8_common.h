// Shared device helpers for the gfx950 W8A8 kernels.
//
// All float arithmetic here is IEEE binary32 in the written order: the library
// is compiled with -ffp-contract=off and every fused multiply-add is spelled
// out as fmaf.  Conversions to 16-bit types round to nearest even.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "w8a8.h"
#include "w8a8_gelu_tables.h"  // generated at build time (imagine_amd/gelu_tables.py)

namespace w8a8 {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- streaming memory access

// Non-temporal (streaming) 16-byte global load, for data a kernel reads
// once: the instruction carries the nt cache policy, so the lines are not
// kept in L2 / the Infinity Cache at the expense of other data.  Measured on
// MI355X (same box, bit-identical outputs): the adaLN GEMV's weight stream
// 11.99 -> 11.04 us; the per-token quantizer at 11712 x 3072 24.2 -> 22.1 us.
// Outputs keep ordinary stores: the next kernel reads them (codes, normalised
// rows), and non-temporal stores there made the block linear set 0.5% and
// the DiT step's W8A8 linears 1.5% slower although the kernels that wrote
// them got faster.  Only for loads whose wave covers whole lines at once: in
// the ConvRot quantizer, where each lane reads its own 128-byte span 16 bytes
// per instruction, it made the kernel 35% slower (lines evicted between the
// instructions that share them).
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 load_stream(const void* p) {
    const v4u t = __builtin_nontemporal_load(static_cast<const v4u*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
}

// ---------------------------------------------------------------- 16-bit floats

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round to nearest even, one v_cvt_pk_bf16_f32 (gfx950).  Bit-identical to
// the software form u += 0x7fff + ((u >> 16) & 1) for every finite input,
// denormals included, and NaN -> (u >> 16) | 0x40 (checked on all 2^32
// inputs on the device).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

// Two values rounded as above and packed (a in the low half), one instruction.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
    const f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    // The empty asm pins f as an fp32 register value: without it the compiler
    // may fuse the fp32 multiply-add that produced f and this conversion into
    // one mixed-precision v_fma_mixlo_f16, which does not round like the two
    // separate roundings (fp32, then fp16) this library computes.  The
    // conversion itself (v_cvt_f16_f32) rounds to nearest even.
    asm("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <int DT> struct DType;
template <> struct DType<W8A8_F32> {
    using storage = float;
    static constexpr int bytes = 4;
    __device__ static float load(const storage v) { return v; }
    __device__ static storage store(float f) { return f; }
    __device__ static float round(float f) { return f; }
    static constexpr float finite_max = 3.40282347e38f;
    static constexpr float tiny = 1.17549435e-38f;
};
template <> struct DType<W8A8_F16> {
    using storage = uint16_t;
    static constexpr int bytes = 2;
    __device__ static float load(const storage v) { return f16_to_f32(v); }
    __device__ static storage store(float f) { return f32_to_f16(f); }
    __device__ static uint32_t store2(float a, float b) {
        return static_cast<uint32_t>(f32_to_f16(a)) | (static_cast<uint32_t>(f32_to_f16(b)) << 16);
    }
    __device__ static float round(float f) { return f16_to_f32(f32_to_f16(f)); }
    static constexpr float finite_max = 65504.0f;
    static constexpr float tiny = 6.103515625e-5f;
};
template <> struct DType<W8A8_BF16> {
    using storage = uint16_t;
    static constexpr int bytes = 2;
    __device__ static float load(const storage v) { return bf16_to_f32(v); }
    __device__ static storage store(float f) { return f32_to_bf16(f); }
    __device__ static uint32_t store2(float a, float b) { return pack2_bf16(a, b); }
    __device__ static float round(float f) { return bf16_to_f32(f32_to_bf16(f)); }
    static constexpr float finite_max = 3.38953139e38f;
    static constexpr float tiny = 1.17549435e-38f;
};

// ---------------------------------------------------------------- GELU (tanh)

// gelu_tanh(x) = 0.5 * x * (1 + tanh(u)),  u = sqrt(2/pi) * (x + 0.044715 * x^3),
// the reference's input_act "gelu_tanh" (inference/src/int8_linear.rs:37-41):
// ATen's operation order in fp32, tanh correctly rounded to fp32, the result
// rounded to the tensor's dtype.  Three forms, each exact for its dtype:
//   bf16  gelu_tanh_fast below, then RNE to bf16.  A bf16 input has 65536
//         values; for every finite one the result equals the correctly
//         rounded form (GPU tests run all of them through the quantizer and
//         through each GEMM main loop's epilogue against the oracle).
//   fp16  a lookup in kGeluF16Table (w8a8_gelu_tables.h, generated at build
//         time by imagine_amd/gelu_tables.py): the formula misses 5 of the
//         63488 finite fp16 inputs.
//   fp32  evaluated with the double-precision tanh of the fp32 argument,
//         rounded once (the correctly rounded fp32 tanh in all but vanishingly
//         rare cases).

// Structure 0.5 x (1 + tanh(u)) as the reference's:
//   e = x (a + b x^2) = 2u / ln 2           (sqrt(2/pi) and 0.044715 pre-scaled
//                                            by 2 / ln 2, so exp2 takes -|e|
//                                            through its input modifiers; u
//                                            has the sign of x)
//   t = exp(-2|u|),  r = 1 - 2 t / (1 + t)  (|tanh u| as one fma; the
//                                            subtraction rounds like an fp32
//                                            tanh, so 1 + tanh u cancels as it
//                                            does: exactly 0 once |u| > 9)
//   gelu = x (1/2 + copysign(1/2, x) r)     (= (x/2) RN(1 + copysign(r, x)),
//                                            the reference's two roundings, for
//                                            every x: halving commutes with
//                                            rounding here, and x/2 is exact;
//                                            the saturated negative tail gives
//                                            x * +0 = -0 as the reference does)
// exp2 and the reciprocal are the hardware approximations (about 1 ulp); the
// fp32 result carries a few ulps of error, which bf16 rounding never shows.
// About 13 VALU slots, two of them quarter-rate.  The GEMM's staged epilogue
// looks its results up instead (gelu_bf16x8_lut below, about 4 operations and
// one LDS read per value).
__device__ __forceinline__ float gelu_tanh_fast(float x) {
    const float kA = 2.302208198144325f;      // sqrt(2/pi) * 2 / ln 2
    const float kB = 0.1029432395800235f;     // sqrt(2/pi) * 0.044715 * 2 / ln 2
    const float e = x * fmaf(kB, x * x, kA);
    const float t = __builtin_amdgcn_exp2f(-fabsf(e));   // (0, 1]
    const float q = t * __builtin_amdgcn_rcpf(1.0f + t);
    const float r = fmaf(-2.0f, q, 1.0f);
    return x * fmaf(__builtin_copysignf(0.5f, x), r, 0.5f);
}

// Two bf16 values packed in one word (low half first) -> their GELU, rounded
// and packed the same way (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t gelu_bf16x2(uint32_t p) {
    return pack2_bf16(gelu_tanh_fast(__uint_as_float(p << 16)), gelu_tanh_fast(__uint_as_float(p & 0xffff0000u)));
}

// fp16 pattern b (low 16 bits) -> fp16 pattern of gelu_tanh(b); the table
// covers |x| < 6, beyond which the result is x (x > 0) or -0 (finite x < 0).
__device__ __forceinline__ uint32_t gelu_f16_bits(uint32_t b) {
    const uint32_t a = b & 0x7fffu;
    const uint32_t looked = kGeluF16Table[(b >> 15) * kGeluF16Span + (a < kGeluF16Hi ? a : kGeluF16Hi - 1)];
    uint32_t big = (b & 0x8000u) ? (a == 0x7c00u ? 0xfe00u : 0x8000u) : b;   // -inf: 0 * -inf
    big = a > 0x7c00u ? (b | 0x200u) : big;                                 // NaN: the input, quieted
    return a < kGeluF16Hi ? looked : big;
}

__device__ __forceinline__ float gelu_f32(float x) {
    const float kBeta = 0.79788456080286535588f;  // sqrt(2) * (2/sqrt(pi)) * 0.5
    const float kKappa = 0.044715f;
    const float x_cube = x * x * x;
    const float inner = kBeta * (x + kKappa * x_cube);
    const float t = static_cast<float>(tanh(static_cast<double>(inner)));
    return 0.5f * x * (1.0f + t);
}

// GELU of the 16-bit pattern b of dtype DT.
template <int DT>
__device__ __forceinline__ uint32_t gelu_bits(uint32_t b) {
    static_assert(DT != W8A8_F32, "16-bit dtypes only");
    if constexpr (DT == W8A8_BF16) return f32_to_bf16(gelu_tanh_fast(bf16_to_f32(static_cast<uint16_t>(b))));
    else return gelu_f16_bits(b);
}

// Two 16-bit patterns of dtype DT packed in one word -> their GELU, packed.
template <int DT>
__device__ __forceinline__ uint32_t gelu_x2(uint32_t p) {
    if constexpr (DT == W8A8_BF16) return gelu_bf16x2(p);
    else return gelu_f16_bits(p & 0xffffu) | (gelu_f16_bits(p >> 16) << 16);
}

// bf16 GELU by lookup in a 16 KB LDS table of gelu_bf16x2's own results, for
// the VALU-bound epilogue of the GEMM.  Word u of the table holds the GELU of
// the patterns kGeluLutLo + u (low half) and 0x8000 | (kGeluLutLo + u) (high
// half): magnitudes 2^-18 up to 2^14 of either sign.  For a pattern b,
// d = (b - kGeluLutLo) mod 2^16 is in range iff bits 12-14 of d are clear,
// and its entry's byte offset is then (4 d mod 2^16) | (d >> 14) = 4u + 2s, s
// the sign: both halves of a word are offset by the same three packed 16-bit
// operations.  An out-of-range offset is still below 64 KB, so the reads stay
// inside a block LDS array of at least 64 KB with the table at its start.
// Filled per block from gelu_bf16x2, the lookup equals gelu_bf16x2 bit for
// bit wherever it applies.
constexpr uint32_t kGeluLutLo = 0x3680u;        // bf16 2^-18
constexpr int kGeluLutBytes = 4096 * 4;

// Fills the table: thread t of nthreads writes words t, t + nthreads, ...
__device__ __forceinline__ void gelu_lut_fill(int8_t* tab, int t, int nthreads) {
    for (int u = t; u < kGeluLutBytes / 4; u += nthreads) {
        const uint32_t b = kGeluLutLo + u;
        reinterpret_cast<uint32_t*>(tab)[u] = gelu_bf16x2(b | ((b | 0x8000u) << 16));
    }
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// Table offsets of the 8 bf16 values of a chunk (see gelu_bf16x8_lut); `miss`
// collects the bits that flag an out-of-range value (0x70007000).
__device__ __forceinline__ void gelu_lut_offsets(uint4 v, uint32_t base, uint32_t (&off)[8], uint32_t& miss) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    const u16x2 lo2 = {static_cast<unsigned short>(kGeluLutLo), static_cast<unsigned short>(kGeluLutLo)};
    miss = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const u16x2 d = __builtin_bit_cast(u16x2, w[k]) - lo2;
        const uint32_t q = __builtin_bit_cast(uint32_t, static_cast<u16x2>((d << 2) | (d >> 14)));
        miss |= __builtin_bit_cast(uint32_t, d);
        off[2 * k] = (q & 0xffffu) + base;
        off[2 * k + 1] = (q >> 16) + base;
    }
}

// GELU of two chunks, all 16 lookups issued before the first result is used
// (otherwise as gelu_bf16x8_lut).
__device__ __forceinline__ void gelu_bf16x16_lut(uint4& a, uint4& b, uint32_t base) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(3))) unsigned short* lds_u16;
    uint32_t oa[8], ob[8], ma, mb;
    gelu_lut_offsets(a, base, oa, ma);
    gelu_lut_offsets(b, base, ob, mb);
    u16x2 ga[4], gb[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        ga[k].x = *(lds_u16)static_cast<uintptr_t>(oa[2 * k]);
        ga[k].y = *(lds_u16)static_cast<uintptr_t>(oa[2 * k + 1]);
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        gb[k].x = *(lds_u16)static_cast<uintptr_t>(ob[2 * k]);
        gb[k].y = *(lds_u16)static_cast<uintptr_t>(ob[2 * k + 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint4 ra = make_uint4(__builtin_bit_cast(uint32_t, ga[0]), __builtin_bit_cast(uint32_t, ga[1]),
                          __builtin_bit_cast(uint32_t, ga[2]), __builtin_bit_cast(uint32_t, ga[3]));
    uint4 rb = make_uint4(__builtin_bit_cast(uint32_t, gb[0]), __builtin_bit_cast(uint32_t, gb[1]),
                          __builtin_bit_cast(uint32_t, gb[2]), __builtin_bit_cast(uint32_t, gb[3]));
    if (__builtin_expect((ma & 0x70007000u) != 0, 0))
        ra = make_uint4(gelu_bf16x2(a.x), gelu_bf16x2(a.y), gelu_bf16x2(a.z), gelu_bf16x2(a.w));
    if (__builtin_expect((mb & 0x70007000u) != 0, 0))
        rb = make_uint4(gelu_bf16x2(b.x), gelu_bf16x2(b.y), gelu_bf16x2(b.z), gelu_bf16x2(b.w));
    a = ra;
    b = rb;
}

// GELU of 8 bf16 values (a 16-byte chunk): table lookups when all 8 are in the
// table's range, else gelu_bf16x2 for the whole chunk.  `base` is the table's
// LDS address; [base, base + 64 KB) lies inside the block's LDS.  All eight
// lookups are issued before the first result is used; each pair's results
// are packed into one word.
__device__ __forceinline__ uint4 gelu_bf16x8_lut(uint4 v, uint32_t base) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(3))) unsigned short* lds_u16;
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    const u16x2 lo2 = {static_cast<unsigned short>(kGeluLutLo), static_cast<unsigned short>(kGeluLutLo)};
    uint32_t off[8], miss = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const u16x2 d = __builtin_bit_cast(u16x2, w[k]) - lo2;
        const uint32_t q = __builtin_bit_cast(uint32_t, static_cast<u16x2>((d << 2) | (d >> 14)));
        miss |= __builtin_bit_cast(uint32_t, d);
        off[2 * k] = (q & 0xffffu) + base;
        off[2 * k + 1] = (q >> 16) + base;
    }
    u16x2 g[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        g[k].x = *(lds_u16)static_cast<uintptr_t>(off[2 * k]);
        g[k].y = *(lds_u16)static_cast<uintptr_t>(off[2 * k + 1]);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint32_t r[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) r[k] = __builtin_bit_cast(uint32_t, g[k]);
    if (__builtin_expect((miss & 0x70007000u) != 0, 0)) {
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = gelu_bf16x2(w[k]);
    }
    return make_uint4(r[0], r[1], r[2], r[3]);
}

// GELU of a value v already rounded to dtype T, as a float.
template <int DT>
__device__ __forceinline__ float gelu_value(float v) {
    if constexpr (DT == W8A8_F32) return gelu_f32(v);
    else return DType<DT>::load(static_cast<typename DType<DT>::storage>(gelu_bits<DT>(DType<DT>::store(v))));
}

// ---------------------------------------------------------------- input activations

// Codes of the linear's input activation (Kitchen's input_act_codes.h; SiTU
// is 4 as the crate passes it, inference/src/convrot.rs:211-238).  SwiGLU and
// SiTU read a [gate | up] row twice as wide as the K they write.
constexpr int kActNone = W8A8_ACT_NONE, kActGeluTanh = W8A8_ACT_GELU, kActSwiGLU = W8A8_ACT_SWIGLU,
              kActRmsNorm = W8A8_ACT_RMSNORM, kActSiTU = W8A8_ACT_SITU;

__host__ __device__ constexpr bool act_gated(int act) { return act == kActSwiGLU || act == kActSiTU; }

// Correctly rounded fp32 exp and tanh (the double-precision function of the
// fp32 argument, rounded once): ATen's CPU silu, sigmoid and tanh give these
// values on every 16-bit input once rounded to the dtype.
__device__ __forceinline__ float exp_cr(float v) { return static_cast<float>(exp(static_cast<double>(v))); }
__device__ __forceinline__ float tanh_cr(float v) { return static_cast<float>(tanh(static_cast<double>(v))); }

// The eager activations of the crate's apply_input (inference/src/int8_linear.rs:
// 37-97): ATen ops on tensors of dtype T, each result rounded to T.  a is the
// value (the gate for the gated ones), b the up value; the result is in T.
template <int DT, int ACT>
__device__ __forceinline__ float act_eager(float a, float b) {
    using D = DType<DT>;
    if constexpr (ACT == kActGeluTanh) {
        return gelu_value<DT>(a);
    } else if constexpr (ACT == kActSwiGLU) {
        return D::round(D::round(a / (1.0f + exp_cr(-a))) * b);                   // silu(a) * b
    } else if constexpr (ACT == kActSiTU) {
        const float t4 = D::round(D::round(tanh_cr(D::round(b / 4.0f))) * 4.0f);  // tanh(b / 4) * 4
        const float sg = D::round(1.0f / (1.0f + exp_cr(-b)));                   // sigmoid(b)
        const float gated = D::round(t4 * sg);
        const float t25 = D::round(D::round(tanh_cr(D::round(a / 25.0f))) * 25.0f);
        return D::round(t25 * gated);
    } else {
        return a;
    }
}

// The fused activations of Kitchen's ConvRot quantizer
// (native/comfy-port/kitchen/int8_linear.cu:1175-1200,1230-1262): fp32, not
// rounded to the dtype (RMSNorm is applied by the kernel from its row rstd).
template <int ACT>
__device__ __forceinline__ float act_fused(float a, float b) {
    if constexpr (ACT == kActGeluTanh) {
        const float kBeta = 0.79788456080286535588f;
        const float inner = kBeta * (a + 0.044715f * a * a * a);
        return 0.5f * a * (1.0f + tanh_cr(inner));
    } else if constexpr (ACT == kActSwiGLU) {
        return (a / (1.0f + exp_cr(-a))) * b;
    } else if constexpr (ACT == kActSiTU) {
        return (tanh_cr(a / 25.0f) * 25.0f) * ((tanh_cr(b / 4.0f) * 4.0f) * (1.0f / (1.0f + exp_cr(-b))));
    } else {
        return a;
    }
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).  Used
// where an index selects a register array element (MFMA accumulators), so the
// array can never be indexed dynamically (which would demote it to scratch).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// ---------------------------------------------------------------- quantizer math

// Row scale from the row's absolute maximum.
//   IEEE form:  max(amax / 127, 1e-30)                 (eager.rs:159-165)
//   RECIP form: max(min(amax, T_max) * (1/127), 1e-30) (int8_linear.cu:36-39,205-208)
template <int DT>
__device__ __forceinline__ float row_scale(float amax, bool recip) {
    float s;
    if (recip) {
        s = fminf(amax, DType<DT>::finite_max) * (1.0f / 127.0f);
    } else {
        s = amax / 127.0f;  // correctly rounded: no fast-math in this library
    }
    return fmaxf(s, 1.0e-30f);
}

// Per-row constants of the element quantizer: the divisor sT = T(s) (zero
// replaced by T's tiny, eager.rs:94-109) and its correctly rounded reciprocal.
struct RowQuant {
    float d;  // sT
    float r;  // RN(1 / sT)
};

template <int DT>
__device__ __forceinline__ RowQuant row_quant(float s) {
    RowQuant rq;
    float d = DType<DT>::round(s);
    if (d == 0.0f) d = DType<DT>::tiny;
    rq.d = d;
    rq.r = 1.0f / d;
    return rq;
}

// The quotient as far as the int8 code needs it.  For 16-bit T the plain
// product RN(x * RN(1/sT)) can differ from RN(x / sT) in the last fp32 bit,
// but clamp(rint(T(.))) of the two is the same for every 16-bit x and every
// reachable divisor (checked exhaustively, tests/divide_check.c); fp32 inputs
// divide in IEEE.
template <int DT>
__device__ __forceinline__ float code_quotient(float x, const RowQuant& rq) {
    if constexpr (DT == W8A8_F32) return x / rq.d;
    else return DType<DT>::round(x * rq.r);
}

// One element: q = clamp(rint(T(x / sT)), -128, 127) as int.
template <int DT>
__device__ __forceinline__ int quant_elem(float x, const RowQuant& rq) {
    const float quot = code_quotient<DT>(x, rq);
    float v = __builtin_rintf(quot);
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return static_cast<int>(v);
}

// The same code as an int8 in the low byte of the result (upper bits are
// garbage): clamp first, then add 1.5 * 2^23, whose round-to-nearest-even
// leaves rint(v) in the low mantissa bits (two's complement, since 2^22 sits
// above them).  Equal to quant_elem for every non-NaN quotient (checked over
// all 2^32 floats; clamping before rounding is exact because the clamp
// bounds are integers), and NaN clamps to -128 in both forms.
template <int DT>
__device__ __forceinline__ uint32_t quant_byte(float x, const RowQuant& rq) {
    const float quot = code_quotient<DT>(x, rq);
    const float v = fminf(fmaxf(quot, -128.0f), 127.0f);
    return __float_as_uint(v + 12582912.0f);
}

// Pack the low bytes of four quant_byte results (a lowest).
__device__ __forceinline__ uint32_t pack4_low_bytes(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x0c0c0400u);   // bytes: a0, b0, 0, 0
    const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x04000c0cu);   // bytes: 0, 0, c0, d0
    return ab | cd;
}

// Round two values to T and widen them back; bf16 rounds both in one
// v_cvt_pk_bf16_f32 (the same bits as DType::round on each).
template <int DT>
__device__ __forceinline__ void round2(float& a, float& b) {
    if constexpr (DT == W8A8_BF16) {
        const uint32_t u = pack2_bf16(a, b);
        a = __uint_as_float(u << 16);
        b = __uint_as_float(u & 0xffff0000u);
    } else {
        a = DType<DT>::round(a);
        b = DType<DT>::round(b);
    }
}

// Four int8 codes packed (a lowest) for four values already in T: the same
// codes as quant_byte, with the 16-bit quotient roundings done in pairs.
template <int DT>
__device__ __forceinline__ uint32_t quant4_packed(float a, float b, float c, float d, const RowQuant& rq) {
    if constexpr (DT == W8A8_F32) {
        return pack4_low_bytes(quant_byte<DT>(a, rq), quant_byte<DT>(b, rq), quant_byte<DT>(c, rq),
                               quant_byte<DT>(d, rq));
    } else {
        float q0 = a * rq.r, q1 = b * rq.r, q2 = c * rq.r, q3 = d * rq.r;
        round2<DT>(q0, q1);
        round2<DT>(q2, q3);
        auto byte = [](float q) {
            return __float_as_uint(fminf(fmaxf(q, -128.0f), 127.0f) + 12582912.0f);
        };
        return pack4_low_bytes(byte(q0), byte(q1), byte(q2), byte(q3));
    }
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
           ((static_cast<uint32_t>(c) & 0xffu) << 16) | ((static_cast<uint32_t>(d) & 0xffu) << 24);
}

// ---------------------------------------------------------------- epilogue

// out = O( fma(float(acc) * xs, ws, bias) ), optional gelu on the O-rounded value.
template <int ODT>
__device__ __forceinline__ float epilogue_value(int acc, float xs, float ws, float bias, bool gelu) {
    float t = static_cast<float>(acc) * xs;
    float v = fmaf(t, ws, bias);
    if (gelu) v = gelu_value<ODT>(DType<ODT>::round(v));
    return v;
}

// Residual of the pre-norm block fused into an epilogue:
//   out = O( fma(O(lin), rscale[n], resid[m, n]) )
// with rscale (1 or N entries) and resid ([M, N]) in the output dtype: the
// reference's fused CUTLASS residual (archived cutlass_gemm_int8.cu:122-188)
// and, bit for bit, its eager addcmul on the GPU (int8_linear.rs:99-111).
struct Residual {
    const void* rscale;
    int64_t rs_size;
    const void* resid;
};

template <int ODT>
__device__ __forceinline__ float residual_value(float lin, const Residual& res, int64_t m, int n, int N) {
    using OS = typename DType<ODT>::storage;
    const float s = DType<ODT>::load(static_cast<const OS*>(res.rscale)[res.rs_size == 1 ? 0 : n]);
    const float r = DType<ODT>::load(static_cast<const OS*>(res.resid)[m * N + n]);
    return fmaf(DType<ODT>::round(lin), s, r);
}

// ---------------------------------------------------------------- wave reductions

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

}  // namespace w8a8
