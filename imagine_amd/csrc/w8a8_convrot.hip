// ConvRot activation quantization for gfx950: a regular Hadamard rotation of
// every `group`-wide slice of a token row, then per-token absmax INT8.
//
// Replaces Kitchen's quantize_int8_rowwise_convrot64_kernel
// (native/comfy-port/kitchen/int8_linear.cu:1204-1314, launcher :1609-1719)
// for the fused route and rotate_activation + quantize_int8_rowwise
// (inference/src/convrot.rs:474-484, int8_utils.rs:97-106) for the others.
//
// Rotation: y = x_g . H_G, H_G = (H4 (x) ... (x) H4) / sqrt(G),
// H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] (int8_utils.rs:21-58),
// computed as radix-4 stages at strides 1, 4, 16, 64 in fp32, each output
// 0.5 * (x0 + x1 + x2 - x3) (or a sign variant) with its operands added left
// to right: the fused reference kernel's operation order (int8_linear.cu:881-895).
//
// Fused route (group 256, K % 256 == 0, 256 <= K <= 16384): the rotated
// values stay in fp32 for the row's absmax and are rounded to the input dtype
// T only for the quotient, q = clamp(rint(T(T(y) / T(s)))).
// Rotate route (any other power-of-4 group): y is rounded to T and written
// out; the plain per-token quantizer then runs on it.
//
// Layout of the fast kernels: each lane holds 64 consecutive elements of a
// group (digits d0, d1, d2 of the in-group index d3*64 + d2*16 + d1*4 + d0),
// so the first three stages run in registers; the four lanes of a quad hold
// d3 = 0..3 of one 256-group, and the last stage reads them with DPP quad
// broadcasts.  A row never leaves registers between its absmax and quantize
// passes.
#include "w8a8_common.h"

namespace w8a8 {

constexpr int kRotGroup = 256;   // the fused route's group
constexpr int kLaneElems = 64;   // consecutive elements per lane

// 0.5 * (H4 row k) . (x0, x1, x2, x3), in place, operands left to right.
__device__ __forceinline__ void h4_stage(float& a, float& b, float& c, float& d) {
    const float x0 = a, x1 = b, x2 = c, x3 = d;
    a = 0.5f * (x0 + x1 + x2 - x3);
    b = 0.5f * (x0 + x1 - x2 + x3);
    c = 0.5f * (x0 - x1 + x2 + x3);
    d = 0.5f * (-x0 + x1 + x2 + x3);
}

// The fast kernels below leave out the 0.5 of every stage: a power-of-two
// scale commutes with round-to-nearest while values stay normal, so their
// stage outputs are exactly 2^L times the reference's (L stages) and the
// factor 2^-L is applied once (folded into the quotient's divisor on the fused
// route).  That holds for rows whose nonzero inputs lie within [2^-100, 2^120)
// in magnitude (no sum then reaches a subnormal in the reference or overflows
// here); the generic kernels keep the 0.5 per stage.
//
// (H4 row k) . (x0, x1, x2, x3) in place, operands left to right as above:
// x0 + x1 is shared by rows 0 and 1, and row 3's (-x0 + x1) + x2 is
// x2 - (x0 - x1) bit for bit (round-to-nearest-even is odd-symmetric).
__device__ __forceinline__ void h4_sum(float& a, float& b, float& c, float& d) {
    const float x0 = a, x1 = b, x2 = c, x3 = d;
    const float p = x0 + x1, m = x0 - x1;
    a = (p + x2) - x3;
    b = (p - x2) + x3;
    c = (m + x2) + x3;
    d = (x2 - m) + x3;
}

// Stage across the quad, four values a, b, c, d at once: lane d of the quad
// gets (H4 row d) . (x0..x3), x_k being the value of quad lane k; sg[k] is -1
// where row d of H4 has its minus sign (k == 3 - d), else +1.  One DPP
// instruction per term: v_mul_f32_dpp for x0 * sg0, then v_fmac_f32_dpp
// t += x_k * sg_k (exact products, so each is the reference's t +- x_k,
// rounded once).  Written with builtins, the compiler folds the quad
// broadcast into the multiply but not into the fmac (7 instructions per value
// instead of 4), so the block is written out; the
// four chains are interleaved, and s_nop 4 first gives the wait states a DPP
// read needs after a VALU write of its source (and after an EXEC write).
// All lanes of every quad are active wherever this is used.
#define W8A8_DPP_Q(K) "quad_perm:[" #K "," #K "," #K "," #K "] row_mask:0xf bank_mask:0xf bound_ctrl:1\n\t"
__device__ __forceinline__ void h4_across_quad_x4(float& a, float& b, float& c, float& d, const float (&sg)[4]) {
    float ta, tb, tc, td;
    asm("s_nop 4\n\t"
        "v_mul_f32_dpp %0, %4, %8 " W8A8_DPP_Q(0)
        "v_mul_f32_dpp %1, %5, %8 " W8A8_DPP_Q(0)
        "v_mul_f32_dpp %2, %6, %8 " W8A8_DPP_Q(0)
        "v_mul_f32_dpp %3, %7, %8 " W8A8_DPP_Q(0)
        "v_fmac_f32_dpp %0, %4, %9 " W8A8_DPP_Q(1)
        "v_fmac_f32_dpp %1, %5, %9 " W8A8_DPP_Q(1)
        "v_fmac_f32_dpp %2, %6, %9 " W8A8_DPP_Q(1)
        "v_fmac_f32_dpp %3, %7, %9 " W8A8_DPP_Q(1)
        "v_fmac_f32_dpp %0, %4, %10 " W8A8_DPP_Q(2)
        "v_fmac_f32_dpp %1, %5, %10 " W8A8_DPP_Q(2)
        "v_fmac_f32_dpp %2, %6, %10 " W8A8_DPP_Q(2)
        "v_fmac_f32_dpp %3, %7, %10 " W8A8_DPP_Q(2)
        "v_fmac_f32_dpp %0, %4, %11 " W8A8_DPP_Q(3)
        "v_fmac_f32_dpp %1, %5, %11 " W8A8_DPP_Q(3)
        "v_fmac_f32_dpp %2, %6, %11 " W8A8_DPP_Q(3)
        "v_fmac_f32_dpp %3, %7, %11 quad_perm:[3,3,3,3] row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=&v"(ta), "=&v"(tb), "=&v"(tc), "=&v"(td)
        : "v"(a), "v"(b), "v"(c), "v"(d), "v"(sg[0]), "v"(sg[1]), "v"(sg[2]), "v"(sg[3]));
    a = ta;
    b = tb;
    c = tc;
    d = td;
}
#undef W8A8_DPP_Q

// The in-register stages of a lane's 64 elements: strides 1, 4, 16, as many
// as the group has (G = 4, 16, 64 or more), unscaled.
template <int G>
__device__ __forceinline__ void lane_stages(float (&v)[kLaneElems]) {
#pragma unroll
    for (int j = 0; j < 16; ++j) h4_sum(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
    if constexpr (G >= 16) {
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int d0 = 0; d0 < 4; ++d0) {
                const int b = 16 * a + d0;
                h4_sum(v[b], v[b + 4], v[b + 8], v[b + 12]);
            }
    }
    if constexpr (G >= 64) {
#pragma unroll
        for (int r = 0; r < 16; ++r) h4_sum(v[r], v[r + 16], v[r + 32], v[r + 48]);
    }
}

// 64 consecutive elements from a valid address (lanes without work of their
// own read row 0, compute on it and store nothing).
template <int DT>
__device__ __forceinline__ void load_lane(const void* src, float (&v)[kLaneElems]) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;  // elements per 16-byte chunk
    const uint4* p = static_cast<const uint4*>(src);
#pragma unroll
    for (int c = 0; c < kLaneElems / E; ++c) {
        const uint4 raw = p[c];
        const typename D::storage* e = reinterpret_cast<const typename D::storage*>(&raw);
#pragma unroll
        for (int i = 0; i < E; ++i) v[c * E + i] = D::load(e[i]);
    }
}

// Fused route.  A block holds rows_per_block rows of ngroups 256-groups, one
// quad per group; quads past the block's rows (or past M) compute on row 0
// and store nothing, so every lane takes part in the DPP stage and the
// barrier (their group maxima are read by no active lane).
template <int DT>
__global__ __launch_bounds__(1024) void convrot_quant_rows(const void* __restrict__ xv,
                                                           int8_t* __restrict__ q,
                                                           float* __restrict__ xs, int64_t M,
                                                           int K, int rows_per_block, int recip) {
    using D = DType<DT>;
    extern __shared__ float group_amax[];  // one per quad
    const int ngroups = K / kRotGroup;
    const int quad = threadIdx.x / 4;
    const int d3 = threadIdx.x % 4;
    const int rb = quad / ngroups;
    const int g = quad - rb * ngroups;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * rows_per_block + rb;
    const bool active = rb < rows_per_block && row < M;
    const int64_t col = static_cast<int64_t>(g) * kRotGroup + d3 * kLaneElems;

    float v[kLaneElems];
    load_lane<DT>(static_cast<const char*>(xv) + ((active ? row : 0) * K + col) * D::bytes, v);
    lane_stages<kRotGroup>(v);
    float sg[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) sg[k] = (k == 3 - d3) ? -1.0f : 1.0f;
    float m = 0.0f;
#pragma unroll
    for (int r = 0; r < kLaneElems; r += 4) {
        h4_across_quad_x4(v[r], v[r + 1], v[r + 2], v[r + 3], sg);  // 16 y
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(v[r + i]));
    }
    // quad max: quad_perm [1,0,3,2] then [2,3,0,1]
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0xb1, 0xf, 0xf, false)));
    m = fmaxf(m, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(m), 0x4e, 0xf, 0xf, false)));
    if (d3 == 0) group_amax[quad] = m;
    __syncthreads();
    if (!active) return;

    float amax = 0.0f;
    const float* ga = group_amax + rb * ngroups;
    for (int i = 0; i < ngroups; ++i) amax = fmaxf(amax, ga[i]);
    const float s = row_scale<DT>(amax * 0.0625f, recip != 0);
    if (g == 0 && d3 == 0) xs[row] = s;
    // T(y) / T(s) from 16 y: bf16 has fp32's exponent range, so T(16 y) =
    // 16 T(y) and the divisor becomes 16 T(s) (reciprocal / 16, exact); fp16
    // (narrow range, absolute denormal steps) rounds y itself.
    RowQuant rq = row_quant<DT>(s);
    if constexpr (DT != W8A8_F16) {
        rq.d *= 16.0f;
        rq.r *= 0.0625f;
    }
    uint32_t packed[kLaneElems / 4];
#pragma unroll
    for (int j = 0; j < kLaneElems / 4; ++j) {
        float a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = (DT == W8A8_F16) ? v[4 * j + i] * 0.0625f : v[4 * j + i];
        round2<DT>(a[0], a[1]);
        round2<DT>(a[2], a[3]);
        packed[j] = quant4_packed<DT>(a[0], a[1], a[2], a[3], rq);
    }
    uint4* dst = reinterpret_cast<uint4*>(q + row * K + col);
#pragma unroll
    for (int c = 0; c < kLaneElems / 16; ++c)
        dst[c] = make_uint4(packed[4 * c], packed[4 * c + 1], packed[4 * c + 2], packed[4 * c + 3]);
}

// Fused route, any alignment: one block per row, the rotated row in LDS
// (K <= 16384 floats), stage by stage like the reference kernel.  ACT fuses
// an input activation the way that kernel does (int8_linear.cu:1175-1262): in
// fp32, not rounded to T, x being [M, 2K] for the gated ones; RMSNorm scales
// the row by its rstd and the weight w.
template <int DT, int ACT>
__global__ __launch_bounds__(256) void convrot_quant_rows_generic(const void* __restrict__ xv,
                                                                  int8_t* __restrict__ q,
                                                                  float* __restrict__ xs, int64_t M,
                                                                  int K, int recip, const void* __restrict__ wv,
                                                                  float eps) {
    using D = DType<DT>;
    using S = typename D::storage;
    extern __shared__ float rowbuf[];
    __shared__ float part[4];
    __shared__ double dpart[4];
    const int64_t row = blockIdx.x;
    const int64_t in_w = act_gated(ACT) ? 2 * static_cast<int64_t>(K) : K;
    const S* x = static_cast<const S*>(xv) + row * in_w;
    float rstd = 1.0f;
    if constexpr (ACT == kActRmsNorm) {
        double acc = 0.0;
        for (int k = threadIdx.x; k < K; k += blockDim.x) {
            const double v = D::load(x[k]);
            acc += v * v;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, kWave);
        if ((threadIdx.x % kWave) == 0) dpart[threadIdx.x / kWave] = acc;
        __syncthreads();
        const double total = (dpart[0] + dpart[1]) + (dpart[2] + dpart[3]);
        rstd = 1.0f / sqrtf(static_cast<float>(total / static_cast<double>(K)) + eps);
    }
    for (int k = threadIdx.x; k < K; k += blockDim.x) {
        const float a = D::load(x[k]);
        if constexpr (ACT == kActRmsNorm) rowbuf[k] = (a * rstd) * D::load(static_cast<const S*>(wv)[k]);
        else if constexpr (act_gated(ACT)) rowbuf[k] = act_fused<ACT>(a, D::load(x[K + k]));
        else rowbuf[k] = act_fused<ACT>(a, 0.0f);
    }
    __syncthreads();
    for (int S = 1; S < kRotGroup; S *= 4) {
        for (int b = threadIdx.x; b < K / 4; b += blockDim.x) {
            const int j = b % (kRotGroup / 4);
            float* p = rowbuf + (b / (kRotGroup / 4)) * kRotGroup + (j % S) + (j / S) * 4 * S;
            h4_stage(p[0], p[S], p[2 * S], p[3 * S]);
        }
        __syncthreads();
    }
    float amax = 0.0f;
    for (int k = threadIdx.x; k < K; k += blockDim.x) amax = fmaxf(amax, fabsf(rowbuf[k]));
    amax = wave_max(amax);
    if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float s = row_scale<DT>(amax, recip != 0);
    if (threadIdx.x == 0) xs[row] = s;
    const RowQuant rq = row_quant<DT>(s);
    for (int k = threadIdx.x; k < K; k += blockDim.x)
        q[row * K + k] = static_cast<int8_t>(quant_elem<DT>(D::round(rowbuf[k]), rq));
}

// Rotate route, aligned rows with K % 64 == 0 and G <= 256: every lane
// rotates 64 consecutive elements (with its quad for G = 256) and stores them
// rounded to T.
template <int DT, int G>
__global__ __launch_bounds__(256) void convrot_rotate_vec(const void* __restrict__ xv,
                                                          void* __restrict__ yv, int64_t chunks) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;
    const int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const bool ok = c < chunks;
    float v[kLaneElems];
    load_lane<DT>(static_cast<const char*>(xv) + (ok ? c : 0) * kLaneElems * D::bytes, v);
    lane_stages<G>(v);
    float sg[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) sg[k] = (k == 3 - static_cast<int>(threadIdx.x % 4)) ? -1.0f : 1.0f;
    uint4* dst = reinterpret_cast<uint4*>(static_cast<char*>(yv) + (ok ? c : 0) * kLaneElems * D::bytes);
    // G = 256: the quad stage chunk by chunk, each chunk stored as it is done
    // (keeps the live registers to one chunk of stage outputs)
    // 2^-L, L = log4(G) stages
    constexpr float kScale = G == 4 ? 0.5f : G == 16 ? 0.25f : G == 64 ? 0.125f : 0.0625f;
#pragma unroll
    for (int k = 0; k < kLaneElems / E; ++k) {
        if constexpr (G == kRotGroup) {
#pragma unroll
            for (int i = 0; i < E; i += 4)
                h4_across_quad_x4(v[k * E + i], v[k * E + i + 1], v[k * E + i + 2], v[k * E + i + 3], sg);
        }
#pragma unroll
        for (int i = 0; i < E; ++i) v[k * E + i] *= kScale;
        uint4 out;
        uint32_t* w = reinterpret_cast<uint32_t*>(&out);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (DT == W8A8_F32) w[i] = __float_as_uint(v[k * E + i]);
            else w[i] = D::store2(v[k * E + 2 * i], v[k * E + 2 * i + 1]);
        }
        if (ok) dst[k] = out;
    }
}

// Rotate route, any power-of-4 group up to 16384 and any alignment: one block
// per group of the [M, K] tensor (groups are contiguous), the group in LDS.
template <int DT>
__global__ __launch_bounds__(256) void convrot_rotate_generic(const void* __restrict__ xv,
                                                              void* __restrict__ yv, int64_t K,
                                                              int G) {
    using D = DType<DT>;
    extern __shared__ float gbuf[];
    // block b: row b / (K / G), group b % (K / G), i.e. element offset b * G
    const int64_t base = static_cast<int64_t>(blockIdx.x) * G;
    const typename D::storage* x = static_cast<const typename D::storage*>(xv) + base;
    typename D::storage* y = static_cast<typename D::storage*>(yv) + base;
    for (int i = threadIdx.x; i < G; i += blockDim.x) gbuf[i] = D::load(x[i]);
    __syncthreads();
    for (int S = 1; S < G; S *= 4) {
        for (int b = threadIdx.x; b < G / 4; b += blockDim.x) {
            float* p = gbuf + (b % S) + (b / S) * 4 * S;
            h4_stage(p[0], p[S], p[2 * S], p[3 * S]);
        }
        __syncthreads();
    }
    for (int i = threadIdx.x; i < G; i += blockDim.x) y[i] = D::store(gbuf[i]);
}

// ---------------------------------------------------------------- host side

bool convrot_fused_route(int64_t K, int64_t group) {
    return group == kRotGroup && K % kRotGroup == 0 && K >= kRotGroup && K <= 16384;
}

// Weights take the fused numerics up to K = 65536 (a block of 1024 threads
// holds one row); rows above K = 16384 need the aligned (register) kernel,
// i.e. 16-byte aligned weight and code rows.
bool convrot_weight_fused(const void* w, const void* q, int64_t K, int64_t group) {
    if (group != kRotGroup || K % kRotGroup != 0 || K < kRotGroup || K > 65536) return false;
    return K <= 16384 || (reinterpret_cast<uintptr_t>(w) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0);
}

// Rows per block of the fused kernel: whole waves with every quad busy where
// possible (ngroups * rows % 16 == 0), about 256 threads, at most 1024.
static int fused_rows_per_block(int ngroups) {
    int best = 1;
    double best_util = 0.0;
    for (int r = 1; 4 * r * ngroups <= 1024; ++r) {
        const int threads = 4 * r * ngroups;
        const int padded = (threads + kWave - 1) / kWave * kWave;
        const double util = static_cast<double>(threads) / padded;
        if (util > best_util + 1e-9) {
            best = r;
            best_util = util;
        }
        if (util > 1.0 - 1e-9 && threads >= 256) return r;
    }
    return best;
}

// The row in LDS: up to 64 KB beside the kernel's static bytes.
template <int DT, int ACT>
static void launch_fused_generic(const void* x, int8_t* q, float* xs, int64_t M, int64_t K, bool recip, const void* w,
                                 float eps, hipStream_t stream) {
    const size_t lds = K * sizeof(float);
    if (lds > 32 * 1024)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&convrot_quant_rows_generic<DT, ACT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    hipLaunchKernelGGL((convrot_quant_rows_generic<DT, ACT>), dim3(static_cast<unsigned>(M)), dim3(256), lds, stream,
                       x, q, xs, M, static_cast<int>(K), recip ? 1 : 0, w, eps);
}

template <int DT>
static void launch_fused(const void* x, int8_t* q, float* xs, int64_t M, int64_t K, bool recip,
                         hipStream_t stream) {
    constexpr int E = 16 / DType<DT>::bytes;
    const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0;
    static_assert(kLaneElems % E == 0, "lane chunks");
    if (aligned) {
        const int ngroups = static_cast<int>(K / kRotGroup);
        const int rpb = fused_rows_per_block(ngroups);
        const int threads = (4 * rpb * ngroups + kWave - 1) / kWave * kWave;
        const int quads = threads / 4;
        const dim3 grid(static_cast<unsigned>((M + rpb - 1) / rpb));
        hipLaunchKernelGGL((convrot_quant_rows<DT>), grid, dim3(threads), quads * sizeof(float), stream, x, q,
                           xs, M, static_cast<int>(K), rpb, recip ? 1 : 0);
    } else {
        launch_fused_generic<DT, kActNone>(x, q, xs, M, K, recip, nullptr, 0.0f, stream);
    }
}

// Fused route with an input activation (act != 0): the LDS-row kernel.
template <int DT>
static void launch_fused_act(int act, const void* x, int8_t* q, float* xs, int64_t M, int64_t K, bool recip,
                             const void* w, float eps, hipStream_t stream) {
    switch (act) {
        case kActGeluTanh: launch_fused_generic<DT, kActGeluTanh>(x, q, xs, M, K, recip, w, eps, stream); break;
        case kActSwiGLU: launch_fused_generic<DT, kActSwiGLU>(x, q, xs, M, K, recip, w, eps, stream); break;
        case kActRmsNorm: launch_fused_generic<DT, kActRmsNorm>(x, q, xs, M, K, recip, w, eps, stream); break;
        default: launch_fused_generic<DT, kActSiTU>(x, q, xs, M, K, recip, w, eps, stream); break;
    }
}

void launch_convrot_quant_act(const void* x, int x_dtype, int act, const void* w, float eps, int8_t* q, float* xs,
                              int64_t M, int64_t K, bool recip, hipStream_t stream) {
    if (x_dtype == W8A8_BF16) launch_fused_act<W8A8_BF16>(act, x, q, xs, M, K, recip, w, eps, stream);
    else if (x_dtype == W8A8_F16) launch_fused_act<W8A8_F16>(act, x, q, xs, M, K, recip, w, eps, stream);
    else launch_fused_act<W8A8_F32>(act, x, q, xs, M, K, recip, w, eps, stream);
}

void launch_convrot_quant(const void* x, int x_dtype, int8_t* q, float* xs, int64_t M, int64_t K,
                          bool recip, hipStream_t stream) {
    if (x_dtype == W8A8_BF16) launch_fused<W8A8_BF16>(x, q, xs, M, K, recip, stream);
    else if (x_dtype == W8A8_F16) launch_fused<W8A8_F16>(x, q, xs, M, K, recip, stream);
    else launch_fused<W8A8_F32>(x, q, xs, M, K, recip, stream);
}

template <int DT>
static void launch_rotate_dt(const void* x, void* y, int64_t M, int64_t K, int64_t G, hipStream_t stream) {
    const bool vec = G <= kRotGroup && K % kLaneElems == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(y) % 16 == 0;
    if (vec) {
        const int64_t chunks = M * K / kLaneElems;
        const dim3 grid(static_cast<unsigned>((chunks + 255) / 256));
        if (G == 4) hipLaunchKernelGGL((convrot_rotate_vec<DT, 4>), grid, dim3(256), 0, stream, x, y, chunks);
        else if (G == 16) hipLaunchKernelGGL((convrot_rotate_vec<DT, 16>), grid, dim3(256), 0, stream, x, y, chunks);
        else if (G == 64) hipLaunchKernelGGL((convrot_rotate_vec<DT, 64>), grid, dim3(256), 0, stream, x, y, chunks);
        else hipLaunchKernelGGL((convrot_rotate_vec<DT, 256>), grid, dim3(256), 0, stream, x, y, chunks);
        return;
    }
    const size_t lds = G * sizeof(float);
    if (lds > 32 * 1024)
        (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&convrot_rotate_generic<DT>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
    const dim3 grid(static_cast<unsigned>(M * (K / G)));
    hipLaunchKernelGGL((convrot_rotate_generic<DT>), grid, dim3(256), lds, stream, x, y, K, static_cast<int>(G));
}

void launch_convrot_rotate(const void* x, int x_dtype, void* y, int64_t M, int64_t K, int64_t G,
                           hipStream_t stream) {
    if (x_dtype == W8A8_BF16) launch_rotate_dt<W8A8_BF16>(x, y, M, K, G, stream);
    else if (x_dtype == W8A8_F16) launch_rotate_dt<W8A8_F16>(x, y, M, K, G, stream);
    else launch_rotate_dt<W8A8_F32>(x, y, M, K, G, stream);
}

}  // namespace w8a8
