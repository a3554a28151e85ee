// Per-token dynamic absmax INT8 quantization for gfx950.
//
// Replaces Kitchen's quantize_int8_rowwise_kernel
// (native/comfy-port/kitchen/int8_linear.cu:184-227, launcher :1322-1371) with
// the numerics of the reference's CPU route (inference/src/eager.rs:94-171):
//   s = max(amax / 127, 1e-30);  q = clamp(rint(T(x / T(s))), -128, 127)
//
// Bandwidth kernel.  A row is held in registers between its two passes (the
// reference re-reads it from memory): 1 wave per row up to 512 16-byte chunks
// (K = 4096 for 16-bit inputs), 4 waves per row up to 2048 chunks; each lane
// issues 128-bit loads, the absmax is a wave64 butterfly (plus a 4-entry LDS
// exchange for 4-wave rows), and the int8 codes leave as 64-bit stores.
// Rows that do not fit, or unaligned operands, take the generic kernel.
#include "w8a8_common.h"

namespace w8a8 {

template <int DT, int W, int CPL, bool GELU, bool SCALES_ONLY>
__global__ __launch_bounds__(256) void quant_rows_vec(const void* __restrict__ xv,
                                                      int8_t* __restrict__ q,
                                                      float* __restrict__ xs, int64_t M,
                                                      int64_t K, int recip) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;          // elements per 16-byte chunk
    constexpr int ROWS = 4 / W;               // rows per 256-thread block
    const int tid = threadIdx.x % (kWave * W);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * ROWS + threadIdx.x / (kWave * W);
    const int64_t nchunks = K / E;
    __shared__ float wave_amax[4];

    const bool row_ok = row < M;
    const uint4* src = reinterpret_cast<const uint4*>(
        static_cast<const char*>(xv) + (row_ok ? row : 0) * K * D::bytes);

    float v[CPL][E];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + static_cast<int64_t>(j) * kWave * W;
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (row_ok && c < nchunks) raw = src[c];
        const typename D::storage* e = reinterpret_cast<const typename D::storage*>(&raw);
#pragma unroll
        for (int i = 0; i < E; ++i) {
            float f = D::load(e[i]);
            if constexpr (GELU) f = D::round(gelu_tanh(f));
            v[j][i] = f;
            amax = fmaxf(amax, fabsf(f));
        }
    }
    amax = wave_max(amax);
    if constexpr (W > 1) {
        const int wave = threadIdx.x / kWave;
        if ((threadIdx.x % kWave) == 0) wave_amax[wave] = amax;
        __syncthreads();
        const int first = (threadIdx.x / (kWave * W)) * W;
#pragma unroll
        for (int w = 0; w < W; ++w) amax = fmaxf(amax, wave_amax[first + w]);
    }
    if (!row_ok) return;
    const float s = row_scale<DT>(amax, recip != 0);
    if (tid == 0) xs[row] = s;
    if constexpr (SCALES_ONLY) return;

    const RowQuant rq = row_quant<DT>(s);
    int8_t* dst = q + row * K;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + static_cast<int64_t>(j) * kWave * W;
        if (c >= nchunks) break;
        if constexpr (E == 8) {
            uint2 packed;
            packed.x = pack4_i8(quant_elem<DT>(v[j][0], rq), quant_elem<DT>(v[j][1], rq),
                                quant_elem<DT>(v[j][2], rq), quant_elem<DT>(v[j][3], rq));
            packed.y = pack4_i8(quant_elem<DT>(v[j][4], rq), quant_elem<DT>(v[j][5], rq),
                                quant_elem<DT>(v[j][6], rq), quant_elem<DT>(v[j][7], rq));
            *reinterpret_cast<uint2*>(dst + c * E) = packed;
        } else {
            uint32_t packed =
                pack4_i8(quant_elem<DT>(v[j][0], rq), quant_elem<DT>(v[j][1], rq),
                         quant_elem<DT>(v[j][2], rq), quant_elem<DT>(v[j][3], rq));
            *reinterpret_cast<uint32_t*>(dst + c * E) = packed;
        }
    }
}

// Any K, any alignment: one block per row, element loads, two passes.
template <int DT, bool GELU, bool SCALES_ONLY>
__global__ __launch_bounds__(256) void quant_rows_generic(const void* __restrict__ xv,
                                                          int8_t* __restrict__ q,
                                                          float* __restrict__ xs, int64_t M,
                                                          int64_t K, int recip) {
    using D = DType<DT>;
    const int64_t row = blockIdx.x;
    const typename D::storage* x = static_cast<const typename D::storage*>(xv) + row * K;
    __shared__ float part[4];
    float amax = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
        float f = D::load(x[k]);
        if constexpr (GELU) f = D::round(gelu_tanh(f));
        amax = fmaxf(amax, fabsf(f));
    }
    amax = wave_max(amax);
    if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float s = row_scale<DT>(amax, recip != 0);
    if (threadIdx.x == 0) xs[row] = s;
    if constexpr (SCALES_ONLY) return;
    const RowQuant rq = row_quant<DT>(s);
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
        float f = D::load(x[k]);
        if constexpr (GELU) f = D::round(gelu_tanh(f));
        q[row * K + k] = static_cast<int8_t>(quant_elem<DT>(f, rq));
    }
}

template <int DT, int W, int CPL, bool GELU, bool SO>
static void launch_vec(const void* x, int8_t* q, float* xs, int64_t M, int64_t K, int recip,
                       hipStream_t stream) {
    const int64_t rows = 4 / W;
    const dim3 grid(static_cast<unsigned>((M + rows - 1) / rows));
    hipLaunchKernelGGL((quant_rows_vec<DT, W, CPL, GELU, SO>), grid, dim3(256), 0, stream, x, q,
                       xs, M, K, recip);
}

template <int DT, bool GELU, bool SO>
static bool dispatch_vec(const void* x, int8_t* q, float* xs, int64_t M, int64_t K, int recip,
                         hipStream_t stream) {
    constexpr int E = 16 / DType<DT>::bytes;
    const int64_t nchunks = K / E;
    if (nchunks <= 64) launch_vec<DT, 1, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 128) launch_vec<DT, 1, 2, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 256) launch_vec<DT, 1, 4, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 384) launch_vec<DT, 1, 6, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 512) launch_vec<DT, 1, 8, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 1024) launch_vec<DT, 4, 4, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 1536) launch_vec<DT, 4, 6, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 2048) launch_vec<DT, 4, 8, GELU, SO>(x, q, xs, M, K, recip, stream);
    else return false;
    return true;
}

template <int DT, bool GELU, bool SO>
static void quant_dispatch_dt(const void* x, int8_t* q, float* xs, int64_t M, int64_t K,
                              int recip, hipStream_t stream) {
    constexpr int E = 16 / DType<DT>::bytes;
    const bool aligned = (reinterpret_cast<uintptr_t>(x) % 16 == 0) && (K % E == 0) &&
                         (SO || reinterpret_cast<uintptr_t>(q) % E == 0);
    if (aligned && dispatch_vec<DT, GELU, SO>(x, q, xs, M, K, recip, stream)) return;
    hipLaunchKernelGGL((quant_rows_generic<DT, GELU, SO>), dim3(static_cast<unsigned>(M)),
                       dim3(256), 0, stream, x, q, xs, M, K, recip);
}

// Host entry used by the C ABI: x_dtype is a W8A8_* code (validated by the caller).
void launch_quantize(const void* x, int x_dtype, int8_t* q, float* xs, int64_t M, int64_t K,
                     bool recip, bool gelu, bool scales_only, hipStream_t stream) {
#define W8A8_QUANT_CASE(DT)                                                                   \
    if (x_dtype == DT) {                                                                      \
        if (scales_only) {                                                                    \
            if (gelu) quant_dispatch_dt<DT, true, true>(x, q, xs, M, K, recip, stream);       \
            else quant_dispatch_dt<DT, false, true>(x, q, xs, M, K, recip, stream);           \
        } else {                                                                              \
            if (gelu) quant_dispatch_dt<DT, true, false>(x, q, xs, M, K, recip, stream);      \
            else quant_dispatch_dt<DT, false, false>(x, q, xs, M, K, recip, stream);          \
        }                                                                                     \
        return;                                                                               \
    }
    W8A8_QUANT_CASE(W8A8_BF16)
    W8A8_QUANT_CASE(W8A8_F16)
    W8A8_QUANT_CASE(W8A8_F32)
#undef W8A8_QUANT_CASE
}

}  // namespace w8a8
