// Per-token dynamic absmax INT8 quantization for gfx950.
//
// Replaces Kitchen's quantize_int8_rowwise_kernel
// (native/comfy-port/kitchen/int8_linear.cu:184-227, launcher :1322-1371) with
// the numerics of the reference's CPU route (inference/src/eager.rs:94-171):
//   s = max(amax / 127, 1e-30);  q = clamp(rint(T(x / T(s))), -128, 127)
//
// Bandwidth kernel.  A row is held in registers between its two passes (the
// reference re-reads it from memory): 1 wave per row up to 128 16-byte chunks
// (K = 1024 for 16-bit inputs), 4 waves per row up to 2048 chunks; each lane
// issues 128-bit loads, the absmax is a wave64 butterfly (plus a 4-entry LDS
// exchange for 4-wave rows), and the int8 codes leave as 64-bit stores.
// Rows that do not fit, or unaligned operands, take the generic kernel.
#include <algorithm>

#include "w8a8_common.h"

namespace w8a8 {

// W waves per row (1 or 4), CPL 16-byte chunks per lane, RPW rows per wave
// group (the dispatch uses 1: two rows per wave measured slower at the DiT
// shapes).  Every load of the group's rows is issued before any arithmetic,
// and the rows stay in registers as raw 16-bit data (converted again in the
// quantize pass, one shift each).
template <int DT, int W, int CPL, int RPW, bool GELU, bool SCALES_ONLY>
__global__ __launch_bounds__(256) void quant_rows_vec(const void* __restrict__ xv,
                                                      int8_t* __restrict__ q,
                                                      float* __restrict__ xs, int64_t M,
                                                      int64_t K, int recip) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;          // elements per 16-byte chunk
    constexpr int GROUPS = 4 / W;             // wave groups per 256-thread block
    const int tid = threadIdx.x % (kWave * W);
    const int grp = threadIdx.x / (kWave * W);
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * GROUPS + grp) * RPW;
    const int64_t nchunks = K / E;
    __shared__ float wave_amax[RPW][4];

    uint4 raw[RPW][CPL];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const bool row_ok = row0 + r < M;
        const uint4* src = reinterpret_cast<const uint4*>(
            static_cast<const char*>(xv) + (row_ok ? row0 + r : 0) * K * D::bytes);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = tid + static_cast<int64_t>(j) * kWave * W;
            raw[r][j] = (row_ok && c < nchunks) ? load_stream(src + c) : make_uint4(0, 0, 0, 0);
        }
    }
    auto elem = [&](int r, int j, int i) {
        const typename D::storage* e = reinterpret_cast<const typename D::storage*>(&raw[r][j]);
        return D::load(e[i]);
    };
    // The input activation once per element: raw holds T(gelu_tanh(x)) from
    // here on, so both passes read activated values (exact for each dtype,
    // see gelu_bits in w8a8_common.h).
    if constexpr (GELU) {
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                uint32_t* wv = reinterpret_cast<uint32_t*>(&raw[r][j]);
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    if constexpr (D::bytes == 4) {
                        wv[h] = __float_as_uint(gelu_f32(__uint_as_float(wv[h])));
                    } else {
                        wv[h] = gelu_x2<DT>(wv[h]);
                    }
                }
            }
    }

    float amax[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < E; ++i) m = fmaxf(m, fabsf(elem(r, j, i)));
        amax[r] = wave_max(m);
    }
    if constexpr (W > 1) {
        const int wave = threadIdx.x / kWave;
        if ((threadIdx.x % kWave) == 0) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) wave_amax[r][wave] = amax[r];
        }
        __syncthreads();
        const int first = grp * W;
#pragma unroll
        for (int r = 0; r < RPW; ++r)
#pragma unroll
            for (int w = 0; w < W; ++w) amax[r] = fmaxf(amax[r], wave_amax[r][first + w]);
    }

    // The quantize pass converts the raw 16-bit data again: the empty asm makes
    // the registers opaque, so the compiler cannot keep every converted float
    // of the absmax pass alive (which would cost the occupancy the loads need).
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int j = 0; j < CPL; ++j)
            asm volatile("" : "+v"(raw[r][j].x), "+v"(raw[r][j].y), "+v"(raw[r][j].z), "+v"(raw[r][j].w));

#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t row = row0 + r;
        if (row >= M) break;
        const float s = row_scale<DT>(amax[r], recip != 0);
        if (tid == 0) xs[row] = s;
        if constexpr (SCALES_ONLY) continue;
        const RowQuant rq = row_quant<DT>(s);
        int8_t* dst = q + row * K;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = tid + static_cast<int64_t>(j) * kWave * W;
            if (c >= nchunks) break;
            if constexpr (E == 8) {
                uint2 packed;
                packed.x = quant4_packed<DT>(elem(r, j, 0), elem(r, j, 1), elem(r, j, 2), elem(r, j, 3), rq);
                packed.y = quant4_packed<DT>(elem(r, j, 4), elem(r, j, 5), elem(r, j, 6), elem(r, j, 7), rq);
                *reinterpret_cast<uint2*>(dst + c * E) = packed;
            } else {
                *reinterpret_cast<uint32_t*>(dst + c * E) =
                    quant4_packed<DT>(elem(r, j, 0), elem(r, j, 1), elem(r, j, 2), elem(r, j, 3), rq);
            }
        }
    }
}

// Grid-stride form of quant_rows_vec (RPW = 1) for rows of several waves:
// wave group g of the grid quantizes rows g, g + G, g + 2 G, ... (G = wave
// groups in the grid) and loads its next row while reducing and storing the
// current one, so each wave keeps two rows' loads in flight.  The iteration
// count is the same for every wave of the grid (rows past M are masked), as
// the cross-wave absmax exchange is a block barrier.
template <int DT, int W, int CPL, bool GELU, bool SCALES_ONLY>
__global__ __launch_bounds__(256) void quant_rows_stream(const void* __restrict__ xv, int8_t* __restrict__ q,
                                                         float* __restrict__ xs, int64_t M, int64_t K, int recip) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;
    constexpr int GROUPS = 4 / W;
    const int tid = threadIdx.x % (kWave * W);
    const int grp = threadIdx.x / (kWave * W);
    const int wave = threadIdx.x / kWave;
    const int64_t G = static_cast<int64_t>(gridDim.x) * GROUPS;
    const int64_t g = static_cast<int64_t>(blockIdx.x) * GROUPS + grp;
    const int64_t iters = (M + G - 1) / G;
    const int64_t nchunks = K / E;
    __shared__ float wave_amax[2][4];   // by iteration parity: no barrier between write rounds

    auto load_row = [&](uint4 (&raw)[CPL], int64_t row) {
        const bool ok = row < M;
        const uint4* src = reinterpret_cast<const uint4*>(static_cast<const char*>(xv) + (ok ? row : 0) * K * D::bytes);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = tid + static_cast<int64_t>(j) * kWave * W;
            raw[j] = (ok && c < nchunks) ? load_stream(src + c) : make_uint4(0, 0, 0, 0);
        }
    };
    uint4 cur[CPL], nxt[CPL];
    load_row(cur, g);
    for (int64_t it = 0; it < iters; ++it) {
        const int64_t row = g + it * G;
        if (it + 1 < iters) load_row(nxt, row + G);
        if constexpr (GELU) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                uint32_t* wv = reinterpret_cast<uint32_t*>(&cur[j]);
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    if constexpr (D::bytes == 4) wv[h] = __float_as_uint(gelu_f32(__uint_as_float(wv[h])));
                    else wv[h] = gelu_x2<DT>(wv[h]);
                }
            }
        }
        auto elem = [&](int j, int i) {
            const typename D::storage* e = reinterpret_cast<const typename D::storage*>(&cur[j]);
            return D::load(e[i]);
        };
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < E; ++i) m = fmaxf(m, fabsf(elem(j, i)));
        float amax = wave_max(m);
        const int par = static_cast<int>(it & 1);
        if ((threadIdx.x % kWave) == 0) wave_amax[par][wave] = amax;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < W; ++w) amax = fmaxf(amax, wave_amax[par][grp * W + w]);
        if (row < M) {
            const float s = row_scale<DT>(amax, recip != 0);
            if (tid == 0) xs[row] = s;
            if constexpr (!SCALES_ONLY) {
                const RowQuant rq = row_quant<DT>(s);
                int8_t* dst = q + row * K;
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    const int64_t c = tid + static_cast<int64_t>(j) * kWave * W;
                    if (c >= nchunks) break;
                    if constexpr (E == 8) {
                        uint2 packed;
                        packed.x = quant4_packed<DT>(elem(j, 0), elem(j, 1), elem(j, 2), elem(j, 3), rq);
                        packed.y = quant4_packed<DT>(elem(j, 4), elem(j, 5), elem(j, 6), elem(j, 7), rq);
                        *reinterpret_cast<uint2*>(dst + c * E) = packed;
                    } else {
                        *reinterpret_cast<uint32_t*>(dst + c * E) =
                            quant4_packed<DT>(elem(j, 0), elem(j, 1), elem(j, 2), elem(j, 3), rq);
                    }
                }
            }
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) cur[j] = nxt[j];
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
        if constexpr (GELU) f = gelu_value<DT>(f);
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
        if constexpr (GELU) f = gelu_value<DT>(f);
        q[row * K + k] = static_cast<int8_t>(quant_elem<DT>(f, rq));
    }
}

template <int DT, int W, int CPL, int RPW, bool GELU, bool SO>
static void launch_vec(const void* x, int8_t* q, float* xs, int64_t M, int64_t K, int recip,
                       hipStream_t stream) {
    const int64_t rows = (4 / W) * RPW;
    // Rows of several waves stream: two rows per wave group (M = 11712 bf16:
    // K = 3072 24.3 -> 23.5 us, K = 12288 83.7 -> 81.0 us; three or six rows
    // per group measured no better).
    constexpr int kStreamRows = 2;
    if constexpr (W > 1) {
        const int64_t per_block = (4 / W) * kStreamRows;
        const dim3 grid(static_cast<unsigned>((M + per_block - 1) / per_block));
        hipLaunchKernelGGL((quant_rows_stream<DT, W, CPL, GELU, SO>), grid, dim3(256), 0, stream, x, q, xs, M, K,
                           recip);
        return;
    }
    const dim3 grid(static_cast<unsigned>((M + rows - 1) / rows));
    hipLaunchKernelGGL((quant_rows_vec<DT, W, CPL, RPW, GELU, SO>), grid, dim3(256), 0, stream, x, q,
                       xs, M, K, recip);
}

// Rows of up to 128 chunks take one wave each; longer rows two or four waves
// in the streaming kernel (K = 3072 bf16, 384 chunks: two waves of 3 chunks
// per lane, every lane busy; four waves of 2 and one wave of 6 measured
// slower; a plain copy of the same bytes 21.8 us).
template <int DT, bool GELU, bool SO>
static bool dispatch_vec(const void* x, int8_t* q, float* xs, int64_t M, int64_t K, int recip,
                         hipStream_t stream) {
    constexpr int E = 16 / DType<DT>::bytes;
    const int64_t nchunks = K / E;
    if (nchunks <= 64) launch_vec<DT, 1, 1, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 128) launch_vec<DT, 1, 2, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 256) launch_vec<DT, 4, 1, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 384) launch_vec<DT, 2, 3, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 512) launch_vec<DT, 4, 2, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 768) launch_vec<DT, 4, 3, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 1024) launch_vec<DT, 4, 4, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 1536) launch_vec<DT, 4, 6, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
    else if (nchunks <= 2048) launch_vec<DT, 4, 8, 1, GELU, SO>(x, q, xs, M, K, recip, stream);
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

// ---------------------------------------------------------------- input activations

// Sum of a double over a 256-thread block (4 waves); part holds 4 doubles.
__device__ __forceinline__ double block_sum_256(double v, double* part) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = v;
    __syncthreads();
    return (part[0] + part[1]) + (part[2] + part[3]);
}

// 1 / sqrt(mean(x^2) + eps) of a row of K values, as ATen's rms_norm forms it
// in fp32.  The squares are summed in double: exact for rows of ordinary
// dynamic range, so the fp32 mean does not depend on the summation order.
template <int DT>
__device__ __forceinline__ float row_rstd(const typename DType<DT>::storage* x, int64_t K, float eps, double* part) {
    double acc = 0.0;
    for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
        const double v = DType<DT>::load(x[k]);
        acc += v * v;
    }
    const double total = block_sum_256(acc, part);
    return 1.0f / sqrtf(static_cast<float>(total / static_cast<double>(K)) + eps);
}

// The crate's eager input activation (inference/src/int8_linear.rs:37-97) of
// one row per block of 256 threads: x is [M, K] ([M, 2K] for the gated
// ones), the activated value of column k is act_eager (RMSNorm: T(x * rstd *
// w)).  WRITE: store the activated [M, K] tensor in T (the ConvRot rotate
// route rotates it next); else quantize it per token, two passes over the row
// (the activation recomputed in the second), codes and scale as
// quant_rows_generic.
template <int DT, int ACT, bool WRITE>
__global__ __launch_bounds__(256) void act_rows(const void* __restrict__ xv, const void* __restrict__ wv, float eps,
                                                int8_t* __restrict__ q, float* __restrict__ xs,
                                                void* __restrict__ yv, int64_t K, int recip) {
    using D = DType<DT>;
    using S = typename D::storage;
    __shared__ double dpart[4];
    __shared__ float part[4];
    const int64_t row = blockIdx.x;
    const int64_t in_w = act_gated(ACT) ? 2 * K : K;
    const S* x = static_cast<const S*>(xv) + row * in_w;
    float rstd = 1.0f;
    if constexpr (ACT == kActRmsNorm) rstd = row_rstd<DT>(x, K, eps, dpart);
    auto value = [&](int64_t k) -> float {
        const float a = D::load(x[k]);
        if constexpr (ACT == kActRmsNorm) return D::round((a * rstd) * D::load(static_cast<const S*>(wv)[k]));
        else if constexpr (act_gated(ACT)) return act_eager<DT, ACT>(a, D::load(x[K + k]));
        else return act_eager<DT, ACT>(a, 0.0f);
    };
    if constexpr (WRITE) {
        S* y = static_cast<S*>(yv) + row * K;
        for (int64_t k = threadIdx.x; k < K; k += blockDim.x) y[k] = D::store(value(k));
    } else {
        float amax = 0.0f;
        for (int64_t k = threadIdx.x; k < K; k += blockDim.x) amax = fmaxf(amax, fabsf(value(k)));
        amax = wave_max(amax);
        if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
        const float s = row_scale<DT>(amax, recip != 0);
        if (threadIdx.x == 0) xs[row] = s;
        const RowQuant rq = row_quant<DT>(s);
        for (int64_t k = threadIdx.x; k < K; k += blockDim.x)
            q[row * K + k] = static_cast<int8_t>(quant_elem<DT>(value(k), rq));
    }
}

template <int DT, int ACT>
static void act_rows_dt(const void* x, const void* w, float eps, int8_t* q, float* xs, void* y, int64_t M, int64_t K,
                        int recip, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(M));
    if (y) hipLaunchKernelGGL((act_rows<DT, ACT, true>), grid, dim3(256), 0, stream, x, w, eps, q, xs, y, K, recip);
    else hipLaunchKernelGGL((act_rows<DT, ACT, false>), grid, dim3(256), 0, stream, x, w, eps, q, xs, y, K, recip);
}

template <int DT>
static void act_rows_act(int act, const void* x, const void* w, float eps, int8_t* q, float* xs, void* y, int64_t M,
                         int64_t K, int recip, hipStream_t stream) {
    switch (act) {
        case kActGeluTanh: act_rows_dt<DT, kActGeluTanh>(x, w, eps, q, xs, y, M, K, recip, stream); break;
        case kActSwiGLU: act_rows_dt<DT, kActSwiGLU>(x, w, eps, q, xs, y, M, K, recip, stream); break;
        case kActRmsNorm: act_rows_dt<DT, kActRmsNorm>(x, w, eps, q, xs, y, M, K, recip, stream); break;
        default: act_rows_dt<DT, kActSiTU>(x, w, eps, q, xs, y, M, K, recip, stream); break;
    }
}

// y != nullptr: write the activated [M, K] tensor to y; else quantize it to q, xs.
void launch_act_rows(const void* x, int x_dtype, int act, const void* w, float eps, int8_t* q, float* xs, void* y,
                     int64_t M, int64_t K, bool recip, hipStream_t stream) {
    const int r = recip ? 1 : 0;
    if (x_dtype == W8A8_BF16) act_rows_act<W8A8_BF16>(act, x, w, eps, q, xs, y, M, K, r, stream);
    else if (x_dtype == W8A8_F16) act_rows_act<W8A8_F16>(act, x, w, eps, q, xs, y, M, K, r, stream);
    else act_rows_act<W8A8_F32>(act, x, w, eps, q, xs, y, M, K, r, stream);
}

// ---------------------------------------------------------------- tensorwise

// Tensorwise quantization: one scale for the whole tensor (the reference's
// quantize_int8_tensorwise, inference/src/eager.rs:134-151).  Three kernels
// on one stream: the absolute maximum into the scale slot (an atomic max of
// the bits of non-negative floats, which order like the floats), the codes
// from it, then the scale written over it once every block has read it.

__global__ void tensor_amax_clear(float* acc) {
    if (threadIdx.x == 0) acc[0] = 0.0f;
}

template <int DT>
__global__ __launch_bounds__(256) void tensor_amax(const void* __restrict__ xv, int64_t n, bool vec,
                                                   unsigned* __restrict__ acc_bits) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;
    __shared__ float part[4];
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    float m = 0.0f;
    if (vec) {
        const uint4* x = static_cast<const uint4*>(xv);
        for (int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < n / E; c += stride) {
            const uint4 raw = x[c];
            const typename D::storage* e = reinterpret_cast<const typename D::storage*>(&raw);
#pragma unroll
            for (int i = 0; i < E; ++i) m = fmaxf(m, fabsf(D::load(e[i])));
        }
    } else {
        const typename D::storage* x = static_cast<const typename D::storage*>(xv);
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
            m = fmaxf(m, fabsf(D::load(x[i])));
    }
    m = wave_max(m);
    if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        m = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
        atomicMax(acc_bits, __float_as_uint(m));
    }
}

// scale_src holds the given scale (given) or the maximum (else).
template <int DT>
__global__ __launch_bounds__(256) void tensor_quant(const void* __restrict__ xv, int8_t* __restrict__ q,
                                                    int64_t n, bool vec, const float* __restrict__ scale_src,
                                                    bool given, int recip) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;
    const float s = given ? scale_src[0] : row_scale<DT>(scale_src[0], recip != 0);
    const RowQuant rq = row_quant<DT>(s);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    if (vec) {
        const uint4* x = static_cast<const uint4*>(xv);
        for (int64_t c = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; c < n / E; c += stride) {
            const uint4 raw = x[c];
            const typename D::storage* e = reinterpret_cast<const typename D::storage*>(&raw);
            if constexpr (E == 8) {
                uint2 packed;
                packed.x = quant4_packed<DT>(D::load(e[0]), D::load(e[1]), D::load(e[2]), D::load(e[3]), rq);
                packed.y = quant4_packed<DT>(D::load(e[4]), D::load(e[5]), D::load(e[6]), D::load(e[7]), rq);
                reinterpret_cast<uint2*>(q)[c] = packed;
            } else {
                reinterpret_cast<uint32_t*>(q)[c] =
                    quant4_packed<DT>(D::load(e[0]), D::load(e[1]), D::load(e[2]), D::load(e[3]), rq);
            }
        }
    } else {
        const typename D::storage* x = static_cast<const typename D::storage*>(xv);
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
            q[i] = static_cast<int8_t>(quant_elem<DT>(D::load(x[i]), rq));
    }
}

template <int DT>
__global__ void tensor_scale_store(float* scale, int recip) {
    if (threadIdx.x == 0) scale[0] = row_scale<DT>(scale[0], recip != 0);
}

template <int DT>
static void tensorwise_dt(const void* x, int8_t* q, float* scale, int64_t n, bool given, bool recip,
                          hipStream_t stream) {
    constexpr int E = 16 / DType<DT>::bytes;
    const bool vec = n % E == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(q) % E == 0;
    const int64_t work = vec ? n / E : n;
    const dim3 grid(static_cast<unsigned>(std::max<int64_t>(1, std::min<int64_t>((work + 255) / 256, 4096))));
    if (!given) {
        hipLaunchKernelGGL(tensor_amax_clear, dim3(1), dim3(64), 0, stream, scale);
        hipLaunchKernelGGL((tensor_amax<DT>), grid, dim3(256), 0, stream, x, n, vec,
                           reinterpret_cast<unsigned*>(scale));
    }
    hipLaunchKernelGGL((tensor_quant<DT>), grid, dim3(256), 0, stream, x, q, n, vec, scale, given,
                       recip ? 1 : 0);
    if (!given) hipLaunchKernelGGL((tensor_scale_store<DT>), dim3(1), dim3(64), 0, stream, scale, recip ? 1 : 0);
}

void launch_quantize_tensorwise(const void* x, int x_dtype, int8_t* q, float* scale, int64_t n, bool given,
                                bool recip, hipStream_t stream) {
    if (x_dtype == W8A8_BF16) tensorwise_dt<W8A8_BF16>(x, q, scale, n, given, recip, stream);
    else if (x_dtype == W8A8_F16) tensorwise_dt<W8A8_F16>(x, q, scale, n, given, recip, stream);
    else tensorwise_dt<W8A8_F32>(x, q, scale, n, given, recip, stream);
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
