// M = 1 / 2 INT8 GEMV with the dequant epilogue, for gfx950.
//
// Replaces Kitchen's int8_gemv2_dequant_warp_kernel / int8_gemv_dequant_warp_kernel
// (native/comfy-port/kitchen/int8_linear.cu:628-708, launcher :1800-1854): the
// adaLN modulation projection, M = 2 rows (conditional + unconditional), a
// weight-streaming, HBM-bound kernel.
//
// Layout of the work: each block stages the M activation rows in LDS and every
// wave copies its chunks into registers (K <= 64 lanes * XC chunks * 16 B),
// then walks output channels RPW at a time with a grid stride, streaming each
// weight row once with 128-bit non-temporal loads (all chunks of a row in
// flight at once)
// and v_dot4_i32_i8 (sdot4), reducing the per-lane partial dot products with a
// wave64 butterfly.  Larger K re-reads the activation chunks from L1 instead
// of holding them.  K % 16 != 0 or unaligned operands take the generic kernel
// (one wave per channel, byte loads).
#include "w8a8_common.h"

namespace w8a8 {

template <int ODT>
__device__ __forceinline__ float load_bias(const void* bias, int64_t n) {
    return DType<ODT>::load(static_cast<const typename DType<ODT>::storage*>(bias)[n]);
}

template <int ODT>
__device__ __forceinline__ void store_out(void* out, int64_t idx, float v) {
    static_cast<typename DType<ODT>::storage*>(out)[idx] = DType<ODT>::store(v);
}

__device__ __forceinline__ int dot16(const uint4 a, const uint4 b, int acc) {
    acc = __builtin_amdgcn_sdot4(static_cast<int>(a.x), static_cast<int>(b.x), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(a.y), static_cast<int>(b.y), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(a.z), static_cast<int>(b.z), acc, false);
    acc = __builtin_amdgcn_sdot4(static_cast<int>(a.w), static_cast<int>(b.w), acc, false);
    return acc;
}

// XC: activation chunks per lane held in registers (0 = stream them from cache).
// Launched with kGemvThreads threads per block.
constexpr int kGemvThreads = 512;

template <int ODT, int MR, int RPW, int XC>
__global__ __launch_bounds__(kGemvThreads) void gemv_vec(const int8_t* __restrict__ q,
                                                         const int8_t* __restrict__ w,
                                                         const float* __restrict__ xs,
                                                         const float* __restrict__ ws, int64_t ws_size,
                                                         const void* __restrict__ bias, Residual res,
                                                         void* __restrict__ out, int64_t N, int64_t K,
                                                         int gelu) {
    const int lane = threadIdx.x % kWave;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * (blockDim.x / kWave);
    const int64_t nchunks = K / 16;
    const uint4* qv = reinterpret_cast<const uint4*>(q);
    const int64_t stride = nwaves * RPW;
    int64_t n0 = wave * RPW;

    // Weight chunks of RPW rows: all of them are loaded before the first dot
    // product, so one memory round trip covers them; lanes past K load chunk 0
    // again and multiply it by their zero activation chunk.
    uint4 wv[RPW][XC > 0 ? XC : 1];
    auto load_rows = [&](int64_t nb) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int64_t n = nb + r < N ? nb + r : N - 1;
#pragma unroll
            for (int j = 0; j < (XC > 0 ? XC : 1); ++j) {
                const int64_t c = lane + j * kWave;
                wv[r][j] = load_stream(reinterpret_cast<const uint4*>(w + n * K) + (c < nchunks ? c : 0));
            }
        }
    };
    // XC > 0: the block stages the M activation rows in LDS once (one pass of
    // 16-byte loads) and every wave takes its chunks from there, instead of
    // each wave loading them from L2.
    uint4 xr[MR][XC > 0 ? XC : 1];
    if constexpr (XC > 0) {
        __shared__ uint4 xl[MR * XC * kWave];
        for (int64_t i = threadIdx.x; i < MR * nchunks; i += blockDim.x) xl[i] = qv[i];
        __syncthreads();
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int j = 0; j < XC; ++j) {
                const int64_t c = lane + j * kWave;
                xr[m][j] = c < nchunks ? xl[m * nchunks + c] : make_uint4(0, 0, 0, 0);
            }
    }
    float xsc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) xsc[m] = xs[m];

    for (; n0 < N; n0 += stride) {
        int acc[MR][RPW];
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[m][r] = 0;

        if constexpr (XC > 0) {
            // (a prefetch of the next rows here raises the register count past
            // 64 and so the occupancy below 8 waves per SIMD: measured slower)
            load_rows(n0);
#pragma unroll
            for (int j = 0; j < XC; ++j)
#pragma unroll
                for (int r = 0; r < RPW; ++r)
#pragma unroll
                    for (int m = 0; m < MR; ++m) acc[m][r] = dot16(xr[m][j], wv[r][j], acc[m][r]);
        } else {
            for (int64_t c = lane; c < nchunks; c += kWave) {
                uint4 xv[MR];
#pragma unroll
                for (int m = 0; m < MR; ++m) xv[m] = qv[m * nchunks + c];
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const int64_t n = n0 + r < N ? n0 + r : N - 1;
                    const uint4 wc = reinterpret_cast<const uint4*>(w + n * K)[c];
#pragma unroll
                    for (int m = 0; m < MR; ++m) acc[m][r] = dot16(xv[m], wc, acc[m][r]);
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int r = 0; r < RPW; ++r) acc[m][r] = wave_sum(acc[m][r]);

        if (lane < RPW) {
            // lane r stores channel n0 + r (all lanes hold every reduced sum)
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                if (r != lane) continue;
                const int64_t n = n0 + r;
                if (n < N) {
                    const float wsn = ws[ws_size == 1 ? 0 : n];
                    const float b = bias ? load_bias<ODT>(bias, n) : 0.0f;
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        float v = epilogue_value<ODT>(acc[m][r], xsc[m], wsn, b, gelu != 0);
                        if (res.resid) v = residual_value<ODT>(v, res, m, static_cast<int>(n), static_cast<int>(N));
                        store_out<ODT>(out, m * N + n, v);
                    }
                }
            }
        }
    }
}

// Any K / alignment: one wave per output channel, byte loads.
template <int ODT>
__global__ __launch_bounds__(256) void gemv_generic(const int8_t* __restrict__ q,
                                                    const int8_t* __restrict__ w,
                                                    const float* __restrict__ xs,
                                                    const float* __restrict__ ws,
                                                    int64_t ws_size, const void* __restrict__ bias,
                                                    Residual res, void* __restrict__ out, int64_t M,
                                                    int64_t N, int64_t K, int gelu) {
    const int lane = threadIdx.x % kWave;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave;
    if (n >= N) return;
    for (int64_t m = 0; m < M; ++m) {
        int acc = 0;
        for (int64_t k = lane; k < K; k += kWave)
            acc += static_cast<int>(q[m * K + k]) * static_cast<int>(w[n * K + k]);
        acc = wave_sum(acc);
        if (lane == 0) {
            const float b = bias ? load_bias<ODT>(bias, n) : 0.0f;
            float v = epilogue_value<ODT>(acc, xs[m], ws[ws_size == 1 ? 0 : n], b, gelu != 0);
            if (res.resid) v = residual_value<ODT>(v, res, m, static_cast<int>(n), static_cast<int>(N));
            store_out<ODT>(out, m * N + n, v);
        }
    }
}

template <int ODT, int MR, int RPW, int XC>
static void launch_gemv_vec(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                            int64_t ws_size, const void* bias, const Residual& res, void* out, int64_t N, int64_t K,
                            int gelu, int blocks, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_vec<ODT, MR, RPW, XC>), dim3(blocks), dim3(kGemvThreads), 0, stream, q, w, xs,
                       ws, ws_size, bias, res, out, N, K, gelu);
}

template <int ODT, int MR>
static void gemv_dispatch_m(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                            int64_t ws_size, const void* bias, const Residual& res, void* out, int64_t N, int64_t K,
                            int gelu, hipStream_t stream) {
    // One channel per wave iteration and 32 waves per CU (8 per SIMD), each
    // walking its channels with a grid stride: at the adaLN shape (K = 3072,
    // N = 18432) this measured fastest of 1-9 channels per wave, 256- to
    // 1024-thread blocks and 4096-18432 waves.
    constexpr int RPW = 1;
    constexpr int kWavesPerBlock = kGemvThreads / kWave;
    const int64_t waves_needed = (N + RPW - 1) / RPW;
    int64_t blocks = (waves_needed + kWavesPerBlock - 1) / kWavesPerBlock;
    if (blocks > 8192 / kWavesPerBlock) blocks = 8192 / kWavesPerBlock;
    const int64_t nchunks = K / 16;
    const int b = static_cast<int>(blocks);
    if (nchunks <= 64) launch_gemv_vec<ODT, MR, RPW, 1>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, b, stream);
    else if (nchunks <= 128) launch_gemv_vec<ODT, MR, RPW, 2>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, b, stream);
    else if (nchunks <= 192) launch_gemv_vec<ODT, MR, RPW, 3>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, b, stream);
    else if (nchunks <= 256) launch_gemv_vec<ODT, MR, RPW, 4>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, b, stream);
    else if (nchunks <= 384) launch_gemv_vec<ODT, MR, RPW, 6>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, b, stream);
    else launch_gemv_vec<ODT, MR, RPW, 0>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, b, stream);
}

template <int ODT>
static void gemv_dispatch(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                          int64_t ws_size, const void* bias, const Residual& res, void* out,
                          int64_t M, int64_t N, int64_t K, int gelu, hipStream_t stream) {
    const bool vec = K % 16 == 0 && reinterpret_cast<uintptr_t>(q) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(w) % 16 == 0 && (M == 1 || M == 2);
    if (vec) {
        if (M == 1) gemv_dispatch_m<ODT, 1>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, stream);
        else gemv_dispatch_m<ODT, 2>(q, w, xs, ws, ws_size, bias, res, out, N, K, gelu, stream);
        return;
    }
    const dim3 grid(static_cast<unsigned>((N + 3) / 4));
    hipLaunchKernelGGL((gemv_generic<ODT>), grid, dim3(256), 0, stream, q, w, xs, ws, ws_size, bias,
                       res, out, M, N, K, gelu);
}

// res == nullptr: no residual.
void launch_gemv(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                 int64_t ws_size, const void* bias, const Residual* res, void* out, int out_dtype,
                 int64_t M, int64_t N, int64_t K, bool gelu, hipStream_t stream) {
    const Residual r = res ? *res : Residual{nullptr, 0, nullptr};
    const int g = gelu ? 1 : 0;
    switch (out_dtype) {
        case W8A8_BF16: gemv_dispatch<W8A8_BF16>(q, w, xs, ws, ws_size, bias, r, out, M, N, K, g, stream); break;
        case W8A8_F16: gemv_dispatch<W8A8_F16>(q, w, xs, ws, ws_size, bias, r, out, M, N, K, g, stream); break;
        default: gemv_dispatch<W8A8_F32>(q, w, xs, ws, ws_size, bias, r, out, M, N, K, g, stream); break;
    }
}

}  // namespace w8a8
