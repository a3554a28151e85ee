// INT8 x INT8 -> INT32 GEMM with the fused dequant epilogue, for gfx950 MFMA.
//
// Replaces Kitchen's CUTLASS FusedInt8Gemm (cutlass_gemm_int8.cu:63-120, entry
// launch_cutlass_int8_dequant :373-388) and, in the int32 mode, the cuBLASLt
// int32 GEMM (cublas_gemm_int8.cu:176-221):
//   out[m, n] = O( fma(float(sum_k q[m,k] * w[n,k]) * xs[m], ws[n], bias[n]) )
//
// Tiling (CDNA4, wave64):
//   * block tile BN (weight rows n) x BM (activation rows m) x BK (k bytes),
//     256 threads = 4 waves in a 2 x 2 grid, each wave WN x WM;
//   * v_mfma_i32_32x32x32_i8: the weight tile is the MFMA A operand and the
//     activation tile the B operand, so the accumulator registers of a lane
//     hold 4 consecutive output channels n of one token m -> 8-byte bf16 stores;
//   * K tiles staged through LDS, double buffered: global 128-bit loads of
//     tile k+1 are in flight while tile k is multiplied; LDS rows are padded by
//     16 bytes so the 128-bit fragment reads of 8/16 consecutive rows hit
//     distinct banks;
//   * tile order: blocks are remapped so that the blocks one XCD runs are
//     contiguous in tile space (the hardware deals blocks to the 8 XCDs
//     round-robin), then grouped GROUP_M activation tiles at a time, so each
//     XCD's L2 sees a small window of weight and activation rows.
// With XQ the activation tile is loaded as bf16/fp16 and quantized while it is
// written to LDS (row constants from the row scales computed beforehand);
// the codes are bit-identical to the standalone quantizer's.
#include "w8a8_common.h"

namespace w8a8 {

constexpr int kXcds = 8;

struct TileCoord {
    int tm, tn;
};

// Bijective remap of the launch order so that consecutive blocks dealt to one
// XCD take consecutive tiles, then a grouped (GROUP_M tall) walk of tile space.
__device__ __forceinline__ TileCoord tile_of_block(int bid, int tiles_m, int tiles_n, int group_m) {
    const int total = tiles_m * tiles_n;
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = bid % kXcds;
    const int logical = xcd * per + (xcd < rem ? xcd : rem) + bid / kXcds;
    const int group_size = group_m * tiles_n;
    const int group = logical / group_size;
    const int first_m = group * group_m;
    const int gm = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
    const int in_group = logical % group_size;
    TileCoord t;
    t.tm = first_m + in_group % gm;
    t.tn = in_group / gm;
    return t;
}

template <int BN, int BM, int BK, int WN, int WM>
struct GemmShape {
    static constexpr int kThreads = 256;
    static constexpr int kWaves = 4;
    static_assert((BN / WN) * (BM / WM) == kWaves, "4 waves per block");
    static constexpr int TN = WN / 32, TM = WM / 32;   // MFMA tiles per wave
    static constexpr int kRow = BK + 16;                // padded LDS row, bytes
    static constexpr int kChunksPerRow = BK / 16;
    static constexpr int kWChunks = BN * kChunksPerRow / kThreads;   // per thread
    static constexpr int kXChunks = BM * kChunksPerRow / kThreads;   // per thread (int8 source)
    static constexpr int kStage = (BN + BM) * kRow;                  // bytes per LDS stage
};

// MODE: 0 = dtype output with bias (if any) and optional GELU; 1 = int32 output.
template <int ODT, int MODE, bool GELU, int XDT, int BN, int BM, int BK, int WN, int WM>
__global__ __launch_bounds__(256, 1) void gemm_mfma(
    const int8_t* __restrict__ q, const void* __restrict__ xsrc, const int8_t* __restrict__ w,
    const float* __restrict__ xs, const float* __restrict__ ws, int64_t ws_size,
    const void* __restrict__ bias, void* __restrict__ out, int M, int N, int K, int group_m) {
    using S = GemmShape<BN, BM, BK, WN, WM>;
    constexpr bool XQ = XDT >= 0;          // activation quantized in the tile load
    constexpr int XDTq = XQ ? XDT : W8A8_BF16;
    using XD = DType<XDTq>;
    constexpr int XE = 16 / XD::bytes;     // float elements per 16-byte source chunk (XQ)
    constexpr int kXSrcChunksPerRow = XQ ? BK / XE : S::kChunksPerRow;
    constexpr int kXLoads = BM * kXSrcChunksPerRow / S::kThreads;

    __shared__ __attribute__((aligned(16))) int8_t lds[2 * S::kStage];

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    const TileCoord tc = tile_of_block(blockIdx.x, tiles_m, tiles_n, group_m);
    const int m_base = tc.tm * BM, n_base = tc.tn * BN;

    const int t = threadIdx.x;
    const int lane = t % kWave, wave = t / kWave;
    const int wave_n = (wave % (BN / WN)) * WN;
    const int wave_m = (wave / (BN / WN)) * WM;
    const int KT = (K + BK - 1) / BK;

    // ---- global -> register staging
    uint4 wreg[S::kWChunks];
    uint4 xreg[kXLoads];
    // per-row quantizer constants of the rows this thread loads (XQ)
    RowQuant xrq[XQ ? kXLoads : 1];
    if constexpr (XQ) {
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int cid = t + i * S::kThreads;
            int m = m_base + cid / kXSrcChunksPerRow;
            m = m < M ? m : M - 1;
            xrq[i] = row_quant<XDTq>(xs[m]);
        }
    }

    auto load_tile = [&](int kt) {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < S::kWChunks; ++i) {
            const int cid = t + i * S::kThreads;
            const int r = cid / S::kChunksPerRow, c = cid % S::kChunksPerRow;
            int n = n_base + r;
            n = n < N ? n : N - 1;
            const int k = k0 + c * 16;
            wreg[i] = k < K ? *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(n) * K + k)
                            : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int cid = t + i * S::kThreads;
            const int r = cid / kXSrcChunksPerRow, c = cid % kXSrcChunksPerRow;
            int m = m_base + r;
            m = m < M ? m : M - 1;
            if constexpr (XQ) {
                const int k = k0 + c * XE;
                const char* base = static_cast<const char*>(xsrc) +
                                   (static_cast<int64_t>(m) * K + k) * XD::bytes;
                xreg[i] = k < K ? *reinterpret_cast<const uint4*>(base) : make_uint4(0, 0, 0, 0);
            } else {
                const int k = k0 + c * 16;
                xreg[i] = k < K ? *reinterpret_cast<const uint4*>(q + static_cast<int64_t>(m) * K + k)
                                : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto store_tile = [&](int stage) {
        int8_t* wl = lds + stage * S::kStage;
        int8_t* xl = wl + BN * S::kRow;
#pragma unroll
        for (int i = 0; i < S::kWChunks; ++i) {
            const int cid = t + i * S::kThreads;
            const int r = cid / S::kChunksPerRow, c = cid % S::kChunksPerRow;
            *reinterpret_cast<uint4*>(wl + r * S::kRow + c * 16) = wreg[i];
        }
#pragma unroll
        for (int i = 0; i < kXLoads; ++i) {
            const int cid = t + i * S::kThreads;
            const int r = cid / kXSrcChunksPerRow, c = cid % kXSrcChunksPerRow;
            if constexpr (XQ) {
                const typename XD::storage* e = reinterpret_cast<const typename XD::storage*>(&xreg[i]);
                int code[XE];
#pragma unroll
                for (int j = 0; j < XE; ++j) code[j] = quant_elem<XDTq>(XD::load(e[j]), xrq[i]);
                if constexpr (XE == 8) {
                    uint2 p;
                    p.x = pack4_i8(code[0], code[1], code[2], code[3]);
                    p.y = pack4_i8(code[4], code[5], code[6], code[7]);
                    *reinterpret_cast<uint2*>(xl + r * S::kRow + c * 8) = p;
                } else {
                    *reinterpret_cast<uint32_t*>(xl + r * S::kRow + c * 4) =
                        pack4_i8(code[0], code[1], code[2], code[3]);
                }
            } else {
                *reinterpret_cast<uint4*>(xl + r * S::kRow + c * 16) = xreg[i];
            }
        }
    };

    v16i acc[S::TN][S::TM];
#pragma unroll
    for (int i = 0; i < S::TN; ++i)
#pragma unroll
        for (int j = 0; j < S::TM; ++j) acc[i][j] = v16i{};

    if (KT > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();

    const int frag_row = lane % 32;
    const int frag_k = (lane / 32) * 16;
    for (int kt = 0; kt < KT; ++kt) {
        const int stage = kt & 1;
        if (kt + 1 < KT) load_tile(kt + 1);
        const int8_t* wl = lds + stage * S::kStage;
        const int8_t* xl = wl + BN * S::kRow;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            v4i a[S::TN], b[S::TM];
#pragma unroll
            for (int i = 0; i < S::TN; ++i)
                a[i] = *reinterpret_cast<const v4i*>(wl + (wave_n + i * 32 + frag_row) * S::kRow +
                                                     ks * 32 + frag_k);
#pragma unroll
            for (int j = 0; j < S::TM; ++j)
                b[j] = *reinterpret_cast<const v4i*>(xl + (wave_m + j * 32 + frag_row) * S::kRow +
                                                     ks * 32 + frag_k);
#pragma unroll
            for (int i = 0; i < S::TN; ++i)
#pragma unroll
                for (int j = 0; j < S::TM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < KT) store_tile(stage ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane holds, for tile (i, j), token m = .. + lane % 32 and
    // channels n = .. + 8 * g + 4 * (lane / 32) + {0,1,2,3} in acc[i][j][4g..4g+3].
    const int lane_m = lane % 32;
    const int lane_n = 4 * (lane / 32);
    float xsv[S::TM];
    if constexpr (MODE == 0) {
#pragma unroll
        for (int j = 0; j < S::TM; ++j) {
            const int m = m_base + wave_m + j * 32 + lane_m;
            xsv[j] = xs[m < M ? m : M - 1];
        }
    }
    const bool vec_ok = (N % 4) == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
#pragma unroll
    for (int i = 0; i < S::TN; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n0 = n_base + wave_n + i * 32 + 8 * g + lane_n;
            float wsv[4], bv[4];
            if constexpr (MODE == 0) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int n = n0 + e < N ? n0 + e : N - 1;
                    wsv[e] = ws[ws_size == 1 ? 0 : n];
                    bv[e] = bias ? DType<ODT>::load(
                                       static_cast<const typename DType<ODT>::storage*>(bias)[n])
                                 : 0.0f;
                }
            }
#pragma unroll
            for (int j = 0; j < S::TM; ++j) {
                const int m = m_base + wave_m + j * 32 + lane_m;
                if (m >= M) continue;
                const int64_t row = static_cast<int64_t>(m) * N;
                if constexpr (MODE == 1) {
                    int32_t* o = static_cast<int32_t*>(out) + row;
                    if (vec_ok && n0 + 3 < N) {
                        *reinterpret_cast<v4i*>(o + n0) =
                            v4i{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n0 + e < N) o[n0 + e] = acc[i][j][4 * g + e];
                    }
                } else {
                    float v[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = epilogue_value<ODT>(acc[i][j][4 * g + e], xsv[j], wsv[e], bv[e], GELU);
                    using OS = typename DType<ODT>::storage;
                    OS* o = static_cast<OS*>(out) + row;
                    if (vec_ok && n0 + 3 < N) {
                        if constexpr (ODT == W8A8_F32) {
                            *reinterpret_cast<float4*>(o + n0) = make_float4(v[0], v[1], v[2], v[3]);
                        } else {
                            uint2 p;
                            p.x = static_cast<uint32_t>(DType<ODT>::store(v[0])) |
                                  (static_cast<uint32_t>(DType<ODT>::store(v[1])) << 16);
                            p.y = static_cast<uint32_t>(DType<ODT>::store(v[2])) |
                                  (static_cast<uint32_t>(DType<ODT>::store(v[3])) << 16);
                            *reinterpret_cast<uint2*>(o + n0) = p;
                        }
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            if (n0 + e < N) o[n0 + e] = DType<ODT>::store(v[e]);
                    }
                }
            }
        }
    }
}

// Generic GEMM for shapes the MFMA kernel does not take (K % 16 != 0,
// unaligned operands, fused quant of fp32 inputs): one thread per output.
template <int ODT, int MODE, bool GELU>
__global__ __launch_bounds__(256) void gemm_generic(const int8_t* __restrict__ q,
                                                    const int8_t* __restrict__ w,
                                                    const float* __restrict__ xs,
                                                    const float* __restrict__ ws, int64_t ws_size,
                                                    const void* __restrict__ bias,
                                                    void* __restrict__ out, int64_t M, int64_t N,
                                                    int64_t K) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t m = idx / N, n = idx % N;
    int acc = 0;
    for (int64_t k = 0; k < K; ++k) acc += static_cast<int>(q[m * K + k]) * static_cast<int>(w[n * K + k]);
    if constexpr (MODE == 1) {
        static_cast<int32_t*>(out)[idx] = acc;
    } else {
        const float b = bias ? DType<ODT>::load(static_cast<const typename DType<ODT>::storage*>(bias)[n]) : 0.0f;
        static_cast<typename DType<ODT>::storage*>(out)[idx] =
            DType<ODT>::store(epilogue_value<ODT>(acc, xs[m], ws[ws_size == 1 ? 0 : n], b, GELU));
    }
}

// Standalone dequant of int32 accumulators (the reference's cuBLAS route's
// second kernel, int8_linear.cu:517-583).
template <int ODT, bool GELU>
__global__ __launch_bounds__(256) void dequant_linear(const int32_t* __restrict__ acc,
                                                      const float* __restrict__ xs,
                                                      const float* __restrict__ ws, int64_t ws_size,
                                                      const void* __restrict__ bias,
                                                      void* __restrict__ out, int64_t M, int64_t N) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t m = idx / N, n = idx % N;
    const float b = bias ? DType<ODT>::load(static_cast<const typename DType<ODT>::storage*>(bias)[n]) : 0.0f;
    static_cast<typename DType<ODT>::storage*>(out)[idx] =
        DType<ODT>::store(epilogue_value<ODT>(acc[idx], xs[m], ws[ws_size == 1 ? 0 : n], b, GELU));
}

// ------------------------------------------------------------------ host side

constexpr int kBN = 256, kBM = 256, kBK = 64, kWN = 128, kWM = 128;
constexpr int kGroupM = 4;

template <int ODT, int MODE, bool GELU, int XDT>
static void launch_mfma(const int8_t* q, const void* x, const int8_t* w, const float* xs,
                        const float* ws, int64_t ws_size, const void* bias, void* out, int64_t M,
                        int64_t N, int64_t K, hipStream_t stream) {
    const int tiles = static_cast<int>(((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN));
    hipLaunchKernelGGL((gemm_mfma<ODT, MODE, GELU, XDT, kBN, kBM, kBK, kWN, kWM>), dim3(tiles),
                       dim3(256), 0, stream, q, x, w, xs, ws, ws_size, bias, out,
                       static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), kGroupM);
}

bool gemm_mfma_supported(const void* a, size_t a_elem, const int8_t* w, int64_t M, int64_t N,
                         int64_t K) {
    return K % 16 == 0 && M < (1ll << 31) / 2 && N < (1ll << 31) / 2 &&
           reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
           M * K * static_cast<int64_t>(a_elem) < (1ll << 40);
}

template <int ODT, bool GELU>
static void gemm_dispatch_odt(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                              int64_t ws_size, const void* bias, void* out, int64_t M, int64_t N,
                              int64_t K, bool int32_out, hipStream_t stream) {
    const bool fast = gemm_mfma_supported(q, 1, w, M, N, K);
    if (int32_out) {
        if (fast) launch_mfma<ODT, 1, false, -1>(q, nullptr, w, xs, ws, ws_size, bias, out, M, N, K, stream);
        else hipLaunchKernelGGL((gemm_generic<ODT, 1, false>), dim3(static_cast<unsigned>((M * N + 255) / 256)),
                                dim3(256), 0, stream, q, w, xs, ws, ws_size, bias, out, M, N, K);
        return;
    }
    if (fast) launch_mfma<ODT, 0, GELU, -1>(q, nullptr, w, xs, ws, ws_size, bias, out, M, N, K, stream);
    else hipLaunchKernelGGL((gemm_generic<ODT, 0, GELU>), dim3(static_cast<unsigned>((M * N + 255) / 256)),
                            dim3(256), 0, stream, q, w, xs, ws, ws_size, bias, out, M, N, K);
}

void launch_gemm(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                 int64_t ws_size, const void* bias, void* out, int out_dtype, int64_t M, int64_t N,
                 int64_t K, bool gelu, bool int32_out, hipStream_t stream) {
#define W8A8_GEMM_CASE(ODT)                                                                       \
    if (out_dtype == ODT) {                                                                       \
        if (gelu && !int32_out) gemm_dispatch_odt<ODT, true>(q, w, xs, ws, ws_size, bias, out, M, N, K, false, stream); \
        else gemm_dispatch_odt<ODT, false>(q, w, xs, ws, ws_size, bias, out, M, N, K, int32_out, stream); \
        return;                                                                                   \
    }
    W8A8_GEMM_CASE(W8A8_BF16)
    W8A8_GEMM_CASE(W8A8_F16)
    W8A8_GEMM_CASE(W8A8_F32)
#undef W8A8_GEMM_CASE
}

// Fused quant + GEMM; returns false when the shape/dtype needs the unfused path.
bool launch_gemm_xq(const void* x, int x_dtype, const float* xs, const int8_t* w, const float* ws,
                    int64_t ws_size, const void* bias, void* out, int out_dtype, int64_t M,
                    int64_t N, int64_t K, bool gelu, hipStream_t stream) {
    if (x_dtype == W8A8_F32) return false;
    if (!gemm_mfma_supported(x, 2, w, M, N, K)) return false;
#define W8A8_XQ_CASE(ODT, XDT)                                                                    \
    if (out_dtype == ODT && x_dtype == XDT) {                                                     \
        if (gelu) launch_mfma<ODT, 0, true, XDT>(nullptr, x, w, xs, ws, ws_size, bias, out, M, N, K, stream); \
        else launch_mfma<ODT, 0, false, XDT>(nullptr, x, w, xs, ws, ws_size, bias, out, M, N, K, stream); \
        return true;                                                                              \
    }
    W8A8_XQ_CASE(W8A8_BF16, W8A8_BF16)
    W8A8_XQ_CASE(W8A8_F16, W8A8_BF16)
    W8A8_XQ_CASE(W8A8_F32, W8A8_BF16)
    W8A8_XQ_CASE(W8A8_BF16, W8A8_F16)
    W8A8_XQ_CASE(W8A8_F16, W8A8_F16)
    W8A8_XQ_CASE(W8A8_F32, W8A8_F16)
#undef W8A8_XQ_CASE
    return false;
}

void launch_dequant(const int32_t* acc, const float* xs, const float* ws, int64_t ws_size,
                    const void* bias, void* out, int out_dtype, int64_t M, int64_t N, bool gelu,
                    hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((M * N + 255) / 256));
#define W8A8_DQ_CASE(ODT)                                                                         \
    if (out_dtype == ODT) {                                                                       \
        if (gelu) hipLaunchKernelGGL((dequant_linear<ODT, true>), grid, dim3(256), 0, stream, acc, xs, ws, ws_size, bias, out, M, N); \
        else hipLaunchKernelGGL((dequant_linear<ODT, false>), grid, dim3(256), 0, stream, acc, xs, ws, ws_size, bias, out, M, N); \
        return;                                                                                   \
    }
    W8A8_DQ_CASE(W8A8_BF16)
    W8A8_DQ_CASE(W8A8_F16)
    W8A8_DQ_CASE(W8A8_F32)
#undef W8A8_DQ_CASE
}

}  // namespace w8a8
