// Host-side dispatch of the W8A8 GEMM kernels (w8a8_gemm_kernels.h): choice
// of main loop and tile configuration (gemm_config) and the C-ABI-facing
// launchers.  The per-dtype instantiations of gemm_dispatch live in
// w8a8_gemm_{bf16,f16,f32}.hip.
#include "w8a8_gemm_launch.h"

namespace w8a8 {

bool gemm_mfma_supported(const void* a, size_t a_elem, const int8_t* w, int64_t M, int64_t N,
                         int64_t K) {
    return K % 16 == 0 && M < (1ll << 31) / 2 && N < (1ll << 31) / 2 &&
           reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
           M * K * static_cast<int64_t>(a_elem) < (1ll << 40);
}

// Compute units of the current device (cached per device).
int device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = n;
    }
    return cus[dev];
}

// Default tile choice among the three one-block-per-CU configurations: the
// estimated time of a shape is (rounds of tiles over the CUs) x (tile area),
// divided by the configuration's measured per-area speed relative to
// 256 x 192.  Without GELU (the mean over the DiT's QKV / out / FFN-down
// GEMMs at M = 11712 and 19904): 256 x 256 1.10, 384 x 192 1.09; both load
// 15% fewer bytes per MFMA operation than 256 x 192.  With the GELU epilogue
// (FFN-up at both M, same box): 256 x 256 1.07, 384 x 192 0.975, whose LDS
// has no room for the GELU table and whose write-out evaluates the formula.
// With these factors the choice is the fastest measured, or within 1% of it,
// at all eight shapes.  192-token tiles cut M = 11712 exactly; 384 x 192
// tiles fill the N = 3072 GEMMs in 2 rounds of 488 tiles (95%), where
// 256 x 256 makes 552 tiles (3 rounds, 72% full).
static int default_tile(int64_t M, int64_t N, bool gelu) {
    const int64_t cus = device_cus();
    auto cost = [&](int64_t bn, int64_t bm, double speed) {
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        return static_cast<double>((tiles + cus - 1) / cus) * static_cast<double>(bn * bm) / speed;
    };
    const double c0 = cost(256, 192, 1.0), c1 = cost(256, 256, gelu ? 1.07 : 1.10),
                 c2 = cost(384, 192, gelu ? 0.975 : 1.09);
    if (c1 < c0 && c1 <= c2) return W8A8_GEMM_TILE_256x256;
    if (c2 < c0) return W8A8_GEMM_TILE_384x192;
    return W8A8_GEMM_TILE_256x192;
}

// The main loop w8a8_gemm_dequant runs for a shape (operands 16-byte aligned),
// its epilogue (GELU or not) and a requested tile (W8A8_GEMM_TILE_* code,
// AUTO = by shape).  A requested DMA tile that does not take the shape falls
// back to the automatic choice.
int gemm_config(int64_t M, int64_t N, int64_t K, int requested, bool gelu) {
    if (!(K % 16 == 0 && M < (1ll << 31) / 2 && N < (1ll << 31) / 2 && M * K < (1ll << 40)))
        return W8A8_GEMM_TILE_GENERIC;
    switch (requested) {
        case W8A8_GEMM_TILE_256x192: if (dma_fits<CfgN256M192W8>(K)) return requested; break;
        case W8A8_GEMM_TILE_256x256: if (dma_fits<CfgN256M256W8>(K)) return requested; break;
        case W8A8_GEMM_TILE_384x192: if (dma_fits<CfgN384M192W8>(K)) return requested; break;
        case W8A8_GEMM_TILE_256x128: if (dma_fits<CfgN256M128>(K)) return requested; break;
        case W8A8_GEMM_TILE_REGS: return requested;
        case W8A8_GEMM_TILE_GENERIC: return requested;
        default: break;
    }
    const int tile = default_tile(M, N, gelu);
    if (tile == W8A8_GEMM_TILE_256x256 && dma_fits<CfgN256M256W8>(K)) return tile;
    if (tile == W8A8_GEMM_TILE_384x192 && dma_fits<CfgN384M192W8>(K)) return tile;
    if (dma_fits<CfgN256M192W8>(K)) return W8A8_GEMM_TILE_256x192;
    if (dma_fits<CfgN256M128>(K)) return W8A8_GEMM_TILE_256x128;
    return W8A8_GEMM_TILE_REGS;
}

#define W8A8_GEMM_EXTERN(ODT, MODE, GELU)                                                          \
    extern template void gemm_dispatch<ODT, MODE, GELU>(const int8_t*, const int8_t*, const float*, const float*, \
                                                        int64_t, const void*, const Residual&, void*, int64_t,  \
                                                        int64_t, int64_t, int, hipStream_t);
W8A8_GEMM_EXTERN(W8A8_BF16, 0, false)
W8A8_GEMM_EXTERN(W8A8_BF16, 0, true)
W8A8_GEMM_EXTERN(W8A8_BF16, 2, false)
W8A8_GEMM_EXTERN(W8A8_F16, 0, false)
W8A8_GEMM_EXTERN(W8A8_F16, 0, true)
W8A8_GEMM_EXTERN(W8A8_F16, 2, false)
W8A8_GEMM_EXTERN(W8A8_F32, 0, false)
W8A8_GEMM_EXTERN(W8A8_F32, 0, true)
W8A8_GEMM_EXTERN(W8A8_F32, 2, false)
W8A8_GEMM_EXTERN(W8A8_F32, 1, false)
#undef W8A8_GEMM_EXTERN

// res == nullptr: no residual.  The int32 mode is instantiated once (f32
// storage type), the residual mode without GELU.
void launch_gemm(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                 int64_t ws_size, const void* bias, const Residual* res, void* out, int out_dtype,
                 int64_t M, int64_t N, int64_t K, bool gelu, bool int32_out, int tile, hipStream_t stream) {
    if (int32_out) {
        gemm_dispatch<W8A8_F32, 1, false>(q, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, tile, stream);
        return;
    }
#define W8A8_GEMM_CASE(ODT)                                                                       \
    if (out_dtype == ODT) {                                                                       \
        if (res) gemm_dispatch<ODT, 2, false>(q, w, xs, ws, ws_size, bias, *res, out, M, N, K, tile, stream); \
        else if (gelu) gemm_dispatch<ODT, 0, true>(q, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, tile, stream); \
        else gemm_dispatch<ODT, 0, false>(q, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, tile, stream); \
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
        if (gelu) launch_mfma<ODT, 0, true, XDT>(nullptr, x, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, stream); \
        else launch_mfma<ODT, 0, false, XDT>(nullptr, x, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, stream); \
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

// Standalone residual step over an existing output: out = O(fma(out, rscale, resid)).
// The reference's eager apply_residual (inference/src/int8_linear.rs:99-111),
// for routes whose epilogue did not fuse it.
template <int ODT>
__global__ __launch_bounds__(256) void residual_apply(void* __restrict__ out, const void* __restrict__ resid,
                                                      const void* __restrict__ rscale, int64_t rs_size,
                                                      int64_t M, int64_t N) {
    using OS = typename DType<ODT>::storage;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t n = idx % N;
    OS* o = static_cast<OS*>(out);
    const float s = DType<ODT>::load(static_cast<const OS*>(rscale)[rs_size == 1 ? 0 : n]);
    const float r = DType<ODT>::load(static_cast<const OS*>(resid)[idx]);
    o[idx] = DType<ODT>::store(fmaf(DType<ODT>::load(o[idx]), s, r));
}

void launch_residual(void* out, const void* resid, const void* rscale, int64_t rs_size, int dtype,
                     int64_t M, int64_t N, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((M * N + 255) / 256));
    switch (dtype) {
        case W8A8_BF16:
            hipLaunchKernelGGL((residual_apply<W8A8_BF16>), grid, dim3(256), 0, stream, out, resid, rscale, rs_size, M, N);
            break;
        case W8A8_F16:
            hipLaunchKernelGGL((residual_apply<W8A8_F16>), grid, dim3(256), 0, stream, out, resid, rscale, rs_size, M, N);
            break;
        default:
            hipLaunchKernelGGL((residual_apply<W8A8_F32>), grid, dim3(256), 0, stream, out, resid, rscale, rs_size, M, N);
            break;
    }
}

}  // namespace w8a8
