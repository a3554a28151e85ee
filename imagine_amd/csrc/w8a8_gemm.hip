// Host-side dispatch of the W8A8 GEMM kernels (w8a8_gemm_kernels.h): choice
// of main loop and tile configuration, launch, and the C-ABI-facing launchers.
#include <cstdlib>
#include <cstring>

#include "w8a8_gemm_kernels.h"

namespace w8a8 {

// ------------------------------------------------------------------ host side

constexpr int kBN = 256, kBM = 256, kBK = 64, kWN = 128, kWM = 128;
constexpr int kGroupM = 4;

constexpr Residual kNoResidual{nullptr, 0, nullptr};

template <int ODT, int MODE, bool GELU, int XDT>
static void launch_mfma(const int8_t* q, const void* x, const int8_t* w, const float* xs,
                        const float* ws, int64_t ws_size, const void* bias, const Residual& res,
                        void* out, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    const int tiles = static_cast<int>(((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN));
    hipLaunchKernelGGL((gemm_mfma<ODT, MODE, GELU, XDT, kBN, kBM, kBK, kWN, kWM>), dim3(tiles),
                       dim3(256), 0, stream, q, x, w, xs, ws, ws_size, bias, res, out,
                       static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), kGroupM);
}

bool gemm_mfma_supported(const void* a, size_t a_elem, const int8_t* w, int64_t M, int64_t N,
                         int64_t K) {
    return K % 16 == 0 && M < (1ll << 31) / 2 && N < (1ll << 31) / 2 &&
           reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0 &&
           M * K * static_cast<int64_t>(a_elem) < (1ll << 40);
}

// Main-loop configurations of the int8-input GEMM (weights BN x activations BM
// per block, wave tile WN x WM, BK bytes per K tile, ring depth, waves per SIMD).
//   N256M192W8: 8 waves of 64 x 96 on a 256 x 192 tile, 2-stage ring of
//               128-byte K tiles (112 KB of LDS), one block per CU.  The
//               default: 192-token tiles cut M = 11712 (2 x 5856) exactly and
//               fill the 256 CUs in rounds that are ~95% full at N = 3072,
//               9216 and 12288.
//   N256M256W8: 8 waves of 128 x 64 on a 256 x 256 tile, 2-stage ring of
//               128-byte K tiles (128 KB of LDS), one block per CU.
//   N256M128:   4 waves of 128 x 64 on a 256 x 128 tile, 3-stage ring of 64-byte
//               K tiles (72 KB), two blocks per CU.
//   N256M256:   4 waves of 128 x 128, 2-stage ring of 128-byte tiles, one wave
//               per SIMD.
//   N384M192W8: 8 waves of 96 x 96 on a 384 x 192 tile, 2-stage ring of
//               128-byte K tiles (144 KB of LDS, the staged output exactly
//               fills it), one block per CU.
using CfgN256M192W8 = DmaCfg<256, 192, 64, 96, 128, 2, 2>;
using CfgN256M256W8 = DmaCfg<256, 256, 128, 64, 128, 2, 2>;
using CfgN384M192W8 = DmaCfg<384, 192, 96, 96, 128, 2, 2>;
using CfgN256M128 = DmaCfg<256, 128, 128, 64, 64, 3, 2>;
using CfgN256M256 = DmaCfg<256, 256, 128, 128, 128, 2, 1>;

// W8A8_GEMM_MAINLOOP = n256m192w8 | n256m256w8 | n384m192w8 | n256m128 | n256m256 | regs
// forces one (a tuning knob; every choice produces identical results).  By
// default the shape picks among N256M192W8, N256M256W8 and N384M192W8
// (default_tile).
static int mainloop_choice() {
    static int choice = [] {
        const char* e = std::getenv("W8A8_GEMM_MAINLOOP");
        if (!e) return 5;
        if (std::strcmp(e, "regs") == 0) return 0;
        if (std::strcmp(e, "n256m128") == 0) return 1;
        if (std::strcmp(e, "n256m256") == 0) return 3;
        if (std::strcmp(e, "n256m256w8") == 0) return 4;
        if (std::strcmp(e, "n256m192w8") == 0) return 6;
        if (std::strcmp(e, "n384m192w8") == 0) return 7;
        return 5;
    }();
    return choice;
}

// W8A8_GEMM_GLOBAL_LOADS=1 forces the global_load_lds form (tuning knob;
// identical results).
static bool buffer_loads_disabled() {
    static bool off = [] {
        const char* e = std::getenv("W8A8_GEMM_GLOBAL_LOADS");
        return e && e[0] == '1';
    }();
    return off;
}

template <int ODT, int MODE, bool GELU, class C>
static void launch_dma(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                       int64_t ws_size, const void* bias, const Residual& res, void* out, int64_t M,
                       int64_t N, int64_t K, hipStream_t stream) {
    const int tiles = static_cast<int>(((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN));
    // buffer-resource loads take 32-bit offsets: both operands below 2 GiB
    const int64_t kBufLimit = (1ll << 31) - 4096;
    if (M * K < kBufLimit && N * K < kBufLimit && !buffer_loads_disabled())
        hipLaunchKernelGGL((gemm_mfma_dma<ODT, MODE, GELU, C, true>), dim3(tiles), dim3(C::kThreads), 0, stream,
                           q, w, xs, ws, ws_size, bias, res, out, static_cast<int>(M), static_cast<int>(N),
                           static_cast<int>(K), kGroupM);
    else
        hipLaunchKernelGGL((gemm_mfma_dma<ODT, MODE, GELU, C, false>), dim3(tiles), dim3(C::kThreads), 0, stream,
                           q, w, xs, ws, ws_size, bias, res, out, static_cast<int>(M), static_cast<int>(N),
                           static_cast<int>(K), kGroupM);
}

// Compute units of the current device (cached per device).
static int device_cus() {
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
// divided by the configuration's measured per-area speed (relative to
// 256 x 192 at the DiT shapes: 256 x 256 1.06, 384 x 192 1.045; both load
// 15% fewer bytes per MFMA operation than 256 x 192).  192-token tiles cut
// M = 11712 exactly; 384 x 192 tiles fill the N = 3072 GEMMs in 2 rounds of
// 488 tiles (95%), where 256 x 256 makes 552 tiles (3 rounds, 72% full).
// Returns 0 (256 x 192), 1 (256 x 256) or 2 (384 x 192).
static int default_tile(int64_t M, int64_t N) {
    const int64_t cus = device_cus();
    auto cost = [&](int64_t bn, int64_t bm, double speed) {
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        return static_cast<double>((tiles + cus - 1) / cus) * static_cast<double>(bn * bm) / speed;
    };
    const double c0 = cost(256, 192, 1.0), c1 = cost(256, 256, 1.06), c2 = cost(384, 192, 1.045);
    if (c1 < c0 && c1 <= c2) return 1;
    if (c2 < c0) return 2;
    return 0;
}

template <int ODT, int MODE, bool GELU>
static bool try_dma(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                    int64_t ws_size, const void* bias, const Residual& res, void* out, int64_t M,
                    int64_t N, int64_t K, hipStream_t stream) {
    const int choice = mainloop_choice();
    // whole K tiles only (the DMA ring has no tail masking)
    if (choice == 0) return false;
    const int tile = choice == 5 ? default_tile(M, N) : -1;
    if (tile == 1 && K % CfgN256M256W8::BK == 0) {
        launch_dma<ODT, MODE, GELU, CfgN256M256W8>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
        return true;
    }
    if ((tile == 2 || choice == 7) && K % CfgN384M192W8::BK == 0) {
        launch_dma<ODT, MODE, GELU, CfgN384M192W8>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
        return true;
    }
    if ((choice == 5 || choice == 6) && K % CfgN256M192W8::BK == 0) {
        launch_dma<ODT, MODE, GELU, CfgN256M192W8>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
        return true;
    }
    if (choice == 4 && K % CfgN256M256W8::BK == 0) {
        launch_dma<ODT, MODE, GELU, CfgN256M256W8>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
        return true;
    }
    if (choice == 3 && K % CfgN256M256::BK == 0) {
        launch_dma<ODT, MODE, GELU, CfgN256M256>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
        return true;
    }
    if (K % CfgN256M128::BK != 0) return false;
    launch_dma<ODT, MODE, GELU, CfgN256M128>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
    return true;
}

// One output mode of one output dtype: the DMA main loop where it applies, the
// register-staged main loop for other K % 16 == 0 shapes, else the generic kernel.
template <int ODT, int MODE, bool GELU>
static void gemm_dispatch(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                          int64_t ws_size, const void* bias, const Residual& res, void* out, int64_t M,
                          int64_t N, int64_t K, hipStream_t stream) {
    const bool fast = gemm_mfma_supported(q, 1, w, M, N, K);
    if (fast && try_dma<ODT, MODE, GELU>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream)) return;
    if (fast) launch_mfma<ODT, MODE, GELU, -1>(q, nullptr, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
    else hipLaunchKernelGGL((gemm_generic<ODT, MODE, GELU>), dim3(static_cast<unsigned>((M * N + 255) / 256)),
                            dim3(256), 0, stream, q, w, xs, ws, ws_size, bias, res, out, M, N, K);
}

// res == nullptr: no residual.  The int32 mode is instantiated once (f32
// storage type), the residual mode without GELU.
void launch_gemm(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                 int64_t ws_size, const void* bias, const Residual* res, void* out, int out_dtype,
                 int64_t M, int64_t N, int64_t K, bool gelu, bool int32_out, hipStream_t stream) {
    if (int32_out) {
        gemm_dispatch<W8A8_F32, 1, false>(q, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, stream);
        return;
    }
#define W8A8_GEMM_CASE(ODT)                                                                       \
    if (out_dtype == ODT) {                                                                       \
        if (res) gemm_dispatch<ODT, 2, false>(q, w, xs, ws, ws_size, bias, *res, out, M, N, K, stream); \
        else if (gelu) gemm_dispatch<ODT, 0, true>(q, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, stream); \
        else gemm_dispatch<ODT, 0, false>(q, w, xs, ws, ws_size, bias, kNoResidual, out, M, N, K, stream); \
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
