// Host-side launch templates of the W8A8 GEMM (kernels: w8a8_gemm_kernels.h).
// gemm_dispatch<ODT, MODE, GELU> is instantiated once per output dtype in
// w8a8_gemm_{bf16,f16,f32}.hip (compiled in parallel); the shape -> main loop
// choice (gemm_config) and the C-ABI-facing launchers are in w8a8_gemm.hip.
#pragma once

#include "w8a8_gemm_kernels.h"

namespace w8a8 {

constexpr int kBN = 256, kBM = 256, kBK = 64, kWN = 128, kWM = 128;
constexpr int kGroupM = 4;

constexpr Residual kNoResidual{nullptr, 0, nullptr};

template <int ODT, int MODE, bool GELU, int XDT>
inline void launch_mfma(const int8_t* q, const void* x, const int8_t* w, const float* xs,
                        const float* ws, int64_t ws_size, const void* bias, const Residual& res,
                        void* out, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
    const int tiles = static_cast<int>(((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN));
    hipLaunchKernelGGL((gemm_mfma<ODT, MODE, GELU, XDT, kBN, kBM, kBK, kWN, kWM>), dim3(tiles),
                       dim3(256), 0, stream, q, x, w, xs, ws, ws_size, bias, res, out,
                       static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), kGroupM);
}

// Main-loop configurations of the int8-input GEMM (weights BN x activations BM
// per block, wave tile WN x WM, BK bytes per K tile, ring depth, waves per SIMD).
//   N256M192W8: 8 waves of 64 x 96 on a 256 x 192 tile, 2-stage ring of
//               128-byte K tiles (112 KB of LDS), one block per CU.
//   N256M256W8: 8 waves of 128 x 64 on a 256 x 256 tile, 2-stage ring of
//               128-byte K tiles (128 KB of LDS), one block per CU.
//   N384M192W8: 8 waves of 96 x 96 on a 384 x 192 tile, 2-stage ring of
//               128-byte K tiles (144 KB of LDS, the staged output exactly
//               fills it), one block per CU.
//   N256M128:   4 waves of 128 x 64 on a 256 x 128 tile, 3-stage ring of 64-byte
//               K tiles (72 KB), two blocks per CU: the K % 64 == 0 shapes the
//               128-byte rings do not take.
using CfgN256M192W8 = DmaCfg<256, 192, 64, 96, 128, 2, 2>;
using CfgN256M256W8 = DmaCfg<256, 256, 128, 64, 128, 2, 2>;
using CfgN384M192W8 = DmaCfg<384, 192, 96, 96, 128, 2, 2>;
using CfgN256M128 = DmaCfg<256, 128, 128, 64, 64, 3, 2>;

// Compute units of the current device (cached per device; w8a8_gemm.hip).
int device_cus();

template <class C, int ODT, int MODE, bool GELU>
inline void launch_dma(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                       int64_t ws_size, const void* bias, const Residual& res, void* out, int64_t M,
                       int64_t N, int64_t K, hipStream_t stream) {
    const int tiles = static_cast<int>(((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN));
    // one block per CU looping over tiles, or one block per tile
    const int cus = device_cus();
    const int grid = DmaPlan<C, ODT, MODE>::kPersist && tiles > cus ? cus : tiles;
    hipLaunchKernelGGL((gemm_mfma_dma<ODT, MODE, GELU, C>), dim3(grid), dim3(C::kThreads), 0, stream, q, w, xs,
                       ws, ws_size, bias, res, out, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                       kGroupM);
}

// Whether configuration C takes the shape: whole K tiles (the DMA ring has no
// tail masking) and buffer offsets of one block's rows below 2^31.
template <class C>
inline bool dma_fits(int64_t K) {
    const int64_t rows = (C::BN > C::BM ? C::BN : C::BM) + 1;
    return K % C::BK == 0 && rows * K < (1ll << 31) - 4096;
}

// The main loop chosen for a shape, its epilogue and a requested
// W8A8_GEMM_TILE_* code (w8a8_gemm.hip).
int gemm_config(int64_t M, int64_t N, int64_t K, int requested, bool gelu);

// One output mode of one output dtype: the configuration gemm_config picks
// (the generic kernel also for unaligned operands).
template <int ODT, int MODE, bool GELU>
void gemm_dispatch(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                          int64_t ws_size, const void* bias, const Residual& res, void* out, int64_t M,
                          int64_t N, int64_t K, int requested, hipStream_t stream) {
    const bool aligned = reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(w) % 16 == 0;
    const int cfg = aligned ? gemm_config(M, N, K, requested, GELU) : W8A8_GEMM_TILE_GENERIC;
    switch (cfg) {
        case W8A8_GEMM_TILE_256x192:
            launch_dma<CfgN256M192W8, ODT, MODE, GELU>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
            return;
        case W8A8_GEMM_TILE_256x256:
            launch_dma<CfgN256M256W8, ODT, MODE, GELU>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
            return;
        case W8A8_GEMM_TILE_384x192:
            launch_dma<CfgN384M192W8, ODT, MODE, GELU>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
            return;
        case W8A8_GEMM_TILE_256x128:
            launch_dma<CfgN256M128, ODT, MODE, GELU>(q, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
            return;
        case W8A8_GEMM_TILE_REGS:
            launch_mfma<ODT, MODE, GELU, -1>(q, nullptr, w, xs, ws, ws_size, bias, res, out, M, N, K, stream);
            return;
        default:
            hipLaunchKernelGGL((gemm_generic<ODT, MODE, GELU>), dim3(static_cast<unsigned>((M * N + 255) / 256)),
                               dim3(256), 0, stream, q, w, xs, ws, ws_size, bias, res, out, M, N, K);
            return;
    }
}

}  // namespace w8a8
