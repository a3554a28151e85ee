// Device side of the W8A8 GEMM: kernel templates and their helpers.  The
// host-side dispatch that instantiates them is w8a8_gemm.hip.
//
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
#pragma once

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

// Epilogue shared by both main loops.  For MFMA tile (i, j) a lane holds token
// m = m_base + wave_m + 32 j + lane % 32 and channels
// n = n_base + wave_n + 32 i + 8 g + 4 (lane / 32) + {0,1,2,3} in acc[i][j][4g .. 4g+3].
// All accumulator indices are compile-time constants (static_for).
// MODE: 0 = output dtype, 1 = int32 accumulators, 2 = output dtype + residual.
template <int ODT, int MODE, bool GELU, int TN, int TM>
__device__ __forceinline__ void store_tiles(const v16i (&acc)[TN][TM], int lane, int m_base,
                                            int n_base, int wave_m, int wave_n, int M, int N,
                                            const float* __restrict__ xs,
                                            const float* __restrict__ ws, int64_t ws_size,
                                            const void* __restrict__ bias, const Residual& res,
                                            void* __restrict__ out) {
    const int lane_m = lane % 32;
    const int lane_n = 4 * (lane / 32);
    float xsv[TM];
    if constexpr (MODE != 1) {
        static_for<0, TM>([&](auto j) {
            const int m = m_base + wave_m + j * 32 + lane_m;
            xsv[j] = xs[m < M ? m : M - 1];
        });
    }
    const bool vec_ok = (N % 4) == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
    static_for<0, TN>([&](auto i) {
        static_for<0, 4>([&](auto g) {
            const int n0 = n_base + wave_n + i * 32 + 8 * g + lane_n;
            float wsv[4], bv[4];
            if constexpr (MODE != 1) {
                static_for<0, 4>([&](auto e) {
                    const int n = n0 + e < N ? n0 + e : N - 1;
                    wsv[e] = ws[ws_size == 1 ? 0 : n];
                    bv[e] = bias ? DType<ODT>::load(
                                       static_cast<const typename DType<ODT>::storage*>(bias)[n])
                                 : 0.0f;
                });
            }
            static_for<0, TM>([&](auto j) {
                const int m = m_base + wave_m + j * 32 + lane_m;
                if (m < M) {
                    const int64_t row = static_cast<int64_t>(m) * N;
                    if constexpr (MODE == 1) {
                        int32_t* o = static_cast<int32_t*>(out) + row;
                        if (vec_ok && n0 + 3 < N) {
                            *reinterpret_cast<v4i*>(o + n0) =
                                v4i{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                    acc[i][j][4 * g + 3]};
                        } else {
                            static_for<0, 4>([&](auto e) {
                                if (n0 + e < N) o[n0 + e] = acc[i][j][4 * g + e];
                            });
                        }
                    } else {
                        float v[4];
                        static_for<0, 4>([&](auto e) {
                            v[e] = epilogue_value<ODT>(acc[i][j][4 * g + e], xsv[j], wsv[e], bv[e], GELU);
                            if constexpr (MODE == 2) {
                                const int n = n0 + e < N ? n0 + e : N - 1;
                                v[e] = residual_value<ODT>(v[e], res, m, n, N);
                            }
                        });
                        using OS = typename DType<ODT>::storage;
                        OS* o = static_cast<OS*>(out) + row;
                        if (vec_ok && n0 + 3 < N) {
                            if constexpr (ODT == W8A8_F32) {
                                *reinterpret_cast<float4*>(o + n0) = make_float4(v[0], v[1], v[2], v[3]);
                            } else {
                                uint2 p;
                                p.x = DType<ODT>::store2(v[0], v[1]);
                                p.y = DType<ODT>::store2(v[2], v[3]);
                                *reinterpret_cast<uint2*>(o + n0) = p;
                            }
                        } else {
                            static_for<0, 4>([&](auto e) {
                                if (n0 + e < N) o[n0 + e] = DType<ODT>::store(v[e]);
                            });
                        }
                    }
                }
            });
        });
    });
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
    const void* __restrict__ bias, Residual res, void* __restrict__ out, int M, int N, int K,
    int group_m) {
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

    store_tiles<ODT, MODE, GELU, S::TN, S::TM>(acc, lane, m_base, n_base, wave_m, wave_n, M, N, xs, ws,
                                               ws_size, bias, res, out);
}

// ---------------------------------------------------------------- LDS-DMA main loop
//
// Same MFMA tiling and accumulator layout as gemm_mfma, but the K tiles travel
// from global memory straight into LDS (buffer_load_dwordx4 ... lds: each lane
// moves 16 bytes, a wave fills 1 KB of contiguous LDS), through a ring of
// STAGES buffers, so no VGPRs stage the tiles and no LDS write instructions
// are issued.  The LDS tile is unpadded (BK bytes per row).  Bank conflicts of
// the 128-bit fragment reads are avoided by an XOR swizzle of the 16-byte
// chunk index that depends only on row mod 32 (so it is a per-lane constant):
//   BK =  64 (4 chunks/row): chunk' = chunk ^ (((row >> 1) ^ (row >> 3)) & 3)
//   BK = 128 (8 chunks/row): chunk' = chunk ^ ((row & 7) ^ ((row >> 3) & 3))
//   BK =  96 (6 chunks/row): no swizzle; rows start 24 banks apart, so any 8
//                            consecutive rows read at one chunk are distinct
// Either makes the rows read in one LDS cycle (8 consecutive rows for a
// 128-byte-wide LDS, 16 for a 256-byte-wide one) land in distinct banks.  The
// swizzle is applied on the load side by choosing which global chunk each
// lane fetches.
//
// Blocks of 4 or 8 waves (a (BN / WN) x (BM / WM) wave grid).  OCC is the
// number of waves per SIMD the launch bounds ask for: 2 keeps each wave within
// 256 registers (128 of them accumulators), so two waves share every SIMD and
// one wave's epilogue and barrier waits run under the other's MFMAs (with
// 4-wave blocks, two blocks per CU).
//
// Synchronisation: one raw s_barrier per K tile, preceded by
// s_waitcnt vmcnt(loads of later tiles) lgkmcnt(0): the wave's own DMA for
// the tile about to be read has landed and its reads of the tile just
// consumed have completed, so after the barrier every wave may read the new
// tile and the buffer of the consumed one may be refilled.  The barrier is
// crossed before the last k32 substep of a tile, so the LDS latency of the
// next tile's first fragments hides under that substep's MFMAs.  Inside a
// substep the fragment reads of the next substep are interleaved one by one
// with the MFMAs (sched_group_barrier), which keeps two fragment sets live.
//
// Epilogue of 16-bit outputs: the block's dequantized tile is staged through
// the (then idle) LDS ring, rows of BN values with the 16-byte chunk index
// XOR-swizzled by the row, and leaves as full-row 16-byte-per-lane stores, so
// every output line is written whole.
template <int BK>
__device__ __forceinline__ int swz(int row) {
    if constexpr (BK == 64) return ((row >> 1) ^ (row >> 3)) & 3;
    else if constexpr (BK == 128) return (row & 7) ^ ((row >> 3) & 3);
    else return 0;   // BK = 96: the 96-byte pitch alone spreads 8 rows over distinct banks
}

// s_waitcnt immediate for gfx9: vmcnt = n (0..63), expcnt unconstrained, lgkmcnt = 0.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0x0 << 8) | (((N >> 4) & 3) << 14));
}

#define W8A8_LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

// Word 3 of a raw buffer resource on gfx9 (32-bit data format, no swizzle).
// Offsets are checked by the host to stay below 2^31 - the tile bytes.
constexpr int kBufferDword3 = 0x00020000;

// Buffer-resource LDS-DMA load of 16 bytes per lane from base + voff + soff.
// The buffer builtins exist only for the device target, so the resource is
// built here, in device-only code (a kernel template whose host-pass
// instantiation touches them gets no host launch stub); it is loop-invariant
// and hoisted by the compiler.
__device__ __forceinline__ void buffer_load_lds16(const void* base, int8_t* lds, uint32_t voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7fffffff, kBufferDword3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, W8A8_LDS_PTR(lds), 16, voff, soff, 0, 0);
#endif
}

// sched_group_barrier masks
constexpr int kSchedMfma = 0x008;
constexpr int kSchedVmem = 0x010;
constexpr int kSchedDsRead = 0x100;

template <int BN_, int BM_, int WN_, int WM_, int BK_, int STAGES_, int OCC_>
struct DmaCfg {
    static constexpr int BN = BN_, BM = BM_, WN = WN_, WM = WM_, BK = BK_, STAGES = STAGES_, OCC = OCC_;
    static constexpr int kWaves = (BN / WN) * (BM / WM);
    static_assert(kWaves == 4 || kWaves == 8, "4 or 8 waves per block");
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int TN = WN / 32, TM = WM / 32;       // MFMA tiles per wave
    static constexpr int CPR = BK / 16;                    // 16-byte chunks per LDS row
    static constexpr int KS = BK / 32;                     // k32 substeps per tile
    static constexpr int kTileBytes = (BN + BM) * BK;      // one stage: weights then activations
    static_assert(kTileBytes % 1024 == 0, "whole 1 KB wave-loads per stage");
    static constexpr int kWaveLoads = kTileBytes / 1024;   // 1 KB per wave-load
    // Wave-load L = j * kWaves + wave: the first kWaveLoads % kWaves waves
    // issue one more per tile than the others when the split is uneven.
    static constexpr int kLoadsPerThread = (kWaveLoads + kWaves - 1) / kWaves;
    static constexpr int kLoadsFew = kWaveLoads / kWaves;
    static constexpr int kWavesWithMore = kWaveLoads % kWaves;
    static constexpr int kWWaveLoads = BN * BK / 1024;
    static_assert(kLoadsPerThread * (STAGES - 2) < 64, "vmcnt range");
    static_assert(BK == 64 || BK == 96 || BK == 128, "K tile of 64, 96 or 128 bytes");
    static constexpr int kLds = STAGES * kTileBytes;
    // 16-bit output tile staged through LDS for whole-line stores
    static constexpr bool kStageOut = BN * BM * 2 <= kLds;
    // one block fills a CU (4 SIMDs x OCC waves): the LDS beyond the ring is
    // then free for the epilogue's side area
    static constexpr bool kOneBlockPerCU = kWaves == 4 * OCC;
};

constexpr int kLdsPerCU = 160 * 1024;

// Side area of the staged epilogue, after the ring: the block's row scales,
// channel scales and bias as fp32, [BM xs | BN ws | BN bias].  Each thread
// loads at most kIters of these values at kernel start (their latency hides
// under the prologue's tile loads), keeps them in registers through the main
// loop and writes them here at the epilogue, whose dequantization then reads
// its scales from LDS instead of issuing global loads after the last MFMA.
template <class C, int ODT, int MODE>
struct SideArea {
    static constexpr int kValues = C::BM + C::BN;
    static constexpr int kBytesIfUsed = (kValues + C::BN) * 4;
    static constexpr bool kUse = MODE != 1 && ODT != W8A8_F32 && C::kStageOut && C::kOneBlockPerCU &&
                                 C::kLds + kBytesIfUsed <= kLdsPerCU;
    static constexpr int kBytes = kUse ? kBytesIfUsed : 0;
    static constexpr int kIters = kUse ? (kValues + C::kThreads - 1) / C::kThreads : 1;
};

// bf16 GELU table of the staged epilogue (gelu_bf16x8_lut) at the start of
// the block's LDS array, where the LDS has room for it: the ring (and the side
// area after it) then start at byte kRing.
template <class C, int ODT, int MODE, bool GELU>
struct GeluLut {
    using Side = SideArea<C, ODT, MODE>;
    static constexpr bool kUse = GELU && ODT == W8A8_BF16 && Side::kUse &&
                                 kGeluLutBytes + C::kLds + Side::kBytes <= kLdsPerCU;
    static constexpr int kRing = kUse ? kGeluLutBytes : 0;
    static constexpr int kArrayBytes = kRing + C::kLds + Side::kBytes;
    static_assert(!kUse || kArrayBytes >= 65536, "lookups read up to 64 KB past the table's start");
};

// The 16-byte output chunk c of staged row r sits at chunk c ^ (r mod P), P
// the largest power of two up to 32 dividing the chunks per row (48 for
// 384-wide tiles: P = 16), so the swizzled chunk stays inside its row.
template <int BN>
__device__ __forceinline__ int out_swz(int row) {
    constexpr int kChunks = BN / 8;
    constexpr int kPeriod = kChunks % 32 == 0 ? 32 : kChunks % 16 == 0 ? 16 : kChunks % 8 == 0 ? 8 : 1;
    return row & (kPeriod - 1);
}

// Block barrier for LDS data only: this wave's LDS accesses have completed
// (lgkmcnt(0)), then s_barrier.  Unlike __syncthreads(), whose release fence
// also waits for outstanding LDS-DMA tile loads (vmcnt(0)), it lets loads
// issued into another LDS region stay in flight.  The empty asm statements
// keep the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // gfx9: vmcnt 63, expcnt 7, lgkmcnt 0
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
}

// Epilogue of 16-bit outputs through an LDS staging area, in PASSES passes,
// each of half the tile when PASSES = 2: of its channels (kSplitN below: all
// waves convert the pass's MFMA column tiles) or of its rows (the waves
// holding those rows, [p * W / PASSES, (p + 1) * W / PASSES) of the block's
// W waves, convert).  The converted values are written as staged rows of
// 16-bit values, the 16-byte chunk index XOR-swizzled by the row; then
// threads read staged chunks back, 16 bytes per lane, apply GELU and store
// them, so each output line segment of 128 bytes or more is written whole
// (N % 8 == 0, out 16-byte aligned).  When a wave's pass segment is one
// 128-byte line per row (kWaveLocal), each wave stages and stores its own
// rows; otherwise the block's threads share the write-out.  GELU of the
// rounded linear output is the reference's order (gelu(T(lin)), rounded
// again).  For MFMA tile (i, j) a lane holds
// token m = wave_m + 32 j + lane % 32 and channels n = wave_n + 32 i + 8 g +
// 4 (lane / 32) + {0..3} in acc[i][j][4g .. 4g+3]; the values equal
// store_tiles'.  Scales come from the side area when it is in use (written
// and made visible by the caller), else from global memory.
// before_store() runs once, after the first pass is staged and before its
// first global store (a wait for loads the caller issued earlier).  MODE 2
// adds the residual in the write-out, reading the residual row and the
// scales as 16-byte chunks (resid and a per-channel rscale 16-byte aligned,
// which the caller checks).  Starts with the staging area free; ends with a
// barrier after the last read of it (LDS only: tile loads the caller has in
// flight into other LDS stay in flight).
template <int ODT, int MODE, bool GELU, class C, class Side, int PASSES, class Hook>
__device__ __forceinline__ void store_tiles_staged(const v16i (&acc)[C::TN][C::TM], const int8_t* lds,
                                                   int8_t* stage, int lane, int t, int wave, int m_base,
                                                   int n_base, int wave_m, int wave_n, int M, int N,
                                                   const float* __restrict__ xs, const float* __restrict__ ws,
                                                   int64_t ws_size, const void* __restrict__ bias,
                                                   const Residual& res, void* __restrict__ out,
                                                   Hook before_store) {
    constexpr int BN = C::BN, BM = C::BM, TN = C::TN, TM = C::TM;
    // The passes split the tile by channels when every wave's channel
    // columns split into whole 128-byte line segments (256 x 256 tiles: two
    // passes of 64 channels per wave column): then all waves convert in each
    // pass, two per SIMD.  Otherwise they split it by rows, and only the
    // waves holding a pass's rows convert in it.
    constexpr bool kSplitN = PASSES > 1 && TN % PASSES == 0 && (C::WN / PASSES) % 64 == 0;
    constexpr int kPassCols = kSplitN ? BN / PASSES : BN;   // channels per staged row
    constexpr int kSegCols = kSplitN ? C::WN / PASSES : BN;  // contiguous channels of a segment
    constexpr int kTnPass = kSplitN ? TN / PASSES : TN;     // MFMA column tiles per pass
    constexpr int kRowBytes = kPassCols * 2;
    constexpr int kChunks = kPassCols / 8;   // 16-byte chunks per staged row
    constexpr int kRows = kSplitN ? BM : BM / PASSES;
    constexpr int kWavesPerPass = C::kWaves / PASSES;
    // With kWaveLocal each wave stages its own WM rows of the pass's
    // 64-channel segment (128 bytes a row) in a private WM x 128-byte region
    // of the staging area, the 16-byte chunk index XOR-swizzled by bits 1-3 of
    // the row, and writes them out itself: a wave's LDS accesses complete in
    // order, so conversion and write-out need no block barrier between them,
    // and the waves drift apart, one converting while another stores.
    constexpr bool kWaveLocal = kSplitN && kSegCols * 2 == 128 && C::WM * 128 * C::kWaves <= C::kTileBytes;
    static_assert(kSplitN || (BM / C::WM) % PASSES == 0, "each pass holds whole wave rows");
    static_assert(kRows * kChunks % C::kThreads == 0, "whole write-out passes over the block");
    using OS = typename DType<ODT>::storage;
    // Lane-derived addresses are recomputed here from values the compiler
    // cannot see through, so that in the persistent kernel they are not
    // hoisted out of the tile loop and kept in registers across the K loop.
    int ln = lane, tv = t;
    asm volatile("" : "+v"(ln), "+v"(tv));
    const int lane_m = ln % 32, half = ln / 32;
    const float* const sv = reinterpret_cast<const float*>(lds + C::kLds);   // [BM xs | BN ws]
    const float* const sb = sv + BM + BN;                                      // [BN bias]
    static_for<0, PASSES>([&](auto p_) {
        constexpr int p = decltype(p_)::value;
        if (kSplitN || wave / kWavesPerPass == p) {   // wave-uniform
            float xsv[TM];
            static_for<0, TM>([&](auto j) {
                if constexpr (Side::kUse) {
                    xsv[j] = sv[wave_m + j * 32 + lane_m];
                } else {
                    const int m = m_base + wave_m + j * 32 + lane_m;
                    xsv[j] = xs[m < M ? m : M - 1];
                }
            });
            // Channel scales and bias of group k = 4 i + g (channels
            // wave_n + 32 i + 8 g + 4 half + {0..3}); with the side area the
            // next group's are read while this group is converted.
            auto load_group = [&](int k, float4& w4, float4& b4) {
                const int nl = wave_n + (k / 4) * 32 + 8 * (k % 4) + 4 * half;
                if constexpr (Side::kUse) {
                    w4 = *reinterpret_cast<const float4*>(sv + BM + nl);
                    b4 = *reinterpret_cast<const float4*>(sb + nl);
                } else {
                    float wv[4], bv[4];
                    static_for<0, 4>([&](auto e) {
                        const int n = n_base + nl + e < N ? n_base + nl + e : N - 1;
                        wv[e] = ws[ws_size == 1 ? 0 : n];
                        bv[e] = bias ? DType<ODT>::load(static_cast<const OS*>(bias)[n]) : 0.0f;
                    });
                    w4 = make_float4(wv[0], wv[1], wv[2], wv[3]);
                    b4 = make_float4(bv[0], bv[1], bv[2], bv[3]);
                }
            };
            // the pass's column tiles: i in [i0, i0 + kTnPass)
            constexpr int i0 = kSplitN ? p * kTnPass : 0;
            float4 w_next, b_next;
            load_group(4 * i0, w_next, b_next);
            static_for<0, kTnPass * 4>([&](auto k_) {
                constexpr int k = 4 * i0 + decltype(k_)::value, i = k / 4, g = k % 4;
                const float4 w4 = w_next, b4 = b_next;
                if constexpr (k + 1 < 4 * (i0 + kTnPass)) load_group(k + 1, w_next, b_next);
                const float wsv[4] = {w4.x, w4.y, w4.z, w4.w};
                const float bv[4] = {b4.x, b4.y, b4.z, b4.w};
                const int chunk = kSplitN ? ((wave_n / C::WN) * kSegCols + (i - i0) * 32 + 8 * g) / 8
                                          : (wave_n + i * 32 + 8 * g) / 8;
                static_for<0, TM>([&](auto j) {
                    // the linear outputs rounded to the output dtype; GELU is
                    // applied to them in the write-out below
                    float v[4];
                    static_for<0, 4>([&](auto e) {
                        v[e] = epilogue_value<ODT>(acc[i][j][4 * g + e], xsv[j], wsv[e], bv[e], false);
                    });
                    uint2 pk;
                    pk.x = DType<ODT>::store2(v[0], v[1]);
                    pk.y = DType<ODT>::store2(v[2], v[3]);
                    if constexpr (kWaveLocal) {
                        const int rw = j * 32 + lane_m, cw = (i - i0) * 4 + g;
                        *reinterpret_cast<uint2*>(stage + wave * (C::WM * 128) + rw * 128 +
                                                  (cw ^ ((rw >> 1) & 7)) * 16 + half * 8) = pk;
                    } else {
                        const int ml = wave_m + j * 32 + lane_m - (kSplitN ? 0 : p * kRows);
                        *reinterpret_cast<uint2*>(stage + ml * kRowBytes + (chunk ^ out_swz<kPassCols>(ml)) * 16 +
                                                  half * 8) = pk;
                    }
                });
            });
        }
        if constexpr (kWaveLocal) asm volatile("" ::: "memory");
        else lds_barrier();
        if constexpr (p == 0) before_store();
        // the residual and the store of the 8 outputs of chunk v at (m, n)
        auto finish_plain = [&](uint4 v, int m, int n) {
            if constexpr (MODE == 2) {
                const uint4 rv = *reinterpret_cast<const uint4*>(static_cast<const OS*>(res.resid) +
                                                                 static_cast<int64_t>(m) * N + n);
                uint4 sv4;
                if (res.rs_size == 1) {
                    const uint32_t s1 = static_cast<const OS*>(res.rscale)[0];
                    sv4.x = sv4.y = sv4.z = sv4.w = s1 | (s1 << 16);
                } else {
                    sv4 = *reinterpret_cast<const uint4*>(static_cast<const OS*>(res.rscale) + n);
                }
                auto lo = [](uint32_t w) { return DType<ODT>::load(static_cast<OS>(w & 0xffffu)); };
                auto hi = [](uint32_t w) { return DType<ODT>::load(static_cast<OS>(w >> 16)); };
                auto fuse = [&](uint32_t lin, uint32_t s, uint32_t rr) {
                    return DType<ODT>::store2(fmaf(lo(lin), lo(s), lo(rr)), fmaf(hi(lin), hi(s), hi(rr)));
                };
                v.x = fuse(v.x, sv4.x, rv.x);
                v.y = fuse(v.y, sv4.y, rv.y);
                v.z = fuse(v.z, sv4.z, rv.z);
                v.w = fuse(v.w, sv4.w, rv.w);
            }
            *reinterpret_cast<uint4*>(static_cast<OS*>(out) + static_cast<int64_t>(m) * N + n) = v;
        };
        // GELU, the residual and the store of the 8 outputs of chunk v at (m, n)
        auto finish = [&](uint4 v, int m, int n) {
            if constexpr (GeluLut<C, ODT, MODE, GELU>::kUse) {
                using Lut = GeluLut<C, ODT, MODE, GELU>;
                v = gelu_bf16x8_lut(v, lds_address(lds - Lut::kRing));
            } else if constexpr (GELU) {
                // every thread of the block takes part here (in the
                // conversion above only the waves of the pass do)
                v.x = gelu_x2<ODT>(v.x);
                v.y = gelu_x2<ODT>(v.y);
                v.z = gelu_x2<ODT>(v.z);
                v.w = gelu_x2<ODT>(v.w);
            }
            finish_plain(v, m, n);
        };
        if constexpr (kWaveLocal) {
            // lane: chunk c of rows r0, r0 + 8, ... of the wave's region
            const int8_t* const mine = stage + wave * (C::WM * 128);
            const int c = ln % 8, r0 = ln / 8;
            const int n = n_base + wave_n + p * 64 + c * 8;
            auto staged_w = [&](int r) {
                return *reinterpret_cast<const uint4*>(mine + r * 128 + (c ^ ((r >> 1) & 7)) * 16);
            };
            constexpr int kSteps = C::WM / 8;
            if constexpr (GeluLut<C, ODT, MODE, GELU>::kUse && kSteps % 2 == 0) {
                // two chunks per step: their 16 lookups in flight together;
                // GELU of rows past M is computed and not stored
                using Lut = GeluLut<C, ODT, MODE, GELU>;
                uint4 n0 = staged_w(r0), n1 = staged_w(r0 + 8);
#pragma unroll
                for (int step = 0; step < kSteps; step += 2) {
                    uint4 v0 = n0, v1 = n1;
                    const int r = r0 + step * 8;
                    if (step + 2 < kSteps) {
                        n0 = staged_w(r + 16);
                        n1 = staged_w(r + 24);
                    }
                    gelu_bf16x16_lut(v0, v1, lds_address(lds - Lut::kRing));
                    const int m = m_base + wave_m + r;
                    if (m < M && n < N) finish_plain(v0, m, n);
                    if (m + 8 < M && n < N) finish_plain(v1, m + 8, n);
                }
            } else {
                uint4 v_next = staged_w(r0);
#pragma unroll
                for (int step = 0; step < kSteps; ++step) {
                    const uint4 v = v_next;
                    const int r = r0 + step * 8;
                    v_next = staged_w(step + 1 < kSteps ? r + 8 : r);
                    const int m = m_base + wave_m + r;
                    if (m < M && n < N) finish(v, m, n);
                }
            }
            // the next pass's conversion overwrites the region after these
            // reads (in order); the caller reuses the staging area after the
            // last pass
            if constexpr (p + 1 == PASSES) lds_barrier();
            else asm volatile("" ::: "memory");
            return;
        }
        // Thread tv takes chunk c = tv % kChunks of rows r0, r0 + kRowStep, ...
        // (r0 = tv / kChunks) when the block covers whole rows per step, so
        // the column, the bounds check on it and the row addresses are set up
        // once per pass and stepped; otherwise each chunk index is decoded.
        constexpr bool kWholeRows = C::kThreads % kChunks == 0;
        constexpr int kRowStep = kWholeRows ? C::kThreads / kChunks : 1;
        const int c0 = tv % kChunks, r0 = tv / kChunks;
        const int n0 = kSplitN ? n_base + (c0 / (kSegCols / 8)) * C::WN + p * kSegCols + (c0 % (kSegCols / 8)) * 8
                               : n_base + c0 * 8;
        const int m0 = m_base + (kSplitN ? 0 : p * kRows) + r0;
        constexpr int kSteps = kRows * kChunks / C::kThreads;
        auto coords = [&](int step, int& r, int& c, int& m, int& n) {
            if constexpr (kWholeRows) {
                r = r0 + step * kRowStep;
                c = c0;
                m = m0 + step * kRowStep;
                n = n0;
            } else {
                const int idx = step * C::kThreads + tv;
                r = idx / kChunks;
                c = idx % kChunks;
                m = m_base + (kSplitN ? 0 : p * kRows) + r;
                n = kSplitN ? n_base + (c / (kSegCols / 8)) * C::WN + p * kSegCols + (c % (kSegCols / 8)) * 8
                            : n_base + c * 8;
            }
        };
        auto staged = [&](int r, int c) {
            return *reinterpret_cast<const uint4*>(stage + r * kRowBytes + (c ^ out_swz<kPassCols>(r)) * 16);
        };
        // each step's staged chunk is read one step ahead (the last step
        // re-reads its own), so the read's latency hides under the previous
        // chunk's work
        int r_nx, c_nx, m_nx, n_nx;   // the next step's chunk
        coords(0, r_nx, c_nx, m_nx, n_nx);
        uint4 v_next = staged(r_nx, c_nx);
#pragma unroll 4
        for (int step = 0; step < kSteps; ++step) {
            uint4 v = v_next;
            const int m = m_nx, n = n_nx;
            coords(step + 1 < kSteps ? step + 1 : step, r_nx, c_nx, m_nx, n_nx);
            v_next = staged(r_nx, c_nx);
            if (m < M && n < N) finish(v, m, n);
        }
        lds_barrier();
    });
}

// Epilogue plan of a DMA configuration for an output mode: kStaged = 16-bit
// outputs staged through LDS for whole-line stores; kPersist = the kernel
// loops over output tiles (grid = min(tiles, CUs)) and overlaps each
// epilogue with the next tile's first loads, which needs a 2-stage ring whose
// stage holds half of the output tile, and accumulators of at most 8 MFMA
// tiles (128 VGPRs): the tile loop's own live state then fits beside them,
// while with 3 x 3 tiles (384 x 192) it spilled and measured ~3% slower than
// one block per tile.
template <class C, int ODT, int MODE>
struct DmaPlan {
    static constexpr bool kStaged = MODE != 1 && ODT != W8A8_F32 && C::kStageOut;
    static constexpr bool kPersist = kStaged && C::STAGES == 2 && C::BN * C::BM <= C::kTileBytes &&
                                     (C::BM / C::WM) % 2 == 0 && C::TN * C::TM <= 8;
};

// Persistent INT8 GEMM over LDS-DMA K tiles.  Block b takes output tiles b,
// b + G, b + 2G, ... (G = gridDim.x; with G = the tile count each block takes
// one).  Per tile: the K loop below, then the epilogue.  With a 2-stage ring
// whose stage holds half of the 16-bit output tile, the epilogue overlaps the
// next tile's start: once every wave has left the K loop, K tile 0 of the
// next output tile is loaded into the stage the last K tile did not use, the
// accumulators are dequantized in registers meanwhile, the output is staged
// in two passes through the other stage and stored, and K tile 1 of the next
// tile is issued into it; the stores then drain under the next K loop.
template <int ODT, int MODE, bool GELU, class C>
__global__ __launch_bounds__(C::kThreads, C::OCC) void gemm_mfma_dma(
    const int8_t* __restrict__ q, const int8_t* __restrict__ w, const float* __restrict__ xs,
    const float* __restrict__ ws, int64_t ws_size, const void* __restrict__ bias, Residual res,
    void* __restrict__ out, int M, int N, int K, int group_m) {
    constexpr int BN = C::BN, BM = C::BM, WN = C::WN, WM = C::WM, BK = C::BK, STAGES = C::STAGES;
    constexpr int TN = C::TN, TM = C::TM, CPR = C::CPR, KS = C::KS;
    constexpr int kTileBytes = C::kTileBytes, kLoadsPerThread = C::kLoadsPerThread;
    constexpr int kWWaveLoads = C::kWWaveLoads;
    using Side = SideArea<C, ODT, MODE>;
    constexpr bool kStaged = DmaPlan<C, ODT, MODE>::kStaged;
    constexpr bool kPersist = DmaPlan<C, ODT, MODE>::kPersist;
    using Lut = GeluLut<C, ODT, MODE, GELU>;
    __shared__ __attribute__((aligned(1024))) int8_t lds_all[Lut::kArrayBytes];
    int8_t* const lds = lds_all + Lut::kRing;   // the ring, then the side area

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN, tiles = tiles_m * tiles_n;
    // The wave index is uniform across the wave: in an SGPR, so operand choice,
    // buffer resources and LDS destinations of the tile loads stay scalar.
    const int t = threadIdx.x, lane = t % kWave, wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int wave_n = (wave % (BN / WN)) * WN;
    const int wave_m = (wave / (BN / WN)) * WM;
    const int KT = K / BK;                                 // K % BK == 0 (host checks)
    bool vec_ok = (N % 8) == 0 && (reinterpret_cast<uintptr_t>(out) % 16) == 0;
    if constexpr (MODE == 2)
        vec_ok = vec_ok && (reinterpret_cast<uintptr_t>(res.resid) % 16) == 0 &&
                 (res.rs_size == 1 || (reinterpret_cast<uintptr_t>(res.rscale) % 16) == 0);

    int tile = blockIdx.x;
    TileCoord tc = tile_of_block(tile, tiles_m, tiles_n, group_m);
    int m_base = tc.tm * BM, n_base = tc.tn * BN;

    // Source of each wave-load this lane takes part in: wave-load L (global
    // index j * kWaves + wave, L < kWaveLoads) fills LDS chunks [64 L, 64 L + 64)
    // of the stage; chunk p holds row p / CPR, logical chunk (p % CPR) ^ swz(row).
    // Byte offsets into a buffer resource per operand (the K offset of a
    // tile goes in the scalar offset).  Each operand's resource is based at
    // the loaded tile's first row, so offsets stay below BN * K (or BM * K)
    // bytes whatever the operand's size (the host checks that bound).  The
    // offsets are recomputed per load (a few VALU operations) rather than
    // kept in registers across the loop.
    int ld_mb = m_base, ld_nb = n_base;   // the output tile whose K tiles issue() loads
    auto set_tile = [&](int mb, int nb) {
        ld_mb = mb;
        ld_nb = nb;
    };
    auto voff_of = [&](int j) -> uint32_t {
        const int L = j * C::kWaves + wave < C::kWaveLoads ? j * C::kWaves + wave : C::kWaveLoads - 1;
        const bool is_w = L < kWWaveLoads;
        const int p = (is_w ? L : L - kWWaveLoads) * 64 + lane;
        const int r = p / CPR;
        const int c = (p % CPR) ^ swz<BK>(r);
        const int base = is_w ? ld_nb : ld_mb;
        const int lim = is_w ? N : M;
        const int row = base + r < lim ? r : lim - 1 - base;   // clamped to the last row, relative
        return static_cast<uint32_t>(row) * static_cast<uint32_t>(K) + c * 16;
    };
    // Loads [j0, j1) of this lane's share of K tile kt into ring stage `stage`.
    auto issue = [&](int kt, int stage, int j0, int j1) {
        const int k0 = kt * BK;
        const int8_t* const wb = w + static_cast<int64_t>(ld_nb) * K;
        const int8_t* const qb = q + static_cast<int64_t>(ld_mb) * K;
#pragma unroll
        for (int j = 0; j < kLoadsPerThread; ++j) {
            if (j < j0 || j >= j1) continue;
            const int L = j * C::kWaves + wave;
            if (C::kWavesWithMore != 0 && L >= C::kWaveLoads) break;   // wave-uniform
            int8_t* dst = lds + stage * kTileBytes + L * 1024;
            buffer_load_lds16(L < kWWaveLoads ? static_cast<const void*>(wb) : static_cast<const void*>(qb), dst,
                              voff_of(j), k0);
        }
    };
    // Half of a K tile's loads are issued right after the barrier that frees
    // its stage, the other half one substep later, so the loads of the eight
    // waves do not all queue at the address unit at once.
    constexpr int kFirst = kLoadsPerThread / 2 > 0 ? kLoadsPerThread / 2 : kLoadsPerThread;

    const int fl = swz<BK>(lane % 32);
    int rd[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) rd[ks] = (((2 * ks + lane / 32) ^ fl) * 16);
    const int wrow = (wave_n + lane % 32) * BK;
    const int xrow = (BN + wave_m + lane % 32) * BK;

    // Fragments of one k32 substep: TN weight fragments, TM activation fragments.
    auto read_frags = [&](int stage, int ks, v4i (&a)[TN], v4i (&b)[TM]) {
        const int8_t* base = lds + stage * kTileBytes + rd[ks];
#pragma unroll
        for (int i = 0; i < TN; ++i)
            a[i] = *reinterpret_cast<const v4i*>(base + wrow + i * 32 * BK);
#pragma unroll
        for (int j = 0; j < TM; ++j)
            b[j] = *reinterpret_cast<const v4i*>(base + xrow + j * 32 * BK);
    };
    v16i acc[TN][TM];
    auto mfmas = [&](const v4i (&a)[TN], const v4i (&b)[TM]) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
    };
    // One MFMA, then one fragment read, while reads remain; then the rest of
    // the MFMAs.
    auto interleave = [&]() {
        constexpr int kReads = TN + TM, kMfma = TN * TM;
        constexpr int kPairs = kReads < kMfma ? kReads : kMfma;
        static_for<0, kPairs>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
        });
        if constexpr (kMfma > kPairs) __builtin_amdgcn_sched_group_barrier(kSchedMfma, kMfma - kPairs, 0);
        if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, kReads - kPairs, 0);
    };
    // Wait until this wave's DMA for the next tile has landed (at most `after`
    // later tiles, 0 <= after <= STAGES - 2, still in flight) and its LDS reads
    // have completed.
    auto wait_tile = [&](int after) {
        static_for<0, STAGES - 1>([&](auto a) {
            constexpr int A = decltype(a)::value;
            if (after == A) {
                if (C::kWavesWithMore == 0 || wave < C::kWavesWithMore) wait_vm_lgkm0<A * kLoadsPerThread>();
                else wait_vm_lgkm0<A * C::kLoadsFew>();
            }
        });
    };
    auto next_stage = [](int st) { return st + 1 == STAGES ? 0 : st + 1; };

    // The GELU table is written once; the barriers of the first K loop order
    // it before the first epilogue's reads.
    if constexpr (Lut::kUse) gelu_lut_fill(lds_all, t, C::kThreads);

    int s0 = 0;           // ring stage of the current tile's K tile 0
    bool primed = false;  // K tile 0 landed (and waited for) and K tile 1 issued by the previous epilogue
    for (;;) {
        // Epilogue scales of this tile (side area): value idx < BM is xs of row
        // m_base + idx, else ws and bias of channel n_base + idx - BM (clamped to
        // the last row / channel, as the direct epilogue clamps them).  Their
        // load latency hides under the K loop.
        float side_v[Side::kIters], side_b[Side::kIters];
        if constexpr (Side::kUse) {
            using OS = typename DType<ODT>::storage;
            static_for<0, Side::kIters>([&](auto it) {
                const int idx = t + it * C::kThreads;
                side_v[it] = 0.0f;
                side_b[it] = 0.0f;
                if (idx < BM) {
                    const int m = m_base + idx;
                    side_v[it] = xs[m < M ? m : M - 1];
                } else if (idx < BM + BN) {
                    int n = n_base + idx - BM;
                    n = n < N ? n : N - 1;
                    side_v[it] = ws[ws_size == 1 ? 0 : n];
                    if (bias) side_b[it] = DType<ODT>::load(static_cast<const OS*>(bias)[n]);
                }
            });
        }
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = v16i{};

        v4i fa[2][TN], fb[2][TM];   // two fragment sets, alternating by substep parity
        if (!primed) {
            int st = s0;
#pragma unroll
            for (int s = 0; s < STAGES - 1; ++s) {
                if (s < KT) issue(s, st, 0, kLoadsPerThread);
                st = next_stage(st);
            }
            if (KT > 0) {
                wait_tile(KT - 1 < STAGES - 2 ? KT - 1 : STAGES - 2);
                __builtin_amdgcn_s_barrier();
                __builtin_amdgcn_sched_barrier(0);
                if (STAGES - 1 < KT) issue(STAGES - 1, st, 0, kLoadsPerThread);
            }
        }
        if (KT > 0) read_frags(s0, 0, fa[0], fb[0]);
        // One K tile.  The fragment set of substep ks is fa/fb[(ks + P) & 1]; with an
        // odd number of substeps per tile the parity flips from tile to tile, so
        // tiles are then processed in pairs (P = 0, 1) to keep every register index
        // a compile-time constant.  Synchronisation: one raw s_barrier per K tile,
        // preceded by s_waitcnt vmcnt(loads of later tiles) lgkmcnt(0): the wave's
        // own DMA for the tile about to be read has landed and its reads of the
        // tile just consumed have completed, so after the barrier every wave may
        // read the new tile and the consumed stage may be refilled.  The barrier
        // is crossed before the last k32 substep of a tile, so the LDS latency of
        // the next tile's first fragments hides under that substep's MFMAs.
        auto ktile = [&](int kt, int stage, int next, auto par) {
            constexpr int P = decltype(par)::value;
            static_for<0, KS>([&](auto ks_) {
                constexpr int ks = decltype(ks_)::value;
                constexpr int cur = (ks + P) & 1;
                if constexpr (ks == 0 && kFirst < kLoadsPerThread) {
                    // the second half of the loads issued at the previous barrier
                    if (kt >= 1 && kt - 1 + STAGES < KT)
                        issue(kt - 1 + STAGES, stage == 0 ? STAGES - 1 : stage - 1, kFirst, kLoadsPerThread);
                }
                if constexpr (ks + 1 < KS) {
                    read_frags(stage, ks + 1, fa[cur ^ 1], fb[cur ^ 1]);
                } else {
                    if (kt + 1 < KT) {
                        // tiles issued so far: up to min(KT - 1, kt + STAGES - 1)
                        const int last = KT - 1 < kt + STAGES - 1 ? KT - 1 : kt + STAGES - 1;
                        wait_tile(last - (kt + 1));
                        __builtin_amdgcn_s_barrier();
                        __builtin_amdgcn_sched_barrier(0);
                        if (kt + STAGES < KT) issue(kt + STAGES, stage, 0, kFirst);
                    }
                    // first fragments of the next tile (after the last tile: an
                    // unused in-bounds read, which keeps this one basic block)
                    read_frags(next, 0, fa[cur ^ 1], fb[cur ^ 1]);
                }
                // The single MFMA block of the substep: one copy only, so the
                // accumulators stay in registers.
                mfmas(fa[cur], fb[cur]);
                interleave();
                __builtin_amdgcn_sched_barrier(0);
            });
        };
        int stage = s0;
        if constexpr (KS % 2 == 0) {
            for (int kt = 0; kt < KT; ++kt) {
                const int nx = next_stage(stage);
                ktile(kt, stage, nx, std::integral_constant<int, 0>{});
                stage = nx;
            }
        } else {
            int kt = 0;
            for (; kt + 1 < KT; kt += 2) {
                const int s1 = next_stage(stage), s2 = next_stage(s1);
                ktile(kt, stage, s1, std::integral_constant<int, 0>{});
                ktile(kt + 1, s1, s2, std::integral_constant<int, 1>{});
                stage = s2;
            }
            if (kt < KT) {
                const int s1 = next_stage(stage);
                ktile(kt, stage, s1, std::integral_constant<int, 0>{});
                stage = s1;
            }
        }
        // `stage` is now the one after the last K tile's: for a 2-stage ring the
        // stage the last K tile did not use.
        const int s_last = stage == 0 ? STAGES - 1 : stage - 1;

        const int next = tile + static_cast<int>(gridDim.x);
        const bool has_next = next < tiles;
        bool stored = false;
        if constexpr (kStaged) {
            if (vec_ok) {
                if constexpr (Side::kUse) {
                    float* const sv = reinterpret_cast<float*>(lds + C::kLds);
                    float* const sb = sv + BM + BN;
                    static_for<0, Side::kIters>([&](auto it) {
                        const int idx = t + it * C::kThreads;
                        if (idx < BM + BN) {
                            sv[idx] = side_v[it];
                            if (idx >= BM) sb[idx - BM] = side_b[it];
                        }
                    });
                }
                __syncthreads();   // no wave reads the ring any more; the side area is written
                if constexpr (kPersist) {
                    if (has_next && KT > 0) {
                        const TileCoord nc = tile_of_block(next, tiles_m, tiles_n, group_m);
                        set_tile(nc.tm * BM, nc.tn * BN);
                        issue(0, stage, 0, kLoadsPerThread);   // K tile 0 of the next output tile
                    }
                    // stage through the last K tile's stage in two passes; K tile 0 of
                    // the next tile is waited for before the first store, so no store
                    // is ever pending under a partial vmcnt wait for tile loads
                    store_tiles_staged<ODT, MODE, GELU, C, Side, 2>(
                        acc, lds, lds + s_last * kTileBytes, lane, t, wave, m_base, n_base, wave_m, wave_n, M, N, xs,
                        ws, ws_size, bias, res, out, [&]() { wait_vm_lgkm0<0>(); });
                    if (!has_next) return;
                    if (1 < KT) issue(1, s_last, 0, kLoadsPerThread);
                    tile = next;
                    tc = tile_of_block(tile, tiles_m, tiles_n, group_m);
                    m_base = tc.tm * BM;
                    n_base = tc.tn * BN;
                    s0 = stage;
                    primed = true;
                    continue;
                } else {
                    store_tiles_staged<ODT, MODE, GELU, C, Side, 1>(acc, lds, lds, lane, t, wave, m_base, n_base,
                                                                    wave_m, wave_n, M, N, xs, ws, ws_size, bias,
                                                                    res, out, []() {});
                }
                stored = true;
            }
        }
        if (!stored)
            store_tiles<ODT, MODE, GELU, TN, TM>(acc, lane, m_base, n_base, wave_m, wave_n, M, N, xs, ws,
                                                 ws_size, bias, res, out);
        if (!kPersist || !has_next) return;
        __syncthreads();   // the LDS is free for the next tile's loads
        tile = next;
        tc = tile_of_block(tile, tiles_m, tiles_n, group_m);
        m_base = tc.tm * BM;
        n_base = tc.tn * BN;
        set_tile(m_base, n_base);
        s0 = 0;
        primed = false;
    }
}

// Generic GEMM for shapes the MFMA kernel does not take (K % 16 != 0,
// unaligned operands, fused quant of fp32 inputs): one thread per output.
template <int ODT, int MODE, bool GELU>
__global__ __launch_bounds__(256) void gemm_generic(const int8_t* __restrict__ q,
                                                    const int8_t* __restrict__ w,
                                                    const float* __restrict__ xs,
                                                    const float* __restrict__ ws, int64_t ws_size,
                                                    const void* __restrict__ bias, Residual res,
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
        float v = epilogue_value<ODT>(acc, xs[m], ws[ws_size == 1 ? 0 : n], b, GELU);
        if constexpr (MODE == 2) v = residual_value<ODT>(v, res, m, static_cast<int>(n), static_cast<int>(N));
        static_cast<typename DType<ODT>::storage*>(out)[idx] = DType<ODT>::store(v);
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

}  // namespace w8a8
