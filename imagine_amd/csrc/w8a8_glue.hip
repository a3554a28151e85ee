// Block glue of the Qwen-Image DiT around its W8A8 linears, for gfx950.
//
//   adaln / rms_adaln   Kitchen's native "adaln" call as the crate issues it
//                       (inference/src/backend_eager.rs:176-229): per row i of
//                       x [n, d], out = T(T(T(norm(x_i)) * T(1 + scale_g)) + shift_h)
//                       with g = i / sg, h = i / tg, the op order of the
//                       crate's eager route (:186-199: layer_norm or rms_norm,
//                       mul by scale + 1, add shift, each rounded to T).
//   gated residual      x += y * gate, tokens before the prefix with gate0,
//                       the rest with gate1 (models/qwen_image21/numeric.rs:
//                       110-125, ATen addcmul_: T(fp32(x + y * g))).
//   rms_rope            the attention's QK RMSNorm + RoPE (backend_rope.rs:204-222).
//   modulated quantizer the batch-one modulation of int8_linear_modulated
//                       (backend_bindings.rs:329-405): xm = T(x * T(1 + s_k)),
//                       then the per-token quantizer on xm, in one kernel.
//
// All three are bandwidth kernels over bf16/fp16/fp32 rows, fp32 arithmetic.
// adaln: one block per row (128 threads up to 1024 16-byte chunks, else
// 256); aligned rows of up to 2048 chunks stay in registers (CPL chunks per
// lane) between the reduction passes and the output pass, so x is read once;
// other rows take a generic kernel that re-reads the row.  Gated residual:
// 16-byte chunks, grid-stride.
#include <algorithm>

#include "w8a8_common.h"

namespace w8a8 {

namespace {

constexpr int kGlueThreads = 256;

// Sum over a block of NW waves (part: NW floats of LDS).
template <int NW>
__device__ __forceinline__ float block_sum_w(float v, float* part) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    __syncthreads();   // earlier readers of part are done
    if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = v;
    __syncthreads();
    float s = part[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) s += part[w];
    return s;
}

__device__ __forceinline__ float block_sum(float v, float* part) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    const int wave = threadIdx.x / kWave;
    __syncthreads();   // earlier readers of part are done
    if ((threadIdx.x % kWave) == 0) part[wave] = v;
    __syncthreads();
    return (part[0] + part[1]) + (part[2] + part[3]);
}

// SINGLE: the single-rounding form T(fma(norm, 1 + scale, shift)) in fp32
// (the structure of Kitchen's CUDA adaln kernel, adaln.cu in the reference's
// native-source archive), instead of the eager route's three roundings.
template <int DT, bool RMS, bool SINGLE>
__global__ __launch_bounds__(kGlueThreads) void adaln_rows(const void* __restrict__ x,
                                                           const void* __restrict__ scale,
                                                           const void* __restrict__ shift,
                                                           void* __restrict__ out, int64_t d,
                                                           int64_t sg, int64_t tg, float eps) {
    using D = DType<DT>;
    using OS = typename D::storage;
    __shared__ float part[4];
    const int64_t row = blockIdx.x;
    const OS* xr = static_cast<const OS*>(x) + row * d;
    const OS* sr = static_cast<const OS*>(scale) + (row / sg) * d;
    const OS* hr = static_cast<const OS*>(shift) + (row / tg) * d;
    OS* o = static_cast<OS*>(out) + row * d;
    const float inv_d = 1.0f / static_cast<float>(d);
    float mean = 0.0f, rstd;
    if constexpr (RMS) {
        // aten rms_norm: x * rsqrt(mean(x^2) + eps) in fp32
        float s2 = 0.0f;
        for (int64_t k = threadIdx.x; k < d; k += kGlueThreads) {
            const float v = D::load(xr[k]);
            s2 = fmaf(v, v, s2);
        }
        s2 = block_sum(s2, part);
        rstd = 1.0f / sqrtf(s2 * inv_d + eps);
    } else {
        // aten layer_norm: biased variance, rstd = 1 / sqrt(var + eps)
        float s1 = 0.0f;
        for (int64_t k = threadIdx.x; k < d; k += kGlueThreads) s1 += D::load(xr[k]);
        mean = block_sum(s1, part) * inv_d;
        float s2 = 0.0f;
        for (int64_t k = threadIdx.x; k < d; k += kGlueThreads) {
            const float c = D::load(xr[k]) - mean;
            s2 = fmaf(c, c, s2);
        }
        const float var = block_sum(s2, part) * inv_d;
        rstd = 1.0f / sqrtf(fmaxf(var, 0.0f) + eps);
    }
    const float bias = -rstd * mean;   // aten's y = x * rstd + (-rstd * mean)
    for (int64_t k = threadIdx.x; k < d; k += kGlueThreads) {
        const float v = D::load(xr[k]);
        if constexpr (SINGLE) {
            const float y = RMS ? v * rstd : fmaf(v, rstd, bias);
            o[k] = D::store(fmaf(y, 1.0f + D::load(sr[k]), D::load(hr[k])));
        } else {
            const float y = D::round(RMS ? v * rstd : fmaf(v, rstd, bias));
            const float m = D::round(1.0f + D::load(sr[k]));
            const float z = D::round(y * m);
            o[k] = D::store(z + D::load(hr[k]));
        }
    }
}

// Register-resident adaln: lane chunk c = tid + j * 256 of the row (E values
// per 16-byte chunk); same operations per element as adaln_rows, so the same
// results up to the order of the fp32 row sums.
template <int DT, bool RMS, bool SINGLE, int CPL, int NT>
__global__ __launch_bounds__(NT) void adaln_rows_vec(const void* __restrict__ x,
                                                               const void* __restrict__ scale,
                                                               const void* __restrict__ shift,
                                                               void* __restrict__ out, int64_t d,
                                                               int64_t sg, int64_t tg, float eps) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;
    constexpr int NW = NT / kWave;
    __shared__ float part[NW];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t nchunks = d / E;
    const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * d * D::bytes);
    const uint4* sr = reinterpret_cast<const uint4*>(static_cast<const char*>(scale) + (row / sg) * d * D::bytes);
    const uint4* hr = reinterpret_cast<const uint4*>(static_cast<const char*>(shift) + (row / tg) * d * D::bytes);
    uint4* o = reinterpret_cast<uint4*>(static_cast<char*>(out) + row * d * D::bytes);
    // the row and, for rows of up to 3 chunks per thread (64 VGPRs: full
    // occupancy), its scale and shift chunks, loaded now so that their
    // latency is not a second round trip after the row reductions
    // (2 x 5856 x 3072 bf16: ~5% faster)
    constexpr int PF = CPL <= 3 ? CPL : 1;
    uint4 raw[CPL], svp[PF], hvp[PF];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + static_cast<int64_t>(j) * NT;
        raw[j] = c < nchunks ? load_stream(xr + c) : make_uint4(0, 0, 0, 0);
        if constexpr (CPL <= 3) {
            svp[j] = c < nchunks ? sr[c] : make_uint4(0, 0, 0, 0);
            hvp[j] = c < nchunks ? hr[c] : make_uint4(0, 0, 0, 0);
        }
    }
    auto elem = [&](const uint4& v, int i) {
        return D::load(reinterpret_cast<const typename D::storage*>(&v)[i]);
    };
    const float inv_d = 1.0f / static_cast<float>(d);
    float mean = 0.0f, rstd;
    if constexpr (RMS) {
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const float v = elem(raw[j], i);
                s2 = fmaf(v, v, s2);
            }
        s2 = block_sum_w<NW>(s2, part);
        rstd = 1.0f / sqrtf(s2 * inv_d + eps);
    } else {
        float s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < E; ++i) s1 += elem(raw[j], i);
        mean = block_sum_w<NW>(s1, part) * inv_d;
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = tid + static_cast<int64_t>(j) * NT;
            if (c >= nchunks) break;   // padding chunks are zeros, not row values
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const float cv = elem(raw[j], i) - mean;
                s2 = fmaf(cv, cv, s2);
            }
        }
        const float var = block_sum_w<NW>(s2, part) * inv_d;
        rstd = 1.0f / sqrtf(fmaxf(var, 0.0f) + eps);
    }
    const float bias = -rstd * mean;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + static_cast<int64_t>(j) * NT;
        if (c >= nchunks) break;
        uint4 sv, hv;
        if constexpr (CPL <= 3) {
            sv = svp[j];
            hv = hvp[j];
        } else {
            sv = sr[c];
            hv = hr[c];
        }
        uint4 res;
        typename D::storage* rp = reinterpret_cast<typename D::storage*>(&res);
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float v = elem(raw[j], i);
            if constexpr (SINGLE) {
                const float y = RMS ? v * rstd : fmaf(v, rstd, bias);
                rp[i] = D::store(fmaf(y, 1.0f + elem(sv, i), elem(hv, i)));
            } else {
                const float y = D::round(RMS ? v * rstd : fmaf(v, rstd, bias));
                const float m = D::round(1.0f + elem(sv, i));
                const float z = D::round(y * m);
                rp[i] = D::store(z + elem(hv, i));
            }
        }
        o[c] = res;
    }
}

// Modulated norm fused with the per-token quantizer, for a norm whose only
// consumer is an INT8 linear (the DiT's norm1 -> QKV and norm2 -> FFN-up):
// row r = b * tokens + t of x gets scale / shift rows b of (scale0, shift0)
// for t < prefix, else of (scale1, shift1) (modulated_norm's text prefix in
// one launch); its T outputs, computed exactly as adaln_rows_vec computes
// them, replace the raw row in registers, and their codes and row scale are
// those the quantizer gives for the stored output.
template <int DT, bool RMS, int CPL, int NT>
__global__ __launch_bounds__(NT) void modnorm_quant_rows_vec(
    const void* __restrict__ x, const void* __restrict__ scale0, const void* __restrict__ scale1,
    const void* __restrict__ shift0, const void* __restrict__ shift1, int8_t* __restrict__ q,
    float* __restrict__ xs, int64_t tokens, int64_t d, int64_t prefix, float eps, int recip) {
    using D = DType<DT>;
    using OS = typename D::storage;
    constexpr int E = 16 / D::bytes;
    constexpr int NW = NT / kWave;
    __shared__ float part[NW];
    const int64_t row = blockIdx.x;
    const int64_t b = row / tokens, t = row % tokens;
    const int tid = threadIdx.x;
    const int64_t nchunks = d / E;
    const uint4* xr = reinterpret_cast<const uint4*>(static_cast<const char*>(x) + row * d * D::bytes);
    const uint4* sr = reinterpret_cast<const uint4*>(static_cast<const char*>(t < prefix ? scale0 : scale1) +
                                                     b * d * D::bytes);
    const uint4* hr = reinterpret_cast<const uint4*>(static_cast<const char*>(t < prefix ? shift0 : shift1) +
                                                     b * d * D::bytes);
    uint4 raw[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + static_cast<int64_t>(j) * NT;
        raw[j] = c < nchunks ? load_stream(xr + c) : make_uint4(0, 0, 0, 0);
    }
    auto elem = [&](const uint4& v, int i) { return D::load(reinterpret_cast<const OS*>(&v)[i]); };
    const float inv_d = 1.0f / static_cast<float>(d);
    float mean = 0.0f, rstd;
    if constexpr (RMS) {
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const float v = elem(raw[j], i);
                s2 = fmaf(v, v, s2);
            }
        s2 = block_sum_w<NW>(s2, part);
        rstd = 1.0f / sqrtf(s2 * inv_d + eps);
    } else {
        float s1 = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < E; ++i) s1 += elem(raw[j], i);
        mean = block_sum_w<NW>(s1, part) * inv_d;
        float s2 = 0.0f;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = tid + static_cast<int64_t>(j) * NT;
            if (c >= nchunks) break;
#pragma unroll
            for (int i = 0; i < E; ++i) {
                const float cv = elem(raw[j], i) - mean;
                s2 = fmaf(cv, cv, s2);
            }
        }
        const float var = block_sum_w<NW>(s2, part) * inv_d;
        rstd = 1.0f / sqrtf(fmaxf(var, 0.0f) + eps);
    }
    const float bias = -rstd * mean;
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + static_cast<int64_t>(j) * NT;
        if (c >= nchunks) break;
        const uint4 sv = sr[c], hv = hr[c];
        OS* rp = reinterpret_cast<OS*>(&raw[j]);
#pragma unroll
        for (int i = 0; i < E; ++i) {
            const float v = elem(raw[j], i);
            const float y = D::round(RMS ? v * rstd : fmaf(v, rstd, bias));
            const float m = D::round(1.0f + elem(sv, i));
            const float z = D::round(y * m);
            rp[i] = D::store(z + elem(hv, i));
            amax = fmaxf(amax, fabsf(D::load(rp[i])));
        }
    }
    amax = wave_max(amax);
    __syncthreads();   // block_sum's readers of part are done
    if ((tid % kWave) == 0) part[tid / kWave] = amax;
    __syncthreads();
    amax = part[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) amax = fmaxf(amax, part[w]);
    const float s = row_scale<DT>(amax, recip != 0);
    if (tid == 0) xs[row] = s;
    const RowQuant rq = row_quant<DT>(s);
    int8_t* qr = q + row * d;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + static_cast<int64_t>(j) * NT;
        if (c >= nchunks) break;
        if constexpr (E == 8) {
            uint2 packed;
            packed.x = quant4_packed<DT>(elem(raw[j], 0), elem(raw[j], 1), elem(raw[j], 2), elem(raw[j], 3), rq);
            packed.y = quant4_packed<DT>(elem(raw[j], 4), elem(raw[j], 5), elem(raw[j], 6), elem(raw[j], 7), rq);
            *reinterpret_cast<uint2*>(qr + c * E) = packed;
        } else {
            *reinterpret_cast<uint32_t*>(qr + c * E) =
                quant4_packed<DT>(elem(raw[j], 0), elem(raw[j], 1), elem(raw[j], 2), elem(raw[j], 3), rq);
        }
    }
}

// QK RMSNorm + RoPE of the attention (Kitchen's rms_rope as the crate's eager
// route computes it, backend_rope.rs:204-222 and :146-159, non-split, full
// rotation): for each [head_dim] row of q and of k,
//   m = T(x * rsqrt(mean(x^2) + eps) * scale)   (aten rms_norm with weight: fp32, one rounding)
//   out[2i + j] = T( f[i][j][0] * m[2i] + f[i][j][1] * m[2i + 1] )   (fp32 products and sum)
// with f the token's [d/2][2][2] fp32 rotation from freqs [freq_batch, seq, d/2, 2, 2].
// One wave per token of q or of k: lane l holds rotation pairs l + 64 j (PPL
// pairs per lane) of the rotation row and both weights in registers for all
// the token's heads, which it walks kHeadGroup at a time (independent row
// sums, one wave butterfly each).  q tokens come first, then k tokens; tokens
// are [batch, seq] in order.  Token (b, t) of q and k starts x_stride
// elements after token (b, t - 1) (heads * d when packed, 3 * heads * d for
// q / k read straight out of a fused QKV output), its heads d apart; the
// outputs are packed [batch, seq, heads, d].  PAIR: every pair is read and
// written as one 2-element access (row bases aligned to two elements).
// NORM = false is the rotation alone (Kitchen's apply_rope / apply_rope1, the
// eager route backend_rope.rs:146-159): m = x, exact in fp32.  k == nullptr
// (ntensors = 1) is the one-tensor form (rms_rope1 / apply_rope1).  Output
// tokens are o_stride elements apart: heads * d (packed), or x_stride for
// the in-place forms (outputs equal to the inputs; every lane reads a group
// of rows into registers before it writes the same elements, and groups are
// disjoint).
constexpr int kHeadGroup = 8;

template <int DT, bool PAIR>
__device__ __forceinline__ void load_pair(const typename DType<DT>::storage* x, int64_t i, float& a, float& c) {
    using D = DType<DT>;
    if constexpr (PAIR && DT == W8A8_F32) {
        const float2 v = *reinterpret_cast<const float2*>(x + i);
        a = v.x;
        c = v.y;
    } else if constexpr (PAIR) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(x + i);
        a = D::load(static_cast<uint16_t>(v & 0xffffu));
        c = D::load(static_cast<uint16_t>(v >> 16));
    } else {
        a = D::load(x[i]);
        c = D::load(x[i + 1]);
    }
}

template <int DT, bool PAIR>
__device__ __forceinline__ void store_pair(typename DType<DT>::storage* o, int64_t i, float a, float c) {
    using D = DType<DT>;
    if constexpr (PAIR && DT == W8A8_F32) {
        *reinterpret_cast<float2*>(o + i) = make_float2(a, c);
    } else if constexpr (PAIR) {
        *reinterpret_cast<uint32_t*>(o + i) =
            static_cast<uint32_t>(D::store(a)) | (static_cast<uint32_t>(D::store(c)) << 16);
    } else {
        o[i] = D::store(a);
        o[i + 1] = D::store(c);
    }
}

template <int DT, int PPL, bool PAIR, bool NORM>
__global__ __launch_bounds__(256) void rms_rope_tokens(const void* q, const void* k,
                                                       const float* __restrict__ freqs,
                                                       const void* __restrict__ q_scale,
                                                       const void* __restrict__ k_scale, void* q_out,
                                                       void* k_out, int64_t tokens, int64_t seq,
                                                       int64_t heads, int64_t d, int64_t x_stride,
                                                       int64_t o_stride, int ntensors, int freq_per_batch,
                                                       float eps) {
    using D = DType<DT>;
    using OS = typename D::storage;
    const int lane = threadIdx.x % kWave;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (wave >= ntensors * tokens) return;   // whole waves only; the kernel has no block barrier
    const bool is_k = wave >= tokens;
    const int64_t tok = is_k ? wave - tokens : wave;
    const OS* x = static_cast<const OS*>(is_k ? k : q) + tok * x_stride;
    const OS* w = static_cast<const OS*>(is_k ? k_scale : q_scale);
    OS* o = static_cast<OS*>(is_k ? k_out : q_out) + tok * o_stride;
    const int64_t b = tok / seq, t = tok % seq;
    const float4* f = reinterpret_cast<const float4*>(freqs + ((freq_per_batch ? b * seq : 0) + t) * (d / 2) * 4);
    float4 fv[PPL];
    float w0[PPL], w1[PPL];
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int64_t p = lane + j * kWave;
        fv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        w0[j] = w1[j] = 0.0f;
        if (2 * p < d) {
            fv[j] = f[p];   // f[p][0][0], f[p][0][1], f[p][1][0], f[p][1][1]
            if constexpr (NORM) {
                w0[j] = D::load(w[2 * p]);
                w1[j] = D::load(w[2 * p + 1]);
            }
        }
    }
    for (int64_t h0 = 0; h0 < heads; h0 += kHeadGroup) {
        float a[kHeadGroup][PPL], c[kHeadGroup][PPL], sum[kHeadGroup];
#pragma unroll
        for (int g = 0; g < kHeadGroup; ++g) {
            sum[g] = 0.0f;
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const int64_t p = lane + j * kWave;
                a[g][j] = c[g][j] = 0.0f;
                if (h0 + g < heads && 2 * p < d) load_pair<DT, PAIR>(x, (h0 + g) * d + 2 * p, a[g][j], c[g][j]);
                sum[g] += a[g][j] * a[g][j];
                sum[g] += c[g][j] * c[g][j];
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
#pragma unroll
                for (int g = 0; g < kHeadGroup; ++g) sum[g] += __shfl_xor(sum[g], off, kWave);
            }
        }
#pragma unroll
        for (int g = 0; g < kHeadGroup; ++g) {
            if (h0 + g >= heads) break;
            const float r = NORM ? 1.0f / sqrtf(sum[g] / static_cast<float>(d) + eps) : 1.0f;
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const int64_t p = lane + j * kWave;
                if (2 * p >= d) break;
                const float m0 = NORM ? D::round(a[g][j] * r * w0[j]) : a[g][j];
                const float m1 = NORM ? D::round(c[g][j] * r * w1[j]) : c[g][j];
                store_pair<DT, PAIR>(o, (h0 + g) * d + 2 * p, fv[j].x * m0 + fv[j].y * m1,
                                     fv[j].z * m0 + fv[j].w * m1);
            }
        }
    }
}

// The same operation for 16-bit rows of d = 8 * LPR (64, 128, 256), aligned
// to 16 bytes: LPR lanes per row, each lane 8 consecutive elements (one
// 16-byte load and store), 64 / LPR of the token's heads per wave
// instruction, so a row costs log2(LPR) butterfly steps and one rsqrt over 8
// elements per lane.  The lane's 4 rotation pairs and 8 weights sit in
// registers for the whole token.  Same numerics per element as
// rms_rope_tokens (the fp32 row sum adds in another order).
template <int DT, int LPR, bool NORM>
__global__ __launch_bounds__(256) void rms_rope_tokens_vec(const void* q, const void* k,
                                                           const float* __restrict__ freqs,
                                                           const void* __restrict__ q_scale,
                                                           const void* __restrict__ k_scale,
                                                           void* q_out, void* k_out,
                                                           int64_t tokens, int64_t seq, int64_t heads,
                                                           int64_t x_stride, int64_t o_stride, int ntensors,
                                                           int freq_per_batch, float eps) {
    using D = DType<DT>;
    using OS = typename D::storage;
    static_assert(sizeof(OS) == 2, "16-bit rows only");
    constexpr int d = 8 * LPR, kRows = kWave / LPR, kGroup = 3;
    const int lane = threadIdx.x % kWave;
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (wave >= ntensors * tokens) return;   // whole waves only; the kernel has no block barrier
    const bool is_k = wave >= tokens;
    const int64_t tok = is_k ? wave - tokens : wave;
    const int sub = lane / LPR, col = lane % LPR;
    const OS* x = static_cast<const OS*>(is_k ? k : q) + tok * x_stride + col * 8;
    OS* o = static_cast<OS*>(is_k ? k_out : q_out) + tok * o_stride + col * 8;
    const int64_t b = tok / seq, t = tok % seq;
    const float4* f = reinterpret_cast<const float4*>(freqs + ((freq_per_batch ? b * seq : 0) + t) * (d / 2) * 4) +
                      col * 4;
    float4 fv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) fv[i] = f[i];   // pair i: f[0][0], f[0][1], f[1][0], f[1][1]
    float w[8] = {};
    if constexpr (NORM) {
        const uint4 wv = *reinterpret_cast<const uint4*>(static_cast<const OS*>(is_k ? k_scale : q_scale) + col * 8);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[2 * i] = D::load(static_cast<uint16_t>(ww[i] & 0xffffu));
            w[2 * i + 1] = D::load(static_cast<uint16_t>(ww[i] >> 16));
        }
    }
    for (int64_t h0 = 0; h0 < heads; h0 += kRows * kGroup) {
        float v[kGroup][8], sum[kGroup];
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            const int64_t h = h0 + g * kRows + sub;
            uint4 u = make_uint4(0u, 0u, 0u, 0u);
            if (h < heads) u = load_stream(x + h * d);
            const uint32_t uu[4] = {u.x, u.y, u.z, u.w};
            sum[g] = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[g][2 * i] = D::load(static_cast<uint16_t>(uu[i] & 0xffffu));
                v[g][2 * i + 1] = D::load(static_cast<uint16_t>(uu[i] >> 16));
                sum[g] += v[g][2 * i] * v[g][2 * i];
                sum[g] += v[g][2 * i + 1] * v[g][2 * i + 1];
            }
        }
        if constexpr (NORM) {
#pragma unroll
            for (int off = LPR / 2; off > 0; off >>= 1) {
#pragma unroll
                for (int g = 0; g < kGroup; ++g) sum[g] += __shfl_xor(sum[g], off, kWave);
            }
        }
#pragma unroll
        for (int g = 0; g < kGroup; ++g) {
            const int64_t h = h0 + g * kRows + sub;
            if (h >= heads) continue;
            const float r = NORM ? 1.0f / sqrtf(sum[g] / static_cast<float>(d) + eps) : 1.0f;
            uint32_t out[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float m0 = NORM ? D::round(v[g][2 * i] * r * w[2 * i]) : v[g][2 * i];
                const float m1 = NORM ? D::round(v[g][2 * i + 1] * r * w[2 * i + 1]) : v[g][2 * i + 1];
                out[i] = D::store2(fv[i].x * m0 + fv[i].y * m1, fv[i].z * m0 + fv[i].w * m1);
            }
            *reinterpret_cast<uint4*>(o + h * d) = make_uint4(out[0], out[1], out[2], out[3]);
        }
    }
}

// x[b, t, :] += y[b, t, :] * gate[b, :], gate = gate0 for t < prefix else gate1;
// gates are [batch, d].  out may alias x (the reference updates x in place).
template <int DT>
__global__ __launch_bounds__(kGlueThreads) void gated_residual_rows(const void* x,
                                                                    const void* __restrict__ y,
                                                                    const void* __restrict__ gate0,
                                                                    const void* __restrict__ gate1,
                                                                    void* out, int64_t tokens,
                                                                    int64_t d, int64_t prefix) {
    using D = DType<DT>;
    using OS = typename D::storage;
    const int64_t row = blockIdx.x;   // b * tokens + t
    const int64_t b = row / tokens, t = row % tokens;
    const OS* g = static_cast<const OS*>(t < prefix ? gate0 : gate1) + b * d;
    const OS* xr = static_cast<const OS*>(x) + row * d;
    const OS* yr = static_cast<const OS*>(y) + row * d;
    OS* o = static_cast<OS*>(out) + row * d;
    for (int64_t k = threadIdx.x; k < d; k += kGlueThreads) {
        // y * g of two 16-bit values is exact in fp32: one fp32 rounding of
        // the sum, then the rounding to T, as ATen's addcmul.
        const float v = D::load(xr[k]) + D::load(yr[k]) * D::load(g[k]);
        o[k] = D::store(v);
    }
}

// The same over 16-byte chunks (d % E == 0, 16-byte aligned operands): chunk
// c of the [rows, d] tensor lies in row c / (d / E).
template <int DT>
__global__ __launch_bounds__(kGlueThreads) void gated_residual_vec(const uint4* x,
                                                                   const uint4* __restrict__ y,
                                                                   const uint4* __restrict__ gate0,
                                                                   const uint4* __restrict__ gate1,
                                                                   uint4* out, int64_t tokens, int64_t dc,
                                                                   int64_t prefix, int64_t total) {
    using D = DType<DT>;
    constexpr int E = 16 / D::bytes;
    for (int64_t c = static_cast<int64_t>(blockIdx.x) * kGlueThreads + threadIdx.x; c < total;
         c += static_cast<int64_t>(gridDim.x) * kGlueThreads) {
        const int64_t row = c / dc, k = c % dc;
        const int64_t b = row / tokens, t = row % tokens;
        const uint4 xv = load_stream(x + c), yv = load_stream(y + c), gv = (t < prefix ? gate0 : gate1)[b * dc + k];
        const typename D::storage* xe = reinterpret_cast<const typename D::storage*>(&xv);
        const typename D::storage* ye = reinterpret_cast<const typename D::storage*>(&yv);
        const typename D::storage* ge = reinterpret_cast<const typename D::storage*>(&gv);
        uint4 res;
        typename D::storage* re = reinterpret_cast<typename D::storage*>(&res);
#pragma unroll
        for (int i = 0; i < E; ++i) re[i] = D::store(D::load(xe[i]) + D::load(ye[i]) * D::load(ge[i]));
        out[c] = res;
    }
}

// Modulated per-token quantizer: xm = T(x * T(1 + s_k)), s = modulation_scale[K];
// scale = max(amax(xm) / 127, 1e-30) (or the CUDA form), codes as the plain
// quantizer.  xm is recomputed in the code pass (same operations, same bits).
template <int DT>
__global__ __launch_bounds__(kGlueThreads) void quant_rows_modulated(const void* __restrict__ x,
                                                                     const void* __restrict__ mod,
                                                                     int8_t* __restrict__ q,
                                                                     float* __restrict__ xs,
                                                                     int64_t K, int recip) {
    using D = DType<DT>;
    using OS = typename D::storage;
    __shared__ float part[4];
    const int64_t row = blockIdx.x;
    const OS* xr = static_cast<const OS*>(x) + row * K;
    const OS* mr = static_cast<const OS*>(mod);
    auto xm = [&](int64_t k) { return D::round(D::load(xr[k]) * D::round(1.0f + D::load(mr[k]))); };
    float amax = 0.0f;
    for (int64_t k = threadIdx.x; k < K; k += kGlueThreads) amax = fmaxf(amax, fabsf(xm(k)));
    amax = wave_max(amax);
    if ((threadIdx.x % kWave) == 0) part[threadIdx.x / kWave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(part[0], part[1]), fmaxf(part[2], part[3]));
    const float s = row_scale<DT>(amax, recip != 0);
    if (threadIdx.x == 0) xs[row] = s;
    const RowQuant rq = row_quant<DT>(s);
    for (int64_t k = threadIdx.x; k < K; k += kGlueThreads)
        q[row * K + k] = static_cast<int8_t>(quant_elem<DT>(xm(k), rq));
}

}  // namespace

namespace {

// Rows of up to 1024 16-byte chunks take 128 threads (2 waves), longer rows
// 256: at the DiT width (3072 bf16 = 384 chunks) every lane then holds 3
// chunks, where 256 threads would leave a quarter of them idle.
template <int DT, bool RMS, bool SINGLE, int CPL>
void launch_adaln_vec(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
                      int64_t sg, int64_t tg, float eps, bool narrow, hipStream_t stream) {
    if (narrow)
        hipLaunchKernelGGL((adaln_rows_vec<DT, RMS, SINGLE, CPL, 128>), dim3(static_cast<unsigned>(n)), dim3(128), 0,
                           stream, x, scale, shift, out, d, sg, tg, eps);
    else
        hipLaunchKernelGGL((adaln_rows_vec<DT, RMS, SINGLE, CPL, 256>), dim3(static_cast<unsigned>(n)), dim3(256), 0,
                           stream, x, scale, shift, out, d, sg, tg, eps);
}

template <int DT, bool RMS, bool SINGLE>
bool adaln_vec_dispatch(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
                        int64_t sg, int64_t tg, float eps, hipStream_t stream) {
    constexpr int E = 16 / DType<DT>::bytes;
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (d % E != 0 || !al(x) || !al(scale) || !al(shift) || !al(out)) return false;
    const bool narrow = d / E <= 1024;
    const int nt = narrow ? 128 : 256;
    const int64_t per_lane = (d / E + nt - 1) / nt;
    switch (per_lane) {
        case 1: launch_adaln_vec<DT, RMS, SINGLE, 1>(x, scale, shift, out, n, d, sg, tg, eps, narrow, stream); return true;
        case 2: launch_adaln_vec<DT, RMS, SINGLE, 2>(x, scale, shift, out, n, d, sg, tg, eps, narrow, stream); return true;
        case 3: launch_adaln_vec<DT, RMS, SINGLE, 3>(x, scale, shift, out, n, d, sg, tg, eps, narrow, stream); return true;
        case 4: launch_adaln_vec<DT, RMS, SINGLE, 4>(x, scale, shift, out, n, d, sg, tg, eps, narrow, stream); return true;
        case 5:
        case 6: launch_adaln_vec<DT, RMS, SINGLE, 6>(x, scale, shift, out, n, d, sg, tg, eps, narrow, stream); return true;
        case 7:
        case 8: launch_adaln_vec<DT, RMS, SINGLE, 8>(x, scale, shift, out, n, d, sg, tg, eps, narrow, stream); return true;
        default: return false;
    }
}

}  // namespace

namespace {

template <int DT, bool RMS>
bool modnorm_quant_dispatch(const void* x, const void* s0, const void* s1, const void* h0, const void* h1,
                            int8_t* q, float* xs, int64_t rows, int64_t tokens, int64_t d, int64_t prefix,
                            float eps, int recip, hipStream_t stream) {
    constexpr int E = 16 / DType<DT>::bytes;
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (d % E != 0 || !al(x) || !al(s0) || !al(s1) || !al(h0) || !al(h1) || reinterpret_cast<uintptr_t>(q) % E != 0)
        return false;
    const bool narrow = d / E <= 1024;   // 128 threads per row, as launch_adaln_vec
    const int nt = narrow ? 128 : 256;
    const int64_t per_lane = (d / E + nt - 1) / nt;
    const dim3 grid(static_cast<unsigned>(rows)), block(nt);
#define W8A8_MNQ(CPL)                                                                                     \
    do {                                                                                                  \
        if (narrow)                                                                                       \
            hipLaunchKernelGGL((modnorm_quant_rows_vec<DT, RMS, CPL, 128>), grid, block, 0, stream, x, s0, s1, h0, h1, q, xs, tokens, d, prefix, eps, recip); \
        else                                                                                              \
            hipLaunchKernelGGL((modnorm_quant_rows_vec<DT, RMS, CPL, 256>), grid, block, 0, stream, x, s0, s1, h0, h1, q, xs, tokens, d, prefix, eps, recip); \
    } while (0)
    switch (per_lane) {
        case 1: W8A8_MNQ(1); return true;
        case 2: W8A8_MNQ(2); return true;
        case 3: W8A8_MNQ(3); return true;
        case 4: W8A8_MNQ(4); return true;
        case 5:
        case 6: W8A8_MNQ(6); return true;
        case 7:
        case 8: W8A8_MNQ(8); return true;
        default: return false;
    }
#undef W8A8_MNQ
}

}  // namespace

bool launch_modnorm_quant(const void* x, const void* s0, const void* s1, const void* h0, const void* h1, int8_t* q,
                          float* xs, int64_t rows, int64_t tokens, int64_t d, int64_t prefix, float eps, int dtype,
                          bool rms, int recip, hipStream_t stream) {
#define W8A8_MNQ_CASE(DT)                                                                                         \
    if (dtype == DT)                                                                                              \
        return rms ? modnorm_quant_dispatch<DT, true>(x, s0, s1, h0, h1, q, xs, rows, tokens, d, prefix, eps, recip, stream) \
                   : modnorm_quant_dispatch<DT, false>(x, s0, s1, h0, h1, q, xs, rows, tokens, d, prefix, eps, recip, stream);
    W8A8_MNQ_CASE(W8A8_BF16)
    W8A8_MNQ_CASE(W8A8_F16)
    W8A8_MNQ_CASE(W8A8_F32)
#undef W8A8_MNQ_CASE
    return false;
}

namespace {

template <int DT, bool RMS, bool SINGLE>
void adaln_dispatch(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
                    int64_t sg, int64_t tg, float eps, hipStream_t stream) {
    if (adaln_vec_dispatch<DT, RMS, SINGLE>(x, scale, shift, out, n, d, sg, tg, eps, stream)) return;
    hipLaunchKernelGGL((adaln_rows<DT, RMS, SINGLE>), dim3(static_cast<unsigned>(n)), dim3(kGlueThreads), 0, stream,
                       x, scale, shift, out, d, sg, tg, eps);
}

template <int DT>
void adaln_dispatch_dt(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
                       int64_t sg, int64_t tg, float eps, bool rms, bool single, hipStream_t stream) {
    if (rms && single) adaln_dispatch<DT, true, true>(x, scale, shift, out, n, d, sg, tg, eps, stream);
    else if (rms) adaln_dispatch<DT, true, false>(x, scale, shift, out, n, d, sg, tg, eps, stream);
    else if (single) adaln_dispatch<DT, false, true>(x, scale, shift, out, n, d, sg, tg, eps, stream);
    else adaln_dispatch<DT, false, false>(x, scale, shift, out, n, d, sg, tg, eps, stream);
}

}  // namespace

void launch_adaln(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
                  int64_t sg, int64_t tg, float eps, int dtype, bool rms, bool single, hipStream_t stream) {
    switch (dtype) {
        case W8A8_BF16: adaln_dispatch_dt<W8A8_BF16>(x, scale, shift, out, n, d, sg, tg, eps, rms, single, stream); return;
        case W8A8_F16: adaln_dispatch_dt<W8A8_F16>(x, scale, shift, out, n, d, sg, tg, eps, rms, single, stream); return;
        default: adaln_dispatch_dt<W8A8_F32>(x, scale, shift, out, n, d, sg, tg, eps, rms, single, stream); return;
    }
}

void launch_gated_residual(const void* x, const void* y, const void* gate0, const void* gate1, void* out,
                           int64_t batch, int64_t tokens, int64_t d, int64_t prefix, int dtype,
                           hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(batch * tokens)), block(kGlueThreads);
    const int esz = dtype == W8A8_F32 ? 4 : 2, E = 16 / esz;
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (d % E == 0 && al(x) && al(y) && al(gate0) && al(gate1) && al(out)) {
        const int64_t dc = d / E, total = batch * tokens * dc;
        const int64_t blocks = std::min<int64_t>((total + kGlueThreads - 1) / kGlueThreads, 256 * 16);
        const dim3 vgrid(static_cast<unsigned>(blocks));
        const uint4 *xv = static_cast<const uint4*>(x), *yv = static_cast<const uint4*>(y);
        const uint4 *g0 = static_cast<const uint4*>(gate0), *g1 = static_cast<const uint4*>(gate1);
        uint4* ov = static_cast<uint4*>(out);
        switch (dtype) {
            case W8A8_BF16:
                hipLaunchKernelGGL((gated_residual_vec<W8A8_BF16>), vgrid, block, 0, stream, xv, yv, g0, g1, ov, tokens, dc, prefix, total);
                return;
            case W8A8_F16:
                hipLaunchKernelGGL((gated_residual_vec<W8A8_F16>), vgrid, block, 0, stream, xv, yv, g0, g1, ov, tokens, dc, prefix, total);
                return;
            default:
                hipLaunchKernelGGL((gated_residual_vec<W8A8_F32>), vgrid, block, 0, stream, xv, yv, g0, g1, ov, tokens, dc, prefix, total);
                return;
        }
    }
    switch (dtype) {
        case W8A8_BF16:
            hipLaunchKernelGGL((gated_residual_rows<W8A8_BF16>), grid, block, 0, stream, x, y, gate0, gate1, out, tokens, d, prefix);
            break;
        case W8A8_F16:
            hipLaunchKernelGGL((gated_residual_rows<W8A8_F16>), grid, block, 0, stream, x, y, gate0, gate1, out, tokens, d, prefix);
            break;
        default:
            hipLaunchKernelGGL((gated_residual_rows<W8A8_F32>), grid, block, 0, stream, x, y, gate0, gate1, out, tokens, d, prefix);
            break;
    }
}

bool launch_rms_rope(const void* q, const void* k, const float* freqs, const void* q_scale, const void* k_scale,
                     void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t heads, int64_t d,
                     int64_t x_stride, bool freq_per_batch, float eps, bool norm, int dtype,
                     hipStream_t stream) {
    const int64_t tokens = batch * seq;
    const int nt = k ? 2 : 1;
    const int64_t o_stride = q_out == q ? x_stride : heads * d;
    const dim3 grid(static_cast<unsigned>((nt * tokens + 3) / 4)), block(256);
    const int fpb = freq_per_batch ? 1 : 0;
    const int ppl = d <= 128 ? 1 : d <= 256 ? 2 : 0;
    if (ppl == 0) return false;
    const auto a16 = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
    if (dtype != W8A8_F32 && (d == 64 || d == 128 || d == 256) && x_stride % 8 == 0 && a16(q) && a16(k) &&
        a16(q_out) && a16(k_out) && a16(q_scale) && a16(k_scale)) {
#define W8A8_RV_N(DT, LPR, N) hipLaunchKernelGGL((rms_rope_tokens_vec<DT, LPR, N>), grid, block, 0, stream, q, k, freqs, q_scale, k_scale, q_out, k_out, tokens, seq, heads, x_stride, o_stride, nt, fpb, eps)
#define W8A8_RV(DT, LPR) do { if (norm) W8A8_RV_N(DT, LPR, true); else W8A8_RV_N(DT, LPR, false); } while (0)
#define W8A8_RV_D(DT) do { if (d == 64) W8A8_RV(DT, 8); else if (d == 128) W8A8_RV(DT, 16); else W8A8_RV(DT, 32); } while (0)
        if (dtype == W8A8_BF16) W8A8_RV_D(W8A8_BF16);
        else W8A8_RV_D(W8A8_F16);
#undef W8A8_RV_D
#undef W8A8_RV
#undef W8A8_RV_N
        return true;
    }
    const uintptr_t al = 2 * (dtype == W8A8_F32 ? 4 : 2);
    const bool pair = x_stride % 2 == 0 && reinterpret_cast<uintptr_t>(q) % al == 0 &&
                      reinterpret_cast<uintptr_t>(k) % al == 0 && reinterpret_cast<uintptr_t>(q_out) % al == 0 &&
                      reinterpret_cast<uintptr_t>(k_out) % al == 0;
#define W8A8_RR_N(DT, PPL, PAIR, N) hipLaunchKernelGGL((rms_rope_tokens<DT, PPL, PAIR, N>), grid, block, 0, stream, q, k, freqs, q_scale, k_scale, q_out, k_out, tokens, seq, heads, d, x_stride, o_stride, nt, fpb, eps)
#define W8A8_RR(DT, PPL, PAIR) do { if (norm) W8A8_RR_N(DT, PPL, PAIR, true); else W8A8_RR_N(DT, PPL, PAIR, false); } while (0)
#define W8A8_RR_P(DT, PPL) do { if (pair) W8A8_RR(DT, PPL, true); else W8A8_RR(DT, PPL, false); } while (0)
#define W8A8_RR_D(DT) do { if (ppl == 1) W8A8_RR_P(DT, 1); else W8A8_RR_P(DT, 2); } while (0)
    if (dtype == W8A8_BF16) W8A8_RR_D(W8A8_BF16);
    else if (dtype == W8A8_F16) W8A8_RR_D(W8A8_F16);
    else W8A8_RR_D(W8A8_F32);
#undef W8A8_RR_D
#undef W8A8_RR_P
#undef W8A8_RR
#undef W8A8_RR_N
    return true;
}

void launch_quant_modulated(const void* x, int dtype, const void* mod, int8_t* q, float* xs, int64_t M,
                            int64_t K, int recip, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(M)), block(kGlueThreads);
    switch (dtype) {
        case W8A8_BF16:
            hipLaunchKernelGGL((quant_rows_modulated<W8A8_BF16>), grid, block, 0, stream, x, mod, q, xs, K, recip);
            break;
        case W8A8_F16:
            hipLaunchKernelGGL((quant_rows_modulated<W8A8_F16>), grid, block, 0, stream, x, mod, q, xs, K, recip);
            break;
        default:
            hipLaunchKernelGGL((quant_rows_modulated<W8A8_F32>), grid, block, 0, stream, x, mod, q, xs, K, recip);
            break;
    }
}

}  // namespace w8a8
