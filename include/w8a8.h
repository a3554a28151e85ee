/*
 * w8a8.h -- C ABI of libw8a8_hip.so, the MI355X (gfx950) W8A8 linear family.
 *
 * Drop-in replacement for the native calls the reference crate's int8_linear
 * operator makes through its C bridge (inference/native/bridge.hpp:29,
 * inference/native/bridge.cpp:415-440 -> Kitchen launchers).  Every entry point
 * takes plain device pointers, sizes, dtype codes and a HIP stream; nothing
 * is allocated or freed inside, nothing synchronizes (the reference's contract:
 * cuda_linear.rs:603-604,638,681,767 preallocate every output; bridge.cpp
 * launches on the caller's stream).
 *
 * Layouts (all row-major, contiguous):
 *   x       [M, K]   fp32 / fp16 / bf16 activations
 *   q       [M, K]   int8 quantized activations
 *   xs      [M]      fp32 per-row (per-token) scales     (the reference's [M,1])
 *   w       [N, K]   int8 weights, one row per output channel
 *   ws      [N] or [1] fp32 per-output-channel (or scalar) weight scales
 *   bias    [N]      in the output dtype, or NULL
 *   out     [M, N]   fp32 / fp16 / bf16
 *
 * Return codes follow the reference bridge (bridge.cpp:75-81,434-439):
 *   0 ok, -1 runtime error, -9 out of memory, -10 accelerator error
 *   (code in w8a8_last_accelerator_code()), -20 ValueError, -21 IndexError.
 * The message of the last failure on the calling thread is w8a8_last_error().
 */
#ifndef W8A8_H
#define W8A8_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: the reference's output codes (cuda_linear.rs:488-497). */
#define W8A8_F32 0
#define W8A8_F16 1
#define W8A8_BF16 2

#define W8A8_OK 0
#define W8A8_ERR_RUNTIME (-1)
#define W8A8_ERR_OOM (-9)
#define W8A8_ERR_ACCELERATOR (-10)
#define W8A8_ERR_VALUE (-20)
#define W8A8_ERR_INDEX (-21)

/* flags */
#define W8A8_SCALE_RECIP (1u << 0)   /* scale = amax * (1/127f), the reference's CUDA
                                        kernel form (int8_linear.cu:205-208); default is
                                        IEEE amax / 127, its CPU form (eager.rs:159-165) */
#define W8A8_ACT_GELU_TANH (1u << 1) /* quantize: gelu_tanh on x first (input_act,
                                        int8_linear.rs:37-41); GEMM/GEMV/dequant:
                                        gelu_tanh on the output-dtype value */
#define W8A8_OUT_INT32 (1u << 2)     /* GEMM: store the int32 accumulators (out is int32) */
#define W8A8_FUSED_QUANT (1u << 3)   /* w8a8_int8_linear: GEMM route quantizes x inside
                                        the GEMM's activation-tile load */
#define W8A8_ROUTE_GEMM (1u << 4)    /* w8a8_int8_linear: skip the M<=2 GEMV routes */
#define W8A8_GIVEN_SCALE (1u << 5)   /* w8a8_quantize_tensorwise: *scale holds the scale
                                        to quantize with (the reference's scale argument) */

/* Input activation codes of the linear (Kitchen's input_act_codes.h, SiTU 4
 * as the crate passes it: inference/src/convrot.rs:211-238): the crate's
 * int8_linear kwarg input_act = None, "gelu_tanh", "swiglu", "rms_norm", "situ"
 * (inference/src/int8_linear.rs:37-97).  SwiGLU and SiTU take a [gate | up] row
 * of 2K values and give K. */
#define W8A8_ACT_NONE 0
#define W8A8_ACT_GELU 1
#define W8A8_ACT_SWIGLU 2
#define W8A8_ACT_RMSNORM 3
#define W8A8_ACT_SITU 4

/* GEMM main loop (w8a8_gemm_dequant, w8a8_gemm_dequant_residual): flag bits
 * 8..11 hold a W8A8_GEMM_TILE_* code, W8A8_GEMM_TILE(code).  AUTO (0) lets
 * the shape choose; any other code requests that main loop, and a DMA tile
 * that does not take the shape (K not a multiple of its K tile) falls back to
 * the automatic choice.  Every main loop gives identical results.  No
 * reference counterpart (CUTLASS picks its tile in its own dispatch,
 * cutlass_gemm_int8.cu:190-269); used to test and time each main loop. */
#define W8A8_GEMM_TILE_AUTO 0
#define W8A8_GEMM_TILE_256x192 1     /* weight rows x tokens per block, 8 waves, 128-byte K tiles */
#define W8A8_GEMM_TILE_256x256 2     /* 8 waves, 128-byte K tiles */
#define W8A8_GEMM_TILE_384x192 3     /* 8 waves, 128-byte K tiles */
#define W8A8_GEMM_TILE_256x128 4     /* 4 waves, two blocks per CU, 64-byte K tiles */
#define W8A8_GEMM_TILE_REGS 5        /* register-staged main loop, K % 16 == 0 */
#define W8A8_GEMM_TILE_GENERIC 6     /* one thread per output, any shape and alignment */
#define W8A8_GEMM_TILE_SHIFT 8
#define W8A8_GEMM_TILE_MASK (0xFu << W8A8_GEMM_TILE_SHIFT)
#define W8A8_GEMM_TILE(code) ((uint32_t)(code) << W8A8_GEMM_TILE_SHIFT)

const char* w8a8_last_error(void);
int w8a8_last_accelerator_code(void);
/* Library version string ("w8a8-hip <major>.<minor> gfx950"). */
const char* w8a8_version(void);

/* Per-token dynamic absmax INT8 quantization.
 * Replaces Kitchen `quantize_int8_rowwise` (int8_linear.cu:184-227, launcher
 * :1322-1371), called by the crate at cuda_linear.rs:600-619.
 *   s[m] = max(amax_m / 127, 1e-30)
 *   q[m,k] = clamp(rint(T(x[m,k] / T(s[m]))), -128, 127)
 * Flags: W8A8_SCALE_RECIP, W8A8_ACT_GELU_TANH. */
int w8a8_quantize_rowwise(const void* x, int x_dtype, int8_t* q, float* xs,
                          int64_t M, int64_t K, uint32_t flags, hipStream_t stream);

/* Row scales only (pass 1 of the fused quant+GEMM): xs[m] as above. */
int w8a8_row_scales(const void* x, int x_dtype, float* xs, int64_t M, int64_t K,
                    uint32_t flags, hipStream_t stream);

/* M = 1 or 2 GEMV with the dequant epilogue.
 * Replaces Kitchen `int8_gemv_dequant` (dlpack_bindings.cpp:3535-3592;
 * int8_linear.cu:628-708, launcher :1800-1854), called at cuda_linear.rs:622-679:
 *   out[m,n] = O(fma(float(sum_k q[m,k] w[n,k]) * xs[m], ws[n], bias[n]))
 * ws_size is 1 or N.  Flags: W8A8_ACT_GELU_TANH. */
int w8a8_gemv_dequant(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                      int64_t ws_size, const void* bias, void* out, int out_dtype,
                      int64_t M, int64_t N, int64_t K, uint32_t flags, hipStream_t stream);

/* INT8 GEMM with the fused dequant epilogue (MFMA, gfx950).
 * Replaces Kitchen `cutlass_int8_dequant` (cutlass_gemm_int8.cu:63-120,373-388),
 * called at cuda_linear.rs:745-763, and, with W8A8_OUT_INT32, `cublas_gemm_int8`
 * (cublas_gemm_int8.cu:176-221, called at cuda_linear.rs:765-779):
 *   out[m,n] = O(fma(float(sum_k q[m,k] w[n,k]) * xs[m], ws[n], bias[n]))
 * Flags: W8A8_ACT_GELU_TANH, W8A8_OUT_INT32 (xs, ws, bias ignored),
 * W8A8_GEMM_TILE(code). */
int w8a8_gemm_dequant(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                      int64_t ws_size, const void* bias, void* out, int out_dtype,
                      int64_t M, int64_t N, int64_t K, uint32_t flags, hipStream_t stream);

/* The W8A8_GEMM_TILE_* code of the main loop w8a8_gemm_dequant launches for
 * M x N x K with these flags (its tile bits and W8A8_ACT_GELU_TANH, which
 * changes the automatic choice), for 16-byte aligned operands
 * (unaligned ones take W8A8_GEMM_TILE_GENERIC), on the current device.  A
 * query with no reference counterpart: tests use it to know which kernel ran. */
int w8a8_gemm_config(int64_t M, int64_t N, int64_t K, uint32_t flags);

/* GEMM with the fused residual epilogue of the pre-norm block:
 *   lin[m,n] = O(fma(float(sum_k q[m,k] w[n,k]) * xs[m], ws[n], bias[n]))
 *   out[m,n] = O(fma(lin[m,n], rscale[n], resid[m,n]))
 * Replaces Kitchen `cutlass_int8_dequant_residual` (archived
 * cutlass_gemm_int8.cu:122-188), called at cuda_linear.rs:724-742; the same
 * single fma as the crate's eager apply_residual on the GPU (int8_linear.rs:99-111).
 * rscale (rscale_size 1 or N entries) and resid ([M, N]) are in the output
 * dtype.  Flags: W8A8_GEMM_TILE(code) only (an output activation or int32
 * output is rejected). */
int w8a8_gemm_dequant_residual(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                               int64_t ws_size, const void* bias, const void* rscale,
                               int64_t rscale_size, const void* resid, void* out, int out_dtype,
                               int64_t M, int64_t N, int64_t K, uint32_t flags, hipStream_t stream);

/* M = 1 or 2 GEMV with the same residual epilogue.  Replaces `int8_gemv_dequant`
 * with its residual arguments (cuda_linear.rs:657-676; gemv_residual_args :171-191). */
int w8a8_gemv_dequant_residual(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                               int64_t ws_size, const void* bias, const void* rscale,
                               int64_t rscale_size, const void* resid, void* out, int out_dtype,
                               int64_t M, int64_t N, int64_t K, uint32_t flags, hipStream_t stream);

/* In place: out[m,n] = O(fma(out[m,n], rscale[n], resid[m,n])), all in dtype.
 * Replaces the eager apply_residual (inference/src/int8_linear.rs:99-111). */
int w8a8_residual_apply(void* out, const void* resid, const void* rscale, int64_t rscale_size,
                        int dtype, int64_t M, int64_t N, hipStream_t stream);

/* GEMM that quantizes the activation inside its tile load: x is the float
 * activation and xs its row scales from w8a8_row_scales (same flags).  Output
 * is bit-identical to w8a8_quantize_rowwise followed by w8a8_gemm_dequant.
 * No reference counterpart as one call: it fuses quantize_int8_rowwise
 * (int8_linear.cu:184-227) into cutlass_int8_dequant (cutlass_gemm_int8.cu:373-388). */
int w8a8_gemm_dequant_xq(const void* x, int x_dtype, const float* xs, const int8_t* w,
                         const float* ws, int64_t ws_size, const void* bias, void* out,
                         int out_dtype, int64_t M, int64_t N, int64_t K, uint32_t flags,
                         hipStream_t stream);

/* Standalone dequant of int32 accumulators.
 * Replaces Kitchen `dequantize_int8_linear` (int8_linear.cu:517-583, launcher
 * :1721-1798), called at cuda_linear.rs:783-794. */
int w8a8_dequantize_linear(const int32_t* acc, const float* xs, const float* ws,
                           int64_t ws_size, const void* bias, void* out, int out_dtype,
                           int64_t M, int64_t N, uint32_t flags, hipStream_t stream);

/* Operator-level W8A8 linear: the crate's int8_dispatch without ConvRot and
 * residual (cuda_linear.rs:419-824): quantize, then the GEMV route for
 * (M == 1 && K % 4 == 0) || (M == 2 && K % 16 == 0) (:498-511, :836-860),
 * else the GEMM route (which, like the reference's, needs K % 4 == 0).
 * The caller provides the workspace for q and xs (the crate allocates them per
 * call, :603-604); w8a8_int8_linear_workspace_bytes gives its size.
 * Flags: W8A8_SCALE_RECIP, W8A8_ACT_GELU_TANH (applied to x, as input_act),
 * W8A8_FUSED_QUANT, W8A8_ROUTE_GEMM. */
int64_t w8a8_int8_linear_workspace_bytes(int64_t M, int64_t K);
int w8a8_int8_linear(const void* x, int x_dtype, const int8_t* w, const float* ws,
                     int64_t ws_size, const void* bias, void* out, int out_dtype,
                     int64_t M, int64_t N, int64_t K, uint32_t flags, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream);

/* w8a8_int8_linear without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, serving loops that forbid hipMalloc).
 * No counterpart in the reference (the crate allocates q and xs per call,
 * cuda_linear.rs:603-604).  The codes and row scales go to a fixed device
 * array of W8A8_NOALLOC_SCRATCH_BYTES, one per device, held from this entry's
 * first call on the device until the process ends; nothing is allocated or
 * freed per call.  Inputs whose w8a8_int8_linear_workspace_bytes(M, K)
 * exceeds it fail with W8A8_ERR_VALUE.  Calls on one device share the array:
 * calls that overlap in time (other streams, other threads) race.  Same
 * routes, flags and results as w8a8_int8_linear. */
#define W8A8_NOALLOC_SCRATCH_BYTES (64ll << 20)
int64_t w8a8_int8_linear_noalloc_max_bytes(void);
int w8a8_int8_linear_noalloc(const void* x, int x_dtype, const int8_t* w, const float* ws, int64_t ws_size,
                             const void* bias, void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                             uint32_t flags, hipStream_t stream);

/* w8a8_int8_linear with the residual of the pre-norm block (the crate's
 * residual / residual_scale kwargs, cuda_linear.rs:700-744 and the eager
 * fallback int8_linear.rs:99-111), fused into the GEMM or GEMV epilogue:
 * out = O(fma(linear(x), rscale[n], resid[m,n])), rscale and resid in the
 * output dtype. */
int w8a8_int8_linear_residual(const void* x, int x_dtype, const int8_t* w, const float* ws,
                              int64_t ws_size, const void* bias, const void* rscale,
                              int64_t rscale_size, const void* resid, void* out, int out_dtype,
                              int64_t M, int64_t N, int64_t K, uint32_t flags, void* workspace,
                              int64_t workspace_bytes, hipStream_t stream);

/* ---- ConvRot (online Hadamard rotation of the activations) ----------------
 * Every `group`-wide slice of a row is multiplied by the regular Hadamard
 * matrix H_G = (H4 (x) ... (x) H4) / sqrt(G) (inference/src/int8_utils.rs:21-58);
 * group is a power of 4 up to 16384 that divides K.  Bad groups return
 * W8A8_ERR_VALUE with the reference's messages (int8_utils.rs:36-46,60-73). */

/* y = dtype(x rotated), [M, K] in x's dtype.  Replaces rotate_activation
 * (int8_utils.rs:97-106) on the crate's unfused route (convrot.rs:474-484). */
int w8a8_convrot_rotate(const void* x, int x_dtype, void* y, int64_t M, int64_t K, int64_t group,
                        hipStream_t stream);

/* Bytes of the rotated-input buffer w8a8_quantize_rowwise_convrot needs: 0 on
 * the fused route (group 256, K % 256 == 0, 256 <= K <= 16384, the crate's
 * predicate cuda_linear.rs:404-417), else M*K elements of x's dtype. */
int64_t w8a8_convrot_workspace_bytes(int64_t M, int64_t K, int64_t group, int x_dtype);

/* ConvRot activation quantization, by the crate's route (cuda_linear.rs:586-599):
 * on the fused route it replaces Kitchen quantize_int8_rowwise_convrot64
 * (native/comfy-port/kitchen/int8_linear.cu:1204-1314, launcher :1609-1719):
 * fp32 rotation, absmax of the fp32 values, q = clamp(rint(T(T(y) / T(s));
 * elsewhere it rotates into `rotated` (rounded to the dtype) and runs
 * w8a8_quantize_rowwise on it.  Flags: W8A8_SCALE_RECIP. */
int w8a8_quantize_rowwise_convrot(const void* x, int x_dtype, int8_t* q, float* xs, int64_t M,
                                  int64_t K, int64_t group, uint32_t flags, void* rotated,
                                  int64_t rotated_bytes, hipStream_t stream);

/* w8a8_int8_linear with convrot=true, convrot_groupsize=group (the crate's
 * int8_linear kwargs, backend_signatures.rs:445-460; route cuda_linear.rs:586-599)
 * and an optional residual (resid == NULL: none).  The workspace holds q, xs
 * and, off the fused route, the rotated input:
 * w8a8_int8_linear_convrot_workspace_bytes gives its size.  W8A8_ACT_GELU_TANH
 * is the gelu_tanh input activation (as w8a8_int8_linear_act). */
int64_t w8a8_int8_linear_convrot_workspace_bytes(int64_t M, int64_t K, int64_t group, int x_dtype);
int w8a8_int8_linear_convrot(const void* x, int x_dtype, const int8_t* w, const float* ws,
                             int64_t ws_size, const void* bias, const void* rscale,
                             int64_t rscale_size, const void* resid, void* out, int out_dtype,
                             int64_t M, int64_t N, int64_t K, int64_t group, uint32_t flags,
                             void* workspace, int64_t workspace_bytes, hipStream_t stream);

/* ---- Input activations (the crate's input_act kwargs) ---------------------
 * act is a W8A8_ACT_* code; act_weight is RMSNorm's [K] weight in x's dtype
 * (NULL for the others; missing for rms_norm: W8A8_ERR_VALUE with the
 * reference's text "input_act 'rms_norm' requires act_weight",
 * int8_linear.rs:79-81), act_eps its epsilon.  K is the output width; x is
 * [M, 2K] ([gate | up] rows) for SwiGLU and SiTU, [M, K] otherwise. */

/* The eager activation of apply_input (inference/src/int8_linear.rs:37-97):
 * ATen ops on x's dtype T, each result rounded to T:
 *   gelu_tanh T(gelu(x)); swiglu T(T(silu(a)) * b);
 *   situ T(T(T(tanh(T(a/25))) * 25) * T(T(T(tanh(T(b/4))) * 4) * T(sigmoid(b))));
 *   rms_norm T(x * rstd * w), rstd = 1 / sqrt(mean(x^2) + eps)  (one rounding)
 * with correctly rounded fp32 exp and tanh.  y is [M, K] in T. */
int w8a8_input_act(const void* x, int x_dtype, int act, const void* act_weight, double act_eps, void* y, int64_t M,
                   int64_t K, hipStream_t stream);

/* The activation quantizer of the crate's int8_dispatch (cuda_linear.rs:
 * 450-481, 586-619): q [M, K] int8 and xs [M] of act(x),
 *   convrot_group == 0: the eager activation fused into the per-token
 *     quantizer (same codes as w8a8_input_act then w8a8_quantize_rowwise);
 *   ConvRot fused route (group 256, K % 256 == 0, 256 <= K <= 16384): Kitchen's
 *     quantize_int8_rowwise_convrot64 with the activation fused in fp32 and not
 *     rounded to T (native/comfy-port/kitchen/int8_linear.cu:1175-1262,
 *     launcher :1618-1706; the crate's predicate cuda_linear.rs:404-417);
 *   other ConvRot groups: the eager activation, rotated, quantized; aux then
 *     holds w8a8_convrot_workspace_bytes(M, K, group, x_dtype) bytes.
 * Flags: W8A8_SCALE_RECIP. */
int w8a8_quantize_rowwise_act(const void* x, int x_dtype, int act, const void* act_weight, double act_eps, int8_t* q,
                              float* xs, int64_t M, int64_t K, int64_t convrot_group, uint32_t flags, void* aux,
                              int64_t aux_bytes, hipStream_t stream);

/* The operator with every kwarg of the crate's int8_linear
 * (backend_signatures.rs:445-460; int8_dispatch cuda_linear.rs:419-824):
 * input activation, ConvRot (convrot_group 0: none) and residual (resid NULL:
 * none) in one call.  Routes as w8a8_int8_linear on the output width K.
 * Workspace: w8a8_int8_linear_workspace_bytes(M, K) without ConvRot,
 * w8a8_int8_linear_convrot_workspace_bytes(M, K, group, x_dtype) with it.
 * Flags: W8A8_SCALE_RECIP, W8A8_ROUTE_GEMM. */
int w8a8_int8_linear_act(const void* x, int x_dtype, int act, const void* act_weight, double act_eps, const int8_t* w,
                         const float* ws, int64_t ws_size, const void* bias, const void* rscale, int64_t rscale_size,
                         const void* resid, void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                         int64_t convrot_group, uint32_t flags, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream);

/* ---- Weight quantizers (TensorWiseINT8Layout.from_float) -----------------
 * The layout's quantize step (inference/src/layout_complete.rs:119-160):
 * per-channel weights use w8a8_quantize_rowwise over the N rows, tensorwise
 * weights w8a8_quantize_tensorwise, ConvRot weights
 * w8a8_quantize_convrot_weight. */

/* One scale for all n elements of x (quantize_int8_tensorwise,
 * inference/src/eager.rs:134-151, which the reference's CUDA backend runs too,
 * backend_bindings.rs:549-585): s = max(amax / 127, 1e-30), or the caller's
 * scale with W8A8_GIVEN_SCALE; q = clamp(rint(T(x / T(s)))).  scale is one
 * fp32 in device memory (written unless W8A8_GIVEN_SCALE).  Flags:
 * W8A8_SCALE_RECIP, W8A8_GIVEN_SCALE. */
int w8a8_quantize_tensorwise(const void* x, int x_dtype, int8_t* q, float* scale, int64_t n,
                             uint32_t flags, hipStream_t stream);

/* ConvRot weight quantization w [N, K] -> q [N, K], per-row scales [N]
 * (quantize_int8_convrot_weight, inference/src/convrot.rs:378-429; path choice
 * weight_path :345-372): group 256 with K % 256 == 0 (up to K = 65536) takes
 * the fused rotation's numerics (fp32 rotated values, absmax over them),
 * like the reference's Rowwise64 and Staged paths; other groups rotate
 * (rounded to the dtype) and quantize rowwise, like its EagerRotation path,
 * using `rotated` (w8a8_convrot_weight_workspace_bytes).  Flags: W8A8_SCALE_RECIP. */
int64_t w8a8_convrot_weight_workspace_bytes(int64_t N, int64_t K, int64_t group, int w_dtype);
int w8a8_quantize_convrot_weight(const void* w, int w_dtype, int8_t* q, float* scale, int64_t N,
                                 int64_t K, int64_t group, uint32_t flags, void* rotated,
                                 int64_t rotated_bytes, hipStream_t stream);

/* ---- DiT block glue around the linears ------------------------------------ */

/* Mode bits of w8a8_adaln's `rms` argument (0 / 1 keep their meaning). */
#define W8A8_ADALN_RMS 1             /* RMSNorm instead of LayerNorm */
#define W8A8_ADALN_SINGLE_ROUNDING 2 /* out = T(fma(norm, 1 + scale, shift)) in fp32 */

/* Adaptive LayerNorm / RMSNorm with modulation, Kitchen's native "adaln" and
 * "rms_adaln" calls as the crate issues them (inference/src/backend_eager.rs:
 * 176-229: input [n, d], scale [n / scale_group, d], shift [n / shift_group, d],
 * out, n, d, sg, tg, eps, dtype): row i gets scale row i / scale_group and
 * shift row i / shift_group, and
 *   out = T( T( T(norm(x)) * T(1 + scale) ) + shift ),
 * norm = layer_norm without affine (biased variance) or, with
 * W8A8_ADALN_RMS, x * rsqrt(mean(x^2) + eps), in fp32: the op order of the
 * crate's eager route (:186-199).  W8A8_ADALN_SINGLE_ROUNDING gives instead
 * the single rounding of Kitchen's CUDA kernel (adaln.cu in the reference's
 * design/reference-local/native-source-candidates.tar.gz: fp32 statistics,
 * (x - mean) * rstd * (1 + scale) + shift rounded once); that kernel's row
 * sums and its approximate rsqrt are not restated, so outputs agree with it
 * to an ulp, not bit for bit.  d == 0 fails with the reference's
 * ZeroDivisionError text as W8A8_ERR_VALUE. */
int w8a8_adaln(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
               int64_t scale_group, int64_t shift_group, double eps, int dtype, int rms,
               hipStream_t stream);

/* modulated_norm fused with the per-token quantizer, for a norm whose only
 * consumer is an INT8 linear (the DiT's norm1 -> QKV and norm2 -> FFN-up):
 * no counterpart in the reference, which runs modulated_norm
 * (inference/src/models/qwen_image21/numeric.rs:63-107, two "adaln" calls)
 * and then quantizes its output inside int8_linear.  x [batch * tokens, d];
 * row b * tokens + t uses scale0 / shift0 row b ([batch, d]) for t < prefix,
 * else scale1 / shift1.  The codes q [rows, d] and row scales xs [rows] are
 * those w8a8_quantize_rowwise gives for w8a8_adaln's output, bit for bit.
 * Needs 16-byte aligned operands, d a multiple of 16 bytes / element size
 * and at most 2048 16-byte chunks per row (else W8A8_ERR_VALUE: run the two
 * steps).  Flags: W8A8_SCALE_RECIP. */
int w8a8_modulated_norm_quant(const void* x, const void* scale0, const void* scale1, const void* shift0,
                              const void* shift1, int8_t* q, float* xs, int64_t batch, int64_t tokens, int64_t d,
                              int64_t prefix, double eps, int dtype, int rms, uint32_t flags, hipStream_t stream);

/* QK RMSNorm + RoPE of the DiT attention: Kitchen's "rms_rope" call
 * (inference/src/backend_rope.rs:311-345) with the numerics of the crate's
 * eager route (eager_rms :204-222, eager_apply :146-159, non-split, whole
 * head rotated).  q, k [batch, seq, heads, d] in dtype with the heads of a
 * token packed d apart and consecutive tokens x_row_stride elements apart
 * (heads * d when packed; 3 * heads * d for views into a fused QKV output);
 * q_out, k_out packed [batch, seq, heads, d]; q_scale, k_scale [d] in dtype;
 * freqs fp32 [freq_per_batch ? batch : 1, seq, d/2, 2, 2] (the reference's
 * [B|1, S, 1, d/2, 2, 2]), 16-byte aligned.  Per row:
 *   m = T(x * rsqrt(mean(x^2) + eps) * scale)   (aten rms_norm: fp32, one rounding)
 *   out[2i + j] = T(f[i][j][0] * m[2i] + f[i][j][1] * m[2i + 1])   (fp32)
 * d even, at most 256; x_row_stride >= heads * d.  k == NULL is Kitchen's
 * one-tensor rms_rope1 (backend_rope.rs:364-440, "x", "scale"): only q is
 * processed and k_scale, k_out are ignored.  q_out == q and k_out == k (both
 * or neither) are the in-place forms (rms_rope_, rms_rope1_): the outputs then
 * keep the inputs' token stride; other overlaps of inputs and outputs are not
 * allowed. */
int w8a8_rms_rope(const void* q, const void* k, const float* freqs, const void* q_scale, const void* k_scale,
                  void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t heads, int64_t d,
                  int64_t x_row_stride, int freq_per_batch, double eps, int dtype, hipStream_t stream);

/* RoPE rotation alone: Kitchen's apply_rope (xq, xk) and, with k == NULL,
 * apply_rope1 (x), native call inference/src/backend_rope.rs:256-299 with the
 * numerics of the eager route (eager_apply :146-159, non-split):
 *   out[2i + j] = T(f[i][j][0] * x[2i] + f[i][j][1] * x[2i + 1])   (fp32)
 * Layouts, strides, freqs and the in-place forms (apply_rope_, apply_rope1_:
 * out == x) as for w8a8_rms_rope; other outputs packed. */
int w8a8_apply_rope(const void* x, const void* k, const float* freqs, void* out, void* k_out, int64_t batch,
                    int64_t seq, int64_t heads, int64_t d, int64_t x_row_stride, int freq_per_batch, int dtype,
                    hipStream_t stream);

/* Gated residual of the DiT block (inference/src/models/qwen_image21/
 * numeric.rs:110-125): x, y [batch, tokens, d], gates [batch, d];
 *   out[b, t] = T( fp32( x[b, t] + y[b, t] * gate[b] ) ),
 * gate = gate0 for t < prefix, else gate1 (ATen addcmul_ on each slice; y *
 * gate is exact in fp32 for 16-bit T).  out may equal x (in place, as the
 * reference). */
int w8a8_gated_residual(const void* x, const void* y, const void* gate0, const void* gate1, void* out,
                        int64_t batch, int64_t tokens, int64_t d, int64_t prefix, int dtype,
                        hipStream_t stream);

/* Per-token quantization of the modulated input of Kitchen's batch-one
 * int8_linear_modulated (inference/src/backend_bindings.rs:329-405):
 *   xm = T( x * T(1 + modulation_scale[k]) ),  then w8a8_quantize_rowwise on xm
 * (modulation_scale: K values in x's dtype), in one kernel.  Flags:
 * W8A8_SCALE_RECIP. */
int w8a8_quantize_rowwise_modulated(const void* x, int x_dtype, const void* modulation_scale, int8_t* q,
                                    float* xs, int64_t M, int64_t K, uint32_t flags, hipStream_t stream);

/* int8_linear_modulated (backend_bindings.rs:329-405): int8_linear of the
 * modulated input above, same routes, workspace (w8a8_int8_linear_workspace_bytes)
 * and epilogue as w8a8_int8_linear.  Flags: W8A8_SCALE_RECIP, W8A8_ROUTE_GEMM. */
int w8a8_int8_linear_modulated(const void* x, int x_dtype, const void* modulation_scale, const int8_t* w,
                               const float* ws, int64_t ws_size, const void* bias, void* out, int out_dtype,
                               int64_t M, int64_t N, int64_t K, uint32_t flags, void* workspace,
                               int64_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* W8A8_H */
