// C ABI of libw8a8_hip.so (declared in include/w8a8.h).
//
// Argument checks and error behaviour mirror the reference's native wrappers
// (Kitchen dlpack_bindings.cpp:2307-2335, :2747-2763, :3485-3660) and the
// bridge's error-code mapping (inference/native/bridge.cpp:75-81,434-439).
// Messages of the checks the crate's callers can trigger are the reference's
// own text, so a caller that matches on them keeps working.
#include <cstdio>
#include <string>

#include "w8a8_common.h"

namespace w8a8 {
void launch_quantize(const void* x, int x_dtype, int8_t* q, float* xs, int64_t M, int64_t K,
                     bool recip, bool gelu, bool scales_only, hipStream_t stream);
void launch_gemv(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                 int64_t ws_size, const void* bias, const Residual* res, void* out, int out_dtype,
                 int64_t M, int64_t N, int64_t K, bool gelu, hipStream_t stream);
void launch_gemm(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                 int64_t ws_size, const void* bias, const Residual* res, void* out, int out_dtype,
                 int64_t M, int64_t N, int64_t K, bool gelu, bool int32_out, int tile, hipStream_t stream);
int gemm_config(int64_t M, int64_t N, int64_t K, int requested, bool gelu);
void launch_residual(void* out, const void* resid, const void* rscale, int64_t rs_size, int dtype,
                     int64_t M, int64_t N, hipStream_t stream);
bool launch_gemm_xq(const void* x, int x_dtype, const float* xs, const int8_t* w, const float* ws,
                    int64_t ws_size, const void* bias, void* out, int out_dtype, int64_t M,
                    int64_t N, int64_t K, bool gelu, hipStream_t stream);
void launch_dequant(const int32_t* acc, const float* xs, const float* ws, int64_t ws_size,
                    const void* bias, void* out, int out_dtype, int64_t M, int64_t N, bool gelu,
                    hipStream_t stream);
bool convrot_fused_route(int64_t K, int64_t group);
void launch_act_rows(const void* x, int x_dtype, int act, const void* w, float eps, int8_t* q, float* xs, void* y,
                     int64_t M, int64_t K, bool recip, hipStream_t stream);
void launch_convrot_quant_act(const void* x, int x_dtype, int act, const void* w, float eps, int8_t* q, float* xs,
                              int64_t M, int64_t K, bool recip, hipStream_t stream);
void launch_convrot_quant(const void* x, int x_dtype, int8_t* q, float* xs, int64_t M, int64_t K,
                          bool recip, hipStream_t stream);
void launch_convrot_rotate(const void* x, int x_dtype, void* y, int64_t M, int64_t K, int64_t G,
                           hipStream_t stream);
bool convrot_weight_fused(const void* w, const void* q, int64_t K, int64_t group);
void launch_quantize_tensorwise(const void* x, int x_dtype, int8_t* q, float* scale, int64_t n, bool given,
                                bool recip, hipStream_t stream);
void launch_adaln(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
                  int64_t sg, int64_t tg, float eps, int dtype, bool rms, bool single, hipStream_t stream);
void launch_gated_residual(const void* x, const void* y, const void* gate0, const void* gate1, void* out,
                           int64_t batch, int64_t tokens, int64_t d, int64_t prefix, int dtype,
                           hipStream_t stream);
void launch_quant_modulated(const void* x, int dtype, const void* mod, int8_t* q, float* xs, int64_t M,
                            int64_t K, int recip, hipStream_t stream);
bool launch_rms_rope(const void* q, const void* k, const float* freqs, const void* q_scale, const void* k_scale,
                     void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t heads, int64_t d,
                     int64_t x_stride, bool freq_per_batch, float eps, bool norm, int dtype,
                     hipStream_t stream);
bool launch_modnorm_quant(const void* x, const void* s0, const void* s1, const void* h0, const void* h1, int8_t* q,
                          float* xs, int64_t rows, int64_t tokens, int64_t d, int64_t prefix, float eps, int dtype,
                          bool rms, int recip, hipStream_t stream);
}  // namespace w8a8

namespace {

thread_local std::string g_last_error;
thread_local int g_last_accel = 0;

int fail(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

}  // namespace

namespace w8a8 {
// The calling thread's error state, for the entry points of other translation units.
int set_error(int code, const std::string& msg) { return fail(code, msg); }
int set_accelerator_error(int hip_code, const std::string& msg) {
    g_last_accel = hip_code;
    return fail(W8A8_ERR_ACCELERATOR, msg);
}
}  // namespace w8a8

namespace {

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_last_accel = static_cast<int>(e);
        return fail(W8A8_ERR_ACCELERATOR, std::string(what) + ": " + hipGetErrorString(e));
    }
    return W8A8_OK;
}

bool valid_dtype(int d) { return d == W8A8_F32 || d == W8A8_F16 || d == W8A8_BF16; }

constexpr uint32_t kKnownFlags = W8A8_SCALE_RECIP | W8A8_ACT_GELU_TANH | W8A8_OUT_INT32 |
                                 W8A8_FUSED_QUANT | W8A8_ROUTE_GEMM | W8A8_GIVEN_SCALE | W8A8_GEMM_TILE_MASK;

int tile_of(uint32_t flags) { return static_cast<int>((flags & W8A8_GEMM_TILE_MASK) >> W8A8_GEMM_TILE_SHIFT); }

int check_tile(uint32_t flags) {
    if (tile_of(flags) > W8A8_GEMM_TILE_GENERIC) return fail(W8A8_ERR_VALUE, "unknown W8A8_GEMM_TILE code");
    return W8A8_OK;
}

int check_common(int64_t M, int64_t N, int64_t K, uint32_t flags) {
    if (M < 0 || N < 0 || K < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (flags & ~kKnownFlags) return fail(W8A8_ERR_VALUE, "unknown flag bits");
    return W8A8_OK;
}

int check_ws(int64_t ws_size, int64_t N, const char* msg) {
    if (ws_size != 1 && ws_size != N) return fail(W8A8_ERR_RUNTIME, msg);
    return W8A8_OK;
}

// Residual operands of the fused residual epilogue (cuda_linear.rs:707-744).
// The reference builds its Hadamard matrix first (int8_utils.rs:36-46) and
// then splits the features into groups (:60-73), with these messages.
int check_convrot_group(int64_t K, int64_t group) {
    if (group < 4 || (group & (group - 1)) != 0 || (group & 0x5555555555555555ll) == 0)
        return fail(W8A8_ERR_VALUE, "Regular Hadamard size must be a power of 4, got " + std::to_string(group));
    if (K % group != 0)
        return fail(W8A8_ERR_VALUE, "features " + std::to_string(K) + " not divisible by group_size " +
                                        std::to_string(group));
    if (group > 16384) return fail(W8A8_ERR_RUNTIME, "ConvRot groups above 16384 are not supported");
    return W8A8_OK;
}

// Input activation arguments (int8_linear.rs:37-97): a known code, and
// RMSNorm's weight (ValueError text of :79-81).
int check_act(int act, const void* act_weight) {
    if (act < W8A8_ACT_NONE || act > W8A8_ACT_SITU) return fail(W8A8_ERR_VALUE, "unknown input activation code");
    if (act == W8A8_ACT_RMSNORM && !act_weight) return fail(W8A8_ERR_VALUE, "input_act 'rms_norm' requires act_weight");
    return W8A8_OK;
}

int check_residual(const void* rscale, int64_t rscale_size, const void* resid, int64_t N) {
    if (!rscale || !resid) return fail(W8A8_ERR_VALUE, "residual requires residual_scale");
    if (rscale_size != 1 && rscale_size != N)
        return fail(W8A8_ERR_RUNTIME, "residual_scale must be scalar or per-output-channel");
    return W8A8_OK;
}

}  // namespace

namespace {

// Shared checks and launch of the RoPE family (norm: rms_rope / rms_rope1;
// otherwise apply_rope / apply_rope1; k == nullptr: the one-tensor forms).
int rope_entry(const char* name, const void* q, const void* k, const float* freqs, const void* q_scale,
               const void* k_scale, void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t heads, int64_t d,
               int64_t x_row_stride, int freq_per_batch, double eps, bool norm, int dtype, hipStream_t stream) {
    const std::string n(name);
    if (batch < 0 || seq < 0 || heads < 0 || d < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (!valid_dtype(dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported dtype for " + n);
    if (d % 2 != 0 || d > 256) return fail(W8A8_ERR_VALUE, n + " needs an even head dimension of at most 256");
    if (batch == 0 || seq == 0 || heads == 0 || d == 0) return W8A8_OK;
    if (x_row_stride < heads * d) return fail(W8A8_ERR_VALUE, n + ": x_row_stride must be at least heads * d");
    if (!q || !freqs || !q_out || (norm && !q_scale)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (k && (!k_out || (norm && !k_scale))) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (k && ((q_out == q) != (k_out == k)))
        return fail(W8A8_ERR_VALUE, n + ": both outputs equal their inputs (in place) or neither does");
    if (reinterpret_cast<uintptr_t>(freqs) % 16 != 0) return fail(W8A8_ERR_VALUE, "freqs must be 16-byte aligned");
    if (2 * batch * seq > 0x7fffffffll * 4) return fail(W8A8_ERR_VALUE, n + ": too many tokens");
    if (!w8a8::launch_rms_rope(q, k, freqs, q_scale, k ? k_scale : nullptr, q_out, k ? k_out : nullptr, batch, seq,
                               heads, d, x_row_stride, freq_per_batch != 0, static_cast<float>(eps), norm, dtype,
                               stream))
        return fail(W8A8_ERR_VALUE, n + " needs an even head dimension of at most 256");
    return check_launch(name);
}

}  // namespace

extern "C" {

const char* w8a8_last_error(void) { return g_last_error.c_str(); }
int w8a8_last_accelerator_code(void) { return g_last_accel; }
const char* w8a8_version(void) { return "w8a8-hip 0.1 gfx950"; }

int w8a8_quantize_rowwise(const void* x, int x_dtype, int8_t* q, float* xs, int64_t M, int64_t K,
                          uint32_t flags, hipStream_t stream) {
    if (int rc = check_common(M, 0, K, flags)) return rc;
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for INT8 quantization");
    if (M == 0) return W8A8_OK;
    if (K > 0 && (!x || !q)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (!xs) return fail(W8A8_ERR_VALUE, "null scale pointer");
    w8a8::launch_quantize(x, x_dtype, q, xs, M, K, flags & W8A8_SCALE_RECIP,
                          flags & W8A8_ACT_GELU_TANH, false, stream);
    return check_launch("quantize_int8_rowwise");
}

int w8a8_quantize_rowwise_modulated(const void* x, int x_dtype, const void* modulation_scale, int8_t* q,
                                    float* xs, int64_t M, int64_t K, uint32_t flags, hipStream_t stream) {
    if (int rc = check_common(M, 0, K, flags)) return rc;
    if (flags & ~W8A8_SCALE_RECIP) return fail(W8A8_ERR_VALUE, "only W8A8_SCALE_RECIP applies to the modulated quantizer");
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for INT8 quantization");
    if (M == 0) return W8A8_OK;
    if (K > 0 && (!x || !q || !modulation_scale)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (!xs) return fail(W8A8_ERR_VALUE, "null scale pointer");
    w8a8::launch_quant_modulated(x, x_dtype, modulation_scale, q, xs, M, K, (flags & W8A8_SCALE_RECIP) ? 1 : 0,
                                 stream);
    return check_launch("quantize_int8_rowwise_modulated");
}

int w8a8_adaln(const void* x, const void* scale, const void* shift, void* out, int64_t n, int64_t d,
               int64_t scale_group, int64_t shift_group, double eps, int dtype, int rms, hipStream_t stream) {
    if (n < 0 || d < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (d == 0) return fail(W8A8_ERR_VALUE, "integer division or modulo by zero");
    if (!valid_dtype(dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported dtype for adaln");
    if (scale_group <= 0 || shift_group <= 0) return fail(W8A8_ERR_VALUE, "modulation group must be positive");
    if (n == 0) return W8A8_OK;
    if (!x || !scale || !shift || !out) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (n > 0x7fffffff) return fail(W8A8_ERR_VALUE, "adaln supports at most 2^31 - 1 rows");
    if (rms & ~(W8A8_ADALN_RMS | W8A8_ADALN_SINGLE_ROUNDING)) return fail(W8A8_ERR_VALUE, "unknown adaln mode bits");
    w8a8::launch_adaln(x, scale, shift, out, n, d, scale_group, shift_group, static_cast<float>(eps), dtype,
                       (rms & W8A8_ADALN_RMS) != 0, (rms & W8A8_ADALN_SINGLE_ROUNDING) != 0, stream);
    return check_launch((rms & W8A8_ADALN_RMS) ? "rms_adaln" : "adaln");
}

int w8a8_modulated_norm_quant(const void* x, const void* scale0, const void* scale1, const void* shift0,
                              const void* shift1, int8_t* q, float* xs, int64_t batch, int64_t tokens, int64_t d,
                              int64_t prefix, double eps, int dtype, int rms, uint32_t flags, hipStream_t stream) {
    if (batch < 0 || tokens < 0 || d < 0 || prefix < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (d == 0) return fail(W8A8_ERR_VALUE, "integer division or modulo by zero");
    if (flags & ~W8A8_SCALE_RECIP) return fail(W8A8_ERR_VALUE, "only W8A8_SCALE_RECIP applies to the fused norm quantizer");
    if (!valid_dtype(dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported dtype for adaln");
    if (batch == 0 || tokens == 0) return W8A8_OK;
    if (!x || !scale1 || !shift1 || !q || !xs || (prefix > 0 && (!scale0 || !shift0)))
        return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (batch * tokens > 0x7fffffff) return fail(W8A8_ERR_VALUE, "modulated_norm_quant supports at most 2^31 - 1 rows");
    const void* s0 = prefix > 0 ? scale0 : scale1;
    const void* h0 = prefix > 0 ? shift0 : shift1;
    if (!w8a8::launch_modnorm_quant(x, s0, scale1, h0, shift1, q, xs, batch * tokens, tokens, d, prefix,
                                    static_cast<float>(eps), dtype, rms != 0, (flags & W8A8_SCALE_RECIP) ? 1 : 0,
                                    stream))
        return fail(W8A8_ERR_VALUE, "modulated_norm_quant needs 16-byte aligned rows of at most 2048 16-byte chunks");
    return check_launch("modulated_norm_quant");
}

int w8a8_rms_rope(const void* q, const void* k, const float* freqs, const void* q_scale, const void* k_scale,
                  void* q_out, void* k_out, int64_t batch, int64_t seq, int64_t heads, int64_t d,
                  int64_t x_row_stride, int freq_per_batch, double eps, int dtype, hipStream_t stream) {
    return rope_entry("rms_rope", q, k, freqs, q_scale, k_scale, q_out, k_out, batch, seq, heads, d, x_row_stride,
                      freq_per_batch, eps, true, dtype, stream);
}

int w8a8_apply_rope(const void* x, const void* k, const float* freqs, void* out, void* k_out, int64_t batch,
                    int64_t seq, int64_t heads, int64_t d, int64_t x_row_stride, int freq_per_batch, int dtype,
                    hipStream_t stream) {
    return rope_entry("apply_rope", x, k, freqs, nullptr, nullptr, out, k_out, batch, seq, heads, d, x_row_stride,
                      freq_per_batch, 0.0, false, dtype, stream);
}

int w8a8_gated_residual(const void* x, const void* y, const void* gate0, const void* gate1, void* out,
                        int64_t batch, int64_t tokens, int64_t d, int64_t prefix, int dtype, hipStream_t stream) {
    if (batch < 0 || tokens < 0 || d < 0 || prefix < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (!valid_dtype(dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported dtype for gated_residual");
    if (batch == 0 || tokens == 0 || d == 0) return W8A8_OK;
    if (!x || !y || !gate1 || !out || (prefix > 0 && !gate0)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (batch * tokens > 0x7fffffff) return fail(W8A8_ERR_VALUE, "gated_residual supports at most 2^31 - 1 rows");
    w8a8::launch_gated_residual(x, y, prefix > 0 ? gate0 : gate1, gate1, out, batch, tokens, d, prefix, dtype,
                                stream);
    return check_launch("gated_residual");
}

int w8a8_input_act(const void* x, int x_dtype, int act, const void* act_weight, double act_eps, void* y, int64_t M,
                   int64_t K, hipStream_t stream) {
    if (M < 0 || K < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (int rc = check_act(act, act_weight)) return rc;
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for the input activation");
    if (M == 0 || K == 0) return W8A8_OK;
    if (!x || !y) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (act == W8A8_ACT_NONE) {
        const int64_t bytes = M * K * (x_dtype == W8A8_F32 ? 4 : 2);
        if (hipMemcpyAsync(y, x, bytes, hipMemcpyDeviceToDevice, stream) != hipSuccess) return check_launch("input_act");
        return W8A8_OK;
    }
    w8a8::launch_act_rows(x, x_dtype, act, act_weight, static_cast<float>(act_eps), nullptr, nullptr, y, M, K, false,
                          stream);
    return check_launch("input_act");
}

int w8a8_quantize_rowwise_act(const void* x, int x_dtype, int act, const void* act_weight, double act_eps, int8_t* q,
                              float* xs, int64_t M, int64_t K, int64_t convrot_group, uint32_t flags, void* aux,
                              int64_t aux_bytes, hipStream_t stream) {
    if (int rc = check_common(M, 0, K, flags)) return rc;
    if (flags & ~W8A8_SCALE_RECIP) return fail(W8A8_ERR_VALUE, "w8a8_quantize_rowwise_act takes only W8A8_SCALE_RECIP");
    if (int rc = check_act(act, act_weight)) return rc;
    if (convrot_group) {
        if (int rc = check_convrot_group(K, convrot_group)) return rc;
    }
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for INT8 quantization");
    if (M == 0) return W8A8_OK;
    if (K > 0 && (!x || !q)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (!xs) return fail(W8A8_ERR_VALUE, "null scale pointer");
    const bool recip = flags & W8A8_SCALE_RECIP;
    const float eps = static_cast<float>(act_eps);
    if (act == W8A8_ACT_NONE) {
        if (!convrot_group) return w8a8_quantize_rowwise(x, x_dtype, q, xs, M, K, flags, stream);
        return w8a8_quantize_rowwise_convrot(x, x_dtype, q, xs, M, K, convrot_group, flags, aux, aux_bytes, stream);
    }
    if (K == 0) return w8a8_quantize_rowwise(x, x_dtype, q, xs, M, K, flags, stream);
    if (!convrot_group) {
        // the activation fused into the quantizer, with the crate's eager numerics
        if (act == W8A8_ACT_GELU) return w8a8_quantize_rowwise(x, x_dtype, q, xs, M, K, flags | W8A8_ACT_GELU_TANH, stream);
        w8a8::launch_act_rows(x, x_dtype, act, act_weight, eps, q, xs, nullptr, M, K, recip, stream);
        return check_launch("quantize_int8_rowwise_act");
    }
    if (w8a8::convrot_fused_route(K, convrot_group)) {
        // Kitchen's fused ConvRot quantizer with the activation in fp32
        w8a8::launch_convrot_quant_act(x, x_dtype, act, act_weight, eps, q, xs, M, K, recip, stream);
        return check_launch("quantize_int8_rowwise_convrot64");
    }
    // other groups: the eager activation into aux, rotated there in place, then quantized
    if (!aux || aux_bytes < w8a8_convrot_workspace_bytes(M, K, convrot_group, x_dtype))
        return fail(W8A8_ERR_VALUE, "aux buffer smaller than w8a8_convrot_workspace_bytes(M, K, group, dtype)");
    w8a8::launch_act_rows(x, x_dtype, act, act_weight, eps, nullptr, nullptr, aux, M, K, false, stream);
    if (int rc = check_launch("input_act")) return rc;
    w8a8::launch_convrot_rotate(aux, x_dtype, aux, M, K, convrot_group, stream);
    if (int rc = check_launch("convrot_rotate")) return rc;
    return w8a8_quantize_rowwise(aux, x_dtype, q, xs, M, K, flags, stream);
}

int w8a8_row_scales(const void* x, int x_dtype, float* xs, int64_t M, int64_t K, uint32_t flags,
                    hipStream_t stream) {
    if (int rc = check_common(M, 0, K, flags)) return rc;
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for INT8 quantization");
    if (M == 0) return W8A8_OK;
    if ((K > 0 && !x) || !xs) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    w8a8::launch_quantize(x, x_dtype, nullptr, xs, M, K, flags & W8A8_SCALE_RECIP,
                          flags & W8A8_ACT_GELU_TANH, true, stream);
    return check_launch("row_scales");
}

int w8a8_gemv_dequant(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                      int64_t ws_size, const void* bias, void* out, int out_dtype, int64_t M,
                      int64_t N, int64_t K, uint32_t flags, hipStream_t stream) {
    if (int rc = check_common(M, N, K, flags)) return rc;
    if (M != 1 && M != 2) return fail(W8A8_ERR_RUNTIME, "INT8 GEMV dequant expects M == 1 or M == 2");
    if (!valid_dtype(out_dtype)) return fail(W8A8_ERR_RUNTIME, "Invalid INT8 GEMV output dtype code");
    if (int rc = check_ws(ws_size, N, "INT8 GEMV weight scale must be scalar or per-output-channel")) return rc;
    if (N == 0) return W8A8_OK;
    if (!out || !xs || !ws || (K > 0 && (!q || !w))) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    w8a8::launch_gemv(q, w, xs, ws, ws_size, bias, nullptr, out, out_dtype, M, N, K,
                      flags & W8A8_ACT_GELU_TANH, stream);
    return check_launch("int8_gemv_dequant");
}

int w8a8_gemv_dequant_residual(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                               int64_t ws_size, const void* bias, const void* rscale,
                               int64_t rscale_size, const void* resid, void* out, int out_dtype,
                               int64_t M, int64_t N, int64_t K, uint32_t flags, hipStream_t stream) {
    if (int rc = check_common(M, N, K, flags)) return rc;
    if (flags & (W8A8_ACT_GELU_TANH | W8A8_OUT_INT32))
        return fail(W8A8_ERR_VALUE, "the residual epilogue takes no output activation");
    if (M != 1 && M != 2) return fail(W8A8_ERR_RUNTIME, "INT8 GEMV dequant expects M == 1 or M == 2");
    if (!valid_dtype(out_dtype)) return fail(W8A8_ERR_RUNTIME, "Invalid INT8 GEMV output dtype code");
    if (int rc = check_ws(ws_size, N, "INT8 GEMV weight scale must be scalar or per-output-channel")) return rc;
    if (int rc = check_residual(rscale, rscale_size, resid, N)) return rc;
    if (N == 0) return W8A8_OK;
    if (!out || !xs || !ws || (K > 0 && (!q || !w))) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    const w8a8::Residual res{rscale, rscale_size, resid};
    w8a8::launch_gemv(q, w, xs, ws, ws_size, bias, &res, out, out_dtype, M, N, K, false, stream);
    return check_launch("int8_gemv_dequant");
}

int w8a8_gemm_dequant(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                      int64_t ws_size, const void* bias, void* out, int out_dtype, int64_t M,
                      int64_t N, int64_t K, uint32_t flags, hipStream_t stream) {
    if (int rc = check_common(M, N, K, flags)) return rc;
    const bool i32 = flags & W8A8_OUT_INT32;
    if (!i32 && !valid_dtype(out_dtype)) return fail(W8A8_ERR_RUNTIME, "Invalid INT8 linear output dtype code");
    if (!i32) {
        if (int rc = check_ws(ws_size, N, "INT8 weight scale must be scalar or per-output-channel")) return rc;
    }
    if (int rc = check_tile(flags)) return rc;
    if (M == 0 || N == 0) return W8A8_OK;
    if (!out || (K > 0 && (!q || !w)) || (!i32 && (!xs || !ws))) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    w8a8::launch_gemm(q, w, xs, ws, ws_size, bias, nullptr, out, i32 ? W8A8_F32 : out_dtype, M, N, K,
                      flags & W8A8_ACT_GELU_TANH, i32, tile_of(flags), stream);
    return check_launch("int8_gemm_dequant");
}

int w8a8_gemm_config(int64_t M, int64_t N, int64_t K, uint32_t flags) {
    if (M < 0 || N < 0 || K < 0 || (flags & ~kKnownFlags) || tile_of(flags) > W8A8_GEMM_TILE_GENERIC) return -1;
    return w8a8::gemm_config(M, N, K, tile_of(flags), (flags & W8A8_ACT_GELU_TANH) != 0);
}

int w8a8_gemm_dequant_residual(const int8_t* q, const int8_t* w, const float* xs, const float* ws,
                               int64_t ws_size, const void* bias, const void* rscale,
                               int64_t rscale_size, const void* resid, void* out, int out_dtype,
                               int64_t M, int64_t N, int64_t K, uint32_t flags, hipStream_t stream) {
    if (int rc = check_common(M, N, K, flags)) return rc;
    if (flags & (W8A8_ACT_GELU_TANH | W8A8_OUT_INT32))
        return fail(W8A8_ERR_VALUE, "the residual epilogue takes no output activation");
    if (!valid_dtype(out_dtype)) return fail(W8A8_ERR_RUNTIME, "Invalid INT8 linear output dtype code");
    if (int rc = check_ws(ws_size, N, "INT8 weight scale must be scalar or per-output-channel")) return rc;
    if (int rc = check_residual(rscale, rscale_size, resid, N)) return rc;
    if (int rc = check_tile(flags)) return rc;
    if (M == 0 || N == 0) return W8A8_OK;
    if (!out || !xs || !ws || (K > 0 && (!q || !w))) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    const w8a8::Residual res{rscale, rscale_size, resid};
    w8a8::launch_gemm(q, w, xs, ws, ws_size, bias, &res, out, out_dtype, M, N, K, false, false, tile_of(flags),
                      stream);
    return check_launch("cutlass_int8_dequant_residual");
}

int w8a8_residual_apply(void* out, const void* resid, const void* rscale, int64_t rscale_size, int dtype,
                        int64_t M, int64_t N, hipStream_t stream) {
    if (M < 0 || N < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (!valid_dtype(dtype)) return fail(W8A8_ERR_RUNTIME, "Invalid output dtype code");
    if (int rc = check_residual(rscale, rscale_size, resid, N)) return rc;
    if (M == 0 || N == 0) return W8A8_OK;
    if (!out) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    w8a8::launch_residual(out, resid, rscale, rscale_size, dtype, M, N, stream);
    return check_launch("apply_residual");
}

int w8a8_gemm_dequant_xq(const void* x, int x_dtype, const float* xs, const int8_t* w,
                         const float* ws, int64_t ws_size, const void* bias, void* out,
                         int out_dtype, int64_t M, int64_t N, int64_t K, uint32_t flags,
                         hipStream_t stream) {
    if (int rc = check_common(M, N, K, flags)) return rc;
    if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype)) return fail(W8A8_ERR_RUNTIME, "Invalid dtype code");
    if (flags & W8A8_OUT_INT32)
        return fail(W8A8_ERR_VALUE, "W8A8_OUT_INT32 is not available with the fused quantizer");
    if (int rc = check_ws(ws_size, N, "INT8 weight scale must be scalar or per-output-channel")) return rc;
    if (M == 0 || N == 0) return W8A8_OK;
    if (!out || !xs || !ws || (K > 0 && (!x || !w))) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (!w8a8::launch_gemm_xq(x, x_dtype, xs, w, ws, ws_size, bias, out, out_dtype, M, N, K,
                              flags & W8A8_ACT_GELU_TANH, stream))
        return fail(W8A8_ERR_RUNTIME,
                    "fused-quant GEMM needs a 16-bit input, K % 16 == 0 and 16-byte aligned operands");
    return check_launch("int8_gemm_dequant_xq");
}

int w8a8_dequantize_linear(const int32_t* acc, const float* xs, const float* ws, int64_t ws_size,
                           const void* bias, void* out, int out_dtype, int64_t M, int64_t N,
                           uint32_t flags, hipStream_t stream) {
    if (int rc = check_common(M, N, 0, flags)) return rc;
    if (!valid_dtype(out_dtype)) return fail(W8A8_ERR_RUNTIME, "Invalid INT8 linear output dtype code");
    if (int rc = check_ws(ws_size, N, "INT8 weight scale must be scalar or per-output-channel")) return rc;
    if (M == 0 || N == 0) return W8A8_OK;
    if (!acc || !xs || !ws || !out) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    w8a8::launch_dequant(acc, xs, ws, ws_size, bias, out, out_dtype, M, N,
                         flags & W8A8_ACT_GELU_TANH, stream);
    return check_launch("dequantize_int8_linear");
}

int64_t w8a8_int8_linear_workspace_bytes(int64_t M, int64_t K) {
    if (M < 0 || K < 0) return -1;
    // q [M, K] int8, padded to 256 bytes, then xs [M] fp32
    return (M * K + 255) / 256 * 256 + M * 4;
}

int64_t w8a8_convrot_workspace_bytes(int64_t M, int64_t K, int64_t group, int x_dtype) {
    if (M < 0 || K < 0 || !valid_dtype(x_dtype)) return -1;
    if (w8a8::convrot_fused_route(K, group)) return 0;
    return M * K * (x_dtype == W8A8_F32 ? 4 : 2);
}

int w8a8_convrot_rotate(const void* x, int x_dtype, void* y, int64_t M, int64_t K, int64_t group,
                        hipStream_t stream) {
    if (M < 0 || K < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (int rc = check_convrot_group(K, group)) return rc;
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for ConvRot rotation");
    if (M == 0 || K == 0) return W8A8_OK;
    if (!x || !y) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    w8a8::launch_convrot_rotate(x, x_dtype, y, M, K, group, stream);
    return check_launch("convrot_rotate");
}

int w8a8_quantize_rowwise_convrot(const void* x, int x_dtype, int8_t* q, float* xs, int64_t M, int64_t K,
                                  int64_t group, uint32_t flags, void* rotated, int64_t rotated_bytes,
                                  hipStream_t stream) {
    if (int rc = check_common(M, 0, K, flags)) return rc;
    if (flags & ~W8A8_SCALE_RECIP)
        return fail(W8A8_ERR_VALUE, "the ConvRot quantizer takes only W8A8_SCALE_RECIP");
    if (int rc = check_convrot_group(K, group)) return rc;
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for INT8 quantization");
    if (M == 0) return W8A8_OK;
    if (K > 0 && (!x || !q)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (!xs) return fail(W8A8_ERR_VALUE, "null scale pointer");
    const bool recip = flags & W8A8_SCALE_RECIP;
    if (K == 0) return w8a8_quantize_rowwise(x, x_dtype, q, xs, M, K, flags, stream);
    if (w8a8::convrot_fused_route(K, group)) {
        w8a8::launch_convrot_quant(x, x_dtype, q, xs, M, K, recip, stream);
        return check_launch("quantize_int8_rowwise_convrot");
    }
    if (!rotated || rotated_bytes < w8a8_convrot_workspace_bytes(M, K, group, x_dtype))
        return fail(W8A8_ERR_VALUE, "rotated buffer smaller than w8a8_convrot_workspace_bytes(M, K, group, dtype)");
    if (int rc = w8a8_convrot_rotate(x, x_dtype, rotated, M, K, group, stream)) return rc;
    return w8a8_quantize_rowwise(rotated, x_dtype, q, xs, M, K, flags, stream);
}

int w8a8_quantize_tensorwise(const void* x, int x_dtype, int8_t* q, float* scale, int64_t n, uint32_t flags,
                             hipStream_t stream) {
    if (n < 0) return fail(W8A8_ERR_VALUE, "negative dimension");
    if (flags & ~(W8A8_SCALE_RECIP | W8A8_GIVEN_SCALE))
        return fail(W8A8_ERR_VALUE, "the tensorwise quantizer takes W8A8_SCALE_RECIP and W8A8_GIVEN_SCALE");
    if (!valid_dtype(x_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for INT8 quantization");
    if (!scale) return fail(W8A8_ERR_VALUE, "null scale pointer");
    if (n > 0 && (!x || !q)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    w8a8::launch_quantize_tensorwise(x, x_dtype, q, scale, n, flags & W8A8_GIVEN_SCALE, flags & W8A8_SCALE_RECIP,
                                     stream);
    return check_launch("quantize_int8_tensorwise");
}

int64_t w8a8_convrot_weight_workspace_bytes(int64_t N, int64_t K, int64_t group, int w_dtype) {
    if (N < 0 || K < 0 || !valid_dtype(w_dtype)) return -1;
    if (group == 256 && K % 256 == 0 && K <= 65536) return 0;
    return N * K * (w_dtype == W8A8_F32 ? 4 : 2);
}

int w8a8_quantize_convrot_weight(const void* w, int w_dtype, int8_t* q, float* scale, int64_t N, int64_t K,
                                 int64_t group, uint32_t flags, void* rotated, int64_t rotated_bytes,
                                 hipStream_t stream) {
    if (int rc = check_common(N, 0, K, flags)) return rc;
    if (flags & ~W8A8_SCALE_RECIP)
        return fail(W8A8_ERR_VALUE, "the ConvRot quantizer takes only W8A8_SCALE_RECIP");
    if (int rc = check_convrot_group(K, group)) return rc;
    if (!valid_dtype(w_dtype)) return fail(W8A8_ERR_RUNTIME, "Unsupported input dtype for INT8 quantization");
    if (N == 0) return W8A8_OK;
    if (K > 0 && (!w || !q)) return fail(W8A8_ERR_VALUE, "null tensor pointer");
    if (!scale) return fail(W8A8_ERR_VALUE, "null scale pointer");
    const bool recip = flags & W8A8_SCALE_RECIP;
    if (K == 0) return w8a8_quantize_rowwise(w, w_dtype, q, scale, N, K, flags, stream);
    if (w8a8_convrot_weight_workspace_bytes(N, K, group, w_dtype) == 0) {
        if (!w8a8::convrot_weight_fused(w, q, K, group))
            return fail(W8A8_ERR_RUNTIME, "ConvRot weight and code rows above K = 16384 must be 16-byte aligned");
        w8a8::launch_convrot_quant(w, w_dtype, q, scale, N, K, recip, stream);
        return check_launch("quantize_int8_convrot_weight");
    }
    if (!rotated || rotated_bytes < w8a8_convrot_weight_workspace_bytes(N, K, group, w_dtype))
        return fail(W8A8_ERR_VALUE,
                    "rotated buffer smaller than w8a8_convrot_weight_workspace_bytes(N, K, group, dtype)");
    if (int rc = w8a8_convrot_rotate(w, w_dtype, rotated, N, K, group, stream)) return rc;
    return w8a8_quantize_rowwise(rotated, w_dtype, q, scale, N, K, flags, stream);
}

int64_t w8a8_int8_linear_convrot_workspace_bytes(int64_t M, int64_t K, int64_t group, int x_dtype) {
    const int64_t rot = w8a8_convrot_workspace_bytes(M, K, group, x_dtype);
    if (rot < 0) return -1;
    // q [M, K] int8 and xs [M] fp32, each padded to 256 bytes, then the rotated input
    return (M * K + 255) / 256 * 256 + (M * 4 + 255) / 256 * 256 + rot;
}

}  // extern "C"

namespace {

// The operator's route policy, shared by the entries with and without a
// residual (res == nullptr: none).  The residual is fused into the GEMM or
// GEMV epilogue; the reference fuses it on its CUTLASS and M = 1 routes and
// applies it eagerly elsewhere, with the same single fma either way.
int int8_linear_impl(const void* x, int x_dtype, const int8_t* w, const float* ws, int64_t ws_size,
                     const void* bias, const w8a8::Residual* res, void* out, int out_dtype, int64_t M,
                     int64_t N, int64_t K, int64_t convrot_group, uint32_t flags, void* workspace,
                     int64_t workspace_bytes, hipStream_t stream, const void* modulation = nullptr,
                     int act = W8A8_ACT_NONE, const void* act_weight = nullptr, double act_eps = 0.0) {
    if (int rc = check_common(M, N, K, flags)) return rc;
    if (flags & W8A8_OUT_INT32) return fail(W8A8_ERR_VALUE, "W8A8_OUT_INT32 is a GEMM-only flag");
    if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype))
        return fail(W8A8_ERR_RUNTIME, "GEMV output requires original floating dtype contract");
    const bool gemv = !(flags & W8A8_ROUTE_GEMM) && ((M == 1 && K % 4 == 0) || (M == 2 && K % 16 == 0));
    if (int rc = check_ws(ws_size, N, gemv ? "INT8 GEMV weight scale must be scalar or per-output-channel"
                                           : "INT8 weight scale must be scalar or per-output-channel"))
        return rc;
    if (res) {
        if (int rc = check_residual(res->rscale, res->rs_size, res->resid, N)) return rc;
    }
    if (!gemv && K % 4 != 0 && M > 0 && N > 0)
        return fail(W8A8_ERR_RUNTIME,
                    "INT8 GEMM not supported on this GPU for these dimensions (requires SM >= 7.5, "
                    "and dimensions multiple of 4).");
    if (int rc = check_act(act, act_weight)) return rc;
    if (act != W8A8_ACT_NONE && (flags & W8A8_ACT_GELU_TANH))
        return fail(W8A8_ERR_VALUE, "W8A8_ACT_GELU_TANH and an input activation code together");
    if (convrot_group) {
        if (int rc = check_convrot_group(K, convrot_group)) return rc;
        if (flags & W8A8_ACT_GELU_TANH) act = W8A8_ACT_GELU;   // the flag's GELU, on the ConvRot route
    }
    if (M == 0) return W8A8_OK;
    const int64_t need = convrot_group ? w8a8_int8_linear_convrot_workspace_bytes(M, K, convrot_group, x_dtype)
                                       : w8a8_int8_linear_workspace_bytes(M, K);
    if (!workspace || workspace_bytes < need)
        return fail(W8A8_ERR_VALUE, convrot_group
                                        ? "workspace smaller than w8a8_int8_linear_convrot_workspace_bytes"
                                        : "workspace smaller than w8a8_int8_linear_workspace_bytes(M, K)");
    if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
        return fail(W8A8_ERR_VALUE, "workspace must be 256-byte aligned");
    int8_t* q = static_cast<int8_t*>(workspace);
    float* xs = reinterpret_cast<float*>(static_cast<char*>(workspace) + (M * K + 255) / 256 * 256);
    const uint32_t qflags = flags & (W8A8_SCALE_RECIP | W8A8_ACT_GELU_TANH);
    // The input activation is applied before quantization; the GEMM/GEMV
    // epilogue itself runs without GELU here.
    // Fused route: row scales, then a GEMM that quantizes its activation tiles
    // (an input activation is only applied by the standalone quantizer); a
    // residual is then applied by the standalone residual kernel.
    if (modulation) {
        if (int rc = w8a8_quantize_rowwise_modulated(x, x_dtype, modulation, q, xs, M, K, qflags, stream))
            return rc;
    } else if (!convrot_group && act == W8A8_ACT_NONE && !gemv && (flags & W8A8_FUSED_QUANT) &&
               !(qflags & W8A8_ACT_GELU_TANH) &&
               N > 0 && x_dtype != W8A8_F32 && K % 16 == 0) {
        if (int rc = w8a8_row_scales(x, x_dtype, xs, M, K, qflags, stream)) return rc;
        if (w8a8::launch_gemm_xq(x, x_dtype, xs, w, ws, ws_size, bias, out, out_dtype, M, N, K,
                                 false, stream)) {
            if (int rc = check_launch("int8_gemm_dequant_xq")) return rc;
            if (!res) return W8A8_OK;
            return w8a8_residual_apply(out, res->resid, res->rscale, res->rs_size, out_dtype, M, N, stream);
        }
    }
    if (modulation) {
        // quantized above
    } else if (act != W8A8_ACT_NONE) {
        void* aux = convrot_group ? static_cast<char*>(workspace) + (M * K + 255) / 256 * 256 + (M * 4 + 255) / 256 * 256
                                  : nullptr;
        const int64_t aux_bytes = convrot_group ? w8a8_convrot_workspace_bytes(M, K, convrot_group, x_dtype) : 0;
        if (int rc = w8a8_quantize_rowwise_act(x, x_dtype, act, act_weight, act_eps, q, xs, M, K, convrot_group,
                                               qflags & W8A8_SCALE_RECIP, aux, aux_bytes, stream))
            return rc;
    } else if (convrot_group) {
        void* rotated = static_cast<char*>(workspace) + (M * K + 255) / 256 * 256 + (M * 4 + 255) / 256 * 256;
        if (int rc = w8a8_quantize_rowwise_convrot(x, x_dtype, q, xs, M, K, convrot_group, qflags, rotated,
                                                   w8a8_convrot_workspace_bytes(M, K, convrot_group, x_dtype),
                                                   stream))
            return rc;
    } else if (int rc = w8a8_quantize_rowwise(x, x_dtype, q, xs, M, K, qflags, stream)) {
        return rc;
    }
    if (N == 0) return W8A8_OK;
    if (res) {
        if (gemv)
            return w8a8_gemv_dequant_residual(q, w, xs, ws, ws_size, bias, res->rscale, res->rs_size,
                                              res->resid, out, out_dtype, M, N, K, 0, stream);
        return w8a8_gemm_dequant_residual(q, w, xs, ws, ws_size, bias, res->rscale, res->rs_size,
                                          res->resid, out, out_dtype, M, N, K, 0, stream);
    }
    if (gemv) return w8a8_gemv_dequant(q, w, xs, ws, ws_size, bias, out, out_dtype, M, N, K, 0, stream);
    return w8a8_gemm_dequant(q, w, xs, ws, ws_size, bias, out, out_dtype, M, N, K, 0, stream);
}

}  // namespace

extern "C" {

int w8a8_int8_linear(const void* x, int x_dtype, const int8_t* w, const float* ws, int64_t ws_size,
                     const void* bias, void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                     uint32_t flags, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
    return int8_linear_impl(x, x_dtype, w, ws, ws_size, bias, nullptr, out, out_dtype, M, N, K, 0, flags,
                            workspace, workspace_bytes, stream);
}

int w8a8_int8_linear_residual(const void* x, int x_dtype, const int8_t* w, const float* ws,
                              int64_t ws_size, const void* bias, const void* rscale,
                              int64_t rscale_size, const void* resid, void* out, int out_dtype,
                              int64_t M, int64_t N, int64_t K, uint32_t flags, void* workspace,
                              int64_t workspace_bytes, hipStream_t stream) {
    const w8a8::Residual res{rscale, rscale_size, resid};
    return int8_linear_impl(x, x_dtype, w, ws, ws_size, bias, &res, out, out_dtype, M, N, K, 0, flags,
                            workspace, workspace_bytes, stream);
}

int w8a8_int8_linear_modulated(const void* x, int x_dtype, const void* modulation_scale, const int8_t* w,
                               const float* ws, int64_t ws_size, const void* bias, void* out, int out_dtype,
                               int64_t M, int64_t N, int64_t K, uint32_t flags, void* workspace,
                               int64_t workspace_bytes, hipStream_t stream) {
    if (flags & (W8A8_ACT_GELU_TANH | W8A8_FUSED_QUANT))
        return fail(W8A8_ERR_VALUE, "int8_linear_modulated takes no input activation or fused quantization");
    if (M > 0 && K > 0 && !modulation_scale) return fail(W8A8_ERR_VALUE, "null modulation_scale");
    return int8_linear_impl(x, x_dtype, w, ws, ws_size, bias, nullptr, out, out_dtype, M, N, K, 0, flags,
                            workspace, workspace_bytes, stream, modulation_scale ? modulation_scale : x);
}

int w8a8_int8_linear_act(const void* x, int x_dtype, int act, const void* act_weight, double act_eps, const int8_t* w,
                         const float* ws, int64_t ws_size, const void* bias, const void* rscale, int64_t rscale_size,
                         const void* resid, void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                         int64_t convrot_group, uint32_t flags, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream) {
    const w8a8::Residual res{rscale, rscale_size, resid};
    return int8_linear_impl(x, x_dtype, w, ws, ws_size, bias, resid ? &res : nullptr, out, out_dtype, M, N, K,
                            convrot_group, flags, workspace, workspace_bytes, stream, nullptr, act, act_weight, act_eps);
}

int w8a8_int8_linear_convrot(const void* x, int x_dtype, const int8_t* w, const float* ws, int64_t ws_size,
                             const void* bias, const void* rscale, int64_t rscale_size, const void* resid,
                             void* out, int out_dtype, int64_t M, int64_t N, int64_t K, int64_t group,
                             uint32_t flags, void* workspace, int64_t workspace_bytes, hipStream_t stream) {
    const w8a8::Residual res{rscale, rscale_size, resid};
    return int8_linear_impl(x, x_dtype, w, ws, ws_size, bias, resid ? &res : nullptr, out, out_dtype, M, N, K,
                            group, flags, workspace, workspace_bytes, stream);
}

}  // extern "C"
