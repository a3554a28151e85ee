// libimagine_kitchen.so -- the W8A8 names of the reference bridge's
// imagine_kitchen_call, over the C ABI of libw8a8_hip.so.
//
// The crate reaches Kitchen's kernels through one dispatcher,
//   int imagine_kitchen_call(const char* name, const KitchenArg* args, size_t n, int64_t* result)
// (inference/native/bridge.hpp:5-6,29, bridge.cpp:415-440; Rust side
// inference/src/native.rs:455-497,1586-1607), with borrowed at::Tensor* handles
// and the caller's stream as an integer.  This file answers the names the
// crate's int8_linear operator issues (cuda_linear.rs:558-582,605-616,657-676,
// 724-762,770-794) with the argument lists, arity rule, operand checks, error
// texts and return values of the pinned Kitchen wrappers
// (dlpack_bindings.cpp:2269-2305,2307-2340,2717-2763,2814-2834,3485-3533,
// 3535-3592,3594-3660) and the bridge's error-code mapping:
//   0 ok; -1 runtime error (message in imagine_last_error()); -20 ValueError;
//   -21 IndexError.  Unknown names fail like the bridge: "Unknown Kitchen kernel".
// The arithmetic is the HIP library's; nothing here allocates, frees or
// synchronizes, and every launch goes to the stream argument.
//
// Scale form: these names stand in for Kitchen's CUDA kernels, so the row
// scale is their amax * (1/127) (W8A8_SCALE_RECIP, int8_linear.cu:205-208).
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

#include "imagine_kitchen.h"
#include "w8a8.h"

namespace {

thread_local std::string last_error;
thread_local int last_accelerator_code = 0;
thread_local std::string last_metadata;

// Failures of the C ABI keep its class: ValueError / IndexError codes pass
// through as the bridge's -20 / -21, everything else is a runtime error (the
// Kitchen launchers throw std::runtime_error on launch failures).
struct AbiError : std::runtime_error {
    int code;
    AbiError(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

void abi(int rc) {
    if (rc == W8A8_OK) return;
    if (rc == W8A8_ERR_ACCELERATOR) last_accelerator_code = w8a8_last_accelerator_code();
    throw AbiError(rc, w8a8_last_error());
}

// The current device follows the first tensor argument for the call
// (bridge.cpp:421-428), restored afterwards.
struct DeviceGuard {
    int saved = -1;
    explicit DeviceGuard(int device) {
        if (device < 0) return;
        if (hipGetDevice(&saved) != hipSuccess) saved = -1;
        if (saved != device && hipSetDevice(device) != hipSuccess) throw std::runtime_error("hipSetDevice failed");
    }
    ~DeviceGuard() {
        if (saved >= 0) (void)hipSetDevice(saved);
    }
};

// Typed access to the argument array, with the bridge's conversion messages
// (bridge.cpp:84-112) and the nanobind-level view checks (tensor_view.hpp).
struct Args {
    const KitchenArg* a;
    size_t n;

    const at::Tensor& tensor(size_t i) const {
        if (a[i].kind != 1 || !a[i].tensor) throw std::runtime_error("Expected tensor argument");
        const at::Tensor& t = *static_cast<const at::Tensor*>(a[i].tensor);
        if (!t.is_cuda()) throw std::runtime_error("Expected CUDA tensor");
        return t;
    }
    const at::Tensor* optional_tensor(size_t i) const {
        if (i >= n || a[i].kind == 0) return nullptr;
        if (a[i].kind != 1) throw std::runtime_error("Expected tensor or None");
        return &tensor(i);
    }
    int64_t integer(size_t i) const {
        if (a[i].kind != 2 && a[i].kind != 4) throw std::runtime_error("Expected integer/bool argument");
        return a[i].integer;
    }
    double real(size_t i) const {
        if (a[i].kind != 3) throw std::runtime_error("Expected floating argument");
        return a[i].real;
    }
};

// Rank and element-type checks of the typed views (tensor_view.hpp:25-37).
const at::Tensor& ranked(const at::Tensor& t, int64_t rank) {
    if (t.dim() != rank) throw std::runtime_error("Tensor rank mismatch");
    return t;
}
const at::Tensor& typed(const at::Tensor& t, at::ScalarType s) {
    if (t.scalar_type() != s) throw std::runtime_error("Typed tensor view dtype mismatch");
    return t;
}

// The kernels read and write rows densely.
const at::Tensor& dense(const at::Tensor& t, const char* what) {
    if (!t.is_contiguous()) throw std::runtime_error(std::string(what) + " must be contiguous");
    return t;
}

// Kitchen's dtype code of a tensor (dlpack_bindings.cpp:33): 0 fp32, 1 fp16,
// 2 bf16, -1 otherwise.
int dtype_code(const at::Tensor& t) {
    switch (t.scalar_type()) {
        case at::kFloat: return W8A8_F32;
        case at::kHalf: return W8A8_F16;
        case at::kBFloat16: return W8A8_BF16;
        default: return -1;
    }
}

hipStream_t stream_of(int64_t s) { return reinterpret_cast<hipStream_t>(static_cast<uintptr_t>(s)); }

// A bias that is absent or empty is "no bias" (dlpack_bindings.cpp:3502,3555);
// a present one must be [N] in the output dtype here: the kernels read it in
// that dtype (the crate always converts it so, cuda_linear.rs:26-51,541-551).
const void* bias_ptr(const at::Tensor* bias, int64_t N, int out_code, const char* shape_msg,
                     const char* dtype_msg) {
    if (!bias || bias->numel() == 0) return nullptr;
    if (bias->size(0) != N) throw std::runtime_error(shape_msg);
    const int code = dtype_code(*bias);
    if (code < 0) throw std::runtime_error(dtype_msg);
    if (code != out_code) throw std::runtime_error("INT8 linear bias must be in the output dtype");
    dense(*bias, "bias");
    return bias->data_ptr();
}

// ---------------------------------------------------------------- routes

// quantize_int8_rowwise(input, output, scales, stochastic, seed, stream)
// (dlpack_bindings.cpp:2307-2340; cuda_linear.rs:605-616)
int64_t quantize_int8_rowwise(const Args& g) {
    const at::Tensor& x = dense(ranked(g.tensor(0), 2), "input");
    const at::Tensor& q = dense(typed(ranked(g.tensor(1), 2), at::kChar), "output");
    const at::Tensor& s = dense(typed(ranked(g.tensor(2), 2), at::kFloat), "scales");
    const bool stochastic = g.integer(3) != 0;
    (void)g.integer(4);
    const int64_t M = x.size(0), K = x.size(1);
    if (q.size(0) != M || q.size(1) != K) throw std::runtime_error("INT8 rowwise quantization output shape mismatch");
    if (s.size(0) != M || s.size(1) != 1) throw std::runtime_error("INT8 rowwise quantization scale shape mismatch");
    const int code = dtype_code(x);
    if (code < 0) throw std::runtime_error("Unsupported input dtype for INT8 rowwise quantization");
    if (stochastic) throw std::runtime_error("stochastic INT8 rounding is not part of this library");
    abi(w8a8_quantize_rowwise(x.data_ptr(), code, static_cast<int8_t*>(q.data_ptr()),
                              static_cast<float*>(s.data_ptr()), M, K, W8A8_SCALE_RECIP, stream_of(g.integer(5))));
    return 0;
}

// Residual operands of the fused residual epilogue: [M, N] and [N] (or one
// value) in the output dtype (cuda_linear.rs:171-191,707-722).
struct Residual {
    const void* resid = nullptr;
    const void* rscale = nullptr;
    int64_t rscale_size = 0;
};

Residual residual_of(const at::Tensor* r, const at::Tensor* s, int64_t M, int64_t N, int out_code, const char* name) {
    Residual out;
    if (!r && !s) return out;
    if (!r || !s) throw std::invalid_argument("residual requires residual_scale");
    if (r->numel() != M * N || dtype_code(*r) != out_code)
        throw std::runtime_error(std::string(name) + ": residual must be [M, N] in the output dtype");
    if ((s->numel() != N && s->numel() != 1) || dtype_code(*s) != out_code)
        throw std::runtime_error(std::string(name) + ": rscale must be a length-N vector in the output dtype");
    out.resid = dense(*r, "residual").data_ptr();
    out.rscale = dense(*s, "residual_scale").data_ptr();
    out.rscale_size = s->numel();
    return out;
}

// int8_gemv_dequant(input, weight, x_scales, weight_scales, bias, output,
// output_dtype_code, stream[, residual, residual_scale])
// (dlpack_bindings.cpp:3535-3592; cuda_linear.rs:657-676 passes the residual pair)
int64_t int8_gemv_dequant(const Args& g) {
    const at::Tensor& q = dense(typed(ranked(g.tensor(0), 2), at::kChar), "input");
    const at::Tensor& w = dense(typed(ranked(g.tensor(1), 2), at::kChar), "weight");
    const at::Tensor& xs = dense(typed(ranked(g.tensor(2), 2), at::kFloat), "x_scales");
    const at::Tensor& ws = dense(typed(g.tensor(3), at::kFloat), "weight_scales");
    const at::Tensor* bias = g.optional_tensor(4);
    const at::Tensor& out = dense(ranked(g.tensor(5), 2), "output");
    const int64_t out_code = g.integer(6);
    const int64_t M = q.size(0), K = q.size(1), N = w.size(0);
    if (M != 1 && M != 2) throw std::runtime_error("INT8 GEMV dequant expects M == 1 or M == 2");
    if (w.size(1) != K) throw std::runtime_error("INT8 GEMV weight K mismatch");
    if (xs.size(0) != M || xs.size(1) != 1) throw std::runtime_error("INT8 GEMV activation scale shape mismatch");
    if (out.size(0) != M || out.size(1) != N) throw std::runtime_error("INT8 GEMV output shape mismatch");
    if (out_code < 0 || out_code > 2) throw std::runtime_error("Invalid INT8 GEMV output dtype code");
    if (dtype_code(out) != out_code) throw std::runtime_error("INT8 GEMV output dtype does not match its code");
    const int oc = static_cast<int>(out_code);
    const void* b = bias_ptr(bias, N, oc, "INT8 GEMV bias shape mismatch", "Unsupported bias dtype for INT8 GEMV");
    const Residual r = g.n == 10 ? residual_of(g.optional_tensor(8), g.optional_tensor(9), M, N, oc, "int8_gemv_dequant")
                                 : Residual{};
    const hipStream_t st = stream_of(g.integer(7));
    auto* qp = static_cast<const int8_t*>(q.data_ptr());
    auto* wp = static_cast<const int8_t*>(w.data_ptr());
    auto* xsp = static_cast<const float*>(xs.data_ptr());
    auto* wsp = static_cast<const float*>(ws.data_ptr());
    if (r.resid)
        abi(w8a8_gemv_dequant_residual(qp, wp, xsp, wsp, ws.numel(), b, r.rscale, r.rscale_size, r.resid,
                                       out.data_ptr(), oc, M, N, K, 0, st));
    else
        abi(w8a8_gemv_dequant(qp, wp, xsp, wsp, ws.numel(), b, out.data_ptr(), oc, M, N, K, 0, st));
    return 0;
}

// Operand checks of the fused-dequant GEMM names (dlpack_bindings.cpp:2717-2745).
struct GemmOperands {
    int64_t M, N, K;
    const void* bias;
};

GemmOperands check_int8_gemm_operands(const char* name, const at::Tensor& a, const at::Tensor& b,
                                      const at::Tensor& xs, const at::Tensor& ws, const at::Tensor* bias,
                                      const at::Tensor& d, int64_t out_code) {
    const int64_t M = a.size(0), K = a.size(1), N = b.size(0);
    const std::string n(name);
    if (b.size(1) != K) throw std::runtime_error(n + ": K mismatch");
    if (d.size(0) != M || d.size(1) != N) throw std::runtime_error(n + ": D shape mismatch");
    if (xs.numel() != M) throw std::runtime_error(n + ": xs must be a length-M vector");
    if (ws.numel() != N) throw std::runtime_error(n + ": ws must be a length-N vector");
    if (bias && bias->numel() != 0 && (bias->numel() != N || dtype_code(*bias) != out_code))
        throw std::runtime_error(n + ": bias must be empty or a length-N vector in the output dtype");
    if (out_code < 0 || out_code > 2)
        throw std::runtime_error(n + ": out_dtype_code must be 0 (fp32), 1 (fp16), or 2 (bf16)");
    if (dtype_code(d) != out_code)
        throw std::runtime_error(n + ": output dtype does not match out_dtype_code (0=fp32, 1=fp16, 2=bf16)");
    return {M, N, K, bias && bias->numel() ? dense(*bias, "bias").data_ptr() : nullptr};
}

// cutlass_int8_dequant(a, b, xs, ws, bias, d, out_dtype_code, stream) -> true
// (dlpack_bindings.cpp:2747-2763; cuda_linear.rs:746-762).  Every shape is
// handled here, so the crate's cuBLAS fallback is never needed.
int64_t cutlass_int8_dequant(const Args& g) {
    const at::Tensor& a = dense(typed(ranked(g.tensor(0), 2), at::kChar), "a");
    const at::Tensor& b = dense(typed(ranked(g.tensor(1), 2), at::kChar), "b");
    const at::Tensor& xs = dense(typed(g.tensor(2), at::kFloat), "xs");
    const at::Tensor& ws = dense(typed(g.tensor(3), at::kFloat), "ws");
    const at::Tensor* bias = g.optional_tensor(4);
    const at::Tensor& d = dense(ranked(g.tensor(5), 2), "d");
    const int64_t code = g.integer(6);
    const GemmOperands o = check_int8_gemm_operands("cutlass_int8_dequant", a, b, xs, ws, bias, d, code);
    abi(w8a8_gemm_dequant(static_cast<const int8_t*>(a.data_ptr()), static_cast<const int8_t*>(b.data_ptr()),
                          static_cast<const float*>(xs.data_ptr()), static_cast<const float*>(ws.data_ptr()), o.N,
                          o.bias, d.data_ptr(), static_cast<int>(code), o.M, o.N, o.K, 0, stream_of(g.integer(7))));
    return 1;
}

// cutlass_int8_dequant_residual(a, b, xs, ws, bias, rscale, resid, d,
// out_dtype_code, stream) -> true (dlpack_bindings.cpp:2814-2834;
// cuda_linear.rs:724-742)
int64_t cutlass_int8_dequant_residual(const Args& g) {
    const at::Tensor& a = dense(typed(ranked(g.tensor(0), 2), at::kChar), "a");
    const at::Tensor& b = dense(typed(ranked(g.tensor(1), 2), at::kChar), "b");
    const at::Tensor& xs = dense(typed(g.tensor(2), at::kFloat), "xs");
    const at::Tensor& ws = dense(typed(g.tensor(3), at::kFloat), "ws");
    const at::Tensor* bias = g.optional_tensor(4);
    const at::Tensor& rscale = dense(g.tensor(5), "rscale");
    const at::Tensor& resid = dense(ranked(g.tensor(6), 2), "resid");
    const at::Tensor& d = dense(ranked(g.tensor(7), 2), "d");
    const int64_t code = g.integer(8);
    const GemmOperands o = check_int8_gemm_operands("cutlass_int8_dequant_residual", a, b, xs, ws, bias, d, code);
    if (resid.size(0) != o.M || resid.size(1) != o.N || dtype_code(resid) != code)
        throw std::runtime_error("cutlass_int8_dequant_residual: residual must be [M, N] in the output dtype");
    if (rscale.numel() != o.N || dtype_code(rscale) != code)
        throw std::runtime_error("cutlass_int8_dequant_residual: rscale must be a length-N vector in the output dtype");
    abi(w8a8_gemm_dequant_residual(static_cast<const int8_t*>(a.data_ptr()), static_cast<const int8_t*>(b.data_ptr()),
                                   static_cast<const float*>(xs.data_ptr()), static_cast<const float*>(ws.data_ptr()),
                                   o.N, o.bias, rscale.data_ptr(), o.N, resid.data_ptr(), d.data_ptr(),
                                   static_cast<int>(code), o.M, o.N, o.K, 0, stream_of(g.integer(9))));
    return 1;
}

// cublas_gemm_int8(a, b, c, workspace, stream): int32 accumulators
// (dlpack_bindings.cpp:2269-2305; cuda_linear.rs:770-779).  The workspace is
// the crate's cuBLASLt buffer; these kernels do not use it.
int64_t cublas_gemm_int8(const Args& g) {
    const at::Tensor& a = dense(typed(ranked(g.tensor(0), 2), at::kChar), "a");
    const at::Tensor& b = dense(typed(ranked(g.tensor(1), 2), at::kChar), "b");
    const at::Tensor& c = dense(typed(ranked(g.tensor(2), 2), at::kInt), "c");
    (void)g.tensor(3);
    const int64_t M = a.size(0), K = a.size(1), N = b.size(0);
    if (b.size(1) != K) throw std::runtime_error("Matrix K dimensions do not match");
    if (c.size(0) != M || c.size(1) != N) throw std::runtime_error("Output matrix C shape does not match");
    abi(w8a8_gemm_dequant(static_cast<const int8_t*>(a.data_ptr()), static_cast<const int8_t*>(b.data_ptr()), nullptr,
                          nullptr, 1, nullptr, c.data_ptr(), W8A8_F32, M, N, K, W8A8_OUT_INT32,
                          stream_of(g.integer(4))));
    return 0;
}

// dequantize_int8_linear(input, x_scales, weight_scales, bias, output,
// output_dtype_code, stream) (dlpack_bindings.cpp:3485-3533; cuda_linear.rs:783-794)
int64_t dequantize_int8_linear(const Args& g) {
    const at::Tensor& acc = dense(typed(ranked(g.tensor(0), 2), at::kInt), "input");
    const at::Tensor& xs = dense(typed(ranked(g.tensor(1), 2), at::kFloat), "x_scales");
    const at::Tensor& ws = dense(typed(g.tensor(2), at::kFloat), "weight_scales");
    const at::Tensor* bias = g.optional_tensor(3);
    const at::Tensor& out = dense(ranked(g.tensor(4), 2), "output");
    const int64_t out_code = g.integer(5);
    const int64_t M = acc.size(0), N = acc.size(1);
    if (xs.size(0) != M || xs.size(1) != 1) throw std::runtime_error("INT8 linear activation scale shape mismatch");
    if (out.size(0) != M || out.size(1) != N) throw std::runtime_error("INT8 linear output shape mismatch");
    if (out_code < 0 || out_code > 2) throw std::runtime_error("Invalid INT8 linear output dtype code");
    if (dtype_code(out) != out_code) throw std::runtime_error("INT8 linear output dtype does not match its code");
    const int oc = static_cast<int>(out_code);
    const void* b = bias_ptr(bias, N, oc, "INT8 linear bias shape mismatch", "Unsupported bias dtype for INT8 linear");
    abi(w8a8_dequantize_linear(static_cast<const int32_t*>(acc.data_ptr()), static_cast<const float*>(xs.data_ptr()),
                               static_cast<const float*>(ws.data_ptr()), ws.numel(), b, out.data_ptr(), oc, M, N, 0,
                               stream_of(g.integer(6))));
    return 0;
}

// int8_linear_m1(input, q_scratch, x_scales, weight, weight_scales, bias,
// output, output_dtype_code, convrot, group_size, act_code, act_weight,
// act_eps, stream, residual, residual_scale) -- the crate's 16-argument list
// (cuda_linear.rs:558-582; the pinned 11-argument wrapper,
// dlpack_bindings.cpp:3594-3660, without the activation and residual ones, is
// taken too): quantize into q_scratch / x_scales, then the M = 1 GEMV.  The
// crate sends activation codes on the ConvRot route only (cuda_linear.rs:
// 525-529); they are fused into the rotation in fp32.
int64_t int8_linear_m1(const Args& g) {
    const bool full = g.n == 16;
    const at::Tensor& x = dense(ranked(g.tensor(0), 2), "input");
    const at::Tensor& q = dense(typed(g.tensor(1), at::kChar), "q_scratch");
    const at::Tensor& xs = dense(typed(g.tensor(2), at::kFloat), "x_scales");
    const at::Tensor& w = dense(typed(ranked(g.tensor(3), 2), at::kChar), "weight");
    const at::Tensor& ws = dense(typed(g.tensor(4), at::kFloat), "weight_scales");
    const at::Tensor* bias = g.optional_tensor(5);
    const at::Tensor& out = dense(ranked(g.tensor(6), 2), "output");
    const int64_t out_code = g.integer(7);
    const bool convrot = g.integer(8) != 0;
    const int64_t group = g.integer(9);
    const int64_t act = full ? g.integer(10) : 0;
    const int64_t st = g.integer(full ? 13 : 10);
    // gated activations take [gate | up] rows of twice the weight's K
    const int64_t M = x.size(0), N = w.size(0);
    const int64_t K = x.size(1) / ((act == W8A8_ACT_SWIGLU || act == W8A8_ACT_SITU) ? 2 : 1);
    if (M != 1) throw std::runtime_error("INT8 M=1 linear expects input M == 1");
    if (w.size(1) != K) throw std::runtime_error("INT8 M=1 linear weight K mismatch");
    if (out.size(0) != 1 || out.size(1) != N) throw std::runtime_error("INT8 M=1 linear output shape mismatch");
    if (out_code < 0 || out_code > 2) throw std::runtime_error("Invalid INT8 M=1 linear output dtype code");
    if (convrot && (group != 256 || K % 256 != 0))
        throw std::runtime_error("INT8 M=1 ConvRot linear requires group_size 256 and K divisible by 256");
    const int code = dtype_code(x);
    if (code < 0) throw std::runtime_error("Unsupported input dtype for INT8 M=1 linear");
    if (act != 0 && !convrot) throw std::runtime_error("INT8 M=1 linear: input activations need the ConvRot route");
    const at::Tensor* aw = full ? g.optional_tensor(11) : nullptr;
    const bool has_w = aw && aw->numel() > 0;
    if (act == W8A8_ACT_RMSNORM && (!has_w || aw->numel() != K))
        throw std::runtime_error("int8 fused convrot GEMV: rms_norm activation requires a weight");
    // the crate passes empty scratch tensors on the ConvRot route (Kitchen
    // fuses that quantizer into its GEMV); here the codes and the scale go
    // through [1, K] / [1, 1] buffers taken from torch's allocator on the
    // current stream, which is the stream the crate passes
    at::Tensor q_own, xs_own;
    const bool own = convrot && (q.numel() < K || xs.numel() < 1);
    if (own) {
        q_own = at::empty({1, K}, x.options().dtype(at::kChar));
        xs_own = at::empty({1, 1}, x.options().dtype(at::kFloat));
    }
    if (!convrot && (q.dim() != 2 || q.size(0) != 1 || q.size(1) != K))
        throw std::runtime_error("INT8 M=1 linear q scratch shape mismatch");
    if (!convrot && (xs.dim() != 2 || xs.size(0) != 1 || xs.size(1) != 1))
        throw std::runtime_error("INT8 M=1 linear activation scale shape mismatch");
    if (dtype_code(out) != out_code) throw std::runtime_error("INT8 M=1 linear output dtype does not match its code");
    const int oc = static_cast<int>(out_code);
    const void* b = bias_ptr(bias, N, oc, "INT8 M=1 linear bias shape mismatch", "Unsupported bias dtype for INT8 M=1 linear");
    const Residual r = full ? residual_of(g.optional_tensor(14), g.optional_tensor(15), 1, N, oc, "int8_linear_m1")
                            : Residual{};
    auto* qp = static_cast<int8_t*>(own ? q_own.data_ptr() : q.data_ptr());
    auto* xsp = static_cast<float*>(own ? xs_own.data_ptr() : xs.data_ptr());
    const hipStream_t s = stream_of(st);
    if (convrot)
        abi(w8a8_quantize_rowwise_act(x.data_ptr(), code, static_cast<int>(act),
                                      has_w ? dense(*aw, "act_weight").data_ptr() : nullptr, full ? g.real(12) : 0.0, qp,
                                      xsp, 1, K, 256, W8A8_SCALE_RECIP, nullptr, 0, s));
    else
        abi(w8a8_quantize_rowwise(x.data_ptr(), code, qp, xsp, 1, K, W8A8_SCALE_RECIP, s));
    auto* wp = static_cast<const int8_t*>(w.data_ptr());
    auto* wsp = static_cast<const float*>(ws.data_ptr());
    if (r.resid)
        abi(w8a8_gemv_dequant_residual(qp, wp, xsp, wsp, ws.numel(), b, r.rscale, r.rscale_size, r.resid,
                                       out.data_ptr(), oc, 1, N, K, 0, s));
    else
        abi(w8a8_gemv_dequant(qp, wp, xsp, wsp, ws.numel(), b, out.data_ptr(), oc, 1, N, K, 0, s));
    return 0;
}

// quantize_int8_rowwise_convrot64(input, output, scales, group_size,
// stochastic, act_code, seed, act_weight, act_eps, stream): the crate's fused
// ConvRot quantizer with an optional input activation (convrot.rs:169-206;
// dlpack_bindings.cpp:3430-3483, SiTU's code 4 and width as the crate passes
// them).  Activations fused in fp32 as Kitchen's kernel does.
int64_t quantize_int8_rowwise_convrot64(const Args& g) {
    const at::Tensor& x = dense(ranked(g.tensor(0), 2), "input");
    const at::Tensor& q = dense(typed(ranked(g.tensor(1), 2), at::kChar), "output");
    const at::Tensor& s = dense(typed(ranked(g.tensor(2), 2), at::kFloat), "scales");
    const int64_t group = g.integer(3);
    const bool stochastic = g.integer(4) != 0;
    const int64_t act = g.integer(5);
    (void)g.integer(6);
    const at::Tensor* aw = g.optional_tensor(7);
    const double eps = g.real(8);
    const int64_t M = x.size(0), K = q.size(1);
    const int64_t in_width = (act == W8A8_ACT_SWIGLU || act == W8A8_ACT_SITU) ? 2 : 1;
    if (q.size(0) != M || x.size(1) != K * in_width) throw std::runtime_error("INT8 rowwise convrot64 output shape mismatch");
    if (s.size(0) != M || s.size(1) != 1) throw std::runtime_error("INT8 rowwise convrot64 scale shape mismatch");
    const int code = dtype_code(x);
    if (code < 0) throw std::runtime_error("Unsupported input dtype for INT8 rowwise convrot64 quantization");
    const bool has_w = aw && aw->numel() > 0;
    if (act == W8A8_ACT_RMSNORM) {
        if (!has_w || aw->numel() != K) throw std::runtime_error("INT8 rowwise convrot64 rms_norm weight must have K elements");
        if (dtype_code(*aw) != code) throw std::runtime_error("INT8 rowwise convrot64 rms_norm weight dtype must match the input");
    }
    if (act < W8A8_ACT_NONE || act > W8A8_ACT_SITU) throw std::runtime_error("Unknown INT8 input activation code");
    if (stochastic) throw std::runtime_error("stochastic INT8 rounding is not part of this library");
    // Kitchen's kernel rotates 256-wide groups whatever group_size says; the
    // crate only takes this route with group 256 (cuda_linear.rs:404-417)
    if (group != 256 || K % 256 != 0 || K < 256 || K > 16384)
        throw std::runtime_error("INT8 rowwise convrot64 needs group 256 and K a multiple of 256 up to 16384");
    abi(w8a8_quantize_rowwise_act(x.data_ptr(), code, static_cast<int>(act), has_w ? dense(*aw, "act_weight").data_ptr() : nullptr,
                                  eps, static_cast<int8_t*>(q.data_ptr()), static_cast<float*>(s.data_ptr()), M, K, 256,
                                  W8A8_SCALE_RECIP, nullptr, 0, stream_of(g.integer(9))));
    return 0;
}

struct Route {
    const char* name;
    int64_t (*fn)(const Args&);
    size_t arity;
    size_t alt_arity;   // a second accepted argument count (0: none)
};

const Route kRoutes[] = {
    {"quantize_int8_rowwise", quantize_int8_rowwise, 6, 0},
    {"int8_gemv_dequant", int8_gemv_dequant, 10, 8},
    {"cutlass_int8_dequant", cutlass_int8_dequant, 8, 0},
    {"cutlass_int8_dequant_residual", cutlass_int8_dequant_residual, 10, 0},
    {"cublas_gemm_int8", cublas_gemm_int8, 5, 0},
    {"dequantize_int8_linear", dequantize_int8_linear, 7, 0},
    {"int8_linear_m1", int8_linear_m1, 16, 11},
    {"quantize_int8_rowwise_convrot64", quantize_int8_rowwise_convrot64, 10, 0},
};

}  // namespace

extern "C" {

__attribute__((visibility("default"))) const char* imagine_last_error() { return last_error.c_str(); }
__attribute__((visibility("default"))) int imagine_last_accelerator_code() { return last_accelerator_code; }
__attribute__((visibility("default"))) const char* imagine_last_metadata() { return last_metadata.c_str(); }

__attribute__((visibility("default"))) int imagine_kitchen_call(const char* name, const KitchenArg* args, size_t n,
                                                                int64_t* result) {
    try {
        if (!name || !result || (!args && n)) throw std::runtime_error("Null bridge argument");
        last_metadata.clear();
        int device = -1;
        for (size_t i = 0; i < n; ++i) {
            if (args[i].kind == 1 && args[i].tensor) {
                device = static_cast<const at::Tensor*>(args[i].tensor)->get_device();
                break;
            }
        }
        DeviceGuard guard(device);
        for (const Route& r : kRoutes) {
            if (std::strcmp(name, r.name) != 0) continue;
            if (n != r.arity && (r.alt_arity == 0 || n != r.alt_arity))
                throw std::runtime_error("Kernel argument count mismatch");
            *result = r.fn(Args{args, n});
            last_error.clear();
            return 0;
        }
        throw std::runtime_error("Unknown Kitchen kernel");
    } catch (const AbiError& e) {
        last_error = e.what();
        return e.code == W8A8_ERR_VALUE ? -20 : e.code == W8A8_ERR_INDEX ? -21 : -1;
    } catch (const std::invalid_argument& e) {
        last_error = e.what();
        return -20;
    } catch (const std::out_of_range& e) {
        last_error = e.what();
        return -21;
    } catch (const std::exception& e) {
        last_error = e.what();
        return -1;
    } catch (...) {
        last_error = "Unknown native exception";
        return -1;
    }
}

}  // extern "C"
