// Test driver of libimagine_kitchen.so (test infrastructure): loads it the way
// the reference crate loads its bridge (dlopen RTLD_NOW | RTLD_LOCAL, dlsym of
// imagine_kitchen_call and imagine_last_error: inference/src/native.rs:1277-1330),
// issues the argument lists of the crate's int8_linear operator
// (inference/src/cuda_linear.rs:558-582, 605-616, 657-676, 724-762, 770-794)
// with borrowed at::Tensor handles, and checks return codes, result values,
// error texts and output bytes; outputs are compared with the oracle
// (oracle/liboracle.so) on host copies.  Prints one line per check, exits 0
// when all pass.
//
//   kitchen_bridge_test <libimagine_kitchen.so> <liboracle.so>
#include <ATen/ATen.h>
#include <dlfcn.h>
#include <hip/hip_runtime_api.h>

#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

struct KitchenArg {
    int64_t kind;
    void* tensor;
    int64_t integer;
    double real;
};

using Call = int (*)(const char*, const KitchenArg*, size_t, int64_t*);
using Text = const char* (*)();

// oracle/w8a8_oracle.c
using OQuant = void (*)(const void*, int, int64_t, int64_t, int, int, int8_t*, float*);
using OGemm = void (*)(const int8_t*, const int8_t*, int64_t, int64_t, int64_t, int32_t*);
using OEpi = void (*)(const int32_t*, const float*, const float*, int64_t, const void*, void*, int, int64_t, int64_t, int,
                      int);
using ORes = void (*)(void*, const void*, const void*, int64_t, int, int64_t, int64_t, int);
using OCrAct = void (*)(const void*, int, int64_t, int64_t, int64_t, int, int, const void*, float, int8_t*, float*,
                        float*);

static Call call;
static Text last_error;
static OQuant o_quant;
static OGemm o_gemm;
static OEpi o_epi;
static ORes o_res;
static OCrAct o_cract;
static int failures = 0;

// The crate's KernelArg -> RawArg (native.rs:462-497).
static KitchenArg T(const at::Tensor& t) { return {1, const_cast<at::Tensor*>(&t), 0, 0.0}; }
static KitchenArg Int(int64_t v) { return {2, nullptr, v, 0.0}; }
static KitchenArg Bool(bool v) { return {4, nullptr, v ? 1 : 0, 0.0}; }
static KitchenArg Float(double v) { return {3, nullptr, 0, v}; }
static KitchenArg None() { return {0, nullptr, 0, 0.0}; }

static void check(bool ok, const std::string& what) {
    std::printf("%s %s\n", ok ? "PASS" : "FAIL", what.c_str());
    std::fflush(stdout);
    if (!ok) ++failures;
}

static int code_of(at::ScalarType s) { return s == at::kFloat ? 0 : s == at::kHalf ? 1 : 2; }

static at::Tensor dev(const at::Tensor& t) { return t.to(at::kCUDA); }

static bool same_bytes(const at::Tensor& a, const at::Tensor& b) {
    const at::Tensor x = a.cpu().contiguous(), y = b.cpu().contiguous();
    return x.nbytes() == y.nbytes() && std::memcmp(x.data_ptr(), y.data_ptr(), x.nbytes()) == 0;
}

static int run(const char* name, const std::vector<KitchenArg>& args, int64_t* result) {
    const int rc = call(name, args.data(), args.size(), result);
    (void)hipDeviceSynchronize();
    return rc;
}

// Oracle of the fused linear: (codes, scales) of x, then acc -> epilogue.
struct Ref {
    at::Tensor q, xs, acc;
};

static Ref oracle_quant_gemm(const at::Tensor& x, const at::Tensor& w) {
    const int64_t M = x.size(0), K = x.size(1), N = w.size(0);
    Ref r;
    r.q = at::empty({M, K}, at::kChar);
    r.xs = at::empty({M, 1}, at::kFloat);
    o_quant(x.data_ptr(), code_of(x.scalar_type()), M, K, /*scale_mode=*/1, 0, r.q.data_ptr<int8_t>(),
            r.xs.data_ptr<float>());
    r.acc = at::empty({M, N}, at::kInt);
    o_gemm(r.q.data_ptr<int8_t>(), w.data_ptr<int8_t>(), M, N, K, r.acc.data_ptr<int32_t>());
    return r;
}

static at::Tensor oracle_epilogue(const Ref& r, const at::Tensor& ws, const at::Tensor* bias, at::ScalarType odt) {
    const int64_t M = r.acc.size(0), N = r.acc.size(1);
    at::Tensor out = at::empty({M, N}, odt);
    o_epi(r.acc.data_ptr<int32_t>(), r.xs.data_ptr<float>(), ws.data_ptr<float>(), ws.numel(),
          bias && bias->numel() ? bias->data_ptr() : nullptr, out.data_ptr(), code_of(odt), M, N, 1, 0);
    return out;
}

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s libimagine_kitchen.so liboracle.so\n", argv[0]);
        return 2;
    }
    void* h = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    void* ho = dlopen(argv[2], RTLD_NOW | RTLD_LOCAL);
    if (!h || !ho) {
        std::fprintf(stderr, "dlopen: %s\n", dlerror());
        return 2;
    }
    call = reinterpret_cast<Call>(dlsym(h, "imagine_kitchen_call"));
    last_error = reinterpret_cast<Text>(dlsym(h, "imagine_last_error"));
    auto accel = dlsym(h, "imagine_last_accelerator_code");
    auto meta = dlsym(h, "imagine_last_metadata");
    o_quant = reinterpret_cast<OQuant>(dlsym(ho, "w8o_quant_rowwise"));
    o_gemm = reinterpret_cast<OGemm>(dlsym(ho, "w8o_gemm_i32"));
    o_epi = reinterpret_cast<OEpi>(dlsym(ho, "w8o_epilogue_kitchen"));
    o_res = reinterpret_cast<ORes>(dlsym(ho, "w8o_residual"));
    o_cract = reinterpret_cast<OCrAct>(dlsym(ho, "w8o_convrot_quant_act"));
    check(call && last_error && accel && meta, "bridge exports imagine_kitchen_call and imagine_last_*");
    if (!call || !o_quant || !o_gemm || !o_epi || !o_res || !o_cract) return 1;

    at::manual_seed(7);
    const int64_t stream = 0;   // the crate passes torch's current stream; the default one here
    int64_t result = -7;

    for (at::ScalarType odt : {at::kBFloat16, at::kHalf, at::kFloat}) {
        const std::string dn = odt == at::kBFloat16 ? "bf16" : odt == at::kHalf ? "f16" : "f32";
        // ---- quantize_int8_rowwise -> cutlass_int8_dequant (GEMM route, M = 300)
        const int64_t M = 300, K = 1024, N = 520;
        const at::Tensor x = at::randn({M, K}).to(at::kBFloat16);
        const at::Tensor w = at::randint(-127, 128, {N, K}, at::kChar);
        const at::Tensor ws = at::rand({N}) * 9e-3 + 1e-3;
        const at::Tensor bias = (at::randn({N}) * 0.02).to(odt);
        const Ref ref = oracle_quant_gemm(x, w);
        const at::Tensor xd = dev(x), wd = dev(w), wsd = dev(ws), bd = dev(bias);
        at::Tensor q = at::empty({M, K}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        at::Tensor xs = at::empty({M, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
        int rc = run("quantize_int8_rowwise", {T(xd), T(q), T(xs), Bool(false), Int(0), Int(stream)}, &result);
        check(rc == 0 && result == 0 && same_bytes(q, ref.q) && same_bytes(xs, ref.xs),
              "quantize_int8_rowwise codes and scales = oracle (" + dn + " pass)");
        at::Tensor out = at::empty({M, N}, at::TensorOptions().dtype(odt).device(at::kCUDA));
        result = -7;
        rc = run("cutlass_int8_dequant", {T(q), T(wd), T(xs), T(wsd), T(bd), T(out), Int(code_of(odt)), Int(stream)},
                 &result);
        check(rc == 0 && result == 1 && same_bytes(out, oracle_epilogue(ref, ws, &bias, odt)),
              "cutlass_int8_dequant returns true and its " + dn + " output = oracle");

        // ---- cutlass_int8_dequant_residual
        const at::Tensor resid = (at::randn({M, N}) * 2).to(odt), rscale = (at::rand({N}) + 0.25).to(odt);
        const at::Tensor rd = dev(resid), sd = dev(rscale);
        at::Tensor out2 = at::empty_like(out);
        result = -7;
        rc = run("cutlass_int8_dequant_residual",
                 {T(q), T(wd), T(xs), T(wsd), T(bd), T(sd), T(rd), T(out2), Int(code_of(odt)), Int(stream)}, &result);
        at::Tensor want2 = oracle_epilogue(ref, ws, &bias, odt);
        o_res(want2.data_ptr(), resid.data_ptr(), rscale.data_ptr(), N, code_of(odt), M, N, 1);
        check(rc == 0 && result == 1 && same_bytes(out2, want2),
              "cutlass_int8_dequant_residual returns true and its " + dn + " output = oracle");

        // ---- cublas_gemm_int8 + dequantize_int8_linear (the fallback route)
        at::Tensor acc = at::empty({M, N}, at::TensorOptions().dtype(at::kInt).device(at::kCUDA));
        at::Tensor wksp = at::empty({4 << 20}, at::TensorOptions().dtype(at::kByte).device(at::kCUDA));
        rc = run("cublas_gemm_int8", {T(q), T(wd), T(acc), T(wksp), Int(stream)}, &result);
        check(rc == 0 && same_bytes(acc, ref.acc), "cublas_gemm_int8 int32 accumulators = oracle");
        at::Tensor out3 = at::empty_like(out);
        rc = run("dequantize_int8_linear", {T(acc), T(xs), T(wsd), T(bd), T(out3), Int(code_of(odt)), Int(stream)},
                 &result);
        check(rc == 0 && same_bytes(out3, out), "dequantize_int8_linear " + dn + " output = the fused route's");

        // ---- int8_gemv_dequant, M = 2 (the adaLN shape, smaller N), and M = 1 with a residual
        {
            const int64_t m = 2, k = 3072, n = 1536;
            const at::Tensor gx = at::randn({m, k}).to(at::kBFloat16);
            const at::Tensor gw = at::randint(-127, 128, {n, k}, at::kChar);
            const at::Tensor gws = at::rand({n}) * 9e-3 + 1e-3;
            const at::Tensor gb = (at::randn({n}) * 0.02).to(odt);
            const Ref gr = oracle_quant_gemm(gx, gw);
            const at::Tensor gxd = dev(gx), gwd = dev(gw), gwsd = dev(gws), gbd = dev(gb);
            at::Tensor gq = at::empty({m, k}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
            at::Tensor gxs = at::empty({m, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
            run("quantize_int8_rowwise", {T(gxd), T(gq), T(gxs), Bool(false), Int(0), Int(stream)}, &result);
            at::Tensor go = at::empty({m, n}, at::TensorOptions().dtype(odt).device(at::kCUDA));
            rc = run("int8_gemv_dequant",
                     {T(gq), T(gwd), T(gxs), T(gwsd), T(gbd), T(go), Int(code_of(odt)), Int(stream), None(), None()},
                     &result);
            check(rc == 0 && same_bytes(go, oracle_epilogue(gr, gws, &gb, odt)), "int8_gemv_dequant M=2 " + dn + " = oracle");

            const at::Tensor x1 = gx.slice(0, 0, 1).contiguous();
            const Ref r1 = oracle_quant_gemm(x1, gw);
            const at::Tensor res1 = (at::randn({1, n}) * 2).to(odt), rs1 = (at::rand({n}) + 0.25).to(odt);
            at::Tensor want1 = oracle_epilogue(r1, gws, &gb, odt);
            o_res(want1.data_ptr(), res1.data_ptr(), rs1.data_ptr(), n, code_of(odt), 1, n, 1);
            const at::Tensor x1d = dev(x1), res1d = dev(res1), rs1d = dev(rs1);
            at::Tensor q1 = at::empty({1, k}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
            at::Tensor s1 = at::empty({1, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
            run("quantize_int8_rowwise", {T(x1d), T(q1), T(s1), Bool(false), Int(0), Int(stream)}, &result);
            at::Tensor o1 = at::empty({1, n}, at::TensorOptions().dtype(odt).device(at::kCUDA));
            rc = run("int8_gemv_dequant",
                     {T(q1), T(gwd), T(s1), T(gwsd), T(gbd), T(o1), Int(code_of(odt)), Int(stream), T(res1d), T(rs1d)},
                     &result);
            check(rc == 0 && same_bytes(o1, want1), "int8_gemv_dequant M=1 with residual " + dn + " = oracle");

            // ---- int8_linear_m1: the crate's 16 arguments (non-ConvRot, no activation)
            const at::Tensor empty_act = at::empty({0}, at::TensorOptions().dtype(at::kBFloat16).device(at::kCUDA));
            at::Tensor q1b = at::empty({1, k}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
            at::Tensor s1b = at::empty({1, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
            at::Tensor o1b = at::empty({1, n}, at::TensorOptions().dtype(odt).device(at::kCUDA));
            rc = run("int8_linear_m1",
                     {T(x1d), T(q1b), T(s1b), T(gwd), T(gwsd), T(gbd), T(o1b), Int(code_of(odt)), Bool(false),
                      Int(256), Int(0), T(empty_act), Float(0.0), Int(stream), T(res1d), T(rs1d)},
                     &result);
            check(rc == 0 && same_bytes(o1b, want1), "int8_linear_m1 (16 arguments) with residual " + dn + " = oracle");
        }
    }

    // ---- quantize_int8_rowwise_convrot64 with each input activation, and
    // int8_linear_m1 on the ConvRot route with empty scratch and an activation
    // (the crate's argument lists: convrot.rs:191-206, cuda_linear.rs:558-582)
    for (at::ScalarType xdt : {at::kBFloat16, at::kHalf, at::kFloat}) {
        const std::string xn = xdt == at::kBFloat16 ? "bf16" : xdt == at::kHalf ? "f16" : "f32";
        const char* names[] = {"none", "gelu_tanh", "swiglu", "rms_norm", "situ"};
        for (int act = 0; act <= 4; ++act) {
            const int64_t m = 5, k = 512, width = (act == 2 || act == 4) ? 2 * k : k;
            const at::Tensor x = (at::randn({m, width}) * 2).to(xdt);
            const at::Tensor aw = act == 3 ? (1 + 0.3 * at::randn({k})).to(xdt) : at::empty({0}, xdt);
            at::Tensor q_ref = at::empty({m, k}, at::kChar), s_ref = at::empty({m, 1}, at::kFloat);
            at::Tensor work = at::empty({k}, at::kFloat);
            o_cract(x.data_ptr(), code_of(xdt), m, k, 256, /*scale_mode=*/1, act, act == 3 ? aw.data_ptr() : nullptr,
                    1e-6f, q_ref.data_ptr<int8_t>(), s_ref.data_ptr<float>(), work.data_ptr<float>());
            const at::Tensor xd = dev(x), awd = dev(aw);
            at::Tensor q = at::empty({m, k}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
            at::Tensor s = at::empty({m, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
            int rc = run("quantize_int8_rowwise_convrot64",
                         {T(xd), T(q), T(s), Int(256), Bool(false), Int(act), Int(0), T(awd), Float(1e-6), Int(stream)},
                         &result);
            check(rc == 0 && same_bytes(q, q_ref) && same_bytes(s, s_ref),
                  std::string("quantize_int8_rowwise_convrot64 ") + names[act] + " " + xn + " = oracle");

            // M = 1 through int8_linear_m1, scratch tensors empty as the crate sends them
            const int64_t n = 384;
            const at::Tensor w = at::randint(-127, 128, {n, k}, at::kChar);
            const at::Tensor ws = at::rand({n}) * 9e-3 + 1e-3;
            const at::Tensor bias = (at::randn({n}) * 0.02).to(at::kBFloat16);
            Ref r1;
            r1.q = q_ref.slice(0, 0, 1).contiguous();
            r1.xs = s_ref.slice(0, 0, 1).contiguous();
            r1.acc = at::empty({1, n}, at::kInt);
            o_gemm(r1.q.data_ptr<int8_t>(), w.data_ptr<int8_t>(), 1, n, k, r1.acc.data_ptr<int32_t>());
            const at::Tensor want = oracle_epilogue(r1, ws, &bias, at::kBFloat16);
            const at::Tensor x1d = dev(x.slice(0, 0, 1).contiguous()), wd = dev(w), wsd = dev(ws), bd = dev(bias);
            const at::Tensor eq = at::empty({0}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
            const at::Tensor es = at::empty({0}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
            at::Tensor o = at::empty({1, n}, at::TensorOptions().dtype(at::kBFloat16).device(at::kCUDA));
            rc = run("int8_linear_m1",
                     {T(x1d), T(eq), T(es), T(wd), T(wsd), T(bd), T(o), Int(2), Bool(true), Int(256), Int(act), T(awd),
                      Float(1e-6), Int(stream), None(), None()},
                     &result);
            check(rc == 0 && same_bytes(o, want), std::string("int8_linear_m1 ConvRot ") + names[act] + " " + xn +
                                                      " (empty scratch) = oracle" + (rc ? ": " + std::string(last_error()) : ""));
        }
        // Kitchen's texts for a bad output width and a missing norm weight
        const at::Tensor x = at::zeros({4, 512}, at::TensorOptions().dtype(xdt).device(at::kCUDA));
        at::Tensor q = at::empty({4, 512}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        at::Tensor s = at::empty({4, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
        const at::Tensor none = at::empty({0}, at::TensorOptions().dtype(xdt).device(at::kCUDA));
        int rc = run("quantize_int8_rowwise_convrot64",
                     {T(x), T(q), T(s), Int(256), Bool(false), Int(2), Int(0), T(none), Float(0.0), Int(stream)}, &result);
        check(rc == -1 && std::string(last_error()) == "INT8 rowwise convrot64 output shape mismatch",
              "convrot64 swiglu width text " + xn);
        rc = run("quantize_int8_rowwise_convrot64",
                 {T(x), T(q), T(s), Int(256), Bool(false), Int(3), Int(0), T(none), Float(0.0), Int(stream)}, &result);
        check(rc == -1 && std::string(last_error()) == "INT8 rowwise convrot64 rms_norm weight must have K elements",
              "convrot64 rms_norm weight text " + xn);
    }

    // ---- errors: codes and texts
    {
        const at::Tensor a = at::zeros({4, 64}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        const at::Tensor b = at::zeros({8, 32}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        const at::Tensor xs = at::ones({4}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
        const at::Tensor ws = at::ones({8}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
        const at::Tensor none = at::empty({0}, at::TensorOptions().dtype(at::kBFloat16).device(at::kCUDA));
        const at::Tensor d = at::empty({4, 8}, at::TensorOptions().dtype(at::kBFloat16).device(at::kCUDA));
        int rc = run("cutlass_int8_dequant", {T(a), T(b), T(xs), T(ws), T(none), T(d), Int(2), Int(0)}, &result);
        check(rc == -1 && std::string(last_error()) == "cutlass_int8_dequant: K mismatch", "K mismatch text");
        rc = run("cutlass_int8_dequant", {T(a), T(b), T(xs), T(ws), T(none), T(d), Int(2)}, &result);
        check(rc == -1 && std::string(last_error()) == "Kernel argument count mismatch", "arity check");
        rc = run("not_a_kitchen_kernel", {}, &result);
        check(rc == -1 && std::string(last_error()) == "Unknown Kitchen kernel", "unknown name");
        const at::Tensor g3 = at::zeros({3, 64}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        const at::Tensor gw = at::zeros({8, 64}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        const at::Tensor gx = at::ones({3, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
        const at::Tensor go = at::empty({3, 8}, at::TensorOptions().dtype(at::kBFloat16).device(at::kCUDA));
        rc = run("int8_gemv_dequant", {T(g3), T(gw), T(gx), T(ws), T(none), T(go), Int(2), Int(0), None(), None()},
                 &result);
        check(rc == -1 && std::string(last_error()) == "INT8 GEMV dequant expects M == 1 or M == 2", "GEMV M text");
        const at::Tensor x = at::zeros({4, 64}, at::TensorOptions().dtype(at::kBFloat16).device(at::kCUDA));
        const at::Tensor qbad = at::empty({4, 32}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        const at::Tensor s = at::empty({4, 1}, at::TensorOptions().dtype(at::kFloat).device(at::kCUDA));
        rc = run("quantize_int8_rowwise", {T(x), T(qbad), T(s), Bool(false), Int(0), Int(0)}, &result);
        check(rc == -1 && std::string(last_error()) == "INT8 rowwise quantization output shape mismatch",
              "quantizer shape text");
        rc = run("quantize_int8_rowwise", {Int(1), T(qbad), T(s), Bool(false), Int(0), Int(0)}, &result);
        check(rc == -1 && std::string(last_error()) == "Expected tensor argument", "argument kind text");
        const at::Tensor bias16 = at::zeros({8}, at::TensorOptions().dtype(at::kHalf).device(at::kCUDA));
        const at::Tensor a2 = at::zeros({4, 32}, at::TensorOptions().dtype(at::kChar).device(at::kCUDA));
        rc = run("cutlass_int8_dequant", {T(a2), T(b), T(xs), T(ws), T(bias16), T(d), Int(2), Int(0)}, &result);
        check(rc == -1 && std::string(last_error()) ==
                              "cutlass_int8_dequant: bias must be empty or a length-N vector in the output dtype",
              "bias dtype text");
    }
    std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
