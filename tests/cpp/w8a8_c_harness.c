/*
 * C caller of libw8a8_hip.so (test infrastructure): compiles against
 * include/w8a8.h as plain C99 with the HIP runtime's C API and nothing else,
 * and runs the operator's routes on device memory it allocates itself:
 * quantize -> GEMM, quantize -> GEMV (M = 2), the operator entry with its
 * workspace, and an argument error.  Results are compared with the oracle
 * (oracle/liboracle.so, loaded with dlopen).  Prints one line per check and
 * exits 0 when all pass.
 *
 *   w8a8_c_harness <liboracle.so>
 */
#include <dlfcn.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "w8a8.h"

typedef void (*oquant_t)(const void*, int, int64_t, int64_t, int, int, int8_t*, float*);
typedef void (*ogemm_t)(const int8_t*, const int8_t*, int64_t, int64_t, int64_t, int32_t*);
typedef void (*oepi_t)(const int32_t*, const float*, const float*, int64_t, const void*, void*, int, int64_t,
                       int64_t, int, int);

static int failures = 0;

static void check(int ok, const char* what) {
    printf("%s %s\n", ok ? "PASS" : "FAIL", what);
    fflush(stdout);
    if (!ok) ++failures;
}

static uint32_t rng = 12345u;
static uint32_t next_u32(void) {
    rng ^= rng << 13;
    rng ^= rng >> 17;
    rng ^= rng << 5;
    return rng;
}
/* bf16 of a value in [-2, 2): top 16 bits of a float, rounded to nearest even */
static uint16_t rand_bf16(void) {
    float f = ((float)(next_u32() >> 8) / 16777216.0f) * 4.0f - 2.0f;
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static void* dalloc(size_t bytes) {
    void* p = NULL;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        fprintf(stderr, "hipMalloc failed\n");
        exit(2);
    }
    return p;
}

static void h2d(void* d, const void* h, size_t n) { (void)hipMemcpy(d, h, n, hipMemcpyHostToDevice); }
static void d2h(void* h, const void* d, size_t n) { (void)hipMemcpy(h, d, n, hipMemcpyDeviceToHost); }

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s liboracle.so\n", argv[0]);
        return 2;
    }
    void* ho = dlopen(argv[1], RTLD_NOW | RTLD_LOCAL);
    if (!ho) {
        fprintf(stderr, "dlopen: %s\n", dlerror());
        return 2;
    }
    oquant_t o_quant = (oquant_t)dlsym(ho, "w8o_quant_rowwise");
    ogemm_t o_gemm = (ogemm_t)dlsym(ho, "w8o_gemm_i32");
    oepi_t o_epi = (oepi_t)dlsym(ho, "w8o_epilogue_kitchen");
    if (!o_quant || !o_gemm || !o_epi) return 2;
    check(strstr(w8a8_version(), "gfx950") != NULL, "w8a8_version names gfx950");

    const int64_t M = 300, K = 768, N = 400;
    uint16_t* x = malloc(M * K * 2);
    int8_t* w = malloc(N * K);
    float* ws = malloc(N * 4);
    uint16_t* bias = malloc(N * 2);
    for (int64_t i = 0; i < M * K; ++i) x[i] = rand_bf16();
    for (int64_t i = 0; i < N * K; ++i) w[i] = (int8_t)((int)(next_u32() % 255u) - 127);
    for (int64_t i = 0; i < N; ++i) ws[i] = 1e-3f + 9e-3f * (float)(next_u32() >> 8) / 16777216.0f;
    for (int64_t i = 0; i < N; ++i) bias[i] = rand_bf16();

    /* oracle: codes, scales, accumulators, bf16 output */
    int8_t* q_ref = malloc(M * K);
    float* xs_ref = malloc(M * 4);
    int32_t* acc_ref = malloc(M * N * 4);
    uint16_t* out_ref = malloc(M * N * 2);
    o_quant(x, W8A8_BF16, M, K, 0, 0, q_ref, xs_ref);
    o_gemm(q_ref, w, M, N, K, acc_ref);
    o_epi(acc_ref, xs_ref, ws, N, bias, out_ref, W8A8_BF16, M, N, 1, 0);

    void* dx = dalloc(M * K * 2);
    int8_t* dq = dalloc(M * K);
    float* dxs = dalloc(M * 4);
    int8_t* dw = dalloc(N * K);
    float* dws = dalloc(N * 4);
    void* db = dalloc(N * 2);
    void* dout = dalloc(M * N * 2);
    h2d(dx, x, M * K * 2);
    h2d(dw, w, N * K);
    h2d(dws, ws, N * 4);
    h2d(db, bias, N * 2);
    hipStream_t stream = NULL;
    (void)hipStreamCreate(&stream);

    int rc = w8a8_quantize_rowwise(dx, W8A8_BF16, dq, dxs, M, K, 0, stream);
    (void)hipStreamSynchronize(stream);
    int8_t* q = malloc(M * K);
    float* xs = malloc(M * 4);
    d2h(q, dq, M * K);
    d2h(xs, dxs, M * 4);
    check(rc == W8A8_OK && memcmp(q, q_ref, M * K) == 0 && memcmp(xs, xs_ref, M * 4) == 0,
          "w8a8_quantize_rowwise codes and scales = oracle");

    rc = w8a8_gemm_dequant(dq, dw, dxs, dws, N, db, dout, W8A8_BF16, M, N, K, 0, stream);
    (void)hipStreamSynchronize(stream);
    uint16_t* out = malloc(M * N * 2);
    d2h(out, dout, M * N * 2);
    check(rc == W8A8_OK && memcmp(out, out_ref, M * N * 2) == 0, "w8a8_gemm_dequant bf16 output = oracle");

    /* the operator entry with a caller-allocated workspace: same output */
    int64_t need = w8a8_int8_linear_workspace_bytes(M, K);
    void* wk = dalloc((size_t)need);
    (void)hipMemset(dout, 0, M * N * 2);
    rc = w8a8_int8_linear(dx, W8A8_BF16, dw, dws, N, db, dout, W8A8_BF16, M, N, K, 0, wk, need, stream);
    (void)hipStreamSynchronize(stream);
    d2h(out, dout, M * N * 2);
    check(rc == W8A8_OK && memcmp(out, out_ref, M * N * 2) == 0, "w8a8_int8_linear (GEMM route) = oracle");

    /* M = 2: the GEMV route of the operator entry equals the oracle on the first two rows */
    rc = w8a8_int8_linear(dx, W8A8_BF16, dw, dws, N, db, dout, W8A8_BF16, 2, N, K, 0, wk, need, stream);
    (void)hipStreamSynchronize(stream);
    d2h(out, dout, 2 * N * 2);
    o_epi(acc_ref, xs_ref, ws, N, bias, out_ref, W8A8_BF16, 2, N, 1, 0);
    check(rc == W8A8_OK && memcmp(out, out_ref, 2 * N * 2) == 0, "w8a8_int8_linear (GEMV route, M = 2) = oracle");

    /* an argument error: its code and message, nothing launched */
    rc = w8a8_gemv_dequant(dq, dw, dxs, dws, N, NULL, dout, W8A8_BF16, 3, N, K, 0, stream);
    check(rc == W8A8_ERR_RUNTIME && strcmp(w8a8_last_error(), "INT8 GEMV dequant expects M == 1 or M == 2") == 0,
          "w8a8_gemv_dequant rejects M = 3 with the reference's text");

    printf("%s: %d failure(s)\n", failures ? "FAILED" : "OK", failures);
    return failures ? 1 : 0;
}
