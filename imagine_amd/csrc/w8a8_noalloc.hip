// w8a8_int8_linear_noalloc: the operator-level W8A8 linear with its workspace
// (the int8 codes and row scales of x) in a file-scope device array instead of
// caller- or library-allocated memory, for callers that cannot allocate
// (code under HIP graph capture, serving loops that forbid hipMalloc).
//
// The array lives in this translation unit's code object, which the runtime
// loads on a device the first time this entry runs there; each device then
// holds its own copy (kScratchBytes) until the process ends.  Host code never
// names the array directly: its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and that address is what
// the kernels receive.
#include <mutex>
#include <string>

#include "w8a8_common.h"

namespace w8a8 {
int set_error(int code, const std::string& msg);
int set_accelerator_error(int hip_code, const std::string& msg);
}  // namespace w8a8

namespace {

constexpr int64_t kScratchBytes = W8A8_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) int8_t scratch[kScratchBytes];

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the current device, looked up on the first
// call per device.  Returns W8A8_OK and sets *ptr, or an error code.
int scratch_of_current_device(void** ptr) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return w8a8::set_accelerator_error(static_cast<int>(e), std::string("hipGetDevice: ") + hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return w8a8::set_error(W8A8_ERR_RUNTIME, "device index out of range for the scratch table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return w8a8::set_accelerator_error(static_cast<int>(e),
                                               std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return W8A8_OK;
}

}  // namespace

extern "C" {

int64_t w8a8_int8_linear_noalloc_max_bytes(void) { return kScratchBytes; }

int w8a8_int8_linear_noalloc(const void* x, int x_dtype, const int8_t* w, const float* ws, int64_t ws_size,
                             const void* bias, void* out, int out_dtype, int64_t M, int64_t N, int64_t K,
                             uint32_t flags, hipStream_t stream) {
    const int64_t need = w8a8_int8_linear_workspace_bytes(M, K);
    if (need < 0) return w8a8::set_error(W8A8_ERR_VALUE, "negative dimension");
    if (need > kScratchBytes)
        return w8a8::set_error(W8A8_ERR_VALUE, "w8a8_int8_linear_noalloc: the codes and scales of a " +
                                                   std::to_string(M) + " x " + std::to_string(K) + " input need " +
                                                   std::to_string(need) + " bytes, above its fixed scratch of " +
                                                   std::to_string(kScratchBytes) + " bytes");
    if (M == 0) return w8a8_int8_linear(x, x_dtype, w, ws, ws_size, bias, out, out_dtype, M, N, K, flags, nullptr, 0,
                                        stream);
    void* ptr = nullptr;
    if (int rc = scratch_of_current_device(&ptr)) return rc;
    return w8a8_int8_linear(x, x_dtype, w, ws, ws_size, bias, out, out_dtype, M, N, K, flags, ptr, kScratchBytes,
                            stream);
}

}  // extern "C"
