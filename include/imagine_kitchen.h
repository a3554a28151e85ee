/*
 * imagine_kitchen.h -- C ABI of libimagine_kitchen.so, the W8A8 names of the
 * reference bridge's Kitchen dispatcher over libw8a8_hip.so.
 *
 * Same record and entry points as the reference bridge
 * (inference/native/bridge.hpp:5-6 KitchenArg, :13-16 imagine_last_*, :29
 * imagine_kitchen_call; behaviour bridge.cpp:415-440), which the crate binds
 * with dlsym (inference/src/native.rs:455-497,1277-1330,1586-1607).  Tensors are
 * borrowed at::Tensor handles of the caller's LibTorch (this build: the ROCm
 * LibTorch of the image).  The names answered and their argument lists are
 * those of the crate's int8_linear operator; see kitchen_bridge.cpp.
 */
#ifndef IMAGINE_KITCHEN_H
#define IMAGINE_KITCHEN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kind: 0 = None, 1 = borrowed at::Tensor*, 2 = int64, 3 = double, 4 = bool
 * (bridge.hpp:5-6). */
struct KitchenArg {
    int64_t kind;
    void* tensor;
    int64_t integer;
    double real;
};

/* Run Kitchen kernel `name` on n arguments; *result receives its return value
 * (1 for the CUTLASS names: handled).  Returns 0, or -1 runtime error, -20
 * ValueError, -21 IndexError, with the text in imagine_last_error()
 * (bridge.hpp:29, bridge.cpp:415-440). */
int imagine_kitchen_call(const char* name, const struct KitchenArg* args, size_t n, int64_t* result);

/* Thread-local diagnostics of the last call (bridge.hpp:13-16). */
const char* imagine_last_error(void);
int imagine_last_accelerator_code(void);
const char* imagine_last_metadata(void);

#ifdef __cplusplus
}
#endif

#endif /* IMAGINE_KITCHEN_H */
