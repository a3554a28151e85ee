// bf16 outputs of the W8A8 GEMM: the gemm_dispatch instantiations for this
// output dtype (plain, GELU and residual epilogues), in a translation
// unit of their own so the kernels of each dtype compile in parallel.
#include "w8a8_gemm_launch.h"

namespace w8a8 {

#define W8A8_GEMM_INST(ODT, MODE, GELU)                                                                      \
    template void gemm_dispatch<ODT, MODE, GELU>(const int8_t*, const int8_t*, const float*, const float*, int64_t, \
                                                 const void*, const Residual&, void*, int64_t, int64_t, int64_t, int, \
                                                 hipStream_t);
W8A8_GEMM_INST(W8A8_BF16, 0, false)
W8A8_GEMM_INST(W8A8_BF16, 0, true)
W8A8_GEMM_INST(W8A8_BF16, 2, false)
#undef W8A8_GEMM_INST

}  // namespace w8a8
