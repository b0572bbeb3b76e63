// gemm_i8.hip -- placeholder for the Q8_0 x Q8 int8 MFMA rung.
#include "krk_kernels.hpp"

namespace krk {
size_t gemm_int8_workspace(int64_t, int64_t) { return 0; }
hipError_t gemm_int8_q8_0(const void *, int64_t, const void *, bool, void *, int64_t, int64_t,
                          int64_t, void *, size_t, hipStream_t) {
    return hipErrorNotSupported;
}
}  // namespace krk
