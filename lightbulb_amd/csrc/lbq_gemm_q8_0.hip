// lbq_gemm_q8_0.hip -- the batched-path MFMA kernels for Q8_0 weights (one unit per
// type, so the library builds them in parallel).
#include "lbq_gemm_kernels.hpp"

namespace lbq {
template hipError_t launch_typed<TYPE_Q8_0>(const Plan &, const uint8_t *, const int8_t *, int64_t, int64_t,
                                          const _Float16 *, const int *, const _Float16 *, int64_t, int64_t,
                                          float *, int64_t, uint32_t *, float *, const float *, hipStream_t);
}  // namespace lbq
