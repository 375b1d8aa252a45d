// lbq_gemm_k23.hip -- the batched-path MFMA kernels for Q2_K and Q3_K weights
// (one unit per type family, so the library builds them in parallel).
#include "lbq_gemm_kernels.hpp"

namespace lbq {
template hipError_t launch_typed<TYPE_Q2_K>(const Plan &, const uint8_t *, const int8_t *, int64_t, int64_t,
                                          const _Float16 *, const int *, const _Float16 *, int64_t, int64_t,
                                          float *, int64_t, uint32_t *, float *, const float *, hipStream_t);
template hipError_t launch_typed<TYPE_Q3_K>(const Plan &, const uint8_t *, const int8_t *, int64_t, int64_t,
                                          const _Float16 *, const int *, const _Float16 *, int64_t, int64_t,
                                          float *, int64_t, uint32_t *, float *, const float *, hipStream_t);
}  // namespace lbq
