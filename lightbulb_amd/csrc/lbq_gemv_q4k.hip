// lbq_gemv_q4k.hip -- decode GEMV instantiations for one weight type (built in
// parallel with the other types; the kernel itself lives in lbq_gemv_impl.hpp).
#include "lbq_gemv_impl.hpp"

namespace lbq {

hipError_t gemv_q4k(const RowMap &rm, int64_t k, int64_t row_bytes, const ActView &act, const float *x, int m,
                       int map, const float *alpha, float eps, hipStream_t st) {
    return run_type<TYPE_Q4_K>(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
}

}  // namespace lbq
