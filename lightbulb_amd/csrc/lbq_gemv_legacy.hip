// lbq_gemv_legacy.hip -- decode GEMV instantiations for the 32-value legacy weight
// types Q4_0, Q4_1, Q5_0, Q5_1 (the kernel itself lives in lbq_gemv_impl.hpp).
#include "lbq_gemv_impl.hpp"

namespace lbq {

hipError_t gemv_legacy(int type, const RowMap &rm, int64_t k, int64_t row_bytes, const ActView &act, const float *x,
                       int m, int map, const float *alpha, float eps, hipStream_t st) {
    switch (type) {
    case TYPE_Q4_0: return run_type<TYPE_Q4_0>(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q4_1: return run_type<TYPE_Q4_1>(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q5_0: return run_type<TYPE_Q5_0>(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q5_1: return run_type<TYPE_Q5_1>(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace lbq
