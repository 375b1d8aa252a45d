// lbq_gemv_k23.hip -- decode GEMV instantiations for Q2_K and Q3_K (the kernel
// itself lives in lbq_gemv_impl.hpp).
#include "lbq_gemv_impl.hpp"

namespace lbq {

hipError_t gemv_k23(int type, const RowMap &rm, int64_t k, int64_t row_bytes, const ActView &act, const float *x,
                    int m, int map, const float *alpha, float eps, hipStream_t st) {
    switch (type) {
    case TYPE_Q2_K: return run_type<TYPE_Q2_K>(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q3_K: return run_type<TYPE_Q3_K>(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace lbq
