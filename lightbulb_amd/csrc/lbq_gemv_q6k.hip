// lbq_gemv_q6k.hip -- decode GEMV instantiations for one weight type (built in
// parallel with the other types; the kernel itself lives in lbq_gemv_impl.hpp).
#include "lbq_gemv_impl.hpp"

namespace lbq {

hipError_t gemv_q6k(int64_t n, int64_t k, int64_t row_bytes, const ActView &act, const float *x, int m, float *y,
                       hipStream_t st, const uint8_t *w) {
    return run_type<TYPE_Q6_K>(w, n, k, row_bytes, act, x, m, y, st);
}

}  // namespace lbq
