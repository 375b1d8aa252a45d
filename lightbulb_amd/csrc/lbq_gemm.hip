// lbq_gemm.hip -- batched path (m > 8).
//
// Until the MFMA tile kernel is in place, the batched path runs the decode
// GEMV over row chunks of 8 activations.  Results are identical in kind to
// the decode path (exact integer sub-block sums, f32 combine); only speed
// differs.
#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

hipError_t launch_gemm(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act,
                       int64_t m, float *y, hipStream_t st) {
    for (int64_t m0 = 0; m0 < m; m0 += 8) {
        const int mc = (int)(m - m0 < 8 ? m - m0 : 8);
        ActView a = act;
        a.xq = act.xq + m0 * k;
        a.xd = act.xd + m0 * act.nb;
        a.xbs = act.xbs ? act.xbs + m0 * (k / 16) : nullptr;
        hipError_t e = launch_gemv(type, w, n, k, row_bytes, a, mc, y + m0 * n, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lbq
