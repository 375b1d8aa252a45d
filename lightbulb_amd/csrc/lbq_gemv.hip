// lbq_gemv.hip -- decode GEMV entry points: per-type dispatch and the fused-quant query.
#include "lbq_gemv_impl.hpp"

namespace lbq {

hipError_t gemv_q4k(const RowMap &, int64_t, int64_t, const ActView &, const float *, int, int, const float *, float, hipStream_t);
hipError_t gemv_q5k(const RowMap &, int64_t, int64_t, const ActView &, const float *, int, int, const float *, float, hipStream_t);
hipError_t gemv_q6k(const RowMap &, int64_t, int64_t, const ActView &, const float *, int, int, const float *, float, hipStream_t);
hipError_t gemv_q8_0(const RowMap &, int64_t, int64_t, const ActView &, const float *, int, int, const float *, float, hipStream_t);
hipError_t gemv_legacy(int, const RowMap &, int64_t, int64_t, const ActView &, const float *, int, int, const float *, float,
                       hipStream_t);
hipError_t gemv_k23(int, const RowMap &, int64_t, int64_t, const ActView &, const float *, int, int, const float *, float,
                    hipStream_t);

bool gemv_fuses_quant(int type, int64_t n, int64_t k, int m, const float *x) {
    (void)n;
    if (m < 1 || m > 8 || (reinterpret_cast<uintptr_t>(x) & 15u)) return false;
    if (m > 1) {
        // m = 2..4: the multi-row kernel quantises the x rows in its prologue (Q8_K
        // rows, at most four (row, 16-block pass) items) instead of a separate
        // quantisation launch before it.  Every workgroup quantises all its rows, so
        // with more items that repeated work outweighs the launch: measured on
        // Q5_K 14336 x 4096 at m = 2 / 4 / 8: 14.3 -> 12.0, 17.3 -> 15.6, 22.8 -> 24.0 us;
        // Q4_K 4096 x 8192 at m = 5 (a four-row chunk of two passes): 17.1 -> 21.3 us
        if (tuning().gemv1_nofuse || tuning().gemv_rows_off) return false;
        const int nbk = (int)(k / QK_K);
        int ppb, rpw, it;
        switch (type) {
        case TYPE_Q4_K:
            return fast_rows_max<TYPE_Q4_K>(nbk) >= 4 && fast_shape<TYPE_Q4_K>(nbk, &ppb, &rpw, &it, 2) && m * it <= 4;
        case TYPE_Q5_K:
            return fast_rows_max<TYPE_Q5_K>(nbk) >= 4 && fast_shape<TYPE_Q5_K>(nbk, &ppb, &rpw, &it, 2) && m * it <= 4;
        case TYPE_Q6_K:
            return fast_rows_max<TYPE_Q6_K>(nbk) >= 4 && fast_shape<TYPE_Q6_K>(nbk, &ppb, &rpw, &it, 2) && m * it <= 4;
        default: return false;
        }
    }
    // Every workgroup quantises all of x before its first dot, so the prologue
    // grows with k, but even at k = 14336 it costs less than a separate
    // quantisation launch (4096 x 14336 Q4_K: fused 10.3 us, quantise + GEMV 11.7).
    if (tuning().gemv1_nofuse) return false;  // tuning switch: always quantise separately
    const int nb = (int)(k / (type == TYPE_Q8_0 ? QK8_0 : QK_K));
    int ppb, rpw, it;
    switch (type) {
    case TYPE_Q4_K: return fast_shape<TYPE_Q4_K>(nb, &ppb, &rpw, &it);
    case TYPE_Q5_K: return fast_shape<TYPE_Q5_K>(nb, &ppb, &rpw, &it);
    case TYPE_Q6_K: return fast_shape<TYPE_Q6_K>(nb, &ppb, &rpw, &it);
    case TYPE_Q8_0: return fast_shape<TYPE_Q8_0>(nb, &ppb, &rpw, &it);
    default: return false;
    }
}

hipError_t launch_gemv(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act, int m,
                       float *y, hipStream_t st) {
    return launch_gemv_x(type, w, n, k, row_bytes, act, nullptr, m, y, st);
}

RowMap single_row_map(const uint8_t *w, int64_t n, float *y) {
    RowMap rm;
    for (int s = 0; s < GROUP_MAX; s++) {
        rm.w[s] = w;
        rm.y[s] = y;
        rm.end[s] = INT32_MAX;
    }
    rm.end[0] = (int32_t)n;
    rm.n = n;
    return rm;
}

static hipError_t dispatch(int type, const RowMap &rm, int64_t k, int64_t row_bytes, const ActView &act, const float *x,
                           int m, int map, hipStream_t st, const float *alpha = nullptr, float eps = 0.f) {
    switch (type) {
    case TYPE_Q4_K: return gemv_q4k(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q5_K: return gemv_q5k(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q6_K: return gemv_q6k(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q8_0: return gemv_q8_0(rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q4_0: case TYPE_Q4_1: case TYPE_Q5_0: case TYPE_Q5_1:
        return gemv_legacy(type, rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    case TYPE_Q2_K: case TYPE_Q3_K: return gemv_k23(type, rm, k, row_bytes, act, x, m, map, alpha, eps, st);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_x(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act,
                         const float *x, int m, float *y, hipStream_t st) {
    return dispatch(type, single_row_map(w, n, y), k, row_bytes, act, x, m, MAP_ONE, st);
}

hipError_t launch_gemv_group(int type, const RowMap &rm, int64_t k, int64_t row_bytes, const ActView &act,
                             const float *x, hipStream_t st, const float *norm_w, float eps) {
    return dispatch(type, rm, k, row_bytes, act, x, 1, MAP_SEGMENTS, st, norm_w, eps);
}

hipError_t launch_gemv_silu_pair(int type, const uint8_t *w_gate, const uint8_t *w_up, int64_t n, int64_t k,
                                 int64_t row_bytes, const float *x, float *out, hipStream_t st, const float *norm_w,
                                 float eps) {
    RowMap rm = single_row_map(w_gate, 2 * n, out);
    rm.w[1] = w_up;
    const ActView none{nullptr, nullptr, nullptr, k, 0};
    return dispatch(type, rm, k, row_bytes, none, x, 1, MAP_SILU_PAIRS, st, norm_w, eps);
}

}  // namespace lbq
