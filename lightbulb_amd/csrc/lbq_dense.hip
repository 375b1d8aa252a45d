// lbq_dense.hip -- QMatMul over dense F32 / F16 / BF16 weights.
//
// candle's QMatMul::from_qtensor does not keep F32 / F16 / BF16 tensors
// quantised: it dequantises them (F16 and BF16 widened exactly to f32) and forward is a
// plain f32 matmul, y = x . W^T (the dense variant; the reference reaches it for
// whatever type output.weight or a projection has, custom_transformer.rs:360-363,
// custom_attention.rs:195-206, mlp_wrapper.rs:127-135).  Here the weight stays
// in its file layout ([n][k], f16, bf16 or f32) and is widened on the fly:
//   m <= 8  k_dense_gemv: waves stream weight rows in 4096-column units with
//           the next unit's 16-byte loads in flight, x staged in LDS, f32 FMA
//           against up to 8 activation rows, DPP row sums -- HBM-bound like the
//           quantised decode GEMV;
//   m > 8   k_dense_gemm: 64 x 128 output tiles on v_mfma_f32_32x32x2_f32
//           (f32 operands, f32 accumulation), operands staged through LDS.
// Both compute in f32 throughout; only the summation order differs from
// candle's, so results agree to f32 rounding (~1e-6 relative on a row).
#include <algorithm>

#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

typedef float floatx16 __attribute__((ext_vector_type(16)));

// 8 consecutive weights of row `row` at column c (c % 8 == 0) widened to f32
template <bool F16, bool BF = false>
__device__ __forceinline__ void load_w8(const uint8_t *row, int64_t c, float w[8]) {
    if constexpr (F16) {
        const uint4 v = *reinterpret_cast<const uint4 *>(row + 2 * c);
        const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            w[2 * i] = w16<BF>(d[i] & 0xffffu);
            w[2 * i + 1] = w16<BF>(d[i] >> 16);
        }
    } else {
        const float4 a = *reinterpret_cast<const float4 *>(row + 4 * c);
        const float4 b = *reinterpret_cast<const float4 *>(row + 4 * c + 16);
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
    }
}

// ---------------------------------------------------------------------------
// m <= 8.  Waves take rows gw, gw + nw, ...; a row is cut into units of 512 UN
// columns (a lane covers 8 consecutive columns per 512-column step; k % 8 == 0,
// a partial last step is masked), and each wave keeps the next unit's weight
// loads in flight while it computes the current one.  With XL the x rows are
// staged in LDS once per workgroup (m k f32 <= 64 KB), else every wave reads
// them through the caches.
// ---------------------------------------------------------------------------
// 8 consecutive values of x at c (vec: 16-byte aligned, else four-byte loads)
__device__ __forceinline__ void load_x8(const float *p, bool vec, float v[8]) {
    load4f(p, vec, v);
    load4f(p + 4, vec, v + 4);
}

constexpr int DENSE_XL_BYTES = 65536;  // x staged in LDS up to this size

template <bool F16>
struct DenseUnit {
    static constexpr int UN = 8;  // 4096 f16 / 4096 f32 weights of a row per unit and wave
    uint4 w[F16 ? UN : 2 * UN];
};

template <bool F16, int MR, bool XL, bool BF = false>
__global__ __launch_bounds__(256) void k_dense_gemv(const uint8_t *__restrict__ W, int64_t N, int64_t K,
                                                    const float *__restrict__ x, int m, float *__restrict__ y) {
    extern __shared__ __align__(16) float xs[];  // XL: x [m][K]
    const bool xv = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;  // K % 8 == 0: every row likewise
    constexpr int UN = DenseUnit<F16>::UN;
    constexpr int64_t WB = F16 ? 2 : 4, CH = 512 * UN;
    const int t = threadIdx.x, lane = t & 63;
    if constexpr (XL) {
        const int64_t total = (int64_t)m * K;
        if (xv) {
            for (int64_t i = 4 * t; i < total; i += 1024)
                *reinterpret_cast<float4 *>(xs + i) = *reinterpret_cast<const float4 *>(x + i);
        } else {
            for (int64_t i = t; i < total; i += 256) xs[i] = x[i];
        }
        __syncthreads();
    }
    const int64_t gw = (int64_t)blockIdx.x * 4 + (t >> 6), nw = (int64_t)gridDim.x * 4;
    const int64_t nch = (K + CH - 1) / CH;
    const int64_t rows = gw < N ? (N - gw + nw - 1) / nw : 0, units = rows * nch;
    auto load = [&](int64_t u, DenseUnit<F16> &d) {
        const uint8_t *row = W + (gw + (u / nch) * nw) * K * WB;
        const int64_t c0 = (u % nch) * CH;
#pragma unroll
        for (int v = 0; v < UN; v++) {
            const int64_t c = c0 + 512 * v + 8 * lane;
            if constexpr (F16) {
                d.w[v] = c < K ? *reinterpret_cast<const uint4 *>(row + 2 * c) : make_uint4(0, 0, 0, 0);
            } else {
                d.w[2 * v] = c < K ? *reinterpret_cast<const uint4 *>(row + 4 * c) : make_uint4(0, 0, 0, 0);
                d.w[2 * v + 1] = c < K ? *reinterpret_cast<const uint4 *>(row + 4 * c + 16) : make_uint4(0, 0, 0, 0);
            }
        }
    };
    float acc[MR];
#pragma unroll
    for (int i = 0; i < MR; i++) acc[i] = 0.f;
    auto compute = [&](int64_t u, const DenseUnit<F16> &d) {
        const int64_t c0 = (u % nch) * CH;
#pragma unroll
        for (int v = 0; v < UN; v++) {
            const int64_t c = c0 + 512 * v + 8 * lane;
            if (c >= K) continue;
            float w[8];
            if constexpr (F16) {
                const uint32_t dw[4] = {d.w[v].x, d.w[v].y, d.w[v].z, d.w[v].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    w[2 * e] = w16<BF>(dw[e] & 0xffffu);
                    w[2 * e + 1] = w16<BF>(dw[e] >> 16);
                }
            } else {
                const uint4 a = d.w[2 * v], b = d.w[2 * v + 1];
                w[0] = __uint_as_float(a.x); w[1] = __uint_as_float(a.y); w[2] = __uint_as_float(a.z); w[3] = __uint_as_float(a.w);
                w[4] = __uint_as_float(b.x); w[5] = __uint_as_float(b.y); w[6] = __uint_as_float(b.z); w[7] = __uint_as_float(b.w);
            }
#pragma unroll
            for (int i = 0; i < MR; i++) {
                if (i < m) {
                    float xv8[8];
                    if constexpr (XL) {
                        const float4 p = *reinterpret_cast<const float4 *>(xs + (int64_t)i * K + c);
                        const float4 q = *reinterpret_cast<const float4 *>(xs + (int64_t)i * K + c + 4);
                        xv8[0] = p.x; xv8[1] = p.y; xv8[2] = p.z; xv8[3] = p.w;
                        xv8[4] = q.x; xv8[5] = q.y; xv8[6] = q.z; xv8[7] = q.w;
                    } else {
                        load_x8(x + (int64_t)i * K + c, xv, xv8);
                    }
#pragma unroll
                    for (int e = 0; e < 8; e++) acc[i] = fmaf(w[e], xv8[e], acc[i]);
                }
            }
        }
        if (u % nch == nch - 1) {  // the row's last unit: its sums
            const int64_t r = gw + (u / nch) * nw;
#pragma unroll
            for (int i = 0; i < MR; i++) {
                if (i < m) {
                    const float s = row_sum_f32(acc[i]);
                    const float tt = __int_as_float(rl(__float_as_uint(s), 0)) + __int_as_float(rl(__float_as_uint(s), 16)) +
                                     __int_as_float(rl(__float_as_uint(s), 32)) + __int_as_float(rl(__float_as_uint(s), 48));
                    if (lane == 0) y[(int64_t)i * N + r] = tt;
                }
                acc[i] = 0.f;
            }
        }
    };
    DenseUnit<F16> ring[2];
    if (units > 0) load(0, ring[0]);
    for (int64_t u = 0; u < units; u += 2) {
        if (u + 1 < units) load(u + 1, ring[1]);
        compute(u, ring[0]);
        if (u + 1 >= units) break;
        if (u + 2 < units) load(u + 2, ring[0]);
        compute(u + 1, ring[1]);
    }
}

// ---------------------------------------------------------------------------
// m > 8.  Workgroup tile 64 (m) x 128 (n), four waves; wave w owns columns
// 32w..32w+31 for all 64 rows (two 32 x 32 MFMA tiles that share the B operand).
// k advances in stages of 64: x [64][64] and W [128][64] (f16 widened) are stored
// k-major into LDS (row stride padded), then 32 k-steps of
// v_mfma_f32_32x32x2_f32: lane l supplies A[row l%32][k 2s + l/32] and
// B[k 2s + l/32][column l%32].  The next stage's global loads are issued into
// registers before the current stage's MFMAs, so their latency hides behind 64
// MFMAs (F16 4096^2 at M = 512: 276 -> 254 us against 32-deep stages loaded
// after the previous stage's MFMAs).  Out-of-range rows, columns and k read as
// zero.
// ---------------------------------------------------------------------------
constexpr int DBM = 64, DBN = 128, DBK = 64;

template <bool F16>
struct DenseStage {
    float4 x[4];                    // x rows (t / 16) + 16 j, k 4 (t % 16)
    uint4 w[F16 ? 4 : 8];           // W rows (t / 8) + 32 j, k 8 (t % 8): f16 x 8, or f32 x 8 as two
};

template <bool F16, bool BF = false>
__global__ __launch_bounds__(256) void k_dense_gemm(const uint8_t *__restrict__ W, int64_t N, int64_t K,
                                                    const float *__restrict__ x, int64_t M, float *__restrict__ y) {
    __shared__ float As[DBK][DBM + 4];
    __shared__ float Bs[DBK][DBN + 4];
    constexpr int64_t WB = F16 ? 2 : 4;
    const bool xv = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, h = lane >> 5, lr = lane & 31;
    const int64_t m0 = (int64_t)blockIdx.y * DBM, n0 = (int64_t)blockIdx.x * DBN;
    floatx16 acc[2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[i][v] = 0.f;
    auto load = [&](int64_t k0, DenseStage<F16> &g) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = (t >> 4) + 16 * j, kk = 4 * (t & 15);
            float v[4] = {0.f, 0.f, 0.f, 0.f};
            if (m0 + r < M && k0 + kk < K) load4f(x + (m0 + r) * K + k0 + kk, xv, v);
            g.x[j] = make_float4(v[0], v[1], v[2], v[3]);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = (t >> 3) + 32 * j, kk = 8 * (t & 7);
            const bool ok = n0 + r < N && k0 + kk < K;
            const uint8_t *src = W + (n0 + r) * K * WB + (k0 + kk) * WB;
            if constexpr (F16) {
                g.w[j] = ok ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0, 0, 0, 0);
            } else {
                g.w[2 * j] = ok ? *reinterpret_cast<const uint4 *>(src) : make_uint4(0, 0, 0, 0);
                g.w[2 * j + 1] = ok ? *reinterpret_cast<const uint4 *>(src + 16) : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto store = [&](const DenseStage<F16> &g) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = (t >> 4) + 16 * j, kk = 4 * (t & 15);
            As[kk][r] = g.x[j].x; As[kk + 1][r] = g.x[j].y; As[kk + 2][r] = g.x[j].z; As[kk + 3][r] = g.x[j].w;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int r = (t >> 3) + 32 * j, kk = 8 * (t & 7);
            float w[8];
            if constexpr (F16) {
                const uint32_t d[4] = {g.w[j].x, g.w[j].y, g.w[j].z, g.w[j].w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    w[2 * e] = w16<BF>(d[e] & 0xffffu);
                    w[2 * e + 1] = w16<BF>(d[e] >> 16);
                }
            } else {
                const uint4 a = g.w[2 * j], b = g.w[2 * j + 1];
                w[0] = __uint_as_float(a.x); w[1] = __uint_as_float(a.y); w[2] = __uint_as_float(a.z); w[3] = __uint_as_float(a.w);
                w[4] = __uint_as_float(b.x); w[5] = __uint_as_float(b.y); w[6] = __uint_as_float(b.z); w[7] = __uint_as_float(b.w);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) Bs[kk + e][r] = w[e];
        }
    };
    DenseStage<F16> g;
    load(0, g);
    store(g);
    __syncthreads();
    for (int64_t k0 = 0; k0 < K; k0 += DBK) {
        const bool more = k0 + DBK < K;
        if (more) load(k0 + DBK, g);  // in flight during this stage's MFMAs
#pragma unroll
        for (int s = 0; s < DBK / 2; s++) {
            const float b = Bs[2 * s + h][32 * wave + lr];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float a = As[2 * s + h][32 * i + lr];
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[i], 0, 0, 0);
            }
        }
        __syncthreads();
        if (more) {
            store(g);
            __syncthreads();
        }
    }
    // D layout of a 32 x 32 tile: lane holds column l%32, rows 8(v/4) + 4h + v%4
    const int64_t n = n0 + 32 * wave + lr;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int64_t m = m0 + 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
            if (m < M && n < N) y[m * N + n] = acc[i][v];
        }
}

template <bool F16, bool BF = false>
static hipError_t dense_typed(const uint8_t *w, int64_t n, int64_t k, const float *x, int64_t m, float *y,
                              hipStream_t st) {
    if (m <= 8) {
        const int64_t waves = std::min<int64_t>(n, (int64_t)num_cus() * 8);
        const unsigned grid = (unsigned)((waves + 3) / 4);
        const int mi = (int)m;
        const size_t xb = (size_t)m * (size_t)k * 4;
        const bool xl = xb <= DENSE_XL_BYTES;
        const size_t lds = xl ? xb : 0;
#define LBQ_DG(MR)                                                                    \
    {                                                                                 \
        if (xl) k_dense_gemv<F16, MR, true, BF><<<grid, 256, lds, st>>>(w, n, k, x, mi, y); \
        else k_dense_gemv<F16, MR, false, BF><<<grid, 256, 0, st>>>(w, n, k, x, mi, y);     \
    }
        if (m == 1) LBQ_DG(1) else if (m <= 2) LBQ_DG(2) else if (m <= 4) LBQ_DG(4) else LBQ_DG(8)
#undef LBQ_DG
        return hipGetLastError();
    }
    const dim3 grid((unsigned)((n + DBN - 1) / DBN), (unsigned)((m + DBM - 1) / DBM));
    k_dense_gemm<F16, BF><<<grid, 256, 0, st>>>(w, n, k, x, m, y);
    return hipGetLastError();
}

hipError_t launch_dense(int type, const uint8_t *w, int64_t n, int64_t k, const float *x, int64_t m, float *y,
                        hipStream_t st) {
    if (k % 8 || m > 65535LL * DBM) return hipErrorInvalidValue;
    if (type == TYPE_F16) return dense_typed<true>(w, n, k, x, m, y, st);
    if (type == TYPE_F32) return dense_typed<false>(w, n, k, x, m, y, st);
    if (type == TYPE_BF16) return dense_typed<true, true>(w, n, k, x, m, y, st);
    return hipErrorInvalidValue;
}

}  // namespace lbq
