// lbq_gemv.hip -- decode GEMV (m <= 8) over GGUF blocks, fused dequant + integer dot.
//
// y[m][n] = sum_k W[n][k] * x[m][k] where x has been quantised to Q8_K (k-quant
// weights) or Q8_0 (Q8_0 weights).  Each output is built the way the reference
// CPU vec_dot builds it (candle-core 0.10.2 k_quants.rs, generic bodies of
// vec_dot for Q8_0/Q4_K/Q5_K/Q6_K): exact int32 sums of code products per
// sub-block, scaled by the integer sub-block scale, then combined in f32 with
// d_w*d_x (and, for Q4_K/Q5_K, minus dmin_w*d_x*sum(m*bsum)).  Only the f32
// summation order across blocks differs from the CPU.
//
// Work decomposition (64-lane waves, 256-thread workgroups):
//   - a "piece" is the unit one lane decodes per step: 16 bytes of 4-bit codes
//     (Q4_K/Q5_K: 32 values in two runs of 16), 32 bytes of Q6_K low bits plus
//     16 of high bits (64 values), or one Q8_0 block (32 values);
//   - a wave owns RPW weight rows; LPR = 64/RPW lanes walk each row's pieces in
//     order, so consecutive lanes read consecutive bytes of a row (coalesced);
//   - S waves of a workgroup may split one row group along k (small-n shapes),
//     combining their partial sums through LDS; no atomics, so results are
//     deterministic.
#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

template <int TYPE>
struct Dec;

// ---- Q4_K: piece p (0..7) = qs[16p .. 16p+16): c = p/2 (64-value chunk), h = p%2.
// low nibbles -> values 64c+16h+[0,16) (sub-block 2c), high -> 64c+32+16h+[0,16) (2c+1).
template <>
struct Dec<TYPE_Q4_K> {
    static constexpr int BYTES = 144, PPB = 8, VALS = 256;
    struct Raw { uint4 hdr, qs; };
    __device__ static Raw load(const uint8_t *blk, int p) {
        Raw r;
        r.hdr = ld_u4(blk);
        r.qs = ld_u4_nt(blk + 16 + 16 * p);
        return r;
    }
    template <int M>
    __device__ static void dot(const Raw &r, int64_t b, int p, const ActView &a, int mrows, float *acc) {
        const int c = p >> 1, h = p & 1;
        uint32_t sc2, m2;
        k4_scale_pair(r.hdr.y, r.hdr.z, r.hdr.w, c, &sc2, &m2);
        const int sc0 = (int)(sc2 & 0xffu), sc1 = (int)(sc2 >> 8), mn0 = (int)(m2 & 0xffu), mn1 = (int)(m2 >> 8);
        const float d = h2f(r.hdr.x & 0xffffu), dmin = h2f(r.hdr.x >> 16);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = q[i] & 0x0f0f0f0fu;
            hi[i] = (q[i] >> 4) & 0x0f0f0f0fu;
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (m < mrows) {
                const int8_t *xr = a.xq + m * a.k + b * QK_K + 64 * c + 16 * h;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xr);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xr + 32);
                int s0 = dot4(lo[0], x0.x, 0);
                s0 = dot4(lo[1], x0.y, s0);
                s0 = dot4(lo[2], x0.z, s0);
                s0 = dot4(lo[3], x0.w, s0);
                int s1 = dot4(hi[0], x1.x, 0);
                s1 = dot4(hi[1], x1.y, s1);
                s1 = dot4(hi[2], x1.z, s1);
                s1 = dot4(hi[3], x1.w, s1);
                const int64_t sb = (int64_t)m * a.nb + b;
                const uint2 bs = *reinterpret_cast<const uint2 *>(a.xbs + sb * 16 + 4 * c);
                const int b0 = (int)(int16_t)(bs.x >> (16 * h)), b1 = (int)(int16_t)(bs.y >> (16 * h));
                const int isum = sc0 * s0 + sc1 * s1;
                const int msum = mn0 * b0 + mn1 * b1;
                const float dx = a.xd[sb];
                acc[m] += (d * dx) * (float)isum - (dmin * dx) * (float)msum;
            }
        }
    }
};

// ---- Q5_K: as Q4_K with the fifth bit from qh[16h .. 16h+16): bit 2c for the low
// run, bit 2c+1 for the high run.
template <>
struct Dec<TYPE_Q5_K> {
    static constexpr int BYTES = 176, PPB = 8, VALS = 256;
    struct Raw { uint4 hdr, qh, qs; };
    __device__ static Raw load(const uint8_t *blk, int p) {
        Raw r;
        r.hdr = ld_u4(blk);
        r.qh = ld_u4(blk + 16 + 16 * (p & 1));
        r.qs = ld_u4_nt(blk + 48 + 16 * p);
        return r;
    }
    template <int M>
    __device__ static void dot(const Raw &r, int64_t b, int p, const ActView &a, int mrows, float *acc) {
        const int c = p >> 1, h = p & 1;
        uint32_t sc2, m2;
        k4_scale_pair(r.hdr.y, r.hdr.z, r.hdr.w, c, &sc2, &m2);
        const int sc0 = (int)(sc2 & 0xffu), sc1 = (int)(sc2 >> 8), mn0 = (int)(m2 & 0xffu), mn1 = (int)(m2 >> 8);
        const float d = h2f(r.hdr.x & 0xffffu), dmin = h2f(r.hdr.x >> 16);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = (q[i] & 0x0f0f0f0fu) | (((qh[i] >> (2 * c)) & 0x01010101u) << 4);
            hi[i] = ((q[i] >> 4) & 0x0f0f0f0fu) | (((qh[i] >> (2 * c + 1)) & 0x01010101u) << 4);
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (m < mrows) {
                const int8_t *xr = a.xq + m * a.k + b * QK_K + 64 * c + 16 * h;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xr);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xr + 32);
                int s0 = dot4(lo[0], x0.x, 0);
                s0 = dot4(lo[1], x0.y, s0);
                s0 = dot4(lo[2], x0.z, s0);
                s0 = dot4(lo[3], x0.w, s0);
                int s1 = dot4(hi[0], x1.x, 0);
                s1 = dot4(hi[1], x1.y, s1);
                s1 = dot4(hi[2], x1.z, s1);
                s1 = dot4(hi[3], x1.w, s1);
                const int64_t sb = (int64_t)m * a.nb + b;
                const uint2 bs = *reinterpret_cast<const uint2 *>(a.xbs + sb * 16 + 4 * c);
                const int b0 = (int)(int16_t)(bs.x >> (16 * h)), b1 = (int)(int16_t)(bs.y >> (16 * h));
                const int isum = sc0 * s0 + sc1 * s1;
                const int msum = mn0 * b0 + mn1 * b1;
                const float dx = a.xd[sb];
                acc[m] += (d * dx) * (float)isum - (dmin * dx) * (float)msum;
            }
        }
    }
};

// ---- Q6_K: piece p (0..3): n = p/2 (128-value half), h = p%2.  It covers
// ql[64n+16h..+16] (qa), ql[64n+32+16h..+16] (qb) and qh[32n+16h..+16]; its four
// runs of 16 values start at 128n+16h+32j (j = 0..3) with int8 scale 8n+h+2j:
//   j=0: qa low | qh bits 0-1;  j=1: qb low | qh bits 2-3;
//   j=2: qa high | qh bits 4-5; j=3: qb high | qh bits 6-7.
// Codes v in [0,63] go through sdot4 unshifted; q = v-32 is restored with the
// Q8_K block sums: sum (v-32)*x = sum v*x - 32*bsum.
template <>
struct Dec<TYPE_Q6_K> {
    static constexpr int BYTES = 210, PPB = 4, VALS = 256;
    struct Raw { uint32_t qa[4], qb[4], qh[4], s0, s1, dbits; };
    __device__ static Raw load(const uint8_t *blk, int p) {
        const int n = p >> 1, h = p & 1;
        Raw r;
        ld16_a2(blk + 64 * n + 16 * h, r.qa);
        ld16_a2(blk + 64 * n + 32 + 16 * h, r.qb);
        ld16_a2(blk + 128 + 32 * n + 16 * h, r.qh);
        r.s0 = ld4_a2(blk + 192 + 8 * n);
        r.s1 = ld4_a2(blk + 196 + 8 * n);
        r.dbits = ld2_a2(blk + 208);
        return r;
    }
    template <int M>
    __device__ static void dot(const Raw &r, int64_t b, int p, const ActView &a, int mrows, float *acc) {
        const int n = p >> 1, h = p & 1;
        const float d = h2f(r.dbits);
        const int sh = 8 * h;
        const int sc[4] = {(int)(int8_t)(r.s0 >> sh), (int)(int8_t)(r.s0 >> (sh + 16)), (int)(int8_t)(r.s1 >> sh),
                           (int)(int8_t)(r.s1 >> (sh + 16))};
        uint32_t v[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[0][i] = (r.qa[i] & 0x0f0f0f0fu) | ((r.qh[i] & 0x03030303u) << 4);
            v[1][i] = (r.qb[i] & 0x0f0f0f0fu) | (((r.qh[i] >> 2) & 0x03030303u) << 4);
            v[2][i] = ((r.qa[i] >> 4) & 0x0f0f0f0fu) | (((r.qh[i] >> 4) & 0x03030303u) << 4);
            v[3][i] = ((r.qb[i] >> 4) & 0x0f0f0f0fu) | (((r.qh[i] >> 6) & 0x03030303u) << 4);
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (m < mrows) {
                const int8_t *xr = a.xq + m * a.k + b * QK_K + 128 * n + 16 * h;
                const int64_t sb = (int64_t)m * a.nb + b;
                const uint4 bs = *reinterpret_cast<const uint4 *>(a.xbs + sb * 16 + 8 * n);
                const uint32_t bsw[4] = {bs.x, bs.y, bs.z, bs.w};
                int isum = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint4 xv = *reinterpret_cast<const uint4 *>(xr + 32 * j);
                    int s = dot4(v[j][0], xv.x, 0);
                    s = dot4(v[j][1], xv.y, s);
                    s = dot4(v[j][2], xv.z, s);
                    s = dot4(v[j][3], xv.w, s);
                    const int bsum = (int)(int16_t)(bsw[j] >> (16 * h));
                    isum += sc[j] * (s - 32 * bsum);
                }
                acc[m] += (d * a.xd[sb]) * (float)isum;
            }
        }
    }
};

// ---- Q8_0: piece = one 34-byte block (2-byte aligned): 9 aligned dwords cover it.
template <>
struct Dec<TYPE_Q8_0> {
    static constexpr int BYTES = 34, PPB = 1, VALS = 32;
    struct Raw { uint32_t w[9]; uint32_t mis; };
    __device__ static Raw load(const uint8_t *blk, int) {
        Raw r;
        const uintptr_t ad = reinterpret_cast<uintptr_t>(blk);
        r.mis = (uint32_t)(ad & 3u);
        const uint8_t *base = reinterpret_cast<const uint8_t *>(ad & ~(uintptr_t)3);
        const u32x4a4 a0 = *reinterpret_cast<const u32x4a4 *>(base);
        const u32x4a4 a1 = *reinterpret_cast<const u32x4a4 *>(base + 16);
        r.w[0] = a0.x; r.w[1] = a0.y; r.w[2] = a0.z; r.w[3] = a0.w;
        r.w[4] = a1.x; r.w[5] = a1.y; r.w[6] = a1.z; r.w[7] = a1.w;
        r.w[8] = *reinterpret_cast<const uint32_t *>(base + 32);
        return r;
    }
    template <int M>
    __device__ static void dot(const Raw &r, int64_t b, int, const ActView &a, int mrows, float *acc) {
        const bool odd = r.mis != 0;  // block starts 2 bytes into a dword
        const float d = h2f(odd ? (r.w[0] >> 16) : (r.w[0] & 0xffffu));
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = odd ? r.w[i + 1] : __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (m < mrows) {
                const int8_t *xr = a.xq + m * a.k + b * QK8_0;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xr);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xr + 16);
                int s = dot4(q[0], x0.x, 0);
                s = dot4(q[1], x0.y, s);
                s = dot4(q[2], x0.z, s);
                s = dot4(q[3], x0.w, s);
                s = dot4(q[4], x1.x, s);
                s = dot4(q[5], x1.y, s);
                s = dot4(q[6], x1.z, s);
                s = dot4(q[7], x1.w, s);
                acc[m] += ((float)s * d) * a.xd[(int64_t)m * a.nb + b];
            }
        }
    }
};

// ---------------------------------------------------------------------------
// The GEMV kernel.  Grid: one workgroup per RPW*(4/S) weight rows.
// ---------------------------------------------------------------------------
template <int TYPE, int M, int RPW, int S, int U>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t *__restrict__ W, int64_t n_rows, int64_t row_bytes, int nb,
                                              ActView act, int mrows, float *__restrict__ y) {
    using D = Dec<TYPE>;
    constexpr int LPR = 64 / RPW;
    constexpr int RG = 4 / S;
    constexpr int STEP = S * LPR;
    static_assert(LPR >= 1 && RG >= 1, "bad config");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rg = wave / S, ks = wave % S;
    const int r = lane / LPR, li = lane % LPR;
    const int64_t row = ((int64_t)blockIdx.x * RG + rg) * RPW + r;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.f;
    if (row < n_rows) {
        const uint8_t *wrow = W + row * row_bytes;
        const int P = nb * D::PPB;
        int q = ks * LPR + li;
        for (; q + (U - 1) * STEP < P; q += U * STEP) {
            typename D::Raw raw[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int qq = q + u * STEP;
                raw[u] = D::load(wrow + (int64_t)(qq / D::PPB) * D::BYTES, qq % D::PPB);
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int qq = q + u * STEP;
                D::template dot<M>(raw[u], qq / D::PPB, qq % D::PPB, act, mrows, acc);
            }
        }
        for (; q < P; q += STEP) {
            const typename D::Raw raw = D::load(wrow + (int64_t)(q / D::PPB) * D::BYTES, q % D::PPB);
            D::template dot<M>(raw, q / D::PPB, q % D::PPB, act, mrows, acc);
        }
    }
    // reduce over the LPR lanes of each row (lanes r*LPR .. r*LPR+LPR-1)
#pragma unroll
    for (int m = 0; m < M; m++) {
#pragma unroll
        for (int off = LPR / 2; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off);
    }
    if constexpr (S == 1) {
        if (li == 0 && row < n_rows) {
#pragma unroll
            for (int m = 0; m < M; m++)
                if (m < mrows) y[(int64_t)m * n_rows + row] = acc[m];
        }
    } else {
        __shared__ float red[RG][S][RPW][M];
        if (li == 0) {
#pragma unroll
            for (int m = 0; m < M; m++) red[rg][ks][r][m] = acc[m];
        }
        __syncthreads();
        if (ks == 0 && li == 0 && row < n_rows) {
#pragma unroll
            for (int m = 0; m < M; m++) {
                float s = red[rg][0][r][m];
#pragma unroll
                for (int t = 1; t < S; t++) s += red[rg][t][r][m];
                if (m < mrows) y[(int64_t)m * n_rows + row] = s;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
template <int TYPE, int M, int RPW, int S, int U>
static void run(const uint8_t *w, int64_t n, int64_t row_bytes, int nb, const ActView &act, int mrows, float *y,
                hipStream_t st) {
    constexpr int ROWS_PER_WG = RPW * (4 / S);
    const dim3 grid((unsigned)((n + ROWS_PER_WG - 1) / ROWS_PER_WG));
    k_gemv<TYPE, M, RPW, S, U><<<grid, 256, 0, st>>>(w, n, row_bytes, nb, act, mrows, y);
}

template <int TYPE, int M, int RPW>
static void run_s(int S, const uint8_t *w, int64_t n, int64_t row_bytes, int nb, const ActView &act, int mrows,
                  float *y, hipStream_t st) {
    constexpr int U = M <= 2 ? 2 : 1;
    if (S == 4) run<TYPE, M, RPW, 4, U>(w, n, row_bytes, nb, act, mrows, y, st);
    else if (S == 2) run<TYPE, M, RPW, 2, U>(w, n, row_bytes, nb, act, mrows, y, st);
    else run<TYPE, M, RPW, 1, U>(w, n, row_bytes, nb, act, mrows, y, st);
}

template <int TYPE, int RPW>
static void run_m(int S, const uint8_t *w, int64_t n, int64_t row_bytes, int nb, const ActView &act, int m, float *y,
                  hipStream_t st) {
    if (m <= 1) run_s<TYPE, 1, RPW>(S, w, n, row_bytes, nb, act, m, y, st);
    else if (m <= 2) run_s<TYPE, 2, RPW>(S, w, n, row_bytes, nb, act, m, y, st);
    else if (m <= 4) run_s<TYPE, 4, RPW>(S, w, n, row_bytes, nb, act, m, y, st);
    else run_s<TYPE, 8, RPW>(S, w, n, row_bytes, nb, act, m, y, st);
}

// Pick the k-split so that the launch has enough waves to cover 256 CUs, but
// never split a row into slices of fewer than ~4 pieces per lane.
static int pick_split(int64_t n, int rpw, int pieces_per_row, int lpr) {
    const int64_t waves1 = (n + rpw - 1) / rpw;
    int s = 1;
    while (s < 4 && waves1 * s < 4096 && pieces_per_row / (lpr * s * 2) >= 2) s *= 2;
    return s;
}

hipError_t launch_gemv(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act, int m,
                       float *y, hipStream_t st) {
    switch (type) {
    case TYPE_Q4_K: {
        const int nb = (int)(k / QK_K);
        run_m<TYPE_Q4_K, 8>(pick_split(n, 8, nb * 8, 8), w, n, row_bytes, nb, act, m, y, st);
        break;
    }
    case TYPE_Q5_K: {
        const int nb = (int)(k / QK_K);
        run_m<TYPE_Q5_K, 8>(pick_split(n, 8, nb * 8, 8), w, n, row_bytes, nb, act, m, y, st);
        break;
    }
    case TYPE_Q6_K: {
        const int nb = (int)(k / QK_K);
        run_m<TYPE_Q6_K, 16>(pick_split(n, 16, nb * 4, 4), w, n, row_bytes, nb, act, m, y, st);
        break;
    }
    case TYPE_Q8_0: {
        const int nb = (int)(k / QK8_0);
        run_m<TYPE_Q8_0, 8>(pick_split(n, 8, nb, 8), w, n, row_bytes, nb, act, m, y, st);
        break;
    }
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lbq
