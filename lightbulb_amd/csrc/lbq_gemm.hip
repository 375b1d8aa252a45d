// lbq_gemm.hip -- batched path (m > 8): k-quant weight tiles dequantised into LDS,
// multiplied on MFMA.
//
// y[m][n] = sum_b d_x[m][b] * sum_{k in block b} q8[m][k] * w[n][k]
//   q8, d_x : the Q8_K activation codes and block scales (as the reference
//             quantises them); the codes are integers in [-128, 127], exact in fp16;
//   w       : the weight dequantised as the reference does it (d*sc)*q - dmin*m in
//             f32, rounded once to fp16 (relative error <= 2^-11 per weight).
// Each 256-value block is accumulated on v_mfma_f32_32x32x16_f16 into its own
// accumulator, which is then scaled by d_x[m][b] and added to the total.  The
// only differences from the reference's integer path are that one rounding of w
// and f32 summation order (about 3e-4 relative on a row).
//
// Tiles: BM x BN = 128 x 128 outputs per 256-thread workgroup, BK = 64 values
// of k per step (a quarter of a block), four waves each owning 64 x 64 outputs
// as 2 x 2 MFMA tiles of 32 x 32.  LDS is double-buffered: while the MFMAs run
// on one step, the next step's weight bytes and codes are already in registers,
// and are dequantised into the other buffer afterwards.
#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 128, GBN = 128, GBK = 64;
constexpr int GLD = GBK + 8;  // LDS row stride in halfs (144 bytes: conflict-free b128 reads)

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    const half2v h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
}

// byte I of v as f32 (the compiler emits v_cvt_f32_ubyteI)
template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t v) { return (float)((v >> (8 * I)) & 0xffu); }

// 4 int8 codes (one dword) -> 4 exact fp16 values (two dwords): byte u = q ^ 0x80 is
// placed in the mantissa of 1024.0 (0x6400 | u = 1024 + u), then 1152 is subtracted.
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, uint32_t *lo, uint32_t *hi) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const half2v bias = {(_Float16)-1152.f, (_Float16)-1152.f};
    *lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, a) + bias);
    *hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, b) + bias);
}

// ---------------------------------------------------------------------------
// Weight staging: one thread owns 32 consecutive values of a row inside the
// step's 64-value window: values 64*kk + 32*hf + [0, 32) of block b.
// ---------------------------------------------------------------------------
template <int TYPE>
struct GemmW;

template <int TYPE>
struct GemmWK45 {
    static constexpr int BYTES = TYPE == TYPE_Q4_K ? 144 : 176;
    struct Raw { uint4 hdr, q0, q1, h0, h1; };
    __device__ static Raw load(const uint8_t *blk, int kk, int hf) {
        (void)hf;
        Raw r;
        r.hdr = ld_u4(blk);
        const uint8_t *qs = blk + (TYPE == TYPE_Q4_K ? 16 : 48) + 32 * kk;
        r.q0 = ld_u4(qs);
        r.q1 = ld_u4(qs + 16);
        if (TYPE == TYPE_Q5_K) {
            r.h0 = ld_u4(blk + 16);
            r.h1 = ld_u4(blk + 32);
        }
        return r;
    }
    // 32 dequantised values -> 16 packed fp16 pairs
    __device__ static void deq(const Raw &r, int kk, int hf, uint32_t out[16]) {
        uint32_t sc2, m2;
        k4_scale_pair(r.hdr.y, r.hdr.z, r.hdr.w, kk, &sc2, &m2);
        const uint32_t sc = hf ? (sc2 >> 8) : (sc2 & 0xffu);
        const uint32_t mn = hf ? (m2 >> 8) : (m2 & 0xffu);
        const float d1 = h2f(r.hdr.x & 0xffffu) * (float)sc;
        const float m1 = h2f(r.hdr.x >> 16) * (float)mn;
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t qh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            uint32_t v = hf ? ((q[i] >> 4) & 0x0f0f0f0fu) : (q[i] & 0x0f0f0f0fu);
            if (TYPE == TYPE_Q5_K) v |= ((qh[i] >> (2 * kk + hf)) & 0x01010101u) << 4;
            const float f0 = d1 * ubyte_f32<0>(v) - m1;
            const float f1 = d1 * ubyte_f32<1>(v) - m1;
            const float f2 = d1 * ubyte_f32<2>(v) - m1;
            const float f3 = d1 * ubyte_f32<3>(v) - m1;
            out[2 * i] = pack_f16x2(f0, f1);
            out[2 * i + 1] = pack_f16x2(f2, f3);
        }
    }
};
template <> struct GemmW<TYPE_Q4_K> : GemmWK45<TYPE_Q4_K> {};
template <> struct GemmW<TYPE_Q5_K> : GemmWK45<TYPE_Q5_K> {};

// Q6_K: window values 64*kk + 32*hf + l (l < 32) are 128n + 32s + l with n = kk/2,
// s = 2*(kk%2) + hf: low bits from ql[64n + 32*(s%2) + l] (nibble s/2), high bits
// from qh[32n + l] (bits 2s, 2s+1), scale index 8n + 2s + l/16.
template <>
struct GemmW<TYPE_Q6_K> {
    static constexpr int BYTES = 210;
    struct Raw { uint32_t ql[8], qh[8], sc, dbits; };
    __device__ static Raw load(const uint8_t *blk, int kk, int hf) {
        const int n = kk >> 1, s = 2 * (kk & 1) + hf;
        Raw r;
        ld16_a2(blk + 64 * n + 32 * (s & 1), r.ql);
        ld16_a2(blk + 64 * n + 32 * (s & 1) + 16, r.ql + 4);
        ld16_a2(blk + 128 + 32 * n, r.qh);
        ld16_a2(blk + 128 + 32 * n + 16, r.qh + 4);
        r.sc = ld4_a2(blk + 192 + 8 * n + 2 * s);
        r.dbits = ld2_a2(blk + 208);
        return r;
    }
    __device__ static void deq(const Raw &r, int kk, int hf, uint32_t out[16]) {
        const int s = 2 * (kk & 1) + hf;
        const float d = h2f(r.dbits);
        const float d1a = d * (float)(int8_t)(r.sc & 0xffu);        // l < 16
        const float d1b = d * (float)(int8_t)((r.sc >> 8) & 0xffu); // l >= 16
        const int shq = 4 * (s >> 1), shh = 2 * s;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t v = ((r.ql[i] >> shq) & 0x0f0f0f0fu) | (((r.qh[i] >> shh) & 0x03030303u) << 4);
            const float d1 = i < 4 ? d1a : d1b;
            const float f0 = d1 * (ubyte_f32<0>(v) - 32.f);
            const float f1 = d1 * (ubyte_f32<1>(v) - 32.f);
            const float f2 = d1 * (ubyte_f32<2>(v) - 32.f);
            const float f3 = d1 * (ubyte_f32<3>(v) - 32.f);
            out[2 * i] = pack_f16x2(f0, f1);
            out[2 * i + 1] = pack_f16x2(f2, f3);
        }
    }
};

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ __launch_bounds__(256, 2) void k_gemm(const uint8_t *__restrict__ W, int64_t N, int64_t row_bytes,
                                                 ActView act, int64_t M, float *__restrict__ y) {
    using GW = GemmW<TYPE>;
    __shared__ __align__(16) _Float16 As[2][GBM][GLD];
    __shared__ __align__(16) _Float16 Bs[2][GBN][GLD];
    __shared__ float Xd[2][GBM];

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wm = wave & 1, wn = wave >> 1;
    const int64_t m0 = (int64_t)blockIdx.x * GBM, n0 = (int64_t)blockIdx.y * GBN;
    const int nb = act.nb;
    const int steps = nb * 4;

    // staging roles: row t/2 of the tile, half hf = t%2 of the 64-value window
    const int srow = t >> 1, hf = t & 1;
    const int64_t am = min(m0 + srow, M - 1);  // clamped: loads stay in range
    const int64_t wn_row = min(n0 + srow, N - 1);
    const int8_t *arow = act.xq + am * act.k;
    const uint8_t *wrow = W + wn_row * row_bytes;

    uint4 ra0, ra1;
    typename GW::Raw rw;
    float rxd = 0.f;
    auto load_step = [&](int s) {
        const int b = s >> 2, kk = s & 3;
        const int8_t *ap = arow + (int64_t)s * GBK + 32 * hf;
        ra0 = *reinterpret_cast<const uint4 *>(ap);
        ra1 = *reinterpret_cast<const uint4 *>(ap + 16);
        rw = GW::load(wrow + (int64_t)b * GW::BYTES, kk, hf);
        if (t < GBM) rxd = act.xd[min(m0 + t, M - 1) * nb + b];
    };
    auto store_step = [&](int s, int buf) {
        const int kk = s & 3;
        uint32_t a16[16];
        const uint32_t aw[8] = {ra0.x, ra0.y, ra0.z, ra0.w, ra1.x, ra1.y, ra1.z, ra1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) i8x4_to_f16(aw[i], &a16[2 * i], &a16[2 * i + 1]);
        uint4 *adst = reinterpret_cast<uint4 *>(&As[buf][srow][32 * hf]);
#pragma unroll
        for (int i = 0; i < 4; i++) adst[i] = make_uint4(a16[4 * i], a16[4 * i + 1], a16[4 * i + 2], a16[4 * i + 3]);
        uint32_t w16[16];
        GW::deq(rw, kk, hf, w16);
        uint4 *bdst = reinterpret_cast<uint4 *>(&Bs[buf][srow][32 * hf]);
#pragma unroll
        for (int i = 0; i < 4; i++) bdst[i] = make_uint4(w16[4 * i], w16[4 * i + 1], w16[4 * i + 2], w16[4 * i + 3]);
        if (kk == 0 && t < GBM) Xd[(s >> 2) & 1][t] = rxd;
    };

    floatx16 acc[2][2], blk[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    load_step(0);
    store_step(0, 0);
    __syncthreads();

    const int lr = lane & 31, lk = 8 * (lane >> 5);
    for (int s = 0; s < steps; s++) {
        const int buf = s & 1;
        if (s + 1 < steps) load_step(s + 1);
        if ((s & 3) == 0) {
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int v = 0; v < 16; v++) blk[i][j][v] = 0.f;
        }
#pragma unroll
        for (int ks = 0; ks < GBK / 16; ks++) {
            half8 a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++)
                a[i] = *reinterpret_cast<const half8 *>(&As[buf][64 * wm + 32 * i + lr][16 * ks + lk]);
#pragma unroll
            for (int j = 0; j < 2; j++)
                b[j] = *reinterpret_cast<const half8 *>(&Bs[buf][64 * wn + 32 * j + lr][16 * ks + lk]);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) blk[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], b[j], blk[i][j], 0, 0, 0);
        }
        if ((s & 3) == 3) {
            // block done: scale by the activation block scale of each output row
            const float *xd = Xd[(s >> 2) & 1];
#pragma unroll
            for (int i = 0; i < 2; i++) {
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const float sx = xd[64 * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3)];
#pragma unroll
                    for (int j = 0; j < 2; j++) acc[i][j][v] += blk[i][j][v] * sx;
                }
            }
        }
        if (s + 1 < steps) store_step(s + 1, buf ^ 1);
        __syncthreads();
    }

    // write y[m][n]: for a fixed v, lanes 0..31 cover 32 consecutive n
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int64_t m = m0 + 64 * wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int64_t n = n0 + 64 * wn + 32 * j + lr;
                if (m < M && n < N) y[m * N + n] = acc[i][j][v];
            }
        }
    }
}

hipError_t launch_gemm(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act,
                       int64_t m, float *y, hipStream_t st) {
    if (type == TYPE_Q4_K || type == TYPE_Q5_K || type == TYPE_Q6_K) {
        const dim3 grid((unsigned)((m + GBM - 1) / GBM), (unsigned)((n + GBN - 1) / GBN));
        switch (type) {
        case TYPE_Q4_K: k_gemm<TYPE_Q4_K><<<grid, 256, 0, st>>>(w, n, row_bytes, act, m, y); break;
        case TYPE_Q5_K: k_gemm<TYPE_Q5_K><<<grid, 256, 0, st>>>(w, n, row_bytes, act, m, y); break;
        case TYPE_Q6_K: k_gemm<TYPE_Q6_K><<<grid, 256, 0, st>>>(w, n, row_bytes, act, m, y); break;
        }
        return hipGetLastError();
    }
    // Q8_0 (activation scale every 32 values): the decode GEMV over row chunks of 8
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
