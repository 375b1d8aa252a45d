// lbq_gemv_impl.hpp -- decode GEMV (m <= 8) over GGUF blocks, fused dequant + integer dot.
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
//   - a wave works on RPW weight rows at a time; LPR = 64/RPW lanes walk each
//     row's pieces in order, so consecutive lanes read consecutive bytes of a
//     row (coalesced); each row is reduced inside one wave (no atomics, so the
//     result is deterministic).
#pragma once
#include <stdio.h>
#include <stdlib.h>
#include <mutex>
#include <utility>
#include <vector>

#include "lbq_device.hpp"
#include "lbq_gemv_fast.hpp"
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
        r.qs = ld_u4(blk + 16 + 16 * p);
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
        r.qs = ld_u4(blk + 48 + 16 * p);
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
        ld16_u2(blk + 64 * n + 16 * h, r.qa);
        ld16_u2(blk + 64 * n + 32 + 16 * h, r.qb);
        ld16_u2(blk + 128 + 32 * n + 16 * h, r.qh);
        r.s0 = ld4_u2(blk + 192 + 8 * n);
        r.s1 = ld4_u2(blk + 196 + 8 * n);
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
        r.mis = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
        const gbytes_c base = align4_global(reinterpret_cast<uintptr_t>(blk));
        const u32x4a4 a0 = gld16(base);
        const u32x4a4 a1 = gld16(base + 16);
        r.w[0] = a0.x; r.w[1] = a0.y; r.w[2] = a0.z; r.w[3] = a0.w;
        r.w[4] = a1.x; r.w[5] = a1.y; r.w[6] = a1.z; r.w[7] = a1.w;
        r.w[8] = gld4(base + 32);
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

// ---- Q2_K / Q3_K: piece p (0..3) = qs[16p .. 16p+16) (h = p/2, t = p%2).  Its
// byte i holds the 2-bit codes of values 128h + 32s + 16t + i for s = 0..3 (bits
// 2s), sub-block j = 8h + 2s + t.  Codes go through sdot4 unsigned (Q2_K 0..3,
// Q3_K 0..7 with the hmask bit as bit 2); Q3_K's -4 offset is restored with the
// Q8_K block sums, sum (u-4)*x = sum u*x - 4*bsum_j.
//   Q2_K (candle vec_dot): d_x*d*sum_j sc_j*(q.x)_j - d_x*dmin*sum_j m_j*bsum_j
//   Q3_K (ggml generic): d*d_x * sum_j (scale_j - 32)*(q.x)_j
template <>
struct Dec<TYPE_Q2_K> {
    static constexpr int BYTES = 84, PPB = 4, VALS = 256;
    struct Raw { uint32_t qs[4], sc0, sc1, dd; };
    __device__ static Raw load(const uint8_t *blk, int p) {
        const int h = p >> 1;
        Raw r;
        const u32x4a4 q = *reinterpret_cast<const u32x4a4 *>(blk + 16 + 16 * p);
        r.qs[0] = q.x; r.qs[1] = q.y; r.qs[2] = q.z; r.qs[3] = q.w;
        r.sc0 = ld_u32(blk + 8 * h);  // scale bytes 8h .. 8h+7 (j = 8h + 2s + t)
        r.sc1 = ld_u32(blk + 8 * h + 4);
        r.dd = ld_u32(blk + 80);
        return r;
    }
    template <int M>
    __device__ static void dot(const Raw &r, int64_t b, int p, const ActView &a, int mrows, float *acc) {
        const int h = p >> 1, t = p & 1;
        const float d = h2f(r.dd & 0xffffu), dmin = h2f(r.dd >> 16);
        int sc[4], mn[4];
        uint32_t v[4][4];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t byte = ((s < 2 ? r.sc0 : r.sc1) >> (8 * ((2 * s + t) & 3))) & 0xffu;
            sc[s] = (int)(byte & 0xFu);
            mn[s] = (int)(byte >> 4);
#pragma unroll
            for (int i = 0; i < 4; i++) v[s][i] = (r.qs[i] >> (2 * s)) & 0x03030303u;
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (m < mrows) {
                const int8_t *xr = a.xq + m * a.k + b * QK_K + 128 * h + 16 * t;
                const int64_t sb = (int64_t)m * a.nb + b;
                const uint4 bs = *reinterpret_cast<const uint4 *>(a.xbs + sb * 16 + 8 * h);
                const uint32_t bsw[4] = {bs.x, bs.y, bs.z, bs.w};
                int isum = 0, summs = 0;
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const uint4 xv = *reinterpret_cast<const uint4 *>(xr + 32 * s);
                    int q = dot4(v[s][0], xv.x, 0);
                    q = dot4(v[s][1], xv.y, q);
                    q = dot4(v[s][2], xv.z, q);
                    q = dot4(v[s][3], xv.w, q);
                    isum += sc[s] * q;
                    summs += mn[s] * (int)(int16_t)(bsw[s] >> (16 * t));
                }
                const float dx = a.xd[sb];
                acc[m] += (dx * d) * (float)isum - (dx * dmin) * (float)summs;
            }
        }
    }
};

// Q3_K blocks are 110 bytes (2-byte aligned).  The 14-byte tail (scales[12], d)
// is read as the 16 bytes from block byte 94, so no dword past the block is read.
template <>
struct Dec<TYPE_Q3_K> {
    static constexpr int BYTES = 110, PPB = 4, VALS = 256;
    struct Raw { uint32_t hm[4], qs[4], tl[4]; };
    __device__ static Raw load(const uint8_t *blk, int p) {
        Raw r;
        ld16_u2(blk + 16 * (p & 1), r.hm);  // hmask[16t .. 16t+16)
        ld16_u2(blk + 32 + 16 * p, r.qs);
        ld16_u2(blk + 94, r.tl);
        return r;
    }
    template <int M>
    __device__ static void dot(const Raw &r, int64_t b, int p, const ActView &a, int mrows, float *acc) {
        const int h = p >> 1, t = p & 1;
        // scales bytes 0..3, 4..7, 8..11 and d (bytes 14, 15 of the tail)
        const uint32_t s0 = __builtin_amdgcn_alignbyte(r.tl[1], r.tl[0], 2);
        const uint32_t s1 = __builtin_amdgcn_alignbyte(r.tl[2], r.tl[1], 2);
        const uint32_t s2 = __builtin_amdgcn_alignbyte(r.tl[3], r.tl[2], 2);
        const float d = h2f(r.tl[3] >> 16);
        int sc[4];
        uint32_t v[4][4];
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int jm = 2 * s + t;  // j % 8 for j = 8h + 2s + t
            const int lo = (int)(((jm < 4 ? s0 : s1) >> (8 * (jm & 3) + 4 * h)) & 0xFu);
            const int hi = (int)((s2 >> (8 * (jm & 3) + 2 * (2 * h + (jm >> 2)))) & 3u);
            sc[s] = (lo | (hi << 4)) - 32;
#pragma unroll
            for (int i = 0; i < 4; i++)
                v[s][i] = ((r.qs[i] >> (2 * s)) & 0x03030303u) | (((r.hm[i] >> (4 * h + s)) & 0x01010101u) << 2);
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (m < mrows) {
                const int8_t *xr = a.xq + m * a.k + b * QK_K + 128 * h + 16 * t;
                const int64_t sb = (int64_t)m * a.nb + b;
                const uint4 bs = *reinterpret_cast<const uint4 *>(a.xbs + sb * 16 + 8 * h);
                const uint32_t bsw[4] = {bs.x, bs.y, bs.z, bs.w};
                int isum = 0;
#pragma unroll
                for (int s = 0; s < 4; s++) {
                    const uint4 xv = *reinterpret_cast<const uint4 *>(xr + 32 * s);
                    int q = dot4(v[s][0], xv.x, 0);
                    q = dot4(v[s][1], xv.y, q);
                    q = dot4(v[s][2], xv.z, q);
                    q = dot4(v[s][3], xv.w, q);
                    isum += sc[s] * (q - 4 * (int)(int16_t)(bsw[s] >> (16 * t)));
                }
                acc[m] += (d * a.xd[sb]) * (float)isum;
            }
        }
    }
};

// ---- 32-value legacy blocks (Q4_0, Q4_1, Q5_0, Q5_1): piece = one block.  Value
// j (j < 16) is the low nibble of qs[j], value j + 16 its high nibble; Q5_* take
// bit 4 of value v from bit v of the u32 qh.  Fields: d f16 | (m f16) | (qh u32) |
// qs[16]; 18- and 22-byte blocks start 2 bytes into a dword every other block.
// The products follow candle's vec_dot bodies: Q4_0 ((sumi*d_w)*d_x), Q5_0
// ((d_w*d_x)*sumi), Q4_1/Q5_1 ((d_w*d_x)*sumi + m_w*s_x) -- with the -8/-16
// code offsets folded into the int8 weight codes.
template <int TYPE>
struct DecLegacy {
    static constexpr bool HAS_M = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;
    static constexpr bool FIVE = TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1;
    static constexpr int BYTES = 18 + (HAS_M ? 2 : 0) + (FIVE ? 4 : 0);
    static constexpr bool ODD = BYTES % 4 != 0;  // may start at 2 mod 4
    static constexpr int NW = FIVE ? 6 : 5;       // aligned dwords covering the block
    static constexpr int PPB = 1, VALS = 32;
    struct Raw { uint32_t w[NW]; uint32_t mis; };
    __device__ static Raw load(const uint8_t *blk, int) {
        Raw r;
        r.mis = ODD ? (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 2u) : 0u;
        const gbytes_c base = align4_global(reinterpret_cast<uintptr_t>(blk));
        const u32x4a4 a0 = gld16(base);
        r.w[0] = a0.x; r.w[1] = a0.y; r.w[2] = a0.z; r.w[3] = a0.w;
        r.w[4] = gld4(base + 16);
        if constexpr (NW == 6) r.w[5] = gld4(base + 20);
        return r;
    }
    // 4 bits b0..b3 -> bit 4 of bytes 0..3
    __device__ static uint32_t spread4(uint32_t b) { return ((b * 0x00204081u) & 0x01010101u) << 4; }
    template <int M>
    __device__ static void dot(const Raw &r, int64_t b, int, const ActView &a, int mrows, float *acc) {
        // the block's dwords from its own byte 0 (c[i] = bytes 4i..4i+3; the top
        // half of the last one is not used)
        constexpr int NC = (BYTES + 3) / 4;
        uint32_t c[NC];
#pragma unroll
        for (int i = 0; i < NC; i++) {
            if constexpr (ODD) c[i] = __builtin_amdgcn_alignbyte(r.w[i + 1 < NW ? i + 1 : i], r.w[i], r.mis);
            else c[i] = r.w[i];
        }
        const float d = h2f(c[0] & 0xffffu);
        const float mw = HAS_M ? h2f(c[0] >> 16) : 0.f;
        // qs dwords: byte offset QS = 2, 4, 6 or 8
        constexpr int QS = (HAS_M ? 4 : 2) + (FIVE ? 4 : 0);
        uint32_t qs[4], qh = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            if constexpr (QS % 4 == 0) qs[i] = c[QS / 4 + i];
            else qs[i] = __builtin_amdgcn_alignbyte(c[QS / 4 + i + 1], c[QS / 4 + i], 2);
        }
        if constexpr (FIVE) {
            constexpr int QH = HAS_M ? 4 : 2;
            if constexpr (QH % 4 == 0) qh = c[QH / 4];
            else qh = __builtin_amdgcn_alignbyte(c[QH / 4 + 1], c[QH / 4], 2);
        }
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            lo[i] = qs[i] & 0x0F0F0F0Fu;
            hi[i] = (qs[i] >> 4) & 0x0F0F0F0Fu;
            if constexpr (FIVE) {
                lo[i] |= spread4((qh >> (4 * i)) & 15u);
                hi[i] |= spread4((qh >> (16 + 4 * i)) & 15u);
            }
            if constexpr (!HAS_M) {
                // code - 8 (Q4_0) / - 16 (Q5_0) per byte as int8, no borrow between bytes
                constexpr uint32_t OFF = FIVE ? 0x10101010u : 0x08080808u;
                lo[i] = ((lo[i] | 0x80808080u) - OFF) ^ 0x80808080u;
                hi[i] = ((hi[i] | 0x80808080u) - OFF) ^ 0x80808080u;
            }
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
            if (m < mrows) {
                const int8_t *xr = a.xq + m * a.k + b * QK8_0;
                const uint4 x0 = *reinterpret_cast<const uint4 *>(xr);
                const uint4 x1 = *reinterpret_cast<const uint4 *>(xr + 16);
                int s = dot4(lo[0], x0.x, 0);
                s = dot4(lo[1], x0.y, s);
                s = dot4(lo[2], x0.z, s);
                s = dot4(lo[3], x0.w, s);
                s = dot4(hi[0], x1.x, s);
                s = dot4(hi[1], x1.y, s);
                s = dot4(hi[2], x1.z, s);
                s = dot4(hi[3], x1.w, s);
                const int64_t xb = (int64_t)m * a.nb + b;
                const float dx = a.xd[xb];
                if constexpr (TYPE == TYPE_Q4_0) acc[m] += ((float)s * d) * dx;
                else if constexpr (TYPE == TYPE_Q5_0) acc[m] += (d * dx) * (float)s;
                else acc[m] += (d * dx) * (float)s + mw * a.xs[xb];
            }
        }
    }
};
template <> struct Dec<TYPE_Q4_0> : DecLegacy<TYPE_Q4_0> {};
template <> struct Dec<TYPE_Q4_1> : DecLegacy<TYPE_Q4_1> {};
template <> struct Dec<TYPE_Q5_0> : DecLegacy<TYPE_Q5_0> {};
template <> struct Dec<TYPE_Q5_1> : DecLegacy<TYPE_Q5_1> {};

// ---------------------------------------------------------------------------
// Persistent GEMV.  The rows are cut into groups of RPW rows; each wave owns a
// contiguous range of groups and walks each group's rows in chunks of
// CH = (64/RPW)*IT pieces, double-buffering the weight loads of the next chunk
// while it computes the current one.  With FUSED the workgroup first quantises
// x itself (the same code as the standalone Q8_K/Q8_0 kernels) into LDS, after
// issuing the loads of its first chunk so that the quantisation overlaps their
// latency; the dot products then read x from LDS.
// ---------------------------------------------------------------------------
struct PGeom {
    int64_t n_rows, row_bytes;
    int nb;                  // weight blocks per row
    int pieces;              // pieces per row
    int cpg;                 // chunks per group
    int64_t ngroups;
};

template <int TYPE, int M, int RPW, int IT, bool FUSED>
__global__ __launch_bounds__(256) void k_gemv_p(const uint8_t *__restrict__ W, PGeom g, ActView act,
                                                const float *__restrict__ x, int mrows, float *__restrict__ y) {
    using D = Dec<TYPE>;
    using Raw = typename D::Raw;
    constexpr int LPR = 64 / RPW;
    constexpr int CH = LPR * IT;
    constexpr bool KQ = is_kquant(TYPE);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane / LPR, li = lane % LPR;
    const int64_t gw = (int64_t)blockIdx.x * 4 + wave, nw = (int64_t)gridDim.x * 4;
    const int64_t per = g.ngroups / nw, rem = g.ngroups % nw;
    const int64_t g0 = gw * per + (gw < rem ? gw : rem);
    const int64_t u0 = g0 * g.cpg, u1 = (g0 + per + (gw < rem ? 1 : 0)) * g.cpg;

    auto load_unit = [&](int64_t u, Raw *raw) {
        const int64_t grp = u / g.cpg;
        const int c = (int)(u - grp * g.cpg);
        const int64_t row = grp * RPW + r;
        const uint8_t *wrow = W + (row < g.n_rows ? row : 0) * g.row_bytes;
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int q = c * CH + it * LPR + li;
            if (row < g.n_rows && q < g.pieces) raw[it] = D::load(wrow + (int64_t)(q / D::PPB) * D::BYTES, q % D::PPB);
        }
    };

    Raw bufA[IT], bufB[IT];
    if (u0 < u1) load_unit(u0, bufA);

    ActView a = act;
    if constexpr (FUSED) {
        extern __shared__ __align__(16) uint8_t smem[];
        const int64_t k = act.k;
        int8_t *sxq = reinterpret_cast<int8_t *>(smem);
        float *sxd = reinterpret_cast<float *>(smem + ((mrows * k + 15) & ~(int64_t)15));
        int16_t *sxbs = reinterpret_cast<int16_t *>(reinterpret_cast<uint8_t *>(sxd) + ((mrows * act.nb * 4 + 15) & ~15));
        const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
        if constexpr (KQ) {
            const int nblk = mrows * act.nb;
            for (int b = wave; b < nblk; b += 4) {
                float v[4];
                load4f(x + (int64_t)b * QK_K + lane * 4, vec, v);
                int s;
                float d;
                const uint32_t packed = q8k_block_wave(v, lane, &s, &d);
                *reinterpret_cast<uint32_t *>(sxq + (int64_t)b * QK_K + lane * 4) = packed;
                if ((lane & 3) == 0) sxbs[b * 16 + (lane >> 2)] = (int16_t)s;
                if (lane == 0) sxd[b] = d;
            }
        } else {
            const int nblk = mrows * act.nb;
            for (int b0 = 0; b0 < nblk; b0 += 32) {
                const int b = b0 + (threadIdx.x >> 3), sub = threadIdx.x & 7;
                float v[4] = {0.f, 0.f, 0.f, 0.f};
                if (b < nblk) load4f(x + (int64_t)b * QK8_0 + sub * 4, vec, v);
                __half dh;
                const uint32_t packed = q8_0_block8(v, &dh);
                if (b < nblk) {
                    *reinterpret_cast<uint32_t *>(sxq + (int64_t)b * QK8_0 + sub * 4) = packed;
                    if (sub == 0) sxd[b] = __half2float(dh);
                }
            }
        }
        __syncthreads();
        a.xq = sxq;
        a.xd = sxd;
        a.xbs = sxbs;
    }

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; m++) acc[m] = 0.f;

    auto compute_unit = [&](int64_t u, const Raw *raw) {
        const int64_t grp = u / g.cpg;
        const int c = (int)(u - grp * g.cpg);
        const int64_t row = grp * RPW + r;
#pragma unroll
        for (int it = 0; it < IT; it++) {
            const int q = c * CH + it * LPR + li;
            if (row < g.n_rows && q < g.pieces) D::template dot<M>(raw[it], q / D::PPB, q % D::PPB, a, mrows, acc);
        }
        if (c == g.cpg - 1) {
#pragma unroll
            for (int m = 0; m < M; m++) {
#pragma unroll
                for (int off = LPR / 2; off >= 1; off >>= 1) acc[m] += __shfl_xor(acc[m], off);
            }
            if (li == 0 && row < g.n_rows) {
#pragma unroll
                for (int m = 0; m < M; m++)
                    if (m < mrows) y[(int64_t)m * g.n_rows + row] = acc[m];
            }
#pragma unroll
            for (int m = 0; m < M; m++) acc[m] = 0.f;
        }
    };

    for (int64_t u = u0; u < u1; u += 2) {
        if (u + 1 < u1) load_unit(u + 1, bufB);
        compute_unit(u, bufA);
        if (u + 1 < u1) {
            if (u + 2 < u1) load_unit(u + 2, bufA);
            compute_unit(u + 1, bufB);
        }
    }
}

// ---------------------------------------------------------------------------
// dispatch
// ---------------------------------------------------------------------------
struct GemvCfg {
    int rpw, it, wpc;  // rows per wave, pieces per lane per chunk, target waves per CU
    bool fused;
};

// LBQ_GEMV="rpw,it,wpc,fused" overrides the choice (tuning; any value is correct).
static GemvCfg pick_cfg(int type, int64_t n, int pieces, int m, int64_t k) {
    GemvCfg c;
    c.fused = (int64_t)m * k <= 32768;
    // rows per wave: enough lanes per row to cover a row in a few chunks
    // must name a pair that run_m compiles for every m
    if (pieces >= 384) { c.rpw = 1; c.it = 7; }
    else if (pieces >= 128) { c.rpw = 2; c.it = 4; }
    else { c.rpw = 4; c.it = 4; }
    c.wpc = 8;
    if (const int *v = tuning().gemv_cfg; v[0] > 0) {
        c.rpw = v[0]; c.it = v[1]; c.wpc = v[2]; c.fused = v[3] != 0 && (int64_t)m * k <= 65536;
    }
    (void)n;
    return c;
}

template <int TYPE, int M, int RPW, int IT, bool FUSED>
static hipError_t run_p(const uint8_t *w, const PGeom &g0, const ActView &act, const float *x, int m, float *y,
                        int wpc, hipStream_t st) {
    PGeom g = g0;
    constexpr int CH = (64 / RPW) * IT;
    g.cpg = (g.pieces + CH - 1) / CH;
    g.ngroups = (g.n_rows + RPW - 1) / RPW;
    int64_t waves = (int64_t)num_cus() * wpc;
    if (waves > g.ngroups) waves = g.ngroups;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    size_t lds = 0;
    if (FUSED) {
        lds = ((size_t)m * act.k + 15) / 16 * 16 + ((size_t)m * act.nb * 4 + 15) / 16 * 16;
        if (is_kquant(TYPE)) lds += (size_t)m * (act.k / 16) * 2;
    }
    k_gemv_p<TYPE, M, RPW, IT, FUSED><<<grid, 256, lds, st>>>(w, g, act, x, m, y);
    return hipGetLastError();
}

// (rpw, it) pairs compiled: the ones pick_cfg returns.
template <int TYPE, int M>
static hipError_t run_m(const GemvCfg &c, const uint8_t *w, const PGeom &g, const ActView &act, const float *x, int m,
                        float *y, hipStream_t st) {
#define LBQ_CASE(R, I)                                                                               \
    if (c.rpw == R && c.it == I) return run_p<TYPE, M, R, I, false>(w, g, act, x, m, y, c.wpc, st);
    LBQ_CASE(1, 7)
    LBQ_CASE(2, 4)
    LBQ_CASE(4, 4)
#undef LBQ_CASE
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// m = 1: the register-activation kernel (lbq_gemv_fast.hpp)
// ---------------------------------------------------------------------------
// Launch shape of the m = 1 kernel for nb blocks per row: lanes per block (ppb:
// 4 = 64-weight pieces, 8 = 32-weight pieces for Q4_K / Q5_K), rows per wave
// group and sweeps.  Measured on Q4_K at Llama-3-8B shapes: 64-weight pieces with
// one row per group for k = 4096; at k = 14336 (56 blocks) 32-weight pieces fill
// seven sweeps of eight blocks exactly, where 64-weight pieces would leave an
// eighth of the lanes idle.
template <int TYPE>
static bool fast_shape(int nb, int *ppb, int *rpw, int *it, int mr = 1) {
    int q = 0, r = 0;
    if (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) {
        // several activation rows: 64-weight pieces throughout (the seven sweeps
        // of 32-weight pieces leave no registers for more than one row)
        if (nb <= 4) { q = 4; r = 4; }
        else if (nb <= 8) { q = 4; r = 2; }
        else if (nb <= 64 && (nb > 56 || nb <= 48 || mr > 1 || TYPE == TYPE_Q4_K)) { q = 4; r = 1; }
        else if (nb <= 56) { q = 8; r = 1; }
    } else if (TYPE == TYPE_Q6_K) {
        if (nb <= 16 && mr == 1) { q = 4; r = 2; }
        else if (nb <= 64) { q = 4; r = 1; }  // several rows: one sweep per row at k <= 4096
    } else if (nb <= 512) {  // Q8_0: nb counts 32-value blocks
        q = 1; r = 1;
    }
    if (tuning().gemv1_ppb > 0) { q = tuning().gemv1_ppb; r = tuning().gemv1_rpw; }  // tuning override
    if (q <= 0 || r <= 0 || 64 % (q * r) != 0) return false;
    const int bpi = 64 / (q * r);
    *ppb = q;
    *rpw = r;
    *it = (nb + bpi - 1) / bpi;  // the smallest sweep count covering the row (the kernel relies on it)
    return true;
}

// The fused m = 1 launch of one weight on the static schedule (k_gemv1 with
// RMAX = R: at most R row groups per wave, the group loop unrolled, no load past
// a wave's last group).  Ring depth: one group ahead of the prologue at k > 8192
// (IT 4: an x of 56 KB per workgroup arrives later behind more weight loads --
// 4096 x 14336 two groups ahead 10.7 us, one 8.7 us), else up to three
// (4096 rows: 4.1 us with all four ahead and with three, 4.5 us in the dynamic
// loop's two).
template <int TYPE, int PPB, int RPW, int IT, int WPG, int R>
static void launch_static(const RowMap &rm, int64_t row_bytes, int nb, const float *x, unsigned grid, size_t lds,
                          hipStream_t st) {
    constexpr int D = IT >= 4 ? 2 : (R < 3 ? R : 3) + 1;
    const ActView none{nullptr, nullptr, nullptr, (int64_t)nb * QK_K, 0};
    k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_ONE, false, WPG, D, R><<<grid, 64 * WPG, lds, st>>>(rm, row_bytes, nb, x,
                                                                                              none, nullptr, 0.f);
}
// The smallest compiled R (1, 2, 4, 7, 8) holding rpw groups per wave; 0: none.
static inline int static_rmax(int64_t rpw) {
    return rpw <= 1 ? 1 : rpw <= 2 ? 2 : rpw <= 4 ? 4 : rpw <= 7 ? 7 : rpw <= 8 ? 8 : 0;
}
template <int TYPE, int PPB, int RPW, int IT, int WPG>
static bool try_static(const RowMap &rm, int64_t row_bytes, int nb, const float *x, int64_t ng, unsigned grid,
                       size_t lds, hipStream_t st) {
    const int64_t nw = (int64_t)grid * WPG;
    switch (static_rmax((ng + nw - 1) / nw)) {
    case 1: launch_static<TYPE, PPB, RPW, IT, WPG, 1>(rm, row_bytes, nb, x, grid, lds, st); return true;
    case 2: launch_static<TYPE, PPB, RPW, IT, WPG, 2>(rm, row_bytes, nb, x, grid, lds, st); return true;
    case 4: launch_static<TYPE, PPB, RPW, IT, WPG, 4>(rm, row_bytes, nb, x, grid, lds, st); return true;
    case 7: launch_static<TYPE, PPB, RPW, IT, WPG, 7>(rm, row_bytes, nb, x, grid, lds, st); return true;
    case 8: launch_static<TYPE, PPB, RPW, IT, WPG, 8>(rm, row_bytes, nb, x, grid, lds, st); return true;
    default: return false;
    }
}

template <int TYPE, int PPB, int RPW, int IT>
static hipError_t launch_fast(const RowMap &rm, int64_t row_bytes, int nb, const float *x, const ActView &act, int map,
                              const float *alpha, float eps, hipStream_t st) {
    const int64_t n = rm.n;
    const int64_t ng = (n + RPW - 1) / RPW;
    // the kernel clamps only the last sweep's block: IT must be the smallest that covers nb
    constexpr int BPI = 64 / RPW / PPB;
    if (!(BPI * (IT - 1) < nb && nb <= BPI * IT)) return hipErrorNotSupported;
    // Waves per CU.  With the fused prologue every workgroup quantises all of x,
    // so for fewer rows (less weight per CU to hide it behind) one workgroup per
    // CU does better, and so it does for k = 14336 and for Q6_K throughout.
    // Measured (fused / pre-quantised x): Q4_K 4096 x 4096 5.0 / 4.5 us at 4 vs
    // 5.7 / 4.6 at 8; 14336 x 4096 9.3 / 8.8 at 4 vs 9.1 / 8.4 at 8; 4096 x 14336
    // 10.1 / 8.2 at 4 vs 11.2 / 9.0 at 8.  Q6_K takes four except from 8192 to 32768
    // rows at k <= 4096 (14336 x 4096 14.0 -> 13.4 us, 28672 x 4096 25.1 -> 24.1 at
    // eight; 4096 / 8192 rows 5.5 / 8.4 -> 5.7 / 8.7 and the 128256-row head 94.1 ->
    // 97.3 us, so those keep four).  Q8_0 takes eight everywhere (4096 x 4096 fused:
    // 6.2 us at 4, 5.7 at 8).
    const bool q6_8 = TYPE == TYPE_Q6_K && n > 8192 && n <= 32768 && nb <= 16;
    int wpc = ((TYPE == TYPE_Q6_K && !q6_8) ||
               (TYPE != TYPE_Q6_K && TYPE != TYPE_Q8_0 && n < 8192 && (x || nb > 32))) ? 4 : 8;
    if (tuning().gemv1_wpc > 0) wpc = tuning().gemv1_wpc;
    int64_t waves = (int64_t)num_cus() * wpc;
    if (waves > ng) waves = ng;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    const size_t lds = (size_t)nb * (TYPE == TYPE_Q8_0 ? XS_0 : XS_K);
    // row maps take the fused quantisation only (the caller runs the rest weight by
    // weight); the RMS norm (alpha != nullptr) only k-quant row maps with k <= 8192
    constexpr bool NORM_OK = TYPE != TYPE_Q8_0 && BPI * IT <= 32;
    if (alpha && (!NORM_OK || nb > 32 || !x || map == MAP_ONE)) return hipErrorNotSupported;
    // Fused launches of Q4_K / Q5_K that run eight waves per CU anyway (n >= 8192)
    // take eight-wave workgroups: one x prologue per CU instead of two, spread
    // over 512 threads (gate/up 14336 x 4096: 9.1 -> 8.7 us; where one four-wave
    // workgroup per CU was chosen, eight waves measured slower).
    constexpr bool W8_OK = TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K;
    // So does the grouped q|k|v launch (6144 rows at k = 4096: grouped step 37.6 -> 37.2 us;
    // at 4096 rows the four-wave workgroups stay ahead).
    bool w8 = W8_OK && (wpc == 8 || (n > 4096 && nb <= 32));
    if (w8 && wpc < 8) waves = std::min<int64_t>((int64_t)num_cus() * 8, ng);
    if (tuning().gemv1_wpg > 0) w8 = W8_OK && tuning().gemv1_wpg == 8;
    const unsigned grid8 = (unsigned)((waves + 7) / 8);
    auto fused = [&](auto k4, auto k8, const float *al, float ep) {
        if (w8) k8<<<grid8, 512, lds, st>>>(rm, row_bytes, nb, x, act, al, ep);
        else k4<<<grid, 256, lds, st>>>(rm, row_bytes, nb, x, act, al, ep);
    };
    constexpr int W8 = W8_OK ? 8 : 4;  // (no eight-wave instantiations for the other types)
    if (map == MAP_SILU_PAIRS) {
        if constexpr (RPW <= 2) {
            if (!x || (n & 1)) return hipErrorNotSupported;
            if constexpr (NORM_OK)
                if (alpha) {
                    fused(k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SILU_PAIRS, true>,
                          k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SILU_PAIRS, true, W8>, alpha, eps);
                    return hipGetLastError();
                }
            fused(k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SILU_PAIRS>,
                  k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SILU_PAIRS, false, W8>, nullptr, 0.f);
        } else {
            return hipErrorNotSupported;
        }
    } else if (map == MAP_SEGMENTS) {
        if (!x) return hipErrorNotSupported;
        if constexpr (NORM_OK)
            if (alpha) {
                fused(k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SEGMENTS, true>,
                      k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SEGMENTS, true, W8>, alpha, eps);
                return hipGetLastError();
            }
        fused(k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SEGMENTS>,
              k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_SEGMENTS, false, W8>, nullptr, 0.f);
    } else if (x) {
        // Q6_K keeps one row group in flight (two-buffer ring: its pieces take 15
        // registers each); a long per-wave stream (the 128256-row head: 62 groups per
        // wave) takes three in flight instead (head 97.6 -> 92.0 us).  Short streams
        // lose with the deeper ring (14336 rows: 13.7 -> 14.8 us; 1024: 6.7 -> 8.8).
        if constexpr (TYPE == TYPE_Q6_K && IT <= 2)
            if (ng >= 32 * waves) {
                fused(k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_ONE, false, 4, 4>,
                      k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_ONE, false, W8, 4>, nullptr, 0.f);
                return hipGetLastError();
            }
        // Q4_K / Q5_K, one row per group, k <= 4096 or k > 12288: the static
        // schedule where every wave holds at most 8 groups.  At k > 12288 eight-wave
        // workgroups (8 per CU): the x prologue over 512 threads, two groups per wave
        // for 4096 rows (4096 x 14336: 10.2 -> 8.7 us with the 64-weight pieces)
        if constexpr ((W8_OK || TYPE == TYPE_Q6_K) && RPW == 1 && (IT == 1 || IT == 4))
            if (!tuning().gemv1_dynamic) {
                // (Q6_K: eight-wave workgroups at k > 12288 only -- its pieces take 15
                // registers, and the two groups per wave fit beside them there)
                const bool s8 = IT == 4 || (W8_OK && w8);
                const int64_t sw = (IT == 4 && s8) ? std::min<int64_t>((int64_t)num_cus() * 8, ng) : waves;
                const unsigned sg = (unsigned)((sw + (s8 ? 7 : 3)) / (s8 ? 8 : 4));
                if (s8 ? try_static<TYPE, PPB, RPW, IT, 8>(rm, row_bytes, nb, x, ng, sg, lds, st)
                       : try_static<TYPE, PPB, RPW, IT, 4>(rm, row_bytes, nb, x, ng, sg, lds, st))
                    return hipGetLastError();
            }
        fused(k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_ONE>, k_gemv1<TYPE, PPB, RPW, IT, 1, true, MAP_ONE, false, W8>,
              nullptr, 0.f);
    } else {
        k_gemv1<TYPE, PPB, RPW, IT, 1, false, MAP_ONE><<<grid, 256, lds, st>>>(rm, row_bytes, nb, x, act, nullptr, 0.f);
    }
    return hipGetLastError();
}

// Lifts a kernel's dynamic LDS limit to the CU's 160 KB, once per (device, kernel).
static hipError_t allow_big_lds(const void *kern) {
    static std::mutex mu;
    static std::vector<std::pair<int, const void *>> done;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    for (const auto &d : done)
        if (d.first == dev && d.second == kern) return hipSuccess;
    e = hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
    if (e == hipSuccess) done.emplace_back(dev, kern);
    return e;
}

// MR pre-quantised activation rows (m = MR) against one weight: the weight is
// streamed once for all MR rows, the activation rows sit in LDS (or registers).
template <int TYPE, int PPB, int RPW, int IT, int MR>
static hipError_t launch_fast_rows(const RowMap &rm, int64_t row_bytes, int nb, const ActView &act, const float *x,
                                   hipStream_t st) {
    const int64_t n = rm.n;
    const int64_t ng = (n + RPW - 1) / RPW;
    constexpr int BPI = 64 / RPW / PPB;
    if (!(BPI * (IT - 1) < nb && nb <= BPI * IT)) return hipErrorNotSupported;
    const size_t lds = (size_t)MR * nb * (TYPE == TYPE_Q8_0 ? XS_0 : XS_K);
    // x: f32 rows quantised in the prologue (Q8_K types), else pre-quantised rows
    constexpr bool FX = TYPE != TYPE_Q8_0 && MR > 1 && MR * IT <= 8;
    if (x && !FX) return hipErrorNotSupported;
    // two workgroups per CU while both fit the CU's 160 KB of LDS
    int wpc = lds <= 80 * 1024 ? 8 : 4;
    if (tuning().gemv1_wpc > 0) wpc = tuning().gemv1_wpc;
    int64_t waves = (int64_t)num_cus() * wpc;
    if (waves > ng) waves = ng;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    // Q6_K keeps one row group in flight; a long per-wave stream with up to four
    // rows takes two (three-buffer ring): head 128256 x 4096 m = 2 / 4 98 -> 94 /
    // 105 -> 99.5 us.  At eight rows (registers) and on short streams (14336 rows:
    // 16.2 -> 16.7 us) the two-buffer ring stays ahead.
    constexpr bool R3 = TYPE == TYPE_Q6_K && MR <= 4;
    const bool ring3 = R3 && ng >= 32 * waves;
    auto kern = x ? (ring3 ? k_gemv1<TYPE, PPB, RPW, IT, MR, FX, MAP_ONE, false, 4, R3 ? 3 : 0>
                           : k_gemv1<TYPE, PPB, RPW, IT, MR, FX, MAP_ONE>)
                  : (ring3 ? k_gemv1<TYPE, PPB, RPW, IT, MR, false, MAP_ONE, false, 4, R3 ? 3 : 0>
                           : k_gemv1<TYPE, PPB, RPW, IT, MR, false, MAP_ONE>);
    if (lds > 65536) {
        const hipError_t attr = allow_big_lds(reinterpret_cast<const void *>(kern));
        if (attr != hipSuccess) return attr;
    }
    kern<<<grid, 256, lds, st>>>(rm, row_bytes, nb, x, act, nullptr, 0.f);
    return hipGetLastError();
}

template <int TYPE, int MR>
static hipError_t run_fast_rows(const RowMap &rm, int64_t row_bytes, int nb, const ActView &act, const float *x,
                                hipStream_t st) {
    int ppb, rpw, it;
    // every chunk of a multi-row call (its single-row remainder too) uses the multi-row shape
    if (!fast_shape<TYPE>(nb, &ppb, &rpw, &it, 2)) return hipErrorNotSupported;
    // only the (shape, rows) pairs fast_rows_max admits are compiled
#define LBQ_FAST(Q, R, I)                                                                                   \
    if constexpr (MR <= (I <= 1 ? 8 : I == 2 ? 4 : 1))                                                     \
        if (ppb == Q && rpw == R && it == I) return launch_fast_rows<TYPE, Q, R, I, MR>(rm, row_bytes, nb, act, x, st);
    if constexpr (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) {
        LBQ_FAST(4, 4, 1) LBQ_FAST(4, 2, 1) LBQ_FAST(4, 1, 1) LBQ_FAST(4, 1, 2) LBQ_FAST(4, 1, 3) LBQ_FAST(4, 1, 4)
    } else if constexpr (TYPE == TYPE_Q6_K) {
        LBQ_FAST(4, 1, 1) LBQ_FAST(4, 1, 2) LBQ_FAST(4, 1, 3) LBQ_FAST(4, 1, 4)
    } else {
        LBQ_FAST(1, 1, 1) LBQ_FAST(1, 1, 2) LBQ_FAST(1, 1, 3) LBQ_FAST(1, 1, 4) LBQ_FAST(1, 1, 5) LBQ_FAST(1, 1, 6)
        LBQ_FAST(1, 1, 7) LBQ_FAST(1, 1, 8)
    }
#undef LBQ_FAST
    return hipErrorNotSupported;
}

// Rows of x one launch can take: their activation registers must fit beside the
// weight ring (8 rows for one sweep per row, 4 for two; beyond, one).
template <int TYPE>
static int fast_rows_max(int nb) {
    int ppb, rpw, it;
    if (!fast_shape<TYPE>(nb, &ppb, &rpw, &it, 2)) return 0;
    return it <= 1 ? 8 : it == 2 ? 4 : 1;
}

template <int TYPE>
static hipError_t run_fast(const RowMap &rm, int64_t row_bytes, int nb, const float *x, const ActView &act, int map,
                           const float *alpha, float eps, hipStream_t st);

// m = 2..8 rows: chunks of 8, 4, 2 and 1 rows, each chunk one launch (the largest
// chunk within fast_rows_max whose activation image fits 80 KB of LDS); rows
// pre-quantised (act), or f32 x that each launch quantises in its prologue.
template <int TYPE>
static hipError_t run_fast_m(const RowMap &rm0, int64_t row_bytes, int nb, const ActView &act, const float *x, int m,
                             hipStream_t st) {
    const size_t row_lds = (size_t)nb * (TYPE == TYPE_Q8_0 ? XS_0 : XS_K);
    const int mr_max = fast_rows_max<TYPE>(nb);
    for (int m0 = 0; m0 < m;) {
        // the smallest allowed chunk that takes every remaining row (padded with
        // rows that repeat the last one and are not stored), else the largest
        int mr = 8;
        while (mr > 1 && (mr > mr_max || (size_t)mr * row_lds > 80 * 1024)) mr >>= 1;
        while (mr > 1 && mr / 2 >= m - m0) mr >>= 1;
        const int real = std::min(mr, m - m0);
        RowMap rm = rm0;
        rm.y[0] = rm0.y[0] + (int64_t)m0 * rm0.n;
        ActView a = act;
        a.xq = act.xq + (int64_t)m0 * act.k;
        a.xd = act.xd + (int64_t)m0 * act.nb;
        if (act.xbs) a.xbs = act.xbs + (int64_t)m0 * (act.k / 16);
        a.rows = real < mr ? real : 0;
        const float *xc = x ? x + (int64_t)m0 * nb * (TYPE == TYPE_Q8_0 ? QK8_0 : QK_K) : nullptr;
        hipError_t e;
        switch (mr) {
        case 8: e = run_fast_rows<TYPE, 8>(rm, row_bytes, nb, a, xc, st); break;
        case 4: e = run_fast_rows<TYPE, 4>(rm, row_bytes, nb, a, xc, st); break;
        case 2: e = run_fast_rows<TYPE, 2>(rm, row_bytes, nb, a, xc, st); break;
        default:  // a single remaining row: the m = 1 kernel (its own fused prologue with x)
            e = x ? run_fast<TYPE>(rm, row_bytes, nb, xc, a, MAP_ONE, nullptr, 0.f, st)
                  : run_fast_rows<TYPE, 1>(rm, row_bytes, nb, a, nullptr, st);
            break;
        }
        if (e != hipSuccess) return e;
        m0 += real;
    }
    return hipSuccess;
}

template <int TYPE>
static hipError_t run_fast(const RowMap &rm, int64_t row_bytes, int nb, const float *x, const ActView &act, int map,
                           const float *alpha, float eps, hipStream_t st) {
    int ppb, rpw, it;
    if (!fast_shape<TYPE>(nb, &ppb, &rpw, &it)) return hipErrorNotSupported;
    // Q6_K at k <= 4096 pairs rows in a wave (two per group) for long streams
    // (128256 x 4096: 97 against 107 us with one row per group; 14336 x 4096: 14.7
    // against 16.2); a weight of at most 8192 rows takes one row per group instead,
    // so every CU gets a workgroup (1024 x 4096: 512 groups would fill half the
    // chip; 4.8 -> 3.4 us).  The choice is the weight's, whatever the launch: fused
    // or not, alone, in a group or a gate/up pair, each row keeps one summation
    // order; a group whose weights fall on both sides runs weight by weight.
    if (TYPE == TYPE_Q6_K && rpw == 2 && tuning().gemv1_ppb == 0) {
        bool small = false, large = false;
        if (map == MAP_SEGMENTS) {
            int32_t prev = 0;
            for (int s = 0; s < GROUP_MAX && prev < rm.n; s++) {
                const int32_t end = (int32_t)std::min<int64_t>(rm.end[s], rm.n);
                (end - prev <= 8192 ? small : large) = true;
                prev = end;
            }
        } else {
            (rm.n / (map == MAP_SILU_PAIRS ? 2 : 1) <= 8192 ? small : large) = true;
        }
        if (small && large) return hipErrorNotSupported;
        if (small) {
            rpw = 1;
            it = (nb + 15) / 16;
        }
    }
#define LBQ_FAST(Q, R, I) \
    if (ppb == Q && rpw == R && it == I) return launch_fast<TYPE, Q, R, I>(rm, row_bytes, nb, x, act, map, alpha, eps, st);
    if constexpr (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) {
        LBQ_FAST(4, 4, 1) LBQ_FAST(4, 2, 1) LBQ_FAST(4, 1, 1) LBQ_FAST(4, 1, 2) LBQ_FAST(4, 1, 3) LBQ_FAST(4, 1, 4)
        LBQ_FAST(8, 1, 7)
    } else if constexpr (TYPE == TYPE_Q6_K) {
        LBQ_FAST(4, 2, 1) LBQ_FAST(4, 2, 2) LBQ_FAST(4, 1, 1) LBQ_FAST(4, 1, 2) LBQ_FAST(4, 1, 3) LBQ_FAST(4, 1, 4)
    } else {
        LBQ_FAST(1, 1, 1) LBQ_FAST(1, 1, 2) LBQ_FAST(1, 1, 3) LBQ_FAST(1, 1, 4) LBQ_FAST(1, 1, 5) LBQ_FAST(1, 1, 6)
        LBQ_FAST(1, 1, 7) LBQ_FAST(1, 1, 8)
    }
#undef LBQ_FAST
    return hipErrorNotSupported;
}

// One weight (rm.n rows, single segment) or, at m = 1, a multi-weight row map
// (map: MAP_ONE / MAP_SEGMENTS, or MAP_SILU_PAIRS for a gate/up pair).
template <int TYPE>
static hipError_t run_type(const RowMap &rm, int64_t k, int64_t row_bytes, const ActView &act, const float *x, int m,
                           int map, const float *alpha, float eps, hipStream_t st) {
    using D = Dec<TYPE>;
    const uint8_t *w = rm.w[0];
    const int64_t n = rm.n;
    float *y = rm.y[0];
    PGeom g{};
    g.n_rows = n;
    g.row_bytes = row_bytes;
    g.nb = (int)(k / D::VALS);
    g.pieces = g.nb * D::PPB;
    if constexpr (has_fast_gemv(TYPE)) {  // the types with a Fast<> decoder
        if (m == 1) {
            const hipError_t e = run_fast<TYPE>(rm, row_bytes, g.nb, x, act, map, alpha, eps, st);
            if (e != hipErrorNotSupported) return e;
        } else if (m <= 8 && !alpha && map == MAP_ONE && rm.end[0] == n && !tuning().gemv_rows_off) {
            // one launch per chunk of rows, each streaming the weight once: worth it
            // while a chunk holds at least half the rows (one or two sweeps per row);
            // f32 x (gemv_fuses_quant) is quantised in each launch's prologue
            if (fast_rows_max<TYPE>(g.nb) >= 4 && (!x || TYPE != TYPE_Q8_0))
                return run_fast_m<TYPE>(rm, row_bytes, g.nb, act, x, m, st);
        }
    }
    if (alpha || map != MAP_ONE || rm.end[0] != n) return hipErrorNotSupported;  // m = 1 fast path only
    GemvCfg c = pick_cfg(TYPE, n, g.pieces, m, k);
    c.fused = false;  // m > 1: x arrives quantised (separate kernel)
    if (x) return hipErrorInvalidValue;
    if (m <= 1) return run_m<TYPE, 1>(c, w, g, act, x, m, y, st);
    if (m <= 2) return run_m<TYPE, 2>(c, w, g, act, x, m, y, st);
    if (m <= 4) return run_m<TYPE, 4>(c, w, g, act, x, m, y, st);
    return run_m<TYPE, 8>(c, w, g, act, x, m, y, st);
}

}  // namespace lbq
