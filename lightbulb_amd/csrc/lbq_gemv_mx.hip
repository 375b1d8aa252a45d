// Batch decode on the matrix cores: y[m][n] = x[m][k] . W[n][k]^T for 2 <= m <= 64
// (the shapes gemv_mx_serves admits),
// Q8_K activation rows against Q4_K / Q5_K / Q6_K weights, in the reference's
// integer arithmetic (candle-core 0.10.2 k_quants.rs, BlockQ4K / BlockQ5K vec_dot
// with BlockQ8K: integer sub-block sums scaled by the 6-bit scales, mins against
// the Q8_K bsums, combined with d, dmin and the activation's d in f32; BlockQ6K:
// mx_block6).
//
// Per 32-value sub-block s of a block, the integer dot of every (activation row,
// weight row) pair is one v_mfma_i32_32x32x32_i8: A = the Q8_K codes of the
// activation rows (A rows past m repeat row m - 1 and are never stored), B = 32
// weight rows' 5-bit (Q5_K) or 4-bit (Q4_K) codes, both as int8, so the int32
// sums are exact.  Each lane owns one weight row (lane % 32), so the sub-block's
// 6-bit scale is one value per lane: isum += sc_s * dot_s.  The mins term
// sum_s m_s * bsum_s (bsum_s: the activation codes summed over sub-block s, from
// the Q8_K 16-value sums) is one v_mfma_f32_32x32x16_f16 per block with each
// bsum split as 64*hi + lo (|hi| <= 64, 0 <= lo < 64) against (64*m_s, m_s):
// every operand and partial sum is an integer below 2^24, so it is exact too.
// The block then adds dx * (d*isum - dmin*msum) in f32.
// Where the multi-row decode kernel re-does its 16 sdot4 per 64 weights for every
// activation row, the matrix core does all rows at once: its MFMA work per weight
// does not grow with m (up to the tile's 32 rows), only the per-row scaling does.
//
// Workgroup: 32 weight rows, four (or, with at most one workgroup per CU, eight)
// waves taking every fourth (eighth) block of the row; the partial tiles are
// added in wave order in LDS.  With few tiles, two workgroups share a tile's
// blocks (split k, MxSplit below).
//
// Activations go through a wave-private LDS stage holding MR rows (8, 16 or 32:
// the launch's m rounded up).  Per block (MR * 256 B of codes, MR * 32 B of
// 16-value sums) every lane fetches its own 16-byte chunks -- MR / 4 code chunks
// and one sums chunk, two blocks ahead, into registers -- which are written to the
// stage one block ahead; the A operands are LDS reads.  At MR = 8 a block then
// costs three activation loads (not nine per-lane A-operand loads) and 24
// activation registers (not 72), for three waves per SIMD.  Stage rows past m hold
// a copy of row m - 1 or stale bytes and are never read.  Rows are 256 bytes apart in the stage, so chunk c of
// row r sits in slot c ^ (r & 15): the 16 distinct chunks an A read touches fall
// in different banks.  Weights: one block ahead in registers (a deeper ring
// measured slower: it costs waves per SIMD).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef int i32x16v __attribute__((ext_vector_type(16)));
typedef float f32x16v __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));

template <int TYPE>
struct MxW {
    uint4 hd, qh, qs[4];  // block header (d, dmin, scales), the lane half's qh, its four 16-byte qs quarters
};
// Q6_K (210-byte blocks, 2-byte aligned): lane half h holds bytes 16h..16h+15 of
// each 32-byte region of ql (four) and qh (two) as loaded; mx_block6 trades
// halves between the lane pairs so that each lane ends with its own 8-byte
// pieces.  sc: the 16 int8 group scales; d: the f16 bits of d.
// With AL (mx_load_w), every field is read as aligned dwords -- the 16 bytes at
// or before it and the dword after (xl, xh, xs) -- and funnel-shifted by sh (0 or
// 16 bits, the block's offset past 4-byte alignment) in mx_block6.
template <>
struct MxW<TYPE_Q6_K> {
    uint32_t ql[4][4], qh[2][4], sc[4], d;
    uint32_t xl[4], xh[2], xs, sh;
};
// Q8_0 (34-byte blocks), eight blocks (256 values) per step.  Rows are a multiple
// of 64 values, so a step starts 4-byte aligned and block s at 34 s: the lane
// half's 16 codes (bytes 34 s + 2 + 16 h ..) are 4-byte aligned in odd blocks
// and 2 bytes past alignment in even ones, which are read as the aligned 16 bytes
// before them plus the dword after (x), funnel-shifted in mx_block8.  The first
// raw dword of an even block holds its d in lane half 0; x of an even block holds
// the next (odd) block's d in lane half 1.
template <>
struct MxW<TYPE_Q8_0> {
    uint32_t c[8][4], x[4];
};
// The legacy 32-value types (ggml block_q4_0 / q4_1 / q5_0 / q5_1), eight blocks
// per step: a step starts 16-byte aligned (8 x 18 / 20 / 22 / 24 bytes), and both
// lane halves of a row read each block's 16 code bytes (half h takes nibble h:
// values 16h .. 16h + 15).  Raw aligned dwords per block (mx_block_leg decodes):
//   Q4_0 (18 B at 18 s): even s: the 16 bytes at 18 s and the dword after (d,
//     codes 2..17 bytes in, the next block's d); odd s: the 16 codes at 18 s + 2
//   Q4_1 (20 B): the codes at 20 s + 4, and d | m << 16 (w[4])
//   Q5_0 (22 B): six dwords from 22 s (even s; codes and qh 2 bytes past
//     alignment) or from 22 s - 2 (odd s; d in the high half of the first)
//   Q5_1 (24 B): six dwords d | m << 16, qh, codes
struct MxWL {
    uint32_t w[8][6];
};
template <> struct MxW<TYPE_Q4_0> : MxWL {};
template <> struct MxW<TYPE_Q4_1> : MxWL {};
template <> struct MxW<TYPE_Q5_0> : MxWL {};
template <> struct MxW<TYPE_Q5_1> : MxWL {};
constexpr bool mx_legacy(int t) { return t == TYPE_Q4_0 || t == TYPE_Q4_1 || t == TYPE_Q5_0 || t == TYPE_Q5_1; }
template <int TYPE, bool AL = false>
__device__ __forceinline__ void mx_load_w(const uint8_t *blk, int h, MxW<TYPE> &r) {
    if constexpr (mx_legacy(TYPE)) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(blk);
        auto ld4 = [&](uintptr_t p, uint32_t *v) {
            const u32x4a4 q = gld16((gbytes_c)p);
            v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
        };
#pragma unroll
        for (int s = 0; s < 8; s++) {
            uint32_t *w = r.w[s];
            if constexpr (TYPE == TYPE_Q4_0) {
                ld4(a + 18 * s + (s & 1 ? 2 : 0), w);
                if (!(s & 1)) w[4] = gld4((gbytes_c)(a + 18 * s + 16));
            } else if constexpr (TYPE == TYPE_Q4_1) {
                w[4] = gld4((gbytes_c)(a + 20 * s));
                ld4(a + 20 * s + 4, w);
            } else {
                constexpr int BS = TYPE == TYPE_Q5_0 ? 22 : 24;
                const uintptr_t p = a + BS * s - (TYPE == TYPE_Q5_0 && (s & 1) ? 2 : 0);
                ld4(p, w);
                w[4] = gld4((gbytes_c)(p + 16));
                w[5] = gld4((gbytes_c)(p + 20));
            }
        }
    } else if constexpr (TYPE == TYPE_Q8_0) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(blk);
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const gbytes_c p = (gbytes_c)(a + 34 * s + 16 * h + (s & 1 ? 2 : 0));
            const u32x4a4 v = gld16(p);
            r.c[s][0] = v.x; r.c[s][1] = v.y; r.c[s][2] = v.z; r.c[s][3] = v.w;
            if (!(s & 1)) r.x[s >> 1] = gld4(p + 16);
        }
    } else if constexpr (TYPE == TYPE_Q6_K && AL) {
        const uintptr_t a = reinterpret_cast<uintptr_t>(blk), a4 = a & ~(uintptr_t)3;
        r.sh = (uint32_t)(a & 2u) * 8u;
        auto ld = [&](uintptr_t off, uint32_t *v, uint32_t &x) {
            const u32x4a4 q = gld16((gbytes_c)(a4 + off));
            v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
            x = gld4((gbytes_c)(a4 + off + 16));
        };
#pragma unroll
        for (int c = 0; c < 4; c++) ld(32 * c + 16 * h, r.ql[c], r.xl[c]);
#pragma unroll
        for (int c = 0; c < 2; c++) ld(128 + 32 * c + 16 * h, r.qh[c], r.xh[c]);
        ld(192, r.sc, r.xs);  // xs: bytes 208..209 (d) in its low (aligned block) or high half
    } else if constexpr (TYPE == TYPE_Q6_K) {
#pragma unroll
        for (int c = 0; c < 4; c++) ld16_u2(blk + 32 * c + 16 * h, r.ql[c]);
#pragma unroll
        for (int c = 0; c < 2; c++) ld16_u2(blk + 128 + 32 * c + 16 * h, r.qh[c]);
        ld16_u2(blk + 192, r.sc);
        r.d = ld2_a2(blk + 208);
    } else {
        constexpr int QS = TYPE == TYPE_Q4_K ? 16 : 48;
        r.hd = ld_u4(blk);
        if constexpr (TYPE == TYPE_Q5_K) r.qh = ld_u4(blk + 16 + 16 * h);
#pragma unroll
        for (int c = 0; c < 4; c++) r.qs[c] = ld_u4(blk + QS + 32 * c + 16 * h);
    }
}

// C row (activation row) of accumulator e in lane half h
__device__ __forceinline__ constexpr int mx_row(int e, int h) { return 8 * (e >> 2) + 4 * h + (e & 3); }

// One block: xa = the 8 sub-blocks' A operands, xbv = the lane half's four pairs
// of 16-value sums; accumulator e (of E = MR / 2) is C row mx_row(e, h).
template <int TYPE, bool JIT, int E>
__device__ __forceinline__ void mx_block(const MxW<TYPE> &r, const uint8_t *st, const int *ro, int h, const float *sdx,
                                         float *acc) {
    // A operands: all nine stage reads up front, or (JIT, fewer registers) each
    // right before its MFMA
    i32x4v xa[8];
    if constexpr (!JIT) {
#pragma unroll
        for (int s = 0; s < 8; s++) xa[s] = *reinterpret_cast<const i32x4v *>(st + ro[s]);
    }
    const uint32_t hw0 = r.hd.x, hw1 = r.hd.y, hw2 = r.hd.z, hw3 = r.hd.w;
    // get_scale_min_k4 for the 8 sub-blocks, as packed bytes: j < 4 from bytes j,
    // j + 4; j >= 4 from the nibbles of bytes j + 4 and the top bits of j - 4, j
    const uint32_t sc03 = hw1 & 0x3f3f3f3fu, m03 = hw2 & 0x3f3f3f3fu;
    const uint32_t sc47 = (hw3 & 0x0f0f0f0fu) | ((hw1 >> 2) & 0x30303030u);
    const uint32_t m47 = ((hw3 >> 4) & 0x0f0f0f0fu) | ((hw2 >> 2) & 0x30303030u);
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    int isum[E];
#pragma unroll
    for (int e = 0; e < E; e++) isum[e] = 0;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        // sub-block s = 2c + hn: nibble hn of qs quarter c, fifth bit s of qh
        const uint4 q = r.qs[s >> 1];
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        i32x4v bw;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t v = (qw[w] >> (4 * (s & 1))) & 0x0f0f0f0fu;
            if constexpr (TYPE == TYPE_Q5_K) v |= ((qh[w] >> s) & 0x01010101u) << 4;
            bw[w] = (int)v;
        }
        const i32x16v zero = {};
        if constexpr (JIT) xa[s] = *reinterpret_cast<const i32x4v *>(st + ro[s]);
        const i32x16v o = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[s], bw, zero, 0, 0, 0);
        const int sc = (int)(((s < 4 ? sc03 : sc47) >> (8 * (s & 3))) & 0xffu);
#pragma unroll
        for (int e = 0; e < E; e++) {
            // one v_mad_i32_i24 per sum (the empty asm keeps the compiler from
            // pairing products into mul + add3: 264 -> 232 VALU per block at E = 8)
            isum[e] += __mul24(sc, o[e]);
            asm volatile("" : "+v"(isum[e]));
        }
    }
    // mins: sub-blocks 4h + t of the lane half (k slots 8h + 2t, 8h + 2t + 1)
    const uint32_t mm = h ? m47 : m03;
    const i32x4v xbv = *reinterpret_cast<const i32x4v *>(st + ro[8]);
    const uint32_t xbw[4] = {(uint32_t)xbv.x, (uint32_t)xbv.y, (uint32_t)xbv.z, (uint32_t)xbv.w};
    f16x8v a, b;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int bs = (int)(int16_t)(xbw[t] & 0xffffu) + ((int)xbw[t] >> 16);  // the sub-block's code sum
        a[2 * t] = (_Float16)(bs >> 6);
        a[2 * t + 1] = (_Float16)(bs & 63);
        const int mv = (int)((mm >> (8 * t)) & 0xffu);
        b[2 * t] = (_Float16)(64 * mv);
        b[2 * t + 1] = (_Float16)mv;
    }
    const f32x16v zf = {};
    const f32x16v ms = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, zf, 0, 0, 0);
    const float d = h2f(hw0 & 0xffffu), dmin = h2f(hw0 >> 16);
#pragma unroll
    for (int e = 0; e < E; e++) {
        const float dx = sdx[mx_row(e, h)];
        acc[e] = fmaf(dx, fmaf(d, (float)isum[e], -(dmin * ms[e])), acc[e]);
    }
}

// lanes 32..63 of a and lanes 0..31 of b trade values (v_permlane32_swap)
__device__ __forceinline__ void swap_halves(uint32_t &a, uint32_t &b) {
    const auto v = __builtin_amdgcn_permlane32_swap(a, b, false, false);
    a = v[0];
    b = v[1];
}

// One Q6_K block (candle-core 0.10.2 k_quants.rs, BlockQ6K vec_dot with BlockQ8K:
// per 16-value group g, the integer dot of the 6-bit codes minus 32 with the
// activation codes, times the group's int8 scale, summed over the block in int32,
// then d * dx in f32).  Value v = 128n + 32u + l (l < 32) of a block is nibble
// u >> 1 of ql byte 64n + 32(u & 1) + l with bits 2u, 2u + 1 of qh byte 32n + l
// above it (ggml's layout), so group g = 8n + 2u + (l >= 16) takes bytes
// 16(g & 1)..+15 of ql region 2n + (u & 1) and of qh region n.
// Per group, one v_mfma_i32_32x32x16_i8 of the activation codes against the codes
// q (0..63), lane half h supplying values 16g + 8h .. 16g + 8h + 7, and isum +=
// sc_g * dot_g.  The -32 of every code is sum_g sc_g * 32 * bsum_g (bsum_g: the
// Q8_K 16-value sums), with bsum_g = 16 hi + lo (hi in -128..127, lo in 0..15) as
// two more v_mfma_i32_32x32x16_i8 against the int8 scales (K = the 16 groups).
// Every sum is exact in int32.  xo: the lane's A-read offset in the stage with
// the chunk bits of group 0 (row ra, byte 8h); sbo: its 16-value sums.
template <int E, bool AL = false>
__device__ __forceinline__ void mx_block6(MxW<TYPE_Q6_K> &r, const uint8_t *st, uint32_t xo, int sbo, int h,
                                          const float *sdx, float *acc) {
    if constexpr (AL) {
        auto funnel = [&](uint32_t *v, uint32_t x) {
            const uint32_t v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
            v[0] = __builtin_amdgcn_alignbit(v1, v0, r.sh);
            v[1] = __builtin_amdgcn_alignbit(v2, v1, r.sh);
            v[2] = __builtin_amdgcn_alignbit(v3, v2, r.sh);
            v[3] = __builtin_amdgcn_alignbit(x, v3, r.sh);
        };
#pragma unroll
        for (int c = 0; c < 4; c++) funnel(r.ql[c], r.xl[c]);
#pragma unroll
        for (int c = 0; c < 2; c++) funnel(r.qh[c], r.xh[c]);
        funnel(r.sc, r.xs);
        r.d = (r.xs >> r.sh) & 0xffffu;
    }
    // half 0 keeps bytes 0..7 of a region and takes 16..23 from its partner lane;
    // half 1 keeps 24..31 and takes 8..15: dwords 0, 1 then hold the lane's
    // piece of the region's first 16 values, dwords 2, 3 of its second 16
    uint32_t(&ql)[4][4] = r.ql;
    uint32_t(&qh)[2][4] = r.qh;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        swap_halves(ql[c][0], ql[c][2]);
        swap_halves(ql[c][1], ql[c][3]);
    }
#pragma unroll
    for (int c = 0; c < 2; c++) {
        swap_halves(qh[c][0], qh[c][2]);
        swap_halves(qh[c][1], qh[c][3]);
    }
    int isum[E];
#pragma unroll
    for (int e = 0; e < E; e++) isum[e] = 0;
    const i32x16v zero = {};
    auto dot = [&](int g) {
        const int n = g >> 3, u = (g >> 1) & 3, p = g & 1, c = 2 * n + (u & 1);
        uint32_t bw[2];
#pragma unroll
        for (int w = 0; w < 2; w++) {
            const uint32_t lo = (ql[c][2 * p + w] >> (4 * (u >> 1))) & 0x0f0f0f0fu;
            const uint32_t hi = ((qh[n][2 * p + w] >> (2 * u)) & 0x03030303u) << 4;
            bw[w] = lo | hi;
        }
        const long b = (long)((uint64_t)bw[0] | (uint64_t)bw[1] << 32);
        const long a = *reinterpret_cast<const long *>(st + (xo ^ (16u * g)));
        return __builtin_amdgcn_mfma_i32_32x32x16_i8(a, b, zero, 0, 0, 0);
    };
    // one group's MFMA in flight while the previous one's sums are scaled: the
    // empty asm pins each group's adds in place (otherwise the sums are
    // reassociated after all 16 MFMAs, which then hold 16 result tiles)
    // (at E = 16 each group waits for its own MFMA: the second result tile would
    // take the wave past 256 registers)
    constexpr bool PIPE = E < 16;
    i32x16v o;
    if constexpr (PIPE) o = dot(0);
#pragma unroll
    for (int g = 0; g < 16; g++) {
        i32x16v on;
        if constexpr (!PIPE) o = dot(g);
        else if (g < 15) on = dot(g + 1);
        const int sc = (int)(int8_t)(uint8_t)(r.sc[g >> 2] >> (8 * (g & 3)));
#pragma unroll
        for (int e = 0; e < E; e++) {
            isum[e] += __mul24(sc, o[e]);
            asm volatile("" : "+v"(isum[e]));
        }
        if (PIPE && g < 15) o = on;
    }
    // the offset: A = hi / lo of the row's sums of groups 8h..8h+7, B = those
    // groups' scales
    const i32x4v xbv = *reinterpret_cast<const i32x4v *>(st + sbo);
    uint32_t ah[2], al[2];
#pragma unroll
    for (int w = 0; w < 2; w++) {
        const uint32_t w0 = (uint32_t)xbv[2 * w], w1 = (uint32_t)xbv[2 * w + 1];
        // bytes 0 and 2 of each: bits 4..11 of both int16 sums, and their low nibbles
        ah[w] = __builtin_amdgcn_perm(w1 >> 4, w0 >> 4, 0x06040200u);
        al[w] = __builtin_amdgcn_perm(w1 & 0x000f000fu, w0 & 0x000f000fu, 0x06040200u);
    }
    const uint32_t s0 = h ? r.sc[2] : r.sc[0], s1 = h ? r.sc[3] : r.sc[1];
    const long bs = (long)((uint64_t)s0 | (uint64_t)s1 << 32);
    const i32x16v oh = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)((uint64_t)ah[0] | (uint64_t)ah[1] << 32), bs, zero, 0, 0, 0);
    const i32x16v ol = __builtin_amdgcn_mfma_i32_32x32x16_i8((long)((uint64_t)al[0] | (uint64_t)al[1] << 32), bs, zero, 0, 0, 0);
    const float d = h2f(r.d);
#pragma unroll
    for (int e = 0; e < E; e++) {
        const int tot = isum[e] - 32 * (16 * oh[e] + ol[e]);
        acc[e] = fmaf(d * sdx[mx_row(e, h)], (float)tot, acc[e]);
    }
}

// Eight Q8_0 blocks (candle-core 0.10.2 k_quants.rs, BlockQ8_0 vec_dot with
// BlockQ8_0: per 32-value block the integer dot of the codes, then
// (sum as f32) * d_w * d_x added in f32).  Block s is one v_mfma_i32_32x32x32_i8
// (its A operand is the stage chunk pair of the Q4_K sub-block s); sdx: [8][MR],
// the activation d of block s and row i.  One block's MFMA is in flight while the
// previous one is scaled.
template <int MR>
__device__ __forceinline__ void mx_block8(const MxW<TYPE_Q8_0> &r, const uint8_t *st, const int *ro, int h,
                                          const float *sdx, float *acc) {
    constexpr int E = MR / 2;
    const i32x16v zero = {};
    // the blocks' d: lane half 0 holds the even blocks' (d0 | d2 << 16, d4 | d6 <<
    // 16), half 1 the odd ones'; one exchange gives every lane both
    uint32_t ev[2], od[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const uint32_t own = h ? ((r.x[2 * q] >> 16) | (r.x[2 * q + 1] & 0xffff0000u))
                               : ((r.c[4 * q][0] & 0xffffu) | (r.c[4 * q + 2][0] << 16));
        ev[q] = own;
        od[q] = own;
        swap_halves(ev[q], od[q]);  // ev: half 0's (even), od: half 1's (odd), in both halves
    }
    auto dot = [&](int s) {
        i32x4v bw;
        if (s & 1) {
            bw = i32x4v{(int)r.c[s][0], (int)r.c[s][1], (int)r.c[s][2], (int)r.c[s][3]};
        } else {
            const uint32_t *v = r.c[s];
            bw[0] = (int)__builtin_amdgcn_alignbit(v[1], v[0], 16);
            bw[1] = (int)__builtin_amdgcn_alignbit(v[2], v[1], 16);
            bw[2] = (int)__builtin_amdgcn_alignbit(v[3], v[2], 16);
            bw[3] = (int)__builtin_amdgcn_alignbit(r.x[s >> 1], v[3], 16);
        }
        const i32x4v xa = *reinterpret_cast<const i32x4v *>(st + ro[s]);
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, bw, zero, 0, 0, 0);
    };
    i32x16v o = dot(0);
#pragma unroll
    for (int s = 0; s < 8; s++) {
        i32x16v on;
        if (s < 7) on = dot(s + 1);
        const float dw = h2f(((s & 1 ? od : ev)[s >> 2] >> (16 * ((s >> 1) & 1))) & 0xffffu);
#pragma unroll
        for (int q = 0; q < E / 4; q++) {
            // C rows 8q + 4h .. 8q + 4h + 3 of accumulators 4q .. 4q + 3
            const float4 dx = *reinterpret_cast<const float4 *>(sdx + s * MR + 8 * q + 4 * h);
            const float dv[4] = {dx.x, dx.y, dx.z, dx.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                acc[4 * q + c] = fmaf((float)o[4 * q + c] * dw, dv[c], acc[4 * q + c]);
                asm volatile("" : "+v"(acc[4 * q + c]));
            }
        }
        if (s < 7) o = on;
    }
}

// Eight legacy blocks (candle-core 0.10.2 k_quants.rs vec_dot: BlockQ4_0 / BlockQ5_0
// with BlockQ8_0, per block (sum of (q - 8 or 16) * y) as f32 * d_w * d_y;
// BlockQ4_1 / BlockQ5_1 with BlockQ8_1, + m_w * s_y).  The codes enter the
// v_mfma_i32_32x32x32_i8 as int8 (q - 8 / q - 16 formed bytewise: adding 0x78 /
// 0x70 to a byte below 32 never carries, then flipping bit 7); the Q5 fifth bits
// spread from qh to bit 4 of each byte by one multiply.  sdx / ssx: [8][MR] of
// this step: the activation d and (Q8_1) s of block s and row i.
template <int TYPE, int MR>
__device__ __forceinline__ void mx_block_leg(const MxW<TYPE> &r, const uint8_t *st, const int *ro, int h,
                                             const float *sdx, const float *ssx, float *acc) {
    constexpr int E = MR / 2;
    constexpr bool Q5 = TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1, MIN = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;
    constexpr uint32_t OFS = TYPE == TYPE_Q4_0 ? 0x78787878u : TYPE == TYPE_Q5_0 ? 0x70707070u : 0u;
    const i32x16v zero = {};
    auto dot = [&](int s) {
        const uint32_t *w = r.w[s];
        uint32_t q[4], qh = 0;
        if constexpr (TYPE == TYPE_Q4_0) {
            if (s & 1) {
                q[0] = w[0]; q[1] = w[1]; q[2] = w[2]; q[3] = w[3];
            } else {
                q[0] = __builtin_amdgcn_alignbit(w[1], w[0], 16);
                q[1] = __builtin_amdgcn_alignbit(w[2], w[1], 16);
                q[2] = __builtin_amdgcn_alignbit(w[3], w[2], 16);
                q[3] = __builtin_amdgcn_alignbit(w[4], w[3], 16);
            }
        } else if constexpr (TYPE == TYPE_Q5_0) {
            if (s & 1) {
                qh = w[1];
                q[0] = w[2]; q[1] = w[3]; q[2] = w[4]; q[3] = w[5];
            } else {
                qh = __builtin_amdgcn_alignbit(w[1], w[0], 16);
                q[0] = __builtin_amdgcn_alignbit(w[2], w[1], 16);
                q[1] = __builtin_amdgcn_alignbit(w[3], w[2], 16);
                q[2] = __builtin_amdgcn_alignbit(w[4], w[3], 16);
                q[3] = __builtin_amdgcn_alignbit(w[5], w[4], 16);
            }
        } else if constexpr (TYPE == TYPE_Q5_1) {
            qh = w[1];
            q[0] = w[2]; q[1] = w[3]; q[2] = w[4]; q[3] = w[5];
        } else {
            q[0] = w[0]; q[1] = w[1]; q[2] = w[2]; q[3] = w[3];
        }
        i32x4v bw;
#pragma unroll
        for (int v = 0; v < 4; v++) {
            uint32_t b = (q[v] >> (4 * h)) & 0x0f0f0f0fu;
            if constexpr (Q5) {
                const uint32_t hb = (qh >> (16 * h + 4 * v)) & 0xfu;  // fifth bits of values 16h + 4v ..
                b |= ((hb * 0x00204081u) & 0x01010101u) << 4;
            }
            if constexpr (OFS != 0u) b = (b + OFS) ^ 0x80808080u;
            bw[v] = (int)b;
        }
        const i32x4v xa = *reinterpret_cast<const i32x4v *>(st + ro[s]);
        return __builtin_amdgcn_mfma_i32_32x32x32_i8(xa, bw, zero, 0, 0, 0);
    };
    auto dm = [&](int s) -> uint32_t {  // d | m << 16 of block s (Q4_0, Q5_0: d only)
        if constexpr (TYPE == TYPE_Q4_0) return s & 1 ? r.w[s - 1][4] >> 16 : r.w[s][0] & 0xffffu;
        else if constexpr (TYPE == TYPE_Q5_0) return s & 1 ? r.w[s][0] >> 16 : r.w[s][0] & 0xffffu;
        else if constexpr (TYPE == TYPE_Q4_1) return r.w[s][4];
        else return r.w[s][0];
    };
    i32x16v o = dot(0);
#pragma unroll
    for (int s = 0; s < 8; s++) {
        i32x16v on;
        if (s < 7) on = dot(s + 1);
        const uint32_t dmv = dm(s);
        const float dw = h2f(dmv & 0xffffu);
#pragma unroll
        for (int q = 0; q < E / 4; q++) {
            const float4 dx = *reinterpret_cast<const float4 *>(sdx + s * MR + 8 * q + 4 * h);
            const float dv[4] = {dx.x, dx.y, dx.z, dx.w};
            float sv[4] = {0.f, 0.f, 0.f, 0.f};
            if constexpr (MIN) {
                const float4 sx = *reinterpret_cast<const float4 *>(ssx + s * MR + 8 * q + 4 * h);
                sv[0] = sx.x; sv[1] = sx.y; sv[2] = sx.z; sv[3] = sx.w;
            }
#pragma unroll
            for (int c = 0; c < 4; c++) {
                float a = fmaf((float)o[4 * q + c] * dw, dv[c], acc[4 * q + c]);
                if constexpr (MIN) a = fmaf(h2f(dmv >> 16), sv[c], a);
                acc[4 * q + c] = a;
                asm volatile("" : "+v"(acc[4 * q + c]));
            }
        }
        if (s < 7) o = on;
    }
}

template <int MR>
struct MxX {
    i32x4v c[MR / 4], s;  // codes (rows 4q + lane/16, chunk lane%16), sums (row lane/2, half lane%2)
};

// Split k: `splits` workgroups share a 32-row tile, each taking a contiguous
// range of its blocks, and store their partial tiles (part[split][m][n]) with
// agent-scope stores, which write through to memory instead of staying in this
// XCD's L2.  Once they have completed (vmcnt(0)), a counter increment publishes
// them; the workgroup that completes the tile's count adds the partials in split
// order (the bits do not depend on which workgroup came last), reading them with
// the same agent-scope policy, writes y and puts the counter back to zero for the
// next call.
constexpr int MX_MAX_SPLITS = 16;

// With two workgroups per tile and a y set to zero beforehand (`add`), each
// workgroup instead adds its half into y atomically: two addends give the same
// bits in either order (a NaN output may carry either half's NaN payload), and no
// partials, counter or read-back are needed (1-2 us less per call on the 4096-row
// shapes).
struct MxSplit {
    int splits;     // workgroups per 32-row tile (1: no partials)
    float *part;    // [splits][prow][n]
    uint32_t *cnt;  // one zeroed word per tile
    int add;        // splits == 2 and y zeroed: atomic adds into y
    int prow = 0;   // rows of the partial buffer (the launch's m)
};

// Row halves (m = 33..64): the activation rows run as two 32-row halves, each
// workgroup of the m <= 32 launch becoming two -- workgroups b and b + 8 of every
// 16, which round-robin placement puts on one XCD at about the same time, so the
// second read of a tile's weight blocks is served by that XCD's L2 and HBM
// carries the weights once.  Each half is exactly a launch over its 32 rows (same
// sums, same bits per row).  mx_half_bid: the half of workgroup bid, and bid
// becomes the workgroup of the m <= 32 launch (-1: a padding workgroup, the grid
// being rounded up to 16).  mx_half_rows: act, m, y and the split state of the
// half.
__device__ __forceinline__ int mx_half_bid(int &bid, int nwg) {
    const int half = (bid >> 3) & 1;
    bid = (bid >> 4) * 8 + (bid & 7);
    return bid < nwg ? half : -1;
}
__device__ __forceinline__ void mx_half_rows(int half, int tiles, ActView &act, int &m, float *__restrict__ &y,
                                             int64_t n, MxSplit &sp) {
    sp.prow = m;
    if (half) {
        act.xq += 32 * act.k;
        act.xd += 32 * act.nb;
        act.xbs += 32 * (act.k / 16);
        y += 32 * n;
        if (sp.part) sp.part += 32 * n;
        if (sp.cnt) sp.cnt += tiles;
        m -= 32;
    } else {
        m = 32;
    }
}

// MR = the activation rows a launch can hold (8, 16 or 32; m <= MR).
// PAIR: a gate/up pair (W gate, W2 up, n rows each; one workgroup per tile, no
// split): a tile holds gate rows 16t..16t+15 in columns 0..15 and the same up rows
// in columns 16..31, and the epilogue writes silu(gate) * up (candle's f32 silu,
// v / (1 + exp(-v)), as the separate product launch computes it) for its 16 rows.
// Every column's sums are those of the single-weight launch with the same wave
// count, so the product has the bits of the separate gate and up calls.
// The body of one workgroup (bid: its index within its weight's launch).
template <int TYPE, int MX_WAVES, int MR, bool PAIR>
__device__ __forceinline__ void mx_workgroup(const uint8_t *__restrict__ W, int64_t row_bytes, int n, int nb,
                                             const ActView &act, int m, float *__restrict__ y, const MxSplit &sp,
                                             const uint8_t *__restrict__ W2, int bid) {
    constexpr int E = MR / 2, STAGE = MR * 256 + MR * 32;  // codes of MR rows, then their 16-value sums
    static_assert(E * 64 * 4 <= STAGE, "the partial tile overlays the wave's stage");
    // [nb][MR] (Q8_0: [8 nb][MR]): dx of activation block b, row i (0 past m)
    // (Q8_1: then the s values, the same way)
    extern __shared__ __align__(16) float sdx[];
    __shared__ __align__(16) uint8_t xs[MX_WAVES][STAGE];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int tile = bid / sp.splits, part = bid % sp.splits;
    const int row0 = tile * (PAIR ? 16 : 32);
    const int64_t k = act.k;
    const uint8_t *wr = PAIR ? (j < 16 ? W : W2) + (int64_t)min(row0 + (j & 15), n - 1) * row_bytes
                             : W + (int64_t)min(row0 + j, n - 1) * row_bytes;
    const int p0 = part * nb / sp.splits, np = (part + 1) * nb / sp.splits - p0;  // this workgroup's blocks
    constexpr int BYTES = TYPE == TYPE_Q4_K   ? 144
                          : TYPE == TYPE_Q5_K ? 176
                          : TYPE == TYPE_Q6_K ? 210
                          : TYPE == TYPE_Q8_0 ? 8 * 34
                          : TYPE == TYPE_Q4_0 ? 8 * 18
                          : TYPE == TYPE_Q4_1 ? 8 * 20
                          : TYPE == TYPE_Q5_0 ? 8 * 22
                                              : 8 * 24;
    // Q8_0 / Q8_1 activations: no 16-value sums, a d (and for Q8_1 an s) per 32 values
    constexpr bool Q80 = TYPE == TYPE_Q8_0 || mx_legacy(TYPE);
    constexpr bool XS = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;
    uint8_t *st = xs[wave];
    // this lane's share of a block's activations: MR / 4 code chunks (row 4q +
    // lane / 16, chunk lane % 16) and a sums chunk (row lane / 2, half lane % 2);
    // rows past m are not loaded (their stage rows are never read)
    const int8_t *xc = act.xq + (int64_t)min(lane >> 4, m - 1) * k + 16 * (lane & 15);
    int wo[MR / 4];
#pragma unroll
    for (int q = 0; q < MR / 4; q++) {
        const int r = 4 * q + (lane >> 4), c = lane & 15;
        wo[q] = r * 256 + 16 * (c ^ (r & 15));
    }
    const int srow = (lane >> 1) & (MR - 1);
    const int16_t *xsum = act.xbs + (int64_t)min(srow, m - 1) * (k / 16) + 8 * (lane & 1);
    const bool sl = lane < 2 * MR;  // lanes past 2 MR load copies and write nothing
    const int so = MR * 256 + 16 * (lane & (2 * MR - 1));
    auto load_x = [&](int b, MxX<MR> &x) {
#pragma unroll
        for (int q = 0; q < MR / 4; q++)
            if (q == 0 || 4 * q + (lane >> 4) < m)
                x.c[q] = *reinterpret_cast<const i32x4v *>(xc + (int64_t)(4 * q) * k + 256 * b);
        if constexpr (!Q80) x.s = *reinterpret_cast<const i32x4v *>(xsum + 16 * b);
    };
    auto write_x = [&](const MxX<MR> &x) {
#pragma unroll
        for (int q = 0; q < MR / 4; q++) *reinterpret_cast<i32x4v *>(st + wo[q]) = x.c[q];
        if constexpr (!Q80)
            if (sl) *reinterpret_cast<i32x4v *>(st + so) = x.s;
    };
    // A-operand reads: row ra (A rows past m read row m - 1), chunk 2s + h
    const int ra = min(j, m - 1);
    int ro[9];
#pragma unroll
    for (int s = 0; s < 8; s++) ro[s] = ra * 256 + 16 * ((2 * s + h) ^ (ra & 15));
    ro[8] = MR * 256 + ra * 32 + 16 * h;
    const uint32_t xo6 = (uint32_t)(ra * 256 + 16 * (ra & 15) + 8 * h);  // Q6_K: 8-byte A reads, group 0
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = 0.f;
    // Loads are unconditional, their block clamped to the wave's last one (the
    // tail re-reads it and never uses the copy).  A wave with no blocks (nb < the
    // wave count) loads nothing.
    // The wave's blocks: every MX_WAVES-th from p0 + wave, so at any time the waves
    // of a workgroup read neighbouring blocks of each weight row (one contiguous
    // span per row in flight instead of one per wave: Q4_K 14336 x 4096 m = 8 / 16
    // / 32 16.8 / 19.2 / 22.9 -> 15.7 / 18.2 / 21.9 us, 4096 x 14336 m = 16 19.3 ->
    // 17.3, against contiguous ranges per wave).  Slot i < cnt is block blk(i); a
    // slot past the last is the last block again (the tail re-reads it and never
    // uses the copy).
    const int cnt = np > wave ? (np - wave + MX_WAVES - 1) / MX_WAVES : 0;
    const int il = cnt - 1;
    auto blk = [&](int i) { return p0 + wave + min(i, il) * MX_WAVES; };
    const bool any = cnt > 0;
    MxW<TYPE> rw[2];
    MxX<MR> xr[2];
    // Q6_K blocks are 2-byte aligned: aligned reads and funnel shifts where the
    // registers allow (up to 16 activation rows)
    constexpr bool AL6 = TYPE == TYPE_Q6_K && MR <= 16;
    auto load_w = [&](int b, MxW<TYPE> &dst) { mx_load_w<TYPE, AL6>(wr + (int64_t)b * BYTES, h, dst); };
    if (any) {
        load_x(blk(0), xr[0]);
        load_x(blk(1), xr[1]);
        load_w(blk(0), rw[0]);
        write_x(xr[0]);
    }
    constexpr int DB = Q80 ? 8 : 1;  // activation d values per 256-value block and row
    for (int q = DB * p0 * MR + t; q < DB * (p0 + np) * MR; q += 64 * MX_WAVES) {
        const int b = q / MR, i = q % MR;
        sdx[q] = i < m ? act.xd[(int64_t)i * (DB * nb) + b] : 0.f;
        if constexpr (XS) sdx[DB * nb * MR + q] = i < m ? act.xs[(int64_t)i * (DB * nb) + b] : 0.f;
    }
    __syncthreads();  // sdx (each wave's first stage is its own)
    if (any) {
        for (int i = 0;; i += 2) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                // xr[1 - q] holds slot i + q + 1 (loaded a block ago); xr[q] takes i + q + 2
                load_x(blk(i + q + 2), xr[q]);
                load_w(blk(i + q + 1), rw[1 - q]);
                if constexpr (mx_legacy(TYPE))
                    mx_block_leg<TYPE, MR>(rw[q], st, ro, h, sdx + DB * MR * blk(i + q),
                                           sdx + DB * nb * MR + DB * MR * blk(i + q), acc);
                else if constexpr (Q80) mx_block8<MR>(rw[q], st, ro, h, sdx + DB * MR * blk(i + q), acc);
                else if constexpr (TYPE == TYPE_Q6_K) mx_block6<E, AL6>(rw[q], st, xo6, ro[8], h, sdx + MR * blk(i + q), acc);
                else mx_block<TYPE, (MX_WAVES > 4), E>(rw[q], st, ro, h, sdx + MR * blk(i + q), acc);
                if (i + q == il) break;
                write_x(xr[1 - q]);  // after this block's stage reads (the MFMAs consumed them)
            }
            if (i + 2 > il) break;
        }
    }
    // the wave's partial tile replaces its own stage (its stage reads are done:
    // LDS operations of one wave complete in order)
    float *red = reinterpret_cast<float *>(st);
#pragma unroll
    for (int e = 0; e < E; e++) red[e * 64 + lane] = acc[e];
    __syncthreads();
    // accumulator e (C row mx_row(e, h)) is stored by wave e % MX_WAVES, the
    // partials added in wave order
    if constexpr (PAIR) {
        const int col = row0 + (lane & 15);
        if (j >= 16) return;
        for (int e = wave; e < E; e += MX_WAVES) {
            float g = reinterpret_cast<const float *>(xs[0])[e * 64 + lane];
            float u = reinterpret_cast<const float *>(xs[0])[e * 64 + lane + 16];
#pragma unroll
            for (int w = 1; w < MX_WAVES; w++) {
                g += reinterpret_cast<const float *>(xs[w])[e * 64 + lane];
                u += reinterpret_cast<const float *>(xs[w])[e * 64 + lane + 16];
            }
            const int i = mx_row(e, h);
            if (i < m && col < n) y[(int64_t)i * n + col] = g / (1.f + expf(-g)) * u;
        }
        return;
    }
    const int col = row0 + j;
    for (int e = wave; e < E; e += MX_WAVES) {
        float s = reinterpret_cast<const float *>(xs[0])[e * 64 + lane];
#pragma unroll
        for (int w = 1; w < MX_WAVES; w++) s += reinterpret_cast<const float *>(xs[w])[e * 64 + lane];
        const int i = mx_row(e, h);
        if (i < m && col < n) {
            if (sp.splits == 1) y[(int64_t)i * n + col] = s;
            else if (sp.add) atomicAdd(y + (int64_t)i * n + col, s);
            else __hip_atomic_store(sp.part + ((int64_t)part * sp.prow + i) * n + col, s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    if (sp.splits == 1 || sp.add) return;
    __shared__ uint32_t last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0) last = __hip_atomic_fetch_add(sp.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (last != (uint32_t)(sp.splits - 1)) return;
    for (int e = wave; e < E; e += MX_WAVES) {
        const int i = mx_row(e, h);
        if (i >= m || col >= n) continue;
        const float *pp = sp.part + (int64_t)i * n + col;
        const int64_t stride = (int64_t)sp.prow * n;
        float s = __hip_atomic_load(pp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int q = 1; q < sp.splits; q++) s += __hip_atomic_load(pp + q * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        y[(int64_t)i * n + col] = s;
    }
    if (t == 0) __hip_atomic_store(sp.cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Q6_K's and Q8_0's 32-row stage kernels: two waves per SIMD (at most 256
// registers), which the register allocator would otherwise give up for a few
// registers more
#define MX_MIN_WAVES(TYPE) ((TYPE) == TYPE_Q6_K || (TYPE) == TYPE_Q8_0 ? 2 : 1)

template <int TYPE, int MX_WAVES, int MR, bool PAIR = false, bool HALVES = false>
__global__ __launch_bounds__(64 * MX_WAVES) __attribute__((amdgpu_waves_per_eu(MX_MIN_WAVES(TYPE))))
void k_gemv_mx(const uint8_t *__restrict__ W, int64_t row_bytes, int n,
                                                         int nb, ActView act, int m, float *__restrict__ y, MxSplit sp,
                                                         const uint8_t *__restrict__ W2, int nwg) {
    int bid = (int)blockIdx.x;
    if constexpr (HALVES) {
        const int half = mx_half_bid(bid, nwg);
        if (half < 0) return;
        mx_half_rows(half, nwg / sp.splits, act, m, y, n, sp);
    } else {
        sp.prow = m;
    }
    mx_workgroup<TYPE, MX_WAVES, MR, PAIR>(W, row_bytes, n, nb, act, m, y, sp, W2, bid);
}

// A grouped call's weights (same type and k) in one launch: segment s owns the
// workgroups [wg_end[s - 1], wg_end[s]) and runs them exactly as its own launch
// would (same tiles, splits and wave count), so every output keeps its bits.
// Two-way split segments add into their y, which the quantisation launch zeroed.
struct MxSegs {
    const uint8_t *w[4];
    float *y[4];
    int n[4], splits[4], wg_end[4];
    int count;
};

template <int TYPE, int MX_WAVES, int MR, bool HALVES = false>
__global__ __launch_bounds__(64 * MX_WAVES) __attribute__((amdgpu_waves_per_eu(MX_MIN_WAVES(TYPE))))
void k_gemv_mx_seg(int64_t row_bytes, int nb, ActView act, int m, MxSegs g) {
    int bid = (int)blockIdx.x, half = 0;
    if constexpr (HALVES) {
        half = mx_half_bid(bid, g.wg_end[g.count - 1]);
        if (half < 0) return;
    }
    int s = 0;
    while (s + 1 < g.count && bid >= g.wg_end[s]) s++;
    MxSplit sp{g.splits[s], nullptr, nullptr, g.splits[s] == 2};
    float *__restrict__ y = g.y[s];
    if constexpr (HALVES) mx_half_rows(half, 0, act, m, y, g.n[s], sp);
    else sp.prow = m;
    mx_workgroup<TYPE, MX_WAVES, MR, false>(g.w[s], row_bytes, g.n[s], nb, act, m, y, sp, nullptr,
                                            bid - (s ? g.wg_end[s - 1] : 0));
}

static int mx_splits(int64_t n, int64_t k, int m);

bool gemv_mx_serves(int type, int64_t n, int64_t k, int m) {
    // Measured against the decode kernels (x quantised by the same separate pass
    // unless noted): Q5_K 14336 x 4096 m = 8 22.8 -> 18.2 us, Q4_K 14336 x 4096
    // 21.4 -> 16.8, 4096 x 4096 13.4 -> 12.5, 2048 x 4096 12.5 -> 11.9, 3072 x
    // 4096 m = 6 12.9 -> 11.9; with 1024 rows (32 eight-wave workgroups) 11.5 ->
    // 11.8, so fewer than 2048 rows keep the multi-row kernel.  At m <= 4
    // that kernel quantises x in its own prologue and stays ahead (m = 2: 12.8 vs
    // 17.9 us) -- except at k > 8192, where it cannot hold the activation rows and
    // the general GEMV runs: Q4_K 4096 x 14336 m = 2 / 3 / 4 / 8 22.2 / 26.3 /
    // 30.2 / 52.8 -> 21.0 / 20.9 / 20.8 / 21.0 us.
    // Q6_K only at k > 8192 and m >= 3, where it is ahead of both the decode
    // kernels and the fp16 GEMM (4096 x 14336 m = 4 / 8 / 16 / 32 / 64: 29.3 / 43.6
    // / 28.5 / 29.7 / 42.8 -> 23.6 / 24.0 / 25.6 / 29.2 / 42.6 us; m = 2: 22.1 ->
    // 23.2); at k = 4096 it is not (1024 x 4096 m = 16 9.2 -> 13.1 us, 14336 x 4096
    // m = 32 29.4 -> 31.1, the 128256-row head m = 8 / 16 128.7 / 159.9 -> 151.5 /
    // 167.6): sixteen MFMAs per block and a scaled sum per group and output.
    if (tuning().gemv_mx_off) return false;
    if (mx_legacy(type)) {
        // Q4_0 / Q4_1 / Q5_0 / Q5_1 at m = 5..16 from 1024 rows, k % 256 == 0
        // (eight blocks per step; the 16-row stage at most: six raw dwords per block)
        if (k % 256 || k / 256 > 64 || m < 2 || m > 16 || n <= 0 || n > (int64_t)MAX_ROWS) return false;
        if (tuning().gemv_mx_all) return true;
        return m >= 5 && n >= 1024 && (m <= 8 || !tuning().gemv_mx_wide_off);
    }
    if (type == TYPE_Q8_0) {
        // m = 5..32 from 1024 rows, k % 256 == 0 (eight blocks per step), against
        // the multi-row decode kernel and the fp16 GEMM (4096 x 4096 m = 5 / 8 / 16 /
        // 32 13.8 / 15.7 / 19.0 / 20.7 -> 13.0 / 13.1 / 14.2 / 16.8 us, 14336 x 4096
        // m = 8 / 16 / 32 31.8 / 40.7 / 42.8 -> 26.3 / 29.5 / 34.4, 4096 x 14336 m =
        // 16 / 32 42.3 / 44.4 -> 28.6 / 33.5; m = 3 / 4: 9.8 / 10.0 -> 12.6 / 12.9),
        // and m = 33..64 as row halves at k <= 8192 (4096 x 4096 m = 48 / 64 23.4 /
        // 25.1 -> 21.2 / 22.5, 1024 x 4096 m = 64 20.6 -> 15.6; 4096 x 14336 m = 64
        // 53.2 -> 56.0)
        if (k % 256 || k / 256 > 64 || m < 2 || m > 64 || n <= 0 || n > (int64_t)MAX_ROWS) return false;
        if (m > 32)
            return (k <= 8192 || tuning().gemv_mx_all) && !tuning().gemv_mx_halves_off &&
                   !tuning().gemv_mx_wide_off && n >= 1024 && (n + 31) / 32 * mx_splits(n, k, 32) <= (int64_t)num_cus();
        if (tuning().gemv_mx_all) return true;
        return m >= 5 && n >= 1024 && (m <= 8 || !tuning().gemv_mx_wide_off);
    }
    if (type != TYPE_Q4_K && type != TYPE_Q5_K && type != TYPE_Q6_K) return false;
    if (k % 256 || k / 256 > 64 || m < 2 || m > 64 || n <= 0 || n > (int64_t)MAX_ROWS) return false;
    if (type == TYPE_Q6_K && (k / 256 <= 32 || m == 2) && !tuning().gemv_mx_all) return false;
    // m = 33..64 as two 32-row halves (mx_half_bid) where the m <= 32 launch has
    // at most one workgroup per CU (up to 8192 rows): against the fp16 GEMM, Q4_K m
    // = 64 4096 x 4096 24.1 -> 16.4 us, 1024 x 4096 17.3 -> 11.1, 4096 x 14336 32.1
    // -> 32.0, m = 40 4096 x 4096 21.3 -> 14.7; with more tiles the halves double a
    // launch that is not HBM-bound (14336 x 4096 m = 64 31.8 -> 36.3 us, m = 33
    // 28.5 -> 31.5) and the GEMM keeps them.
    if (m > 32)
        return !tuning().gemv_mx_halves_off && !tuning().gemv_mx_wide_off && n >= 1024 &&
               (n + 31) / 32 * mx_splits(n, k, 32) <= (int64_t)num_cus();
    // m = 9..32 (the fp16 GEMM otherwise): Q4_K 14336 x 4096 m = 16 / 32 22.1 / 23.4
    // -> 18.3 / 21.8 us, Q5_K m = 12 / 24 23.9 / 24.3 -> 18.4 / 21.8, 4096 x 14336
    // m = 16 23.6 -> 20.3, 4096 x 4096 m = 32 16.1 -> 14.9; with two workgroups per
    // tile adding into y atomically, 1024 / 2048 rows too (1024 x 4096 m = 16 / 32
    // 10.7 / 13.0 -> 10.2 / 11.9, 2048 x 4096 11.3 / 13.9 -> 10.4 / 12.1), and at
    // m = 5..8 from 1024 rows (1024 x 4096 m = 8 11.2 -> 9.5).  Below 1024 rows:
    // not measured, the other kernels keep those.
    if (tuning().gemv_mx_all) return m <= 8 || !tuning().gemv_mx_wide_off;
    if (m > 8) return !tuning().gemv_mx_wide_off && n >= 1024;
    if (k / 256 > 32) return true;  // the multi-row decode kernel cannot hold these rows
    return m >= 5 && n >= 1024;
}

// Workgroups per 32-row tile: two up to 128 tiles (4096 rows), which fills the
// chip's 256 CUs with eight-wave workgroups.  Measured (Q4_K, x quantised by the
// separate pass): 4096 x 14336 m = 8 / 16 / 32 20.6 / 24.1 / 30.5 -> 17.5 / 20.3
// / 25.4 us, 4096 x 4096 m = 8 / 16 / 32 12.0 / 13.0 / 15.6 -> 11.2 / 12.1 /
// 14.9; four workgroups per tile (or four waves each) measured slower.
static int mx_splits(int64_t n, int64_t k, int m) {
    const int64_t tiles = (n + 31) / 32;
    const int nb = (int)(k / 256);
    int s = tuning().gemv_mx_splits;
    if (s <= 0) s = tiles <= 128 ? 2 : 1;
    s = (int)std::min<int64_t>({(int64_t)s, (int64_t)nb, (int64_t)MX_MAX_SPLITS});
    if (tiles * (m > 32 ? 2 : 1) > KS_COUNTERS) s = 1;  // a counter per tile and row half
    return std::max(s, 1);
}

size_t gemv_mx_workspace_bytes(int type, int64_t n, int64_t k, int m) {
    if (!gemv_mx_serves(type, n, k, m)) return 0;
    const int s = mx_splits(n, k, m);
    return s > 1 ? (size_t)s * (size_t)m * (size_t)n * sizeof(float) : 0;
}

bool gemv_mx_adds(int type, int64_t n, int64_t k, int m) {
    return gemv_mx_serves(type, n, k, m) && mx_splits(n, k, m) == 2;
}

// Grid of a launch of nwg workgroups: twice that, rounded up to 16, with row halves
static unsigned mx_grid(int64_t nwg, int m) { return (unsigned)(m > 32 ? (nwg + 7) / 8 * 16 : nwg); }
// activation rows a launch's stage holds: 8, 16 or 32 (each half's 32 with row halves)
static int mx_rows(int m) { return m <= 8 ? 8 : m <= 16 ? 16 : 32; }

// f(std::integral_constant<int, type>) for the types this kernel serves
template <typename F>
static void mx_typed(int type, F &&f) {
    if (type == TYPE_Q4_K) f(std::integral_constant<int, TYPE_Q4_K>{});
    else if (type == TYPE_Q5_K) f(std::integral_constant<int, TYPE_Q5_K>{});
    else if (type == TYPE_Q6_K) f(std::integral_constant<int, TYPE_Q6_K>{});
    else if (type == TYPE_Q8_0) f(std::integral_constant<int, TYPE_Q8_0>{});
    else if (type == TYPE_Q4_0) f(std::integral_constant<int, TYPE_Q4_0>{});
    else if (type == TYPE_Q4_1) f(std::integral_constant<int, TYPE_Q4_1>{});
    else if (type == TYPE_Q5_0) f(std::integral_constant<int, TYPE_Q5_0>{});
    else f(std::integral_constant<int, TYPE_Q5_1>{});
}

// The activation view a launch of `type` reads: Q8_K codes, d per 256 values and
// 16-value sums; Q8_0 codes and d per 32 values.
static bool mx_act_ok(int type, const ActView &act, int64_t k) {
    const bool x32 = type == TYPE_Q8_0 || mx_legacy(type), xs = type == TYPE_Q4_1 || type == TYPE_Q5_1;
    return act.k == k && act.nb == (x32 ? k / 32 : k / 256) && act.xq && act.xd && (x32 || act.xbs) && (!xs || act.xs);
}
// LDS for the activation scales of a launch (see mx_workgroup)
static size_t mx_lds(int type, int64_t k, int m) {
    const bool x32 = type == TYPE_Q8_0 || mx_legacy(type), xs = type == TYPE_Q4_1 || type == TYPE_Q5_1;
    return (size_t)(k / 256) * (x32 ? 8 : 1) * (xs ? 2 : 1) * mx_rows(m) * sizeof(float);
}

template <int TYPE, int WAVES, bool PAIR>
static void mx_launch(int m, unsigned grid, size_t lds, hipStream_t st, const uint8_t *w, int64_t row_bytes, int n,
                      int nb, const ActView &act, float *y, const MxSplit &sp, const uint8_t *w2, int nwg) {
    auto go = [&](auto kern) { kern<<<grid, 64 * WAVES, lds, st>>>(w, row_bytes, n, nb, act, m, y, sp, w2, nwg); };
    if constexpr (mx_legacy(TYPE)) {  // (m <= 16: gemv_mx_serves)
        if (m > 8) go(k_gemv_mx<TYPE, WAVES, 16, PAIR>);
        else go(k_gemv_mx<TYPE, WAVES, 8, PAIR>);
        return;
    } else {
    if constexpr (!PAIR) {  // (a pair has more tiles than CUs: never row halves)
        if (m > 32) return go(k_gemv_mx<TYPE, WAVES, 32, false, true>);
    }
    if (m > 16) go(k_gemv_mx<TYPE, WAVES, 32, PAIR>);
    else if (m > 8) go(k_gemv_mx<TYPE, WAVES, 16, PAIR>);
    else go(k_gemv_mx<TYPE, WAVES, 8, PAIR>);
    }
}

template <int TYPE, int WAVES>
static void mx_seg_launch(int m, unsigned grid, size_t lds, hipStream_t st, int64_t row_bytes, int nb,
                          const ActView &act, const MxSegs &g) {
    auto go = [&](auto kern) { kern<<<grid, 64 * WAVES, lds, st>>>(row_bytes, nb, act, m, g); };
    if constexpr (mx_legacy(TYPE)) {  // (m <= 16: gemv_mx_serves)
        if (m > 8) go(k_gemv_mx_seg<TYPE, WAVES, 16>);
        else go(k_gemv_mx_seg<TYPE, WAVES, 8>);
    } else if (m > 32) go(k_gemv_mx_seg<TYPE, WAVES, 32, true>);
    else if (m > 16) go(k_gemv_mx_seg<TYPE, WAVES, 32>);
    else if (m > 8) go(k_gemv_mx_seg<TYPE, WAVES, 16>);
    else go(k_gemv_mx_seg<TYPE, WAVES, 8>);
}

hipError_t launch_gemv_mx_group(int type, int count, const uint8_t *const *w, const int64_t *n, int64_t k,
                                int64_t row_bytes, const ActView &act, int m, float *const *y, hipStream_t st) {
    if (count < 2 || count > 4) return hipErrorNotSupported;
    const int nb = (int)(k / 256);
    if (!mx_act_ok(type, act, k)) return hipErrorInvalidValue;
    MxSegs g{};
    int waves = 0, wg = 0;
    for (int i = 0; i < count; i++) {
        if (!gemv_mx_serves(type, n[i], k, m)) return hipErrorNotSupported;
        const int s = mx_splits(n[i], k, m);
        if (s > 2) return hipErrorNotSupported;  // only the atomic form of a split
        const int64_t tiles = (n[i] + 31) / 32;
        const int wv = tuning().gemv_mx_waves ? tuning().gemv_mx_waves
                       : (int64_t)mx_grid(tiles * s, m) <= (int64_t)num_cus() ? 8 : 4;
        if (i && wv != waves) return hipErrorNotSupported;  // each weight as its own launch would run it
        waves = wv;
        wg += (int)(tiles * s);
        g.w[i] = w[i];
        g.y[i] = y[i];
        g.n[i] = (int)n[i];
        g.splits[i] = s;
        g.wg_end[i] = wg;
    }
    g.count = count;
    const size_t lds = mx_lds(type, k, m);
    const unsigned grid = mx_grid(wg, m);
    mx_typed(type, [&](auto T) {
        if (waves == 8) mx_seg_launch<T.value, 8>(m, grid, lds, st, row_bytes, nb, act, g);
        else mx_seg_launch<T.value, 4>(m, grid, lds, st, row_bytes, nb, act, g);
    });
    return hipGetLastError();
}

bool gemv_mx_pair_serves(int type, int64_t n, int64_t k, int m) {
    // above 8192 rows the single-weight launches take one four-wave workgroup per
    // 32-row tile, as the pair launch does per 16-row pair tile (the same sums)
    return !tuning().gemv_mx_pair_off && n > 8192 && gemv_mx_serves(type, n, k, m) && mx_splits(n, k, m) == 1 &&
           (n + 31) / 32 > (int64_t)num_cus() && !tuning().gemv_mx_waves;
}

hipError_t launch_gemv_mx_pair(int type, const uint8_t *w_gate, const uint8_t *w_up, int64_t n, int64_t k,
                               int64_t row_bytes, const ActView &act, int m, float *out, hipStream_t st) {
    if (!gemv_mx_pair_serves(type, n, k, m)) return hipErrorNotSupported;
    const int nb = (int)(k / 256);
    if (!mx_act_ok(type, act, k)) return hipErrorInvalidValue;
    const MxSplit sp{1, nullptr, nullptr, 0};
    const int nwg = (int)((n + 15) / 16);
    const size_t lds = mx_lds(type, k, m);
    mx_typed(type, [&](auto T) {
        mx_launch<T.value, 4, true>(m, mx_grid(nwg, m), lds, st, w_gate, row_bytes, (int)n, nb, act, out, sp, w_up, nwg);
    });
    return hipGetLastError();
}

hipError_t launch_gemv_mx(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act, int m,
                          float *y, float *ws, uint32_t *counters, hipStream_t st, bool y_zeroed) {
    if (!gemv_mx_serves(type, n, k, m)) return hipErrorNotSupported;
    const int nb = (int)(k / 256);
    if (!mx_act_ok(type, act, k)) return hipErrorInvalidValue;
    MxSplit sp{mx_splits(n, k, m), ws, counters, 0};
    sp.add = sp.splits == 2 && y_zeroed;
    if (sp.splits > 1 && !sp.add && (!ws || !counters)) return hipErrorInvalidValue;
    const int nwg = (int)((n + 31) / 32 * sp.splits);
    const unsigned grid = mx_grid(nwg, m);
    // Up to one workgroup per CU: eight waves split a row's blocks (2 per wave at
    // k = 4096), A operands read just in time to stay within four waves per SIMD
    // (4096 x 14336 m = 4: 21.8 -> 19.5 us; 4096 x 4096 m = 8: 12.9 -> 12.4).  With
    // more workgroups, four waves (14336 x 4096 m = 8: 16.9 at four, 18.7 at eight).
    const bool w8 = tuning().gemv_mx_waves ? tuning().gemv_mx_waves == 8 : (int64_t)grid <= (int64_t)num_cus();
    const size_t lds = mx_lds(type, k, m);
    mx_typed(type, [&](auto T) {
        if (w8) mx_launch<T.value, 8, false>(m, grid, lds, st, w, row_bytes, (int)n, nb, act, y, sp, nullptr, nwg);
        else mx_launch<T.value, 4, false>(m, grid, lds, st, w, row_bytes, (int)n, nb, act, y, sp, nullptr, nwg);
    });
    return hipGetLastError();
}

}  // namespace lbq
