// lbq_gemm.hip -- host side of the batched path (m > 8): the launch plan, the
// fp16 operand pre-pass (Q8_K / Q8_0 activation rows -> MFMA A operands), the
// split-k sum, the per-row weight exponents and the entry points lbq_api.cpp
// calls.  The MFMA kernels are in lbq_gemm_kernels.hpp, instantiated per weight
// type in lbq_gemm_<type>.hip.
#include "lbq_gemm_kernels.hpp"

namespace lbq {

// the MFMA kernels of each type are compiled in that type's own unit
#define LBQ_GEMM_EXTERN(T)                                                                                          \
    extern template hipError_t launch_typed<T>(const Plan &, const uint8_t *, const int8_t *, int64_t, int64_t,      \
                                               const _Float16 *, const int *, const _Float16 *, int64_t, int64_t,    \
                                               float *, int64_t, uint32_t *, float *, const float *, hipStream_t);
LBQ_GEMM_EXTERN(TYPE_Q4_K)
LBQ_GEMM_EXTERN(TYPE_Q5_K)
LBQ_GEMM_EXTERN(TYPE_Q6_K)
LBQ_GEMM_EXTERN(TYPE_Q8_0)
LBQ_GEMM_EXTERN(TYPE_Q4_0)
LBQ_GEMM_EXTERN(TYPE_Q4_1)
LBQ_GEMM_EXTERN(TYPE_Q5_0)
LBQ_GEMM_EXTERN(TYPE_Q5_1)
LBQ_GEMM_EXTERN(TYPE_Q2_K)
LBQ_GEMM_EXTERN(TYPE_Q3_K)
#undef LBQ_GEMM_EXTERN

// ---------------------------------------------------------------------------
// Pre-pass: Q8_K rows (codes + block scales) -> fp16 operand rows in the GEMM's k
// order, and the row exponent e_m.  One workgroup of T threads per row (T = 1024
// for few rows, so the row's chunks are converted in one pass): the threads
// share the maximum of the row's block scales through LDS, then convert
// 16-code chunks.
// ---------------------------------------------------------------------------
// QB: values per activation scale block (256: Q8_K, 32: Q8_0 / Q8_1).
//
// ofs (Q8_1 rows of Q4_1 / Q5_1 weights): also the extra k-step's A operands,
// per super-block 16 values: position 8h + j (j < 4) holds the stored block sum
// s of block 4h + j times 2^-e_m, exact in f16; positions 8h + 4.. are zero.  So
// that s (up to 32 times the largest activation value) fits f16, e_m is 5 larger
// for these rows: their largest value lies in [2^9, 2^10) -- still 2^23 above
// the f16 subnormal range.
__device__ __forceinline__ int64_t ofs_pos(int64_t m, int64_t k, int64_t blk32) {
    const int j = (int)(blk32 & 7);
    return (m * (k / KB) + blk32 / 8) * 16 + 8 * (j >> 2) + (j & 3);
}

template <int T, int QB>
__global__ __launch_bounds__(T) void k_act_f16(ActView act, int64_t M, _Float16 *__restrict__ A,
                                               int *__restrict__ erow, int opmajor, _Float16 *__restrict__ ofs) {
    __shared__ float wmax[T / 64];
    const int64_t m = blockIdx.x;
    const int t = threadIdx.x;
    const int nb = act.nb;
    const float *xd = act.xd + m * nb;
    float mx = 0.f;
    for (int b = t; b < nb; b += T) mx = fmaxf(mx, fabsf(xd[b]));
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((t & 63) == 0) wmax[t >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < T / 64; w++) mx = fmaxf(mx, wmax[w]);
    // max |d_x| = f*2^E, f in [0.5, 1): |q8*d_x| < 128*2^E, so e = E - 8 keeps the
    // row's values below 2^15 and its largest at or above 2^14 (E - 3 with ofs:
    // below 2^10)
    const int e = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) - (ofs ? 3 : 8) : 0;
    if (t == 0) erow[m] = e;
    const int8_t *q = act.xq + m * act.k;
    for (int64_t c = 16 * t; c < act.k; c += 16 * T) {
        if (ofs) {  // Q8_1 rows (QB = 32): one chunk of each block writes s, the other a zero
            const int64_t blk = c / 32;
            const float sv = (c & 16) ? 0.f : __builtin_amdgcn_ldexpf(act.xs[m * nb + blk], -e);
            ofs[ofs_pos(m, act.k, blk) + ((c & 16) ? 4 : 0)] = (_Float16)sv;
        }
        const uint4 w = *reinterpret_cast<const uint4 *>(q + c);
        const float sx = __builtin_amdgcn_ldexpf(xd[c / QB], -e);
        const float cc = -1152.f * sx;
        uint32_t v[8];
        codes_to_f16(w.x, sx, cc, &v[0], &v[1]);
        codes_to_f16(w.y, sx, cc, &v[2], &v[3]);
        codes_to_f16(w.z, sx, cc, &v[4], &v[5]);
        codes_to_f16(w.w, sx, cc, &v[6], &v[7]);
        const int64_t b = c / KB;
        const int p8 = (int)(c % KB) / 8;
        *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, b, p8, act.k)) = make_uint4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, b, p8 + 1, act.k)) = make_uint4(v[4], v[5], v[6], v[7]);
    }
}

// The same operand rows straight from f32 x (k <= 16384): the workgroup
// quantises its row to Q8_K in registers (q8k_lane16, as the standalone
// quantiser), shares the block scales through LDS for the row exponent, and
// converts with the same arithmetic as k_act_f16 -- one launch instead of two,
// bit-identical operands.  P: passes of T / 16 blocks, the fewest covering the
// row (every load of a pass is issued, so no more passes than the row needs).
template <int T, int P>
__global__ __launch_bounds__(T) void k_quant_f16(const float *__restrict__ x, int64_t K, _Float16 *__restrict__ A,
                                                 int *__restrict__ erow, int opmajor) {
    constexpr int BPP = T / 16, MAXP = P;  // passes of BPP blocks, 64 blocks at most
    static_assert(BPP * P <= 64 && P >= 1, "at most 64 blocks per row");
    __shared__ float wmax[T / 64];
    const int64_t m = blockIdx.x;
    const int t = threadIdx.x, sub = t & 15;
    const int nbx = (int)(K / KB), np = (nbx + BPP - 1) / BPP;
    const float *xr = x + m * K;
    float v[MAXP][16];
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
        const int b = min(BPP * j + (t >> 4), nbx - 1);
        const float4 *src = reinterpret_cast<const float4 *>(xr + (int64_t)b * KB + 16 * sub);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = src[i];
            v[j][4 * i] = f.x; v[j][4 * i + 1] = f.y; v[j][4 * i + 2] = f.z; v[j][4 * i + 3] = f.w;
        }
    }
    uint4 codes[MAXP];
    float dj[MAXP];
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
        codes[j] = make_uint4(0u, 0u, 0u, 0u);
        dj[j] = 0.f;
        if (j < np) {  // workgroup-uniform
            uint32_t packed[4];
            int sum;
            q8k_lane16(v[j], sub, packed, &sum, &dj[j]);
            codes[j] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            if (BPP * j + (t >> 4) < nbx) mx = fmaxf(mx, fabsf(dj[j]));
        }
    }
    // the row's largest |d|: a wave reduction, then across the waves (fmaxf never
    // returns a NaN operand over a number, so the order does not matter)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((t & 63) == 0) wmax[t >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < T / 64; w++) mx = fmaxf(mx, wmax[w]);
    const int e = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) - 8 : 0;  // as k_act_f16
    if (t == 0) erow[m] = e;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
        const int b = BPP * j + (t >> 4);
        if (j < np && b < nbx) {
            const float sx = __builtin_amdgcn_ldexpf(dj[j], -e);
            const float cc = -1152.f * sx;
            uint32_t w8[8];
            codes_to_f16(codes[j].x, sx, cc, &w8[0], &w8[1]);
            codes_to_f16(codes[j].y, sx, cc, &w8[2], &w8[3]);
            codes_to_f16(codes[j].z, sx, cc, &w8[4], &w8[5]);
            codes_to_f16(codes[j].w, sx, cc, &w8[6], &w8[7]);
            *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, b, 2 * sub, K)) = make_uint4(w8[0], w8[1], w8[2], w8[3]);
            *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, b, 2 * sub + 1, K)) = make_uint4(w8[4], w8[5], w8[6], w8[7]);
        }
    }
}

// The operand rows for Q8_0 weights straight from f32 x (k <= 16384): the
// workgroup quantises its row to Q8_0 as candle's BlockQ8_0::from_float does
// (two lanes per 32-value block, the decode prologue's arithmetic), shares the
// stored f16 scales through LDS for the row exponent, and converts with
// k_act_f16's arithmetic -- bit-identical operands, one launch.
// With ofs (Q4_1 / Q5_1 weights: candle's BlockQ8_1::from_float codes are these
// Q8_0 codes), also the extra k-step's operands of k_act_f16, from the block sum
// s = f16(f16(sum of codes) * d) the reference stores.
template <int T>
__global__ __launch_bounds__(T) void k_quant_f16_q80(const float *__restrict__ x, int64_t K, _Float16 *__restrict__ A,
                                                     int *__restrict__ erow, int opmajor, _Float16 *__restrict__ ofs) {
    constexpr int BPP = T / 2, MAXP = 512 / BPP;  // passes of BPP blocks, 512 blocks at most
    __shared__ float wmax[T / 64];
    const int64_t m = blockIdx.x;
    const int t = threadIdx.x, sub = t & 1;
    const int nbx = (int)(K / 32), np = (nbx + BPP - 1) / BPP;
    const float *xr = x + m * K;
    float v[MAXP][16];
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
        const int b = min(BPP * j + (t >> 1), nbx - 1);
        const float4 *src = reinterpret_cast<const float4 *>(xr + (int64_t)b * 32 + 16 * sub);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = src[i];
            v[j][4 * i] = f.x; v[j][4 * i + 1] = f.y; v[j][4 * i + 2] = f.z; v[j][4 * i + 3] = f.w;
        }
    }
    uint32_t codes[MAXP][4];
    float dj[MAXP], sj[MAXP];
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
        codes[j][0] = codes[j][1] = codes[j][2] = codes[j][3] = 0u;
        dj[j] = 0.f;
        if (j < np) {  // workgroup-uniform: the shuffle stays convergent
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[j][i]));
            amax = fmaxf(amax, __shfl_xor(amax, 1));
            const float d = amax / 127.f;
            const float id = d != 0.f ? 1.f / d : 0.f;
            int sum = 0;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float r = roundf(v[j][i] * id);
                const int q = (r != r) ? 0 : (int)fminf(fmaxf(r, -128.f), 127.f);
                codes[j][i >> 2] |= ((uint32_t)q & 0xffu) << (8 * (i & 3));
                sum += q;
            }
            dj[j] = __half2float(__float2half_rn(d));  // the stored scale
            sum += __shfl_xor(sum, 1);
            sj[j] = __half2float(__float2half_rn(__half2float(__float2half_rn((float)sum)) * dj[j]));
            if (BPP * j + (t >> 1) < nbx) mx = fmaxf(mx, fabsf(dj[j]));
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((t & 63) == 0) wmax[t >> 6] = mx;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < T / 64; w++) mx = fmaxf(mx, wmax[w]);
    const int e = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) - (ofs ? 3 : 8) : 0;  // as k_act_f16
    if (t == 0) erow[m] = e;
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
        const int b = BPP * j + (t >> 1);
        if (j < np && b < nbx) {
            if (ofs) ofs[ofs_pos(m, K, b) + 4 * sub] = (_Float16)(sub ? 0.f : __builtin_amdgcn_ldexpf(sj[j], -e));
            const float sx = __builtin_amdgcn_ldexpf(dj[j], -e);
            const float cc = -1152.f * sx;
            uint32_t w8[8];
            codes_to_f16(codes[j][0], sx, cc, &w8[0], &w8[1]);
            codes_to_f16(codes[j][1], sx, cc, &w8[2], &w8[3]);
            codes_to_f16(codes[j][2], sx, cc, &w8[4], &w8[5]);
            codes_to_f16(codes[j][3], sx, cc, &w8[6], &w8[7]);
            const int64_t c = (int64_t)b * 32 + 16 * sub;  // first value of the lane's 16
            const int p8 = (int)(c % KB) / 8;
            *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, c / KB, p8, K)) = make_uint4(w8[0], w8[1], w8[2], w8[3]);
            *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, c / KB, p8 + 1, K)) = make_uint4(w8[4], w8[5], w8[6], w8[7]);
        }
    }
}

// y = sum over s < S of part[s] (fixed order: ((p0 + p1) + p2) + ...), count
// values.  Four values per thread, the partials' loads issued eight slices at a
// time (a runtime trip count would otherwise serialise them).
__global__ __launch_bounds__(256) void k_split_sum(const float *__restrict__ part, int S, int64_t count,
                                                   float *__restrict__ y) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= count) return;
    if (i + 4 <= count && (reinterpret_cast<uintptr_t>(y) & 15u) == 0 && (count & 3) == 0) {
        const float4 *pp = reinterpret_cast<const float4 *>(part + i);
        const int64_t st = count / 4;
        float4 acc = pp[0];
        for (int z0 = 1; z0 < S; z0 += 8) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (z0 + j < S) v[j] = pp[(int64_t)(z0 + j) * st];
#pragma unroll
            for (int j = 0; j < 8; j++)
                if (z0 + j < S) { acc.x += v[j].x; acc.y += v[j].y; acc.z += v[j].z; acc.w += v[j].w; }
        }
        *reinterpret_cast<float4 *>(y + i) = acc;
        return;
    }
    for (int64_t e = i; e < min(i + 4, count); e++) {
        float a = part[e];
        for (int z = 1; z < S; z++) a += part[(int64_t)z * count + e];
        y[e] = a;
    }
}

// The k-sliced layout's operand rows with Q8_K activations: one wave per (row m,
// exponent group g of KS_BLOCKS blocks), 16 lanes per block.  Each block is
// quantised as k_quant_f16 does (q8k_lane16) or read from Q8_K codes; the group's
// largest |d| gives e (as k_act_f16's row exponent, over the group's blocks only),
// stored at erow[g * M + m]; the codes are converted with k_act_f16's arithmetic.
// So every row costs one memory round trip instead of a 1024-thread pass per row.
// SRC_X: quantise f32 x (k <= 16384, 16-byte aligned); otherwise codes from act.
template <bool SRC_X>
__global__ __launch_bounds__(64) void k_ops_ks(const float *__restrict__ x, ActView act, int64_t K, int64_t M,
                                               _Float16 *__restrict__ A, int *__restrict__ erow, int opmajor) {
    const int nb = (int)(K / KB), ng = (nb + KS_BLOCKS - 1) / KS_BLOCKS;
    const int64_t m = blockIdx.x / ng;
    const int g = (int)(blockIdx.x % ng);
    const int lane = threadIdx.x, sub = lane & 15;
    const int b = KS_BLOCKS * g + (lane >> 4);
    const bool live = b < nb;  // a short last group: lanes of missing blocks only help reduce
    const int bc = live ? b : nb - 1;
    uint32_t packed[4];
    float d;
    if constexpr (SRC_X) {
        const float4 *src = reinterpret_cast<const float4 *>(x + m * K + (int64_t)bc * KB + 16 * sub);
        float v[16];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = src[i];
            v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
        }
        int sum;
        q8k_lane16(v, sub, packed, &sum, &d);
    } else {
        const uint4 w = *reinterpret_cast<const uint4 *>(act.xq + m * act.k + (int64_t)bc * KB + 16 * sub);
        packed[0] = w.x; packed[1] = w.y; packed[2] = w.z; packed[3] = w.w;
        d = act.xd[m * act.nb + bc];
    }
    float mx = live ? fabsf(d) : 0.f;
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const int e = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) - 8 : 0;  // as k_act_f16, over the group
    if (lane == 0) erow[(int64_t)g * M + m] = e;
    if (!live) return;
    const float sx = __builtin_amdgcn_ldexpf(d, -e);
    const float cc = -1152.f * sx;
    uint32_t w8[8];
    codes_to_f16(packed[0], sx, cc, &w8[0], &w8[1]);
    codes_to_f16(packed[1], sx, cc, &w8[2], &w8[3]);
    codes_to_f16(packed[2], sx, cc, &w8[4], &w8[5]);
    codes_to_f16(packed[3], sx, cc, &w8[6], &w8[7]);
    *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, b, 2 * sub, K)) = make_uint4(w8[0], w8[1], w8[2], w8[3]);
    *reinterpret_cast<uint4 *>(A + op_pos(opmajor, m, b, 2 * sub + 1, K)) = make_uint4(w8[4], w8[5], w8[6], w8[7]);
}

// ---------------------------------------------------------------------------
// Per-row operand exponents, once per weight: e_n such that the largest value
// any block of row n can produce, B_n, satisfies B_n * 2^-e_n < 2^15.  The
// bound is the largest |d|, |dmin| of the row's blocks times the largest code
// and scale products of the format: Q4_K 63*15 |d| + 63 |dmin|, Q5_K
// 63*31 |d| + 63 |dmin|, Q6_K 128*32 |d|, Q8_0 128 |d|, Q4_0 8 |d|, Q4_1
// 15 |d| + |m|, Q5_0 16 |d|, Q5_1 31 |d| + |m|, Q2_K 3*15 |d| + 15 |dmin|, Q3_K
// 4*32 |d| (the min / offset m in the dmin column).  Non-finite scales are
// left out (their blocks produce non-finite values whatever the exponent); a
// row of zero scales gets e_n = 0.  One thread per row.
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ __launch_bounds__(256) void k_row_exponents(const uint8_t *__restrict__ W, int64_t N, int nb,
                                                        int64_t row_bytes, int8_t *__restrict__ rexp) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    const uint8_t *row = W + n * row_bytes;
    // bytes per block (of 256 values, or 32 for Q8_0 and the legacy types)
    constexpr int SB = TYPE == TYPE_Q4_K ? 144 : TYPE == TYPE_Q5_K ? 176 : TYPE == TYPE_Q6_K ? 210
                     : TYPE == TYPE_Q4_0 ? 18 : TYPE == TYPE_Q4_1 ? 20 : TYPE == TYPE_Q5_0 ? 22
                     : TYPE == TYPE_Q5_1 ? 24 : TYPE == TYPE_Q2_K ? 84 : TYPE == TYPE_Q3_K ? 110 : 34;
    float dm = 0.f, mm = 0.f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = row + (int64_t)b * SB;
        float d, dmin = 0.f;
        if constexpr (TYPE == TYPE_Q6_K) {
            d = h2f(ld2_a2(blk + 208));
        } else if constexpr (TYPE == TYPE_Q3_K) {
            d = h2f(ld2_a2(blk + 108));
        } else if constexpr (TYPE == TYPE_Q8_0 || TYPE == TYPE_Q4_0 || TYPE == TYPE_Q5_0) {
            d = h2f(ld2_a2(blk));
        } else {
            // d | dmin (Q4_K, Q5_K, Q2_K at byte 80) or d | m (Q4_1, Q5_1), 4-byte aligned
            const uint32_t hdr = ld_u32(blk + (TYPE == TYPE_Q2_K ? 80 : 0));
            d = h2f(hdr & 0xffffu);
            dmin = h2f(hdr >> 16);
        }
        d = fabsf(d);
        dmin = fabsf(dmin);
        if (d <= 3.4e38f) dm = fmaxf(dm, d);  // false for NaN and Inf
        if (dmin <= 3.4e38f) mm = fmaxf(mm, dmin);
    }
    const float bound = TYPE == TYPE_Q4_K   ? 945.f * dm + 63.f * mm
                        : TYPE == TYPE_Q5_K ? 1953.f * dm + 63.f * mm
                        : TYPE == TYPE_Q6_K ? 4096.f * dm
                        : TYPE == TYPE_Q4_0 ? 8.f * dm
                        : TYPE == TYPE_Q4_1 ? 15.f * dm + mm
                        : TYPE == TYPE_Q5_0 ? 16.f * dm
                        : TYPE == TYPE_Q5_1 ? 31.f * dm + mm
                        : TYPE == TYPE_Q2_K ? 45.f * dm + 15.f * mm
                                            : 128.f * dm;  // Q3_K, Q8_0
    // bound = f * 2^E, f in [0.5, 1): bound * 2^-(E - 15) = f * 2^15 < 2^15
    rexp[n] = (int8_t)(bound > 0.f ? __builtin_amdgcn_frexp_expf(bound) - 15 : 0);
}

hipError_t launch_row_exponents(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, int8_t *rexp,
                                hipStream_t st) {
    if (!gemm_serves(type, k)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((n + 255) / 256);
    const int nb = (int)(k / (is_kquant(type) ? KB : 32));
    switch (type) {
#define LBQ_REXP(T) case T: k_row_exponents<T><<<grid, 256, 0, st>>>(w, n, nb, row_bytes, rexp); break;
    LBQ_REXP(TYPE_Q4_K) LBQ_REXP(TYPE_Q5_K) LBQ_REXP(TYPE_Q6_K) LBQ_REXP(TYPE_Q8_0) LBQ_REXP(TYPE_Q4_0)
    LBQ_REXP(TYPE_Q4_1) LBQ_REXP(TYPE_Q5_0) LBQ_REXP(TYPE_Q5_1) LBQ_REXP(TYPE_Q2_K) LBQ_REXP(TYPE_Q3_K)
#undef LBQ_REXP
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

namespace {


// mt, rt and tile_rows depend on (type, k, m) only -- the pre-pass plans with n = 1
Plan plan_for(int type, int64_t n, int64_t k, int64_t m) {
    Plan p;
    // two row tiles (m <= 64) for Q6_K (3-19 % faster than its 64-row tiles at
    // m = 48, 64; for Q4_K / Q5_K the 64-row tiles win on the large matrices).
    // The choice -- and so the operand layout -- must not depend on n: a grouped
    // call runs one pre-pass for weights of different n.
    const Tuning &tu = tuning();
    // (the other types with a large per-lane weight state plan as Q6_K)
    const bool heavy = gemm_heavy(type);
    const bool ks2 = heavy || tu.gemm_ks64;
    if (m <= (ks2 ? 64 : 32) && !tu.gemm_no_ks) {
        // k-sliced: 128-column workgroups of one or two 32-row tiles, each a
        // slice of S blocks
        p.mt = MT_KS;
        p.rt = m <= 32 ? 1 : 2;
        p.tiles_m = 1;
        p.tiles_n = (int)((n + KSN - 1) / KSN);
        // blocks per slice: 4, fewer (down to 2) until the grid has a workgroup
        // per CU (measured at m = 16 on the Llama-3 shapes, 1 to 4 blocks); two
        // row tiles: 2 (the activation slice is 32 KB per block)
        const int nb = (int)(k / KB);
        const int smax = p.rt == 1 ? KS_BLOCKS : 2;
        // (1, 2 or 4 blocks: a slice stays inside one exponent group of KS_BLOCKS)
        int bps = smax;
        if (bps == 4 && (int64_t)p.tiles_n * ((nb + 3) / 4) < (int64_t)num_cus()) bps = 2;
        // one-block slices where two-block ones leave half the CUs idle (Q6_K
        // 1024 x 4096, 8 column tiles: m = 16 / 32 11.0 / 13.9 -> 9.2 / 10.6 us;
        // on 4096 x 14336 one-block slices measured 5 us slower at m = 32)
        if (bps == 2 && p.rt == 1 && 2 * (int64_t)p.tiles_n * ((nb + 1) / 2) <= (int64_t)num_cus()) bps = 1;
        if (tu.gemm_ks) bps = std::max(1, std::min(tu.gemm_ks == 3 ? 2 : tu.gemm_ks, smax));  // tuning
        p.bps = bps;
        p.splits = (nb + bps - 1) / bps;
        return p;
    }
    // the wide and tall kernels address a tile's operand rows through a buffer
    // resource of 256 * k * 2 bytes or less, which must stay below 2^31
    const bool big_ok = k * 2 * TBM < (int64_t(1) << 31) && !tu.gemm_no_tall;
    // wide tiles (two waves per SIMD, dequantisation per 128 rows) below 256 rows,
    // and for Q4_K (the cheapest dequantisation) up to 512; tall tiles (one wave
    // per SIMD, dequantisation per 256 rows) where the dequantisation VALU per
    // MFMA decides (measured per type and m: 128, 256, 512, 2048; Q4_K at 2048
    // with the seven-wave wide tiles below is a wash, 14336 x 4096 318 -> 308 us
    // but 4096 x 14336 280 -> 290).  The choice must not depend on n: a grouped
    // call's pre-pass lays out whole tiles of rows for every weight of the group.
    bool wide = m < 256 || (type == TYPE_Q4_K && m <= 512);
    if (tu.gemm_big) wide = tu.gemm_big == 1 || m < 256;  // tuning override: wide or tall
    // (Q6_K from 65 rows: its 64-row tiles took 66 us at m = 100 where the wide
    // tiles take 50 at m = 128, 14336 x 4096)
    if ((m >= 128 || (heavy && m > 64)) && big_ok) p.mt = wide ? MT_WIDE : 8;
    else p.mt = m <= 32 ? 1 : (m <= 64 || heavy) ? 2 : 4;  // heavy weight state leaves no room for MT = 4
    const int rows = tile_rows(p), cols = p.mt == 8 ? TBN : BN;
    p.tiles_m = (int)((m + rows - 1) / rows);
    p.tiles_n = (int)((n + cols - 1) / cols);
    const int nb = (int)(k / KB);
    // split k until the grid has about one workgroup per CU (also where two fit:
    // measured at m = 64, more splits only add partial-sum traffic)
    const int64_t slots = (int64_t)num_cus();
    auto splits_for = [&](int64_t tiles) {
        int s = 1;
        if (tiles * 2 <= slots) s = (int)std::min<int64_t>(slots / tiles, nb);
        if (tu.gemm_splits) s = std::max(1, std::min(tu.gemm_splits, nb));  // tuning override
        return s;
    };
    int s = splits_for((int64_t)p.tiles_m * p.tiles_n);
    if (p.mt == MT_WIDE && n % (7 * 32) == 0 && tu.gemm_wide7 >= 0) {
        // seven-wave tiles (224 columns) where they take fewer wave-rounds of the
        // chip: rounds of workgroups over the CUs x waves x blocks per workgroup
        const int tn7 = (int)(n / (7 * 32));
        const int s7 = splits_for((int64_t)p.tiles_m * tn7);
        auto cost = [&](int64_t wgs, int waves, int sp) { return (wgs + slots - 1) / slots * waves * ((nb + sp - 1) / sp); };
        if (tu.gemm_wide7 > 0 || cost((int64_t)p.tiles_m * tn7 * s7, 7, s7) < cost((int64_t)p.tiles_m * p.tiles_n * s, 8, s)) {
            p.mt = MT_WIDE7;
            p.tiles_n = tn7;
            s = s7;
        }
    }
    p.bps = (nb + s - 1) / s;
    p.splits = (nb + p.bps - 1) / p.bps;
    return p;
}

// workspace: fp16 operand rows [m][k] | row exponents [m] | split-k partials [S][m][n]
struct WsLayout {
    size_t a_off, e_off, o_off, part_off, total;
};

// type: the extra k-step's operand rows (gemm_offset_step types) sit between the
// exponents and the partials, for whole row tiles like the operand rows
WsLayout ws_layout(int type, const Plan &p, int64_t n, int64_t k, int64_t m) {
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    const size_t rows = (size_t)p.tiles_m * tile_rows(p);
    WsLayout L;
    L.a_off = 0;
    L.e_off = L.a_off + up(rows * (size_t)k * sizeof(_Float16));  // whole row tiles
    // exponents: per row, or per (exponent group, row) for the k-sliced layout with Q8_K rows
    const bool grouped_e = operand_major(p) && vec_dot_type(type) == TYPE_Q8_K;
    const size_t ne = grouped_e ? (size_t)m * (size_t)((k / KB + KS_BLOCKS - 1) / KS_BLOCKS) : (size_t)m;
    L.o_off = L.e_off + up(ne * sizeof(int));
    L.part_off = L.o_off + (gemm_offset_step(type) ? up(rows * (size_t)(k / KB) * 16 * sizeof(_Float16)) : 0);
    L.total = L.part_off + (p.splits > 1 ? up((size_t)p.splits * (size_t)(m * n) * sizeof(float)) : 0);
    return L;
}

}  // namespace

size_t gemm_workspace_bytes(int type, int64_t n, int64_t k, int64_t m) {
    if (!gemm_serves(type, k)) return 0;
    return ws_layout(type, plan_for(type, n, k, m), n, k, m).total;
}

bool gemm_prepass_fuses_quant(int type, int64_t k, const float *x) {
    return x && gemm_serves(type, k) && k / KB <= 64 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

hipError_t gemm_prepass(int type, int64_t k, const ActView &act, const float *x, int64_t m, void *ws, hipStream_t st) {
    if (!ws || !gemm_serves(type, k)) return hipErrorInvalidValue;
    const Plan p = plan_for(type, 1, k, m);  // the operand rows do not depend on n
    const WsLayout L = ws_layout(type, p, 1, k, m);
    uint8_t *base = static_cast<uint8_t *>(ws);
    _Float16 *a = reinterpret_cast<_Float16 *>(base + L.a_off);
    int *erow = reinterpret_cast<int *>(base + L.e_off);
    _Float16 *ofs = gemm_offset_step(type) ? reinterpret_cast<_Float16 *>(base + L.o_off) : nullptr;
    // few rows, or long rows up to 1024 of them: one pass of 1024 threads per
    // row; otherwise 256-thread workgroups (measured at m = 512 and 2048)
    const bool wide_wg = m <= 64 || (k > 8192 && m <= 1024);
    const int om = operand_major(p);
    if (om && vec_dot_type(type) == TYPE_Q8_K) {  // k-sliced layout: exponents per (group, row)
        const unsigned grid = (unsigned)(m * ((k / KB + KS_BLOCKS - 1) / KS_BLOCKS));
        if (x) {
            if (!gemm_prepass_fuses_quant(type, k, x)) return hipErrorInvalidValue;
            k_ops_ks<true><<<grid, 64, 0, st>>>(x, act, k, m, a, erow, om);
        } else {
            k_ops_ks<false><<<grid, 64, 0, st>>>(nullptr, act, k, m, a, erow, om);
        }
        return hipGetLastError();
    }
    if (x) {
        if (!gemm_prepass_fuses_quant(type, k, x)) return hipErrorInvalidValue;
        if (vec_dot_type(type) != TYPE_Q8_K) {  // Q8_0 codes (the Q8_1 codes are the same)
            if (wide_wg) k_quant_f16_q80<1024><<<(unsigned)m, 1024, 0, st>>>(x, k, a, erow, om, ofs);
            else k_quant_f16_q80<256><<<(unsigned)m, 256, 0, st>>>(x, k, a, erow, om, ofs);
        } else {
            const int nbx = (int)(k / KB);
            if (wide_wg) {
                k_quant_f16<1024, 1><<<(unsigned)m, 1024, 0, st>>>(x, k, a, erow, om);
            } else {
                auto go = [&](auto kern) { kern<<<(unsigned)m, 256, 0, st>>>(x, k, a, erow, om); };
                if (nbx <= 16) go(k_quant_f16<256, 1>);
                else if (nbx <= 32) go(k_quant_f16<256, 2>);
                else if (nbx <= 48) go(k_quant_f16<256, 3>);
                else go(k_quant_f16<256, 4>);
            }
        }
    } else if (vec_dot_type(type) != TYPE_Q8_K) {  // Q8_0 / Q8_1 activations
        if (ofs && !act.xs) return hipErrorInvalidValue;  // Q4_1 / Q5_1 need the Q8_1 block sums
        if (wide_wg) k_act_f16<1024, 32><<<(unsigned)m, 1024, 0, st>>>(act, m, a, erow, om, ofs);
        else k_act_f16<256, 32><<<(unsigned)m, 256, 0, st>>>(act, m, a, erow, om, ofs);
    } else {
        if (wide_wg) k_act_f16<1024, KB><<<(unsigned)m, 1024, 0, st>>>(act, m, a, erow, om, nullptr);
        else k_act_f16<256, KB><<<(unsigned)m, 256, 0, st>>>(act, m, a, erow, om, nullptr);
    }
    return hipGetLastError();
}

bool gemm_quantises_in_kernel(int type, int64_t n, int64_t k, int64_t m, const float *x) {
    if (!gemm_prepass_fuses_quant(type, k, x) || vec_dot_type(type) != TYPE_Q8_K || tuning().gemm_prepass) return false;
    // every column tile's workgroups quantise their slice again: with many tiles
    // that repeated VALU work costs more than the pre-pass launch (measured at
    // m = 16: 1.8 us faster at 1024 and 4096 columns, 2.5 us slower at 14336)
    const Plan p = plan_for(type, n, k, m);
    return p.mt == MT_KS && p.tiles_n <= KS_FX_MAX_TILES && ks_fx_shape(p.bps, ks_fx_rows(m, p.rt));
}

hipError_t gemm_main(int type, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t k, int64_t row_bytes, int64_t m,
                     float *y, void *ws, uint32_t *counters, const float *x, hipStream_t st) {
    if (!ws || !rexp || !gemm_serves(type, k)) return hipErrorInvalidValue;
    if (x && !gemm_quantises_in_kernel(type, n, k, m, x)) return hipErrorInvalidValue;
    const Plan p = plan_for(type, n, k, m);
    const WsLayout L = ws_layout(type, p, n, k, m);
    uint8_t *base = static_cast<uint8_t *>(ws);
    const _Float16 *a = reinterpret_cast<const _Float16 *>(base + L.a_off);
    const int *erow = reinterpret_cast<const int *>(base + L.e_off);
    const _Float16 *ofs = gemm_offset_step(type) ? reinterpret_cast<const _Float16 *>(base + L.o_off) : nullptr;
    float *part = reinterpret_cast<float *>(base + L.part_off);
    float *out = p.splits > 1 ? part : y;
    const int64_t stride = p.splits > 1 ? m * n : 0;
    // the k-sliced kernel adds its own slices when given zeroed tile counters
    // (with few column tiles the one workgroup per tile that adds the slices is
    // slower than the separate launch, which spreads the sum over the chip)
    uint32_t *cnt = (p.mt == MT_KS && p.splits > 1 && p.splits <= KS_FUSED_SLICES && n % 4 == 0 && counters &&
                     !tuning().gemm_split_launch &&
                     p.tiles_n >= KS_FUSED_MIN_TILES && p.tiles_n <= KS_COUNTERS &&
                     (int64_t)p.splits * m * n * 4 < ((int64_t)1 << 31))
                        ? counters
                        : nullptr;
    hipError_t e;
    switch (type) {
    case TYPE_Q4_K: e = launch_typed<TYPE_Q4_K>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q5_K: e = launch_typed<TYPE_Q5_K>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q6_K: e = launch_typed<TYPE_Q6_K>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q8_0: e = launch_typed<TYPE_Q8_0>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q4_0: e = launch_typed<TYPE_Q4_0>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q4_1: e = launch_typed<TYPE_Q4_1>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q5_0: e = launch_typed<TYPE_Q5_0>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q5_1: e = launch_typed<TYPE_Q5_1>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q2_K: e = launch_typed<TYPE_Q2_K>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    case TYPE_Q3_K: e = launch_typed<TYPE_Q3_K>(p, w, rexp, n, row_bytes, a, erow, ofs, k, m, out, stride, cnt, y, x, st); break;
    default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess || p.splits == 1 || cnt) return e;
    const int64_t count = m * n;
    k_split_sum<<<(unsigned)((count + 1023) / 1024), 256, 0, st>>>(part, p.splits, count, y);
    return hipGetLastError();
}

hipError_t launch_gemm(int type, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t k, int64_t row_bytes,
                       const ActView &act, const float *x, int64_t m, float *y, void *ws, uint32_t *counters,
                       hipStream_t st) {
    if (gemm_serves(type, k)) {
        if (gemm_quantises_in_kernel(type, n, k, m, x))  // no operand pre-pass
            return gemm_main(type, w, rexp, n, k, row_bytes, m, y, ws, counters, x, st);
        hipError_t e = gemm_prepass(type, k, act, x, m, ws, st);
        if (e != hipSuccess) return e;
        return gemm_main(type, w, rexp, n, k, row_bytes, m, y, ws, counters, nullptr, st);
    }
    if (x) return hipErrorInvalidValue;  // the GEMV over row chunks takes quantised activations
    // k % 256 != 0: the decode GEMV over row chunks of 8
    for (int64_t m0 = 0; m0 < m; m0 += 8) {
        const int mc = (int)(m - m0 < 8 ? m - m0 : 8);
        ActView a = act;
        a.xq = act.xq + m0 * k;
        a.xd = act.xd + m0 * act.nb;
        a.xbs = act.xbs ? act.xbs + m0 * (k / 16) : nullptr;
        a.xs = act.xs ? act.xs + m0 * act.nb : nullptr;
        hipError_t e = launch_gemv(type, w, n, k, row_bytes, a, mc, y + m0 * n, st);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace lbq
