// lbq_gemm.hip -- batched path (m > 8): k-quant weights dequantised in registers
// straight into MFMA operands, activation codes staged through LDS.
//
// y[m][n] = 2^(e_m + e_n) * sum_k a[m][k] * w[n][k]   (v_mfma_f32_32x32x16_f16, f32 accumulation)
//   a[m][k] = f16(q8[m][k] * d_x[m][b] * 2^-e_m): the Q8_K activation value as the
//             reference quantises it (codes q8, block scale d_x), rounded once to
//             fp16 after a power-of-two row normalisation e_m chosen so that the
//             row's largest |value| lies in [2^14, 2^15) -- no overflow, and
//             every block within 2^14 of the row's largest keeps full precision;
//   w[n][k] = 2^-e_n times the weight value the reference's integer path
//             implies, (d*sc)*q - dmin*m (Q4_K/Q5_K), (d*sc)*(q-32) (Q6_K) or d*q
//             (Q8_0), formed at f32 precision and rounded once to fp16.  The
//             per-row exponent e_n (computed once per weight, row_exponents)
//             puts the largest value a row's blocks can produce just below 2^15,
//             so small block scales never fall into the fp16 subnormal range;
//   y[m][n] = 2^(e_m + e_n) * sum_k a[m][k] * w[n][k].
// So the products differ from the reference's by two fp16 roundings (relative
// <= 2^-11 each) and the sum by f32 summation order: about 4e-4 relative on a row.
//
// Kernels by m (plan_for): k_gemm_ks, k-sliced 32- or 64-row tiles, for m <= 32
// (Q6_K: 64); k_gemm<MT>, 32*MT-row tiles, up to 127 rows (Q6_K: 64); k_gemm_w,
// eight-wave 128 x 256 tiles, from 128 rows (Q6_K: 65) below 256 (Q4_K: up to
// 512); k_gemm_t, 256 x 128 tiles, above.  Each has its own description below;
// the work split of k_gemm<MT>, on which the others build, follows.
//
// Work split.  A 256-thread workgroup owns BM = 32*MT rows of y and BN = 256
// columns; wave w owns columns 64w..64w+63 (two 32-column MFMA tiles) for all BM
// rows (MT 32-row tiles).  Lane l serves weight rows 32j + l%32 (j = 0, 1) and the
// half h = l/32 of every 256-value block: it loads that half's raw bytes one block
// ahead into registers and expands them into the B operands of the block's 16
// MFMA k-steps.  No weight byte goes through LDS and each is dequantised once per
// workgroup.  The activations are turned into fp16 operands once, by a pre-pass
// (k_act_f16), and each block of them (BM x 256) is loaded one block ahead and
// copied into a double-buffered LDS tile that all four waves read as A operands.
//
// k order.  For k-step s (0..15), lane half h supplies the 8 values
// 128h + 8s + pi(e), e = 0..7, pi = (0,2,1,3,4,6,5,7): nibbles of bytes 0 and 2 of
// a dword land in one f16 pair, bytes 1 and 3 in the next, which saves a shift
// per pair.  The activation tile is stored in the same order (position 4a + e
// holds value 4a + pi(e)), so each A operand is one contiguous 16-byte LDS read.
//
// Shapes with few output tiles split k over S workgroups (split-K) that write
// partial sums to the workspace; a second kernel adds them in a fixed order, so
// results do not depend on scheduling.
#include <algorithm>

#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int KB = 256;      // values per block (weights and Q8_K activations)
constexpr int ALD = KB + 8;  // activation tile row stride in halfs: 528 B, conflict-free b128 reads
constexpr int BN = 256;      // output columns per workgroup

// Weight operands are built from f16 subnormals: the bit pattern u (u < 1024) is
// the f16 value u * 2^-24, exactly, so masking a nibble (or a nibble plus high
// bits) in place in bytes 0 and 2 of a dword yields two f16 operands at once; a
// nibble left in bits 4..7 reads as 16u * 2^-24.  The per-sub-block scale is
// pre-multiplied by 2^24 (or 2^20), and v_fma_mix forms u*d1 - m1 at f32
// precision (the subnormal converts exactly) and rounds it to f16 once.
__device__ __forceinline__ uint32_t scale2(uint32_t p, float d1s, float c1) {
    const half2v h = __builtin_bit_cast(half2v, p);
    const half2v r = {(_Float16)fmaf((float)h.x, d1s, c1), (_Float16)fmaf((float)h.y, d1s, c1)};
    return __builtin_bit_cast(uint32_t, r);
}

// 4 int8 codes times the scale sx -> f16 pairs (x0, x2) and (x1, x3).  Byte
// q ^ 0x80 goes into the mantissa of 1024.0 (the f16 1152 + q, exact), and
// (1152 + q)*sx + c with c = -1152*sx is evaluated at f32 precision and rounded
// once (c carries an f32 rounding, <= 2^-24 * 1152 * |sx|, far below the f16 one).
__device__ __forceinline__ void codes_to_f16(uint32_t w, float sx, float c, uint32_t *lo, uint32_t *hi) {
    const uint32_t u = w ^ 0x80808080u;
    const half2v a = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04020400u));
    const half2v b = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, 0x04030401u));
    const half2v ra = {(_Float16)fmaf((float)a.x, sx, c), (_Float16)fmaf((float)a.y, sx, c)};
    const half2v rb = {(_Float16)fmaf((float)b.x, sx, c), (_Float16)fmaf((float)b.y, sx, c)};
    *lo = __builtin_bit_cast(uint32_t, ra);
    *hi = __builtin_bit_cast(uint32_t, rb);
}

// Where the pre-pass puts the 8 operand values at k-order position 8*p8 of block
// b of row m (p8 = 16h + s: lane half h, k-step s).  Row-major ([m][k], the
// tiled kernels stage it through LDS) or, for the k-sliced kernel (m <= 64),
// operand-major: the 64 lanes' operands of one (block, 32-row tile, k-step) are
// 1 KB in a row, so each k-step's A operand is a single contiguous read.
__device__ __forceinline__ int64_t op_pos(int opmajor, int64_t m, int64_t b, int p8, int64_t K) {
    // opmajor = number of 32-row tiles (0: row-major); operand-major order is
    // block, row tile, k-step, lane
    if (opmajor) return (((b * opmajor + (m >> 5)) * 16 + (p8 & 15)) * 64 + (p8 >> 4) * 32 + (m & 31)) * 8;
    return m * K + b * KB + 8 * p8;
}

// ---------------------------------------------------------------------------
// Pre-pass: Q8_K rows (codes + block scales) -> fp16 operand rows in the GEMM's k
// order, and the row exponent e_m.  One workgroup of T threads per row (T = 1024
// for few rows, so the row's chunks are converted in one pass): the threads
// share the maximum of the row's block scales through LDS, then convert
// 16-code chunks.
// ---------------------------------------------------------------------------
// QB: values per activation scale block (256: Q8_K, 32: Q8_0)
template <int T, int QB>
__global__ __launch_bounds__(T) void k_act_f16(ActView act, int64_t M, _Float16 *__restrict__ A,
                                               int *__restrict__ erow, int opmajor) {
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
    // row's values below 2^15 and its largest at or above 2^14
    const int e = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) - 8 : 0;
    if (t == 0) erow[m] = e;
    const int8_t *q = act.xq + m * act.k;
    for (int64_t c = 16 * t; c < act.k; c += 16 * T) {
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
// bit-identical operands.
template <int T>
__global__ __launch_bounds__(T) void k_quant_f16(const float *__restrict__ x, int64_t K, _Float16 *__restrict__ A,
                                                 int *__restrict__ erow, int opmajor) {
    constexpr int BPP = T / 16, MAXP = 64 / BPP;  // passes of BPP blocks, 64 blocks at most
    __shared__ float ds[64];
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
#pragma unroll
    for (int j = 0; j < MAXP; j++) {
        codes[j] = make_uint4(0u, 0u, 0u, 0u);
        dj[j] = 0.f;
        if (j < np) {  // workgroup-uniform
            uint32_t packed[4];
            int sum;
            q8k_lane16(v[j], sub, packed, &sum, &dj[j]);
            codes[j] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            const int b = BPP * j + (t >> 4);
            if (sub == 0 && b < nbx) ds[b] = dj[j];
        }
    }
    __syncthreads();
    float mx = 0.f;
    for (int b = 0; b < nbx; b++) mx = fmaxf(mx, fabsf(ds[b]));
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
template <int T>
__global__ __launch_bounds__(T) void k_quant_f16_q80(const float *__restrict__ x, int64_t K, _Float16 *__restrict__ A,
                                                     int *__restrict__ erow, int opmajor) {
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
    float dj[MAXP];
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
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float r = roundf(v[j][i] * id);
                const int q = (r != r) ? 0 : (int)fminf(fmaxf(r, -128.f), 127.f);
                codes[j][i >> 2] |= ((uint32_t)q & 0xffu) << (8 * (i & 3));
            }
            dj[j] = __half2float(__float2half_rn(d));  // the stored scale
            if (BPP * j + (t >> 1) < nbx) mx = fmaxf(mx, fabsf(dj[j]));
        }
    }
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
        const int b = BPP * j + (t >> 1);
        if (j < np && b < nbx) {
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

// ---------------------------------------------------------------------------
// B-operand sources.  A lane's raw bytes of one block come in NL loads
// (load_part(i), so the kernel can spread them over its MFMA stream); prep()
// derives the per-block scales; dw(s, d) gives f16 values 2d, 2d+1 of the 8 the
// lane supplies to k-step s.
// ---------------------------------------------------------------------------
template <int TYPE>
struct GB;

// Q4_K / Q5_K: lane half h holds qs bytes 64h..64h+63 (sub-blocks 4h..4h+3) and,
// for Q5_K, all 32 qh bytes (high bit of value 64c + 32*hi + i is bit 2c+hi of qh[i]).
template <int TYPE>
struct GBK45 {
    static constexpr int BYTES = TYPE == TYPE_Q4_K ? 144 : 176;
    static constexpr int QS = TYPE == TYPE_Q4_K ? 16 : 48;
    static constexpr int NL = TYPE == TYPE_Q4_K ? 5 : 7;
    struct Raw { uint4 v[NL]; };  // header, qs x4, (qh x2)
    struct Prep { float d1[4], c1[4]; uint32_t q[16], qh[8]; };
    __device__ static void load_part(const uint8_t *blk, int h, Raw &r, int i) {
        if (i == 0) r.v[0] = ld_u4(blk);
        else if (i <= 4) r.v[i] = ld_u4(blk + QS + 64 * h + 16 * (i - 1));
        else r.v[i] = ld_u4(blk + 16 + 16 * (i - 5));
    }
    // lane sub-block j (0..3) is block sub-block 4h + j: low nibbles for even j,
    // high nibbles (read as 16u) for odd j
    // wsc = 2^-e_n, the row's power-of-two scale (exact in f32)
    __device__ static void prep(const Raw &r, int h, float wsc, Prep &p) {
        const uint4 hdr = r.v[0];
        const float d = h2f(hdr.x & 0xffffu) * wsc, dmin = h2f(hdr.x >> 16) * wsc;
#pragma unroll
        for (int cl = 0; cl < 2; cl++) {
            uint32_t sc2, m2;
            k4_scale_pair(hdr.y, hdr.z, hdr.w, 2 * h + cl, &sc2, &m2);
#pragma unroll
            for (int hi = 0; hi < 2; hi++) {
                p.d1[2 * cl + hi] = d * (float)((sc2 >> (8 * hi)) & 0xffu) * (hi ? 1048576.f : 16777216.f);
                p.c1[2 * cl + hi] = -(dmin * (float)((m2 >> (8 * hi)) & 0xffu));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 q = r.v[1 + i];
            p.q[4 * i] = q.x; p.q[4 * i + 1] = q.y; p.q[4 * i + 2] = q.z; p.q[4 * i + 3] = q.w;
        }
        if (TYPE == TYPE_Q5_K) {
            // bring bit 4h (sub-block 4h) of every qh byte to bit 0
            const uint32_t sh = 4u * (uint32_t)h;
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const uint4 q = r.v[NL - 2 + i];
                p.qh[4 * i] = q.x >> sh; p.qh[4 * i + 1] = q.y >> sh;
                p.qh[4 * i + 2] = q.z >> sh; p.qh[4 * i + 3] = q.w >> sh;
            }
        }
    }
    // dword d (f16 slots 2d, 2d+1 = bytes 0,2 or 1,3 of a qs dword) of the operand of k-step s
    __device__ static uint32_t dw(const Prep &p, int s, int d) {
        const int js = s >> 2, hi = js & 1;
        uint32_t q = p.q[8 * (s >> 3) + 2 * (s & 3) + (d >> 1)];
        if (d & 1) q >>= 8;
        uint32_t v = q & (hi ? 0x00f000f0u : 0x000f000fu);
        if (TYPE == TYPE_Q5_K) {
            // fifth bit: bit js of the qh byte, to bit 4 (8 for high nibbles) of the f16
            uint32_t hq = p.qh[2 * (s & 3) + (d >> 1)];
            if (d & 1) hq >>= 8;
            v |= (hq << ((hi ? 8 : 4) - js)) & (hi ? 0x01000100u : 0x00100010u);
        }
        return scale2(v, p.d1[js], p.c1[js]);
    }
};
template <> struct GB<TYPE_Q4_K> : GBK45<TYPE_Q4_K> {};
template <> struct GB<TYPE_Q5_K> : GBK45<TYPE_Q5_K> {};

// Q6_K: lane half h holds the 128-value half h: ql bytes 64h..64h+63, qh bytes
// 32h..32h+31, scales 8h..8h+7.  Value 128h + 32q + l (l < 32): low bits from
// ql[64h + 32(q%2) + l] (nibble q/2), high bits from qh[32h + l] (bits 2q, 2q+1),
// scale 8h + 2q + l/16.  Blocks are 210 bytes, only 2-byte aligned: each field is
// read as the aligned dwords that hold it (the last one re-read when the field
// is 4-byte aligned, so no dword outside it is touched) and funnel-shifted.
template <>
struct GB<TYPE_Q6_K> {
    static constexpr int BYTES = 210;
    static constexpr int NL = 12;
    struct Raw { u32x4a4 ql[4], qh[2]; uint32_t qlt, qht, sc[3], dw; };
    struct Prep { float d1[8], c1[8]; uint32_t l[16], qh[8]; };
    // aligned dwords of the block's fields, through global pointers (align4_global)
    __device__ static gbytes_c al4(const uint8_t *p) { return align4_global(reinterpret_cast<uintptr_t>(p)); }
    __device__ static void load_part(const uint8_t *blk, int h, Raw &r, int i) {
        const bool mis = (reinterpret_cast<uintptr_t>(blk) & 3u) != 0;
        const gbytes_c ql = al4(blk + 64 * h), qh = al4(blk + 128 + 32 * h), sc = al4(blk + 192 + 8 * h);
        if (i < 4) r.ql[i] = gld16(ql + 16 * i);
        else if (i < 6) r.qh[i - 4] = gld16(qh + 16 * (i - 4));
        else if (i == 6) r.qlt = gld4(ql + (mis ? 64 : 60));
        else if (i == 7) r.qht = gld4(qh + (mis ? 32 : 28));
        else if (i < 10) r.sc[i - 8] = gld4(sc + 4 * (i - 8));
        else if (i == 10) r.sc[2] = gld4(sc + (mis ? 8 : 4));
        else r.dw = ld2_a2(blk + 208);
    }
    // mis: byte misalignment of the block (0 or 2)
    __device__ static void prep(const Raw &r, uint32_t mis, float wsc, Prep &p) {
        uint32_t w[17], x[9];
#pragma unroll
        for (int i = 0; i < 4; i++) { w[4 * i] = r.ql[i].x; w[4 * i + 1] = r.ql[i].y; w[4 * i + 2] = r.ql[i].z; w[4 * i + 3] = r.ql[i].w; }
        w[16] = r.qlt;
#pragma unroll
        for (int i = 0; i < 2; i++) { x[4 * i] = r.qh[i].x; x[4 * i + 1] = r.qh[i].y; x[4 * i + 2] = r.qh[i].z; x[4 * i + 3] = r.qh[i].w; }
        x[8] = r.qht;
#pragma unroll
        for (int i = 0; i < 16; i++) p.l[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], mis);
#pragma unroll
        for (int i = 0; i < 8; i++) p.qh[i] = __builtin_amdgcn_alignbyte(x[i + 1], x[i], mis);
        const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc[1], r.sc[0], mis), s1 = __builtin_amdgcn_alignbyte(r.sc[2], r.sc[1], mis);
        const float d = h2f(r.dw) * wsc;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // scale i covers quarter q = i/2 of the half: high nibbles (read as 16u) for i >= 4
            const int8_t sc = (int8_t)(((i < 4 ? s0 : s1) >> (8 * (i & 3))) & 0xffu);
            const float d1 = d * (float)sc;
            p.d1[i] = d1 * (i >= 4 ? 1048576.f : 16777216.f);
            p.c1[i] = -32.f * d1;  // (u - 32)*d1
        }
    }
    __device__ static uint32_t dw(const Prep &p, int s, int d) {
        const int q = s >> 2, hi = q >> 1;
        uint32_t l = p.l[8 * (q & 1) + 2 * (s & 3) + (d >> 1)], hq = p.qh[2 * (s & 3) + (d >> 1)];
        if (d & 1) { l >>= 8; hq >>= 8; }
        // bits (2q, 2q+1) of the qh byte -> bits 4,5 of the f16 (8,9 for high nibbles)
        const uint32_t v = (l & (hi ? 0x00f000f0u : 0x000f000fu)) |
                           ((hq << ((hi ? 8 : 4) - 2 * q)) & (hi ? 0x03000300u : 0x00300030u));
        return scale2(v, p.d1[s >> 1], p.c1[s >> 1]);
    }
};

// Q8_0: a 256-value super-block of the k loop is 8 consecutive 34-byte blocks
// (272 bytes; rows of k % 256 == 0 keep every super-block 16-byte aligned).
// Lane half h holds blocks 4h..4h+3 (bytes 136h..136h+135, 8-byte aligned):
// block j's f16 d at byte 34j of that range, its 32 codes from byte 34j + 2.
// The weight value is d*q (q int8); each code becomes (1152 + q) in the f16
// mantissa and (1152 + q)*sx - 1152*sx with sx = d * 2^-e_n is formed at f32
// precision and rounded once (as the activation operands are built).
template <>
struct GB<TYPE_Q8_0> {
    static constexpr int BYTES = 272;
    static constexpr int NL = 9;
    struct Raw { u32x4a4 v[8]; uint2 t; };
    struct Prep { float sx[4], c[4]; uint32_t q[32]; };
    __device__ static void load_part(const uint8_t *blk, int h, Raw &r, int i) {
        const uint8_t *base = blk + 136 * h;
        if (i < 8) r.v[i] = gld16(align4_global(reinterpret_cast<uintptr_t>(base + 16 * i)));
        else r.t = *reinterpret_cast<const uint2 *>(base + 128);
    }
    __device__ static void prep(const Raw &r, float wsc, Prep &p) {
        uint32_t w[34];
#pragma unroll
        for (int i = 0; i < 8; i++) { w[4 * i] = r.v[i].x; w[4 * i + 1] = r.v[i].y; w[4 * i + 2] = r.v[i].z; w[4 * i + 3] = r.v[i].w; }
        w[32] = r.t.x;
        w[33] = r.t.y;
        // block j: d at byte 34j, codes at 34j + 2 (dword-aligned for odd j)
        const uint32_t dbits[4] = {w[0] & 0xffffu, w[8] >> 16, w[17] & 0xffffu, w[25] >> 16};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            p.sx[j] = h2f(dbits[j]) * wsc;
            p.c[j] = -1152.f * p.sx[j];
        }
#pragma unroll
        for (int i = 0; i < 8; i++) {
            p.q[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
            p.q[8 + i] = w[9 + i];
            p.q[16 + i] = __builtin_amdgcn_alignbyte(w[18 + i], w[17 + i], 2);
            p.q[24 + i] = w[26 + i];
        }
    }
    // k-step s takes codes 8(s%4)..8(s%4)+7 of block s/4; dword d holds values
    // (0, 2), (1, 3), (4, 6), (5, 7) of those eight
    __device__ static uint32_t dw(const Prep &p, int s, int d) {
        const int j = s >> 2;
        const uint32_t u = p.q[8 * j + 2 * (s & 3) + (d >> 1)] ^ 0x80808080u;
        const half2v a = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, u, (d & 1) ? 0x04030401u : 0x04020400u));
        const half2v r2 = {(_Float16)fmaf((float)a.x, p.sx[j], p.c[j]), (_Float16)fmaf((float)a.y, p.sx[j], p.c[j])};
        return __builtin_bit_cast(uint32_t, r2);
    }
};

template <int TYPE>
__device__ __forceinline__ void gb_prep(const typename GB<TYPE>::Raw &r, int h, const uint8_t *blk, float wsc,
                                        typename GB<TYPE>::Prep &p) {
    if constexpr (TYPE == TYPE_Q6_K) GB<TYPE>::prep(r, (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u), wsc, p);
    else if constexpr (TYPE == TYPE_Q8_0) { (void)blk; (void)h; GB<TYPE>::prep(r, wsc, p); }
    else { (void)blk; GB<TYPE>::prep(r, h, wsc, p); }
}


// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
struct GemmGrid {
    int tiles_m, tiles_n, bps;  // bps: blocks of k per split
    int64_t split_stride;       // floats between the partial outputs of two splits (0: no split)
    int splits;
    const int8_t *rexp;         // per weight row: e_n (w operands carry 2^-e_n)
};

// resident workgroups per CU the register budget allows
template <int TYPE, int MT>
constexpr int gemm_occupancy() {
    return (MT == 4 || TYPE == TYPE_Q6_K || TYPE == TYPE_Q8_0 || (TYPE == TYPE_Q5_K && MT == 2)) ? 1 : 2;
}
// weight bytes loaded two blocks ahead (where the registers allow: Q4_K, 32-row tiles)
template <int TYPE, int MT>
constexpr bool gemm_deep() { return TYPE == TYPE_Q4_K && MT == 1; }

// Pipeline.  The MFMAs of a block run as 16 k-steps of 2*MT MFMAs; each MFMA sits
// in its own scheduling region (sched_barrier) together with a share of the
// other work, so that work issues in the MFMA shadow instead of as a bubble
// (on gfx950 only about four VALU per MFMA co-issue for free):
//   every step s < 15 : the B operands (one dword per MFMA at MT = 4) and the A
//                       operands of step s+1;
//   step 0            : the next block's activation loads;
//   steps 1..3        : the next block's weight loads;
//   step 4            : barrier -- every wave is done with the other LDS buffer;
//   step 8            : the next block's activations into the other LDS buffer;
//   step 13           : barrier -- that buffer is complete;
//   step 14           : the next block's first A operands;
//   step 15           : the next block's scales and first B operands.
template <int TYPE, int MT>
__global__ __launch_bounds__(256, (gemm_occupancy<TYPE, MT>())) void k_gemm(const uint8_t *__restrict__ W, int64_t N,
                                                               int64_t row_bytes, const _Float16 *__restrict__ A,
                                                               const int *__restrict__ erow, int64_t K, int64_t M,
                                                               float *__restrict__ out, GemmGrid g) {
    using B = GB<TYPE>;
    constexpr int BM = 32 * MT;
    constexpr int NG = 2 * MT;                 // MFMAs (regions) per k-step
    constexpr int ALOADS = BM / 8;             // 16-byte activation loads per thread and block (= 2 NG)
    constexpr int WL = 2 * B::NL;              // weight loads per lane and block
    constexpr int WPR = (WL + 3 * NG - 1) / (3 * NG);
    constexpr int PER = 8 / NG;                // B-operand dwords built per region
    constexpr int NPR = (8 + NG - 2) / (NG - 1 > 0 ? NG - 1 : 1);  // step 15: dwords per region after the scales
    __shared__ __align__(16) _Float16 As[2][BM][ALD];
    __shared__ int Es[BM];

    // tile of this workgroup: consecutive workgroup ids go to different XCDs, so
    // renumber them such that each XCD receives a contiguous run of tiles; tiles
    // are ordered split-major, then by column tile, then by row tile, so the row
    // tiles that share weight columns share an L2.
    const int G = (int)gridDim.x, L = (int)blockIdx.x;
    const int T = (G & 7) == 0 ? (L & 7) * (G >> 3) + (L >> 3) : L;
    const int tm = T % g.tiles_m, tn = (T / g.tiles_m) % g.tiles_n, z = T / (g.tiles_m * g.tiles_n);
    const int nb = (int)(K / KB);
    const int b0 = z * g.bps, b1 = min(nb, b0 + g.bps);
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    float *y = out + (int64_t)z * g.split_stride;

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, h = lane >> 5, lr = lane & 31;
    const uint8_t *wrow[2];
    int en[2];
    float wsc[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int64_t row = min(n0 + 64 * wave + 32 * j + lr, N - 1);
        wrow[j] = W + row * row_bytes;
        en[j] = g.rexp[row];
        wsc[j] = __builtin_amdgcn_ldexpf(1.f, -en[j]);
    }
    // activation staging: a block row is 256 halfs = 32 16-byte pieces; load i of
    // thread t moves piece t%32 of tile row 8i + t/32, so every load instruction
    // reads two whole 512-byte rows.  The operand buffer holds whole tiles of rows
    // (rows past M are never stored), so the addresses need no clamping.
    const int pc = t & 31, pr = t >> 5;
    const _Float16 *abase = A + (m0 + pr) * K + pc * 8;
    if (t < BM) Es[t] = erow[min(m0 + t, M - 1)];

    // Raw weight bytes: with DEEP, two sets, so the loads for block b + 2 go out
    // while block b + 1's bytes wait in the other set (a short block's MFMA work
    // does not cover a memory latency); the set roles swap with the LDS buffer.
    constexpr bool DEEP = gemm_deep<TYPE, MT>();
    typename B::Raw raw[DEEP ? 2 : 1][2];
    typename B::Prep p[2];
    uint4 ra[ALOADS];
    auto a_load = [&](int b, int i) { ra[i] = *reinterpret_cast<const uint4 *>(abase + 8 * i * K + (int64_t)b * KB); };
    auto a_store = [&](int buf, int i) {
        *reinterpret_cast<uint4 *>(&As[buf][8 * i + pr][8 * pc]) = make_uint4(ra[i].x, ra[i].y, ra[i].z, ra[i].w);
    };
    auto w_load = [&](int b, int q, int set) {
        B::load_part(wrow[q / B::NL] + (int64_t)b * B::BYTES, h, raw[DEEP ? set : 0][q / B::NL], q % B::NL);
    };
    auto w_prep = [&](int b, int j, int set) {
        gb_prep<TYPE>(raw[DEEP ? set : 0][j], h, wrow[j] + (int64_t)b * B::BYTES, wsc[j], p[j]);
    };

    floatx16 acc[MT][2];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[i][j][v] = 0.f;

    // prologue: block b0 into LDS buffer 0, its scales and first operands (and
    // with DEEP block b0 + 1's bytes into set 0, which the first block preps)
#pragma unroll
    for (int i = 0; i < ALOADS; i++) a_load(b0, i);
#pragma unroll
    for (int q = 0; q < WL; q++) w_load(b0, q, 1);
    if constexpr (DEEP) {
#pragma unroll
        for (int q = 0; q < WL; q++) w_load(min(b0 + 1, b1 - 1), q, 0);
    }
#pragma unroll
    for (int i = 0; i < ALOADS; i++) a_store(0, i);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; j++) w_prep(b0, j, 1);
    const _Float16 *al0 = &As[0][lr][128 * h], *al1 = &As[1][lr][128 * h];
    half8 acur[MT];
    uint32_t bcur[2][4];
#pragma unroll
    for (int i = 0; i < MT; i++) acur[i] = *reinterpret_cast<const half8 *>(al0 + 32 * i * ALD);
#pragma unroll
    for (int q = 0; q < 8; q++) bcur[q >> 2][q & 3] = B::dw(p[q >> 2], 0, q & 3);

    auto block = [&](int b, int buf) {
        const int bn = min(b + 1, b1 - 1);  // clamped: the last block re-stages itself, harmlessly
        const int bl = DEEP ? min(b + 2, b1 - 1) : bn;  // the block whose weight bytes this block loads
        const _Float16 *al = buf ? al1 : al0, *aln = buf ? al0 : al1;
        half8 ablk[MT];
        uint32_t bblk[2][4];
#pragma unroll
        for (int s = 0; s < 16; s++) {
            half8 anxt[MT];
            uint32_t bnxt[2][4];
#pragma unroll
            for (int i = 0; i < MT; i++) {
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int rg = 2 * i + j;
                    const half8 bo = __builtin_bit_cast(half8, make_uint4(bcur[j][0], bcur[j][1], bcur[j][2], bcur[j][3]));
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(acur[i], bo, acc[i][j], 0, 0, 0);
                    if (s < 15) {
#pragma unroll
                        for (int q = rg * PER; q < (rg + 1) * PER; q++) bnxt[q >> 2][q & 3] = B::dw(p[q >> 2], s + 1, q & 3);
                        if (j == 1) anxt[i] = *reinterpret_cast<const half8 *>(al + 32 * i * ALD + 8 * (s + 1));
                    }
                    if (s == 0) { a_load(bn, 2 * rg); a_load(bn, 2 * rg + 1); }
                    if (s >= 1 && s <= 3) {
#pragma unroll
                        for (int w = ((s - 1) * NG + rg) * WPR; w < ((s - 1) * NG + rg + 1) * WPR; w++)
                            if (w < WL) w_load(bl, w, buf ^ 1);
                    }
                    if (s == 4 && rg == 0) __syncthreads();
                    if (s == 8) { a_store(buf ^ 1, 2 * rg); a_store(buf ^ 1, 2 * rg + 1); }
                    if (s == 13 && rg == 0) __syncthreads();
                    if (s == 14 && j == 1) ablk[i] = *reinterpret_cast<const half8 *>(aln + 32 * i * ALD);
                    if (s == 15) {
                        if (rg == 0) {
#pragma unroll
                            for (int jj = 0; jj < 2; jj++) w_prep(bn, jj, buf);
                        }
                        if (NG == 1 || rg > 0) {
                            const int r0 = NG == 1 ? 0 : (rg - 1) * NPR;
#pragma unroll
                            for (int q = r0; q < r0 + (NG == 1 ? 8 : NPR); q++)
                                if (q < 8) bblk[q >> 2][q & 3] = B::dw(p[q >> 2], 0, q & 3);
                        }
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
            if (s < 15) {
#pragma unroll
                for (int i = 0; i < MT; i++) acur[i] = anxt[i];
#pragma unroll
                for (int q = 0; q < 8; q++) bcur[q >> 2][q & 3] = bnxt[q >> 2][q & 3];
            }
        }
#pragma unroll
        for (int i = 0; i < MT; i++) acur[i] = ablk[i];
#pragma unroll
        for (int q = 0; q < 8; q++) bcur[q >> 2][q & 3] = bblk[q >> 2][q & 3];
    };

    int b = b0;
    for (; b + 1 < b1; b += 2) {
        block(b, 0);
        block(b + 1, 1);
    }
    if (b < b1) block(b, 0);

    // D layout of a 32x32 MFMA tile: lane holds column l%32, rows 8(v/4) + 4h + v%4
#pragma unroll
    for (int i = 0; i < MT; i++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
            const int64_t m = m0 + r;
            const int e = Es[r];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int64_t n = n0 + 64 * wave + 32 * j + lr;
                if (m < M && n < N) y[m * N + n] = __builtin_amdgcn_ldexpf(acc[i][j][v], e + en[j]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Tall tiles for m >= 256: each wave owns 256 rows x 32 columns (8 x 1 MFMA
// tiles), so every B operand it builds feeds 8 MFMAs (about 2.3 VALU per MFMA
// including the scale prep -- within what gfx950 co-issues next to MFMA, where
// the 128-row kernel needs 4+).  Workgroup tile 256 x 128.  The activation tile
// is staged in two stages per block: stage t holds, for lane half h, values
// 128h + 64t + [0, 64) -- exactly k-steps 8t..8t+7 of the k order above -- so a
// double-buffered stage (256 rows x 128 values) fits in LDS.
// ---------------------------------------------------------------------------
constexpr int TBM = 256, TBN = 128;
constexpr int TROW = 256;  // stage row: 128 halfs, no padding (chunks are swizzled instead)

// Stage layout: row r of a stage is 256 B = 16 chunks of 8 halfs; logical chunk
// c = 8h + j (lane half h, k-step j of the stage) sits in slot c ^ (r & 15).  A
// wave's A-operand read (rows lr, lr + 32.., one chunk each) then touches 16
// distinct slots per 16 rows: every bank once, with no padding, so a stage is
// exactly 64 KB and fills by direct-to-LDS loads (16 B per lane, a wave writes
// 4 whole rows per instruction; each lane fetches the chunk its slot holds).
//
// Per stage (8 k-steps x 8 MFMA regions), besides the A operands of the k-step
// AH ahead and the B operand of the next one:
//   k-step 0    : barrier -- every wave is done with the other buffer; then the
//                 next stage's direct-to-LDS loads into it (2 per region);
//   k-step 6    : wait for this wave's loads, barrier -- the other buffer is
//                 complete; from k-step 8 - AH on, the next stage's first A
//                 operands are read from it;
//   k-steps 6-7 : in stage 0, the next block's weight loads (after the wait, so
//                 they are not waited for until the next stage's k-step 6);
//   k-step 7    : in stage 1, the next block's scales and first B operand.
template <int TYPE>
__global__ __launch_bounds__(256, 1) void k_gemm_t(const uint8_t *__restrict__ W, int64_t N, int64_t row_bytes,
                                                   const _Float16 *__restrict__ A, const int *__restrict__ erow,
                                                   int64_t K, int64_t M, float *__restrict__ out, GemmGrid g) {
    using B = GB<TYPE>;
    // two separate arrays, so the compiler tells the buffers apart when it
    // places waits for the direct-to-LDS loads
    __shared__ __align__(1024) uint8_t As0[TBM * TROW];
    __shared__ __align__(1024) uint8_t As1[TBM * TROW];
    __shared__ int Es[TBM];

    const int G = (int)gridDim.x, L = (int)blockIdx.x;
    const int T = (G & 7) == 0 ? (L & 7) * (G >> 3) + (L >> 3) : L;
    const int tm = T % g.tiles_m, tn = (T / g.tiles_m) % g.tiles_n, z = T / (g.tiles_m * g.tiles_n);
    const int nb = (int)(K / KB);
    const int b0 = z * g.bps, b1 = min(nb, b0 + g.bps);
    const int64_t m0 = (int64_t)tm * TBM, n0 = (int64_t)tn * TBN;
    float *y = out + (int64_t)z * g.split_stride;

    // the wave index as a scalar: staging addresses and LDS targets are then
    // scalar too (the direct-to-LDS target goes through M0)
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5,
              lr = lane & 31;
    const int64_t wr = min(n0 + 32 * wave + lr, N - 1);
    const uint8_t *wrow = W + wr * row_bytes;
    const int en = g.rexp[wr];
    const float wsc = __builtin_amdgcn_ldexpf(1.f, -en);
    Es[t] = erow[min(m0 + t, M - 1)];

    // direct-to-LDS staging: instruction j of a wave fills stage rows
    // 64 wave + 4j + [0, 4); lane l writes row 64 wave + 4j + l/16, slot l%16,
    // so it fetches logical chunk (l%16) ^ (row & 15), whose pattern repeats
    // every 4 instructions: a scalar offset plus one of four 32-bit lane offsets.
    // Rows past M exist in the operand buffer (whole tiles), so no clamping.
    // Buffer loads, not global ones: the compiler counts a pending global
    // load-to-LDS against the LDS-read counter as well and then drains every
    // LDS read (lgkmcnt(0)) at each A-operand use until the stage's loads land;
    // a buffer load is counted as a vector-memory load only, so the A reads keep
    // their read-ahead.  The resource spans the tile's 256 operand rows
    // (the host keeps 256 * K * 2 bytes below 2^31).
    // (the base passes through readfirstlane so the resource is known to be
    // scalar: otherwise each load becomes a waterfall loop)
    const uint64_t abase = reinterpret_cast<uint64_t>(A + m0 * K);
    const uint64_t abase_s = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)abase) |
                             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(abase >> 32)) << 32);
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void *>(abase_s), (short)0, __builtin_amdgcn_readfirstlane((int)(TBM * K * 2)), 0x00020000);
    uint32_t voff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int c = (lane & 15) ^ ((4 * q + (lane >> 4)) & 15);
        voff[q] = (uint32_t)(((lane >> 4) * (int)K + 128 * (c >> 3) + 8 * (c & 7)) * 2);
    }
    auto a_dma = [&](int u, int buf, int j) {
        const int soff = ((64 * wave + 4 * j) * (int)K + (u >> 1) * KB + 64 * (u & 1)) * 2;
        uint8_t *dst = (buf ? As1 : As0) + (64 * wave + 4 * j) * TROW;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void *)dst, 16, voff[j & 3],
                                                 soff, 0, 0);
    };
    // A-operand read addresses: row lr (+32 i, an immediate offset), chunk 8h + j
    // in slot (8h + j) ^ (lr & 15); one register per k-step and buffer
    // (the offsets pass through an empty asm statement per buffer, so neither
    // buffer's addresses are rebuilt from the other's -- a VALU op per read --
    // while each pointer still names its array, which the placement of waits
    // for the direct-to-LDS loads relies on)
    const uint8_t *rb[2][8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int o0 = lr * TROW + 16 * ((8 * h + j) ^ (lr & 15)), o1 = o0;
        asm volatile("" : "+v"(o0), "+v"(o1));
        rb[0][j] = As0 + o0;
        rb[1][j] = As1 + o1;
    }
    auto a_read = [&](int buf, int j, int i) -> half8 {
        return *reinterpret_cast<const half8 *>(rb[buf][j] + 32 * i * TROW);
    };

    typename B::Raw raw;
    typename B::Prep p;
    auto w_load = [&](int b, int q) { B::load_part(wrow + (int64_t)b * B::BYTES, h, raw, q); };
    auto w_prep = [&](int b) { gb_prep<TYPE>(raw, h, wrow + (int64_t)b * B::BYTES, wsc, p); };

    floatx16 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[i][v] = 0.f;

#pragma unroll
    for (int j = 0; j < 16; j++) a_dma(2 * b0, 0, j);
#pragma unroll
    for (int q = 0; q < B::NL; q++) w_load(b0, q);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    w_prep(b0);
    // A operands are read AH k-steps ahead (ar[j] holds k-step ks + j): with one
    // wave per SIMD, 8 KB of reads per k-step need that depth to keep the LDS
    // busy.  Q6_K's larger weight state leaves registers for one step only.
    constexpr int AH = (TYPE == TYPE_Q6_K || TYPE == TYPE_Q8_0) ? 1 : 2;
    half8 ar[AH][8];
    uint32_t bcur[4];
#pragma unroll
    for (int j = 0; j < AH; j++)
#pragma unroll
        for (int i = 0; i < 8; i++) ar[j][i] = a_read(0, j, i);
#pragma unroll
    for (int d = 0; d < 4; d++) bcur[d] = B::dw(p, 0, d);

    const int u_end = 2 * b1;
    auto stage = [&](int u, int buf) {
        const int ts = u & 1;
        const int un = min(u + 1, u_end - 1);          // clamped: the last stage re-stages itself
        const int bn = min((u >> 1) + 1, b1 - 1);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            const int s = 8 * ts + ks;  // k-step within the block
            half8 an[8];
            uint32_t bnxt[4];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if (ks == 0 && i == 0) __syncthreads();  // every wave is done with the other buffer
                if (ks == 6 && i == 0) {
                    // this wave's direct-to-LDS loads (and nothing later is in
                    // flight: the weight loads come after), then all waves'
                    __builtin_amdgcn_s_waitcnt(0);
                    __syncthreads();
                }
                const half8 bo = __builtin_bit_cast(half8, make_uint4(bcur[0], bcur[1], bcur[2], bcur[3]));
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ar[0][i], bo, acc[i], 0, 0, 0);
                if (ks + AH < 8) an[i] = a_read(buf, ks + AH, i);
                else an[i] = a_read(buf ^ 1, ks + AH - 8, i);
                // B-operand dwords two at a time, so the half-register writes of one
                // interleave with the other's (no hazard stall between them)
                if (s < 15) {
                    if (i == 0 || i == 2) { bnxt[i] = B::dw(p, s + 1, i); bnxt[i + 1] = B::dw(p, s + 1, i + 1); }
                } else {
                    if (i == 0) w_prep(bn);
                    else if (i == 1 || i == 3) { bnxt[i - 1] = B::dw(p, 0, i - 1); bnxt[i] = B::dw(p, 0, i); }
                }
                if (ks == 0) { a_dma(un, buf ^ 1, 2 * i); a_dma(un, buf ^ 1, 2 * i + 1); }
                if (ts == 0 && (ks == 6 || ks == 7)) {
                    const int q = 8 * (ks - 6) + i;
                    if (q < B::NL) w_load(bn, q);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) {
#pragma unroll
                for (int j = 0; j + 1 < AH; j++) ar[j][i] = ar[j + 1][i];
                ar[AH - 1][i] = an[i];
            }
#pragma unroll
            for (int d = 0; d < 4; d++) bcur[d] = bnxt[d];
        }
    };
    for (int u = 2 * b0; u < u_end; u += 2) {
        stage(u, 0);
        stage(u + 1, 1);
    }

#pragma unroll
    for (int i = 0; i < 8; i++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
            const int64_t m = m0 + r;
            const int64_t n = n0 + 32 * wave + lr;
            if (m < M && n < N) y[m * N + n] = __builtin_amdgcn_ldexpf(acc[i][v], Es[r] + en);
        }
    }
}

// ---------------------------------------------------------------------------
// Wide tiles for m >= 128: eight waves (two per SIMD), workgroup tile 128 x 256;
// wave w owns columns 32w..32w+31 for all 128 rows (4 MFMA tiles), so each
// weight byte is dequantised once per workgroup.  One wave per SIMD cannot keep
// the matrix core busy -- even back-to-back independent 32x32x16 MFMAs from a
// single wave issue at about two thirds of the peak rate, and the LDS reads and
// dequantisation VALU between them add to that -- while two waves per SIMD
// overlap one wave's VALU and LDS work with the other's MFMAs.  The activation
// stage is the tall kernel's layout at 128 rows (32 KB per buffer, XOR-swizzled
// chunks, filled by buffer loads to LDS), and the per-stage protocol is the same:
//   k-step 0    : barrier, then the next stage's loads into the other buffer
//                 (4 per wave);
//   k-step 6    : wait for this wave's loads, barrier;
//   k-steps 6-7 : in stage 0, the next block's weight loads;
//   k-step 7    : in stage 1, the next block's scales and first B operand.
// ---------------------------------------------------------------------------
constexpr int WBM = 128, WBN = 256;

template <int TYPE>
__global__ __launch_bounds__(512, 1) void k_gemm_w(const uint8_t *__restrict__ W, int64_t N, int64_t row_bytes,
                                                   const _Float16 *__restrict__ A, const int *__restrict__ erow,
                                                   int64_t K, int64_t M, float *__restrict__ out, GemmGrid g) {
    using B = GB<TYPE>;
    __shared__ __align__(1024) uint8_t As0[WBM * TROW];
    __shared__ __align__(1024) uint8_t As1[WBM * TROW];
    __shared__ int Es[WBM];

    const int G = (int)gridDim.x, L = (int)blockIdx.x;
    const int T = (G & 7) == 0 ? (L & 7) * (G >> 3) + (L >> 3) : L;
    const int tm = T % g.tiles_m, tn = (T / g.tiles_m) % g.tiles_n, z = T / (g.tiles_m * g.tiles_n);
    const int nb = (int)(K / KB);
    const int b0 = z * g.bps, b1 = min(nb, b0 + g.bps);
    const int64_t m0 = (int64_t)tm * WBM, n0 = (int64_t)tn * WBN;
    float *y = out + (int64_t)z * g.split_stride;

    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5,
              lr = lane & 31;
    const int64_t wr = min(n0 + 32 * wave + lr, N - 1);
    const uint8_t *wrow = W + wr * row_bytes;
    const int en = g.rexp[wr];
    const float wsc = __builtin_amdgcn_ldexpf(1.f, -en);
    if (t < WBM) Es[t] = erow[min(m0 + t, M - 1)];

    // staging: instruction j (0..3) of wave w fills stage rows 16w + 4j + [0, 4);
    // lane l writes row 16w + 4j + l/16, slot l%16, holding logical chunk
    // (l%16) ^ (row & 15) = (l%16) ^ ((4j + l/16) & 15)
    const uint64_t abase = reinterpret_cast<uint64_t>(A + m0 * K);
    const uint64_t abase_s = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)abase) |
                             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(abase >> 32)) << 32);
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void *>(abase_s), (short)0, __builtin_amdgcn_readfirstlane((int)(WBM * K * 2)), 0x00020000);
    uint32_t voff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int c = (lane & 15) ^ ((4 * q + (lane >> 4)) & 15);
        voff[q] = (uint32_t)(((lane >> 4) * (int)K + 128 * (c >> 3) + 8 * (c & 7)) * 2);
    }
    auto a_dma = [&](int u, int buf, int j) {
        const int soff = ((16 * wave + 4 * j) * (int)K + (u >> 1) * KB + 64 * (u & 1)) * 2;
        uint8_t *dst = (buf ? As1 : As0) + (16 * wave + 4 * j) * TROW;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void *)dst, 16, voff[j],
                                                 soff, 0, 0);
    };
    // A operand of MFMA tile i at k-step j: row lr + 32i, chunk 8h + j in slot
    // (8h + j) ^ (lr & 15)
    const uint8_t *rb[2][8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        int o0 = lr * TROW + 16 * ((8 * h + j) ^ (lr & 15)), o1 = o0;
        asm volatile("" : "+v"(o0), "+v"(o1));
        rb[0][j] = As0 + o0;
        rb[1][j] = As1 + o1;
    }
    auto a_read = [&](int buf, int j, int i) -> half8 {
        return *reinterpret_cast<const half8 *>(rb[buf][j] + 32 * i * TROW);
    };

    typename B::Raw raw;
    typename B::Prep p;
    auto w_load = [&](int b, int q) { B::load_part(wrow + (int64_t)b * B::BYTES, h, raw, q); };
    auto w_prep = [&](int b) { gb_prep<TYPE>(raw, h, wrow + (int64_t)b * B::BYTES, wsc, p); };

    floatx16 acc[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[i][v] = 0.f;

#pragma unroll
    for (int j = 0; j < 4; j++) a_dma(2 * b0, 0, j);
#pragma unroll
    for (int q = 0; q < B::NL; q++) w_load(b0, q);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    w_prep(b0);
    constexpr int AH = 2;
    half8 ar[AH][4];
    uint32_t bcur[4];
#pragma unroll
    for (int j = 0; j < AH; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) ar[j][i] = a_read(0, j, i);
#pragma unroll
    for (int d = 0; d < 4; d++) bcur[d] = B::dw(p, 0, d);

    const int u_end = 2 * b1;
    auto stage = [&](int u, int buf) {
        const int ts = u & 1;
        const int un = min(u + 1, u_end - 1);  // clamped: the last stage re-stages itself
        const int bn = min((u >> 1) + 1, b1 - 1);
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
            const int s = 8 * ts + ks;
            half8 an[4];
            uint32_t bnxt[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (ks == 0 && i == 0) __syncthreads();  // every wave is done with the other buffer
                if (ks == 6 && i == 0) {
                    __builtin_amdgcn_s_waitcnt(0);  // this wave's stage loads (the weight loads come after)
                    __syncthreads();
                }
                const half8 bo = __builtin_bit_cast(half8, make_uint4(bcur[0], bcur[1], bcur[2], bcur[3]));
                acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ar[0][i], bo, acc[i], 0, 0, 0);
                if (ks + AH < 8) an[i] = a_read(buf, ks + AH, i);
                else an[i] = a_read(buf ^ 1, ks + AH - 8, i);
                if (s < 15) {
                    if (i == 0 || i == 2) { bnxt[i] = B::dw(p, s + 1, i); bnxt[i + 1] = B::dw(p, s + 1, i + 1); }
                } else {
                    if (i == 0) w_prep(bn);
                    else if (i == 1 || i == 3) { bnxt[i - 1] = B::dw(p, 0, i - 1); bnxt[i] = B::dw(p, 0, i); }
                }
                if (ks == 0) a_dma(un, buf ^ 1, i);
                if (ts == 0 && (ks == 6 || ks == 7)) {
#pragma unroll
                    for (int q = 4 * (ks - 6) + i; q < B::NL; q += 8) w_load(bn, q);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) {
#pragma unroll
                for (int j = 0; j + 1 < AH; j++) ar[j][i] = ar[j + 1][i];
                ar[AH - 1][i] = an[i];
            }
#pragma unroll
            for (int d = 0; d < 4; d++) bcur[d] = bnxt[d];
        }
    };
    for (int u = 2 * b0; u < u_end; u += 2) {
        stage(u, 0);
        stage(u + 1, 1);
    }

#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = 32 * i + 8 * (v >> 2) + 4 * h + (v & 3);
            const int64_t m = m0 + r;
            const int64_t n = n0 + 32 * wave + lr;
            if (m < M && n < N) y[m * N + n] = __builtin_amdgcn_ldexpf(acc[i][v], Es[r] + en);
        }
    }
}

// ---------------------------------------------------------------------------
// K-sliced tiles for m <= 32.  A workgroup owns 128 columns (32 per wave) and a
// slice of S consecutive blocks of k that its four waves share.  The slice's
// activation operands (16 KB per block, operand-major) go into LDS by buffer
// loads issued first; then every weight load of the slice is issued at once.
// Memory loads complete in order, so with the activations ahead of the weights
// no wait ever holds a wave for a weight block it does not need yet, and each
// wave has its whole slice of weight bytes in flight (the stream's latency is
// paid once per workgroup, not once per block).  Slices write partial sums that
// k_split_sum adds in a fixed order.
// ---------------------------------------------------------------------------
constexpr int KSN = 128;  // columns per k-sliced workgroup

template <int TYPE>
constexpr int ks_blocks() { return 4; }  // longest slice: 4 x 16 KB of LDS, two workgroups per CU

template <int TYPE, int S, int T>
__global__ __launch_bounds__(256, 2) void k_gemm_ks(const uint8_t *W, int64_t N, int64_t row_bytes,
                                                    const _Float16 *__restrict__ A, const int *__restrict__ erow,
                                                    int64_t K, int64_t M, float *__restrict__ out, GemmGrid g) {
    const int slices = g.splits;
    const int64_t split_stride = g.split_stride;
    using B = GB<TYPE>;
    static_assert(S >= 1 && S <= ks_blocks<TYPE>() && (T == 1 || T == 2), "slice length, row tiles");
    __shared__ __align__(1024) uint8_t As[S * T * 16384];
    const int tn = (int)blockIdx.x / slices, z = (int)blockIdx.x % slices;
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5,
              lr = lane & 31;
    const int nb = (int)(K / KB);
    const int b0 = z * S, cnt = min(S, nb - b0);  // cnt >= 1
    const int64_t n0 = (int64_t)tn * KSN + 32 * wave;
    const int64_t wr = min(n0 + lr, N - 1);
    const uint8_t *wrow = W + wr * row_bytes + (int64_t)b0 * B::BYTES;
    const int en = g.rexp[wr];
    const float wsc = __builtin_amdgcn_ldexpf(1.f, -en);

    // the slice's operands: block b, row tile u, k-step s, lane l at byte
    // (((T b + u) 16 + s) 64 + l) 16; 1 KB per wave instruction, chunk 4i + wave;
    // chunks past the slice's last block read as zero (outside the buffer
    // resource) and are never used
    const uint64_t abase = reinterpret_cast<uint64_t>(A + (int64_t)b0 * T * 16 * 512);
    const uint64_t abase_s = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)abase) |
                             ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(abase >> 32)) << 32);
    const __amdgpu_buffer_rsrc_t arsrc = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<void *>(abase_s), (short)0, __builtin_amdgcn_readfirstlane(cnt * T * 16384), 0x00020000);
#pragma unroll
    for (int i = 0; i < 4 * S * T; i++) {
        const int chunk = 4 * i + wave;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void *)(As + chunk * 1024),
                                                 16, (uint32_t)lane * 16, chunk * 1024, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    // weight loads block by block, in order (each block's wait then covers only
    // the blocks before it)
    typename B::Raw raw[S];
#pragma unroll
    for (int b = 0; b < S; b++) {
#pragma unroll
        for (int q = 0; q < B::NL; q++) B::load_part(wrow + (int64_t)min(b, cnt - 1) * B::BYTES, h, raw[b], q);
        __builtin_amdgcn_sched_barrier(0);
    }
    // The activation loads are the oldest in flight.  The compiler tracks loads
    // to LDS and, before the barrier, waits for exactly those (vmcnt = the number
    // of weight load instructions issued after them, as it emitted them -- it may
    // merge neighbouring loads, so a count written here could be too high).
    __syncthreads();

    floatx16 acc[T];
#pragma unroll
    for (int u = 0; u < T; u++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[u][v] = 0.f;
    const uint8_t *arow = As + lane * 16;
#pragma unroll
    for (int b = 0; b < S; b++) {
        if (b < cnt) {
            typename B::Prep p;
            gb_prep<TYPE>(raw[b], h, wrow + (int64_t)b * B::BYTES, wsc, p);
#pragma unroll
            for (int s = 0; s < 16; s++) {
                uint32_t bw[4];
#pragma unroll
                for (int d = 0; d < 4; d++) bw[d] = B::dw(p, s, d);
                const half8 bo = __builtin_bit_cast(half8, make_uint4(bw[0], bw[1], bw[2], bw[3]));
#pragma unroll
                for (int u = 0; u < T; u++) {
                    const half8 a = *reinterpret_cast<const half8 *>(arow + ((b * T + u) * 16 + s) * 1024);
                    acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bo, acc[u], 0, 0, 0);
                }
            }
        }
    }

    float *y = out + (int64_t)z * split_stride;
    const int64_t n = n0 + lr;
    // D layout of a 32x32 MFMA tile: lane holds column l%32, rows 8(v/4) + 4h + v%4
#pragma unroll
    for (int u = 0; u < T; u++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = 32 * u + 8 * (v >> 2) + 4 * h + (v & 3);
            if (r < M && n < N) y[(int64_t)r * N + n] = __builtin_amdgcn_ldexpf(acc[u][v], erow[r] + en);
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

// ---------------------------------------------------------------------------
// Per-row operand exponents, once per weight: e_n such that the largest value
// any block of row n can produce, B_n, satisfies B_n * 2^-e_n < 2^15.  The
// bound is the largest |d|, |dmin| of the row's blocks times the largest code
// and scale products of the format: Q4_K 63*15 |d| + 63 |dmin|, Q5_K
// 63*31 |d| + 63 |dmin|, Q6_K 128*32 |d|, Q8_0 128 |d|.  Non-finite scales are
// left out (their blocks produce non-finite values whatever the exponent); a
// row of zero scales gets e_n = 0.  One thread per row.
// ---------------------------------------------------------------------------
template <int TYPE>
__global__ __launch_bounds__(256) void k_row_exponents(const uint8_t *__restrict__ W, int64_t N, int nb,
                                                        int64_t row_bytes, int8_t *__restrict__ rexp) {
    const int64_t n = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    const uint8_t *row = W + n * row_bytes;
    constexpr int SB = TYPE == TYPE_Q4_K ? 144 : TYPE == TYPE_Q5_K ? 176 : TYPE == TYPE_Q6_K ? 210 : 34;
    float dm = 0.f, mm = 0.f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = row + (int64_t)b * SB;
        float d, dmin = 0.f;
        if constexpr (TYPE == TYPE_Q6_K) {
            d = h2f(ld2_a2(blk + 208));
        } else if constexpr (TYPE == TYPE_Q8_0) {
            d = h2f(ld2_a2(blk));
        } else {
            const uint32_t hdr = ld_u32(blk);
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
                                            : 128.f * dm;
    // bound = f * 2^E, f in [0.5, 1): bound * 2^-(E - 15) = f * 2^15 < 2^15
    rexp[n] = (int8_t)(bound > 0.f ? __builtin_amdgcn_frexp_expf(bound) - 15 : 0);
}

hipError_t launch_row_exponents(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, int8_t *rexp,
                                hipStream_t st) {
    if (!gemm_serves(type, k)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((n + 255) / 256);
    const int nb = (int)(k / (type == TYPE_Q8_0 ? 32 : KB));
    switch (type) {
    case TYPE_Q4_K: k_row_exponents<TYPE_Q4_K><<<grid, 256, 0, st>>>(w, n, nb, row_bytes, rexp); break;
    case TYPE_Q5_K: k_row_exponents<TYPE_Q5_K><<<grid, 256, 0, st>>>(w, n, nb, row_bytes, rexp); break;
    case TYPE_Q6_K: k_row_exponents<TYPE_Q6_K><<<grid, 256, 0, st>>>(w, n, nb, row_bytes, rexp); break;
    default: k_row_exponents<TYPE_Q8_0><<<grid, 256, 0, st>>>(w, n, nb, row_bytes, rexp); break;
    }
    return hipGetLastError();
}

namespace {

struct Plan {
    int mt, tiles_m, tiles_n, splits, bps;  // bps: blocks of k per split
    int rt = 1;                             // k-sliced kernel: 32-row tiles per workgroup
};

// mt = 8 selects the tall kernel (256 x 128 tiles), MT_WIDE the wide one (128 x 256)
constexpr int MT_WIDE = 16, MT_KS = 32;  // MT_KS: the k-sliced kernel (m <= 64)
int tile_rows(const Plan &p) { return p.mt == MT_KS ? 32 * p.rt : p.mt == 8 ? TBM : p.mt == MT_WIDE ? WBM : 32 * p.mt; }
// the pre-pass layout: 32-row tiles of operand-major rows, or 0 (row-major)
int operand_major(const Plan &p) { return p.mt == MT_KS ? p.rt : 0; }
int ks_blocks_for(int type) {
    return type == TYPE_Q4_K   ? ks_blocks<TYPE_Q4_K>()
           : type == TYPE_Q5_K ? ks_blocks<TYPE_Q5_K>()
           : type == TYPE_Q6_K ? ks_blocks<TYPE_Q6_K>()
                               : ks_blocks<TYPE_Q8_0>();
}

// mt, rt and tile_rows depend on (type, k, m) only -- the pre-pass plans with n = 1
Plan plan_for(int type, int64_t n, int64_t k, int64_t m) {
    Plan p;
    // two row tiles (m <= 64) for Q6_K (3-19 % faster than its 64-row tiles at
    // m = 48, 64; for Q4_K / Q5_K the 64-row tiles win on the large matrices).
    // The choice -- and so the operand layout -- must not depend on n: a grouped
    // call runs one pre-pass for weights of different n.
    const Tuning &tu = tuning();
    // (Q8_0, whose raw super-blocks are the largest, plans as Q6_K)
    const bool heavy = type == TYPE_Q6_K || type == TYPE_Q8_0;
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
        const int smax = p.rt == 1 ? ks_blocks_for(type) : 2;
        int bps = smax;
        while (bps > 2 && (int64_t)p.tiles_n * ((nb + bps - 1) / bps) < (int64_t)num_cus()) bps--;
        if (tu.gemm_ks) bps = std::max(1, std::min(tu.gemm_ks, smax));  // tuning
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
    // MFMA decides (measured per type and m: 128, 256, 512, 2048)
    bool wide = m < 256 || (type == TYPE_Q4_K && m <= 512);
    if (tu.gemm_big) wide = tu.gemm_big == 1 || m < 256;  // tuning override: wide or tall
    // (Q6_K from 65 rows: its 64-row tiles took 66 us at m = 100 where the wide
    // tiles take 50 at m = 128, 14336 x 4096)
    if ((m >= 128 || (heavy && m > 64)) && big_ok) p.mt = wide ? MT_WIDE : 8;
    else p.mt = m <= 32 ? 1 : (m <= 64 || heavy) ? 2 : 4;  // Q6_K's raw blocks leave no room for MT = 4
    const int rows = tile_rows(p), cols = p.mt == 8 ? TBN : BN;
    p.tiles_m = (int)((m + rows - 1) / rows);
    p.tiles_n = (int)((n + cols - 1) / cols);
    const int nb = (int)(k / KB);
    const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
    // split k until the grid has about one workgroup per CU (also where two fit:
    // measured at m = 64, more splits only add partial-sum traffic)
    const int64_t slots = (int64_t)num_cus();
    int s = 1;
    if (tiles * 2 <= slots) s = (int)std::min<int64_t>(slots / tiles, nb);
    if (tu.gemm_splits) s = std::max(1, std::min(tu.gemm_splits, nb));  // tuning override
    p.bps = (nb + s - 1) / s;
    p.splits = (nb + p.bps - 1) / p.bps;
    return p;
}

template <int TYPE>
hipError_t launch_typed(const Plan &p, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t row_bytes,
                        const _Float16 *a, const int *erow, int64_t k, int64_t m, float *out, int64_t split_stride,
                        hipStream_t st) {
    const GemmGrid g{p.tiles_m, p.tiles_n, p.bps, split_stride, p.splits, rexp};
    const dim3 grid((unsigned)(p.tiles_m * p.tiles_n * p.splits));
    if (p.mt == MT_KS) {
        if (p.rt == 2) {  // two row tiles: slices of 1 or 2 blocks
            if (p.bps == 1) k_gemm_ks<TYPE, 1, 2><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g);
            else k_gemm_ks<TYPE, 2, 2><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g);
            return hipGetLastError();
        }
        switch (p.bps) {  // slice length
        case 1: k_gemm_ks<TYPE, 1, 1><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
        case 2: k_gemm_ks<TYPE, 2, 1><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
        case 3: k_gemm_ks<TYPE, 3, 1><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
        default: k_gemm_ks<TYPE, 4, 1><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
        }
        return hipGetLastError();
    }
    switch (p.mt) {
    case 8: k_gemm_t<TYPE><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
    case MT_WIDE: k_gemm_w<TYPE><<<grid, 512, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
    case 1: k_gemm<TYPE, 1><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
    case 2: k_gemm<TYPE, 2><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
    default:
        if constexpr (TYPE != TYPE_Q6_K && TYPE != TYPE_Q8_0)
            k_gemm<TYPE, 4><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g);
        break;
    }
    return hipGetLastError();
}

// workspace: fp16 operand rows [m][k] | row exponents [m] | split-k partials [S][m][n]
struct WsLayout {
    size_t a_off, e_off, part_off, total;
};

WsLayout ws_layout(const Plan &p, int64_t n, int64_t k, int64_t m) {
    auto up = [](size_t v) { return (v + 255) / 256 * 256; };
    WsLayout L;
    L.a_off = 0;
    L.e_off = L.a_off + up((size_t)p.tiles_m * tile_rows(p) * (size_t)k * sizeof(_Float16));  // whole row tiles
    L.part_off = L.e_off + up((size_t)m * sizeof(int));
    L.total = L.part_off + (p.splits > 1 ? up((size_t)p.splits * (size_t)(m * n) * sizeof(float)) : 0);
    return L;
}

}  // namespace

size_t gemm_workspace_bytes(int type, int64_t n, int64_t k, int64_t m) {
    if (!gemm_serves(type, k)) return 0;
    return ws_layout(plan_for(type, n, k, m), n, k, m).total;
}

bool gemm_prepass_fuses_quant(int type, int64_t k, const float *x) {
    return x && gemm_serves(type, k) && k / KB <= 64 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

hipError_t gemm_prepass(int type, int64_t k, const ActView &act, const float *x, int64_t m, void *ws, hipStream_t st) {
    if (!ws || !gemm_serves(type, k)) return hipErrorInvalidValue;
    const Plan p = plan_for(type, 1, k, m);  // the operand rows do not depend on n
    const WsLayout L = ws_layout(p, 1, k, m);
    uint8_t *base = static_cast<uint8_t *>(ws);
    _Float16 *a = reinterpret_cast<_Float16 *>(base + L.a_off);
    int *erow = reinterpret_cast<int *>(base + L.e_off);
    // few rows, or long rows up to 1024 of them: one pass of 1024 threads per
    // row; otherwise 256-thread workgroups (measured at m = 512 and 2048)
    const bool wide_wg = m <= 64 || (k > 8192 && m <= 1024);
    const int om = operand_major(p);
    if (x) {
        if (!gemm_prepass_fuses_quant(type, k, x)) return hipErrorInvalidValue;
        if (type == TYPE_Q8_0) {
            if (wide_wg) k_quant_f16_q80<1024><<<(unsigned)m, 1024, 0, st>>>(x, k, a, erow, om);
            else k_quant_f16_q80<256><<<(unsigned)m, 256, 0, st>>>(x, k, a, erow, om);
        } else {
            if (wide_wg) k_quant_f16<1024><<<(unsigned)m, 1024, 0, st>>>(x, k, a, erow, om);
            else k_quant_f16<256><<<(unsigned)m, 256, 0, st>>>(x, k, a, erow, om);
        }
    } else if (type == TYPE_Q8_0) {
        if (wide_wg) k_act_f16<1024, 32><<<(unsigned)m, 1024, 0, st>>>(act, m, a, erow, om);
        else k_act_f16<256, 32><<<(unsigned)m, 256, 0, st>>>(act, m, a, erow, om);
    } else {
        if (wide_wg) k_act_f16<1024, KB><<<(unsigned)m, 1024, 0, st>>>(act, m, a, erow, om);
        else k_act_f16<256, KB><<<(unsigned)m, 256, 0, st>>>(act, m, a, erow, om);
    }
    return hipGetLastError();
}

hipError_t gemm_main(int type, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t k, int64_t row_bytes, int64_t m,
                     float *y, void *ws, hipStream_t st) {
    if (!ws || !rexp || !gemm_serves(type, k)) return hipErrorInvalidValue;
    const Plan p = plan_for(type, n, k, m);
    const WsLayout L = ws_layout(p, n, k, m);
    uint8_t *base = static_cast<uint8_t *>(ws);
    const _Float16 *a = reinterpret_cast<const _Float16 *>(base + L.a_off);
    const int *erow = reinterpret_cast<const int *>(base + L.e_off);
    float *part = reinterpret_cast<float *>(base + L.part_off);
    float *out = p.splits > 1 ? part : y;
    const int64_t stride = p.splits > 1 ? m * n : 0;
    hipError_t e;
    switch (type) {
    case TYPE_Q4_K: e = launch_typed<TYPE_Q4_K>(p, w, rexp, n, row_bytes, a, erow, k, m, out, stride, st); break;
    case TYPE_Q5_K: e = launch_typed<TYPE_Q5_K>(p, w, rexp, n, row_bytes, a, erow, k, m, out, stride, st); break;
    case TYPE_Q6_K: e = launch_typed<TYPE_Q6_K>(p, w, rexp, n, row_bytes, a, erow, k, m, out, stride, st); break;
    default: e = launch_typed<TYPE_Q8_0>(p, w, rexp, n, row_bytes, a, erow, k, m, out, stride, st); break;
    }
    if (e != hipSuccess || p.splits == 1) return e;
    const int64_t count = m * n;
    k_split_sum<<<(unsigned)((count + 1023) / 1024), 256, 0, st>>>(part, p.splits, count, y);
    return hipGetLastError();
}

hipError_t launch_gemm(int type, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t k, int64_t row_bytes,
                       const ActView &act, const float *x, int64_t m, float *y, void *ws, hipStream_t st) {
    if (gemm_serves(type, k)) {
        hipError_t e = gemm_prepass(type, k, act, x, m, ws, st);
        if (e != hipSuccess) return e;
        return gemm_main(type, w, rexp, n, k, row_bytes, m, y, ws, st);
    }
    if (x) return hipErrorInvalidValue;  // the GEMV over row chunks takes quantised activations
    // Q8_0, the legacy types, Q2_K and Q3_K: the decode GEMV over row chunks of 8
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
