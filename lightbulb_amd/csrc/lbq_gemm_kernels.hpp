// lbq_gemm_kernels.hpp -- the batched path (m > 8): k-quant and legacy weights
// dequantised in registers straight into MFMA operands, activation codes staged
// through LDS.  Device code and the per-type launcher; lbq_gemm.hip plans the
// launch, runs the operand pre-pass and adds split-k partials, and one
// lbq_gemm_<type>.hip unit per weight type instantiates launch_typed.
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
#pragma once
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

// The 32-value legacy blocks, Q4_0 (d, qs[16]: 18 B), Q4_1 (d, m, qs: 20 B),
// Q5_0 (d, qh[4], qs: 22 B) and Q5_1 (d, m, qh, qs: 24 B).  A 256-value
// super-block of the k loop is 8 consecutive blocks (8*BB bytes, a multiple of 16,
// so rows of k % 256 == 0 keep every super-block 16-byte aligned); lane half h
// holds blocks 4h..4h+3, the BB dwords from byte 4*BB*h.  In a block, value
// j < 16 is the low nibble of qs[j] and value j + 16 its high nibble, with (Q5)
// bit j resp. j + 16 of the little-endian u32 qh as the fifth bit; the weight
// value is d*(q - 8) (Q4_0), d*(q - 16) (Q5_0) or d*q + m (Q4_1, Q5_1).  K-step s
// takes values 8(s%4)..8(s%4)+7 of block s/4: qs bytes 8(s%2).., low nibbles for
// s%4 < 2, high for s%4 >= 2 -- in place, as for Q4_K (subnormal operands, the
// scale pre-multiplied by 2^24 or 2^20).
//
// Q4_1 / Q5_1 (OFS): the reference's vec_dot adds m * s per block, s the Q8_1
// activation's stored f16 block sum (itself rounded from the f16 code sum times
// d), not m * sum of the activation values.  So the weight operand is d*q alone,
// and one more MFMA k-step per super-block adds the m * s products exactly: its
// B operand holds the lane half's four m (f16, times 2^-e_n: exact) in slots
// 0..3 and zeros in 4..7; its A operand, written by the pre-pass, the matching
// four s (times 2^-e_m) and zeros (odw, ofs operand rows).
template <int TYPE>
struct GBL {
    static constexpr int BB = TYPE == TYPE_Q4_0 ? 18 : TYPE == TYPE_Q4_1 ? 20 : TYPE == TYPE_Q5_0 ? 22 : 24;
    static constexpr bool Q5 = TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1;
    static constexpr bool OFS = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;  // d*q + m
    static constexpr int BYTES = 8 * BB;
    // 16-byte loads, then (18- and 22-byte blocks) one 8-byte tail, 8-byte aligned
    static constexpr int N16 = BB / 4, NL = N16 + (BB % 4 ? 1 : 0);
    struct Raw { u32x4a4 v[N16]; uint2 t; };
    // per block j: d1 (low nibbles: d*2^24; high: d*2^20 is d1*2^-4), c1; the qs
    // dwords; for Q5, the fifth bits of values 0..15 (e[2j]) and 16..31 (e[2j+1])
    // with bit i+2 moved to i+16, so one shift puts the bits of values i and i+2
    // at the two f16 slots of a dword
    struct Prep { float d1[4], c1[4]; uint32_t q[16], e[8], mw[2]; };
    __device__ static void load_part(const uint8_t *blk, int h, Raw &r, int i) {
        const uint8_t *base = blk + 4 * BB * h;
        if (i < N16) r.v[i] = gld16(align4_global(reinterpret_cast<uintptr_t>(base + 16 * i)));
        else r.t = *reinterpret_cast<const uint2 *>(base + 16 * N16);
    }
    __device__ static void prep(const Raw &r, float wsc, Prep &p) {
        uint32_t w[BB];
#pragma unroll
        for (int i = 0; i < N16; i++) { w[4 * i] = r.v[i].x; w[4 * i + 1] = r.v[i].y; w[4 * i + 2] = r.v[i].z; w[4 * i + 3] = r.v[i].w; }
#pragma unroll
        for (int i = 4 * N16; i < BB; i++) w[i] = i == 4 * N16 ? r.t.x : r.t.y;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // block j starts at byte BB*j: 2 mod 4 for odd j of the 18- and 22-byte
            // blocks, so its fields are funnel-shifted out of aligned dwords
            const int o = BB * j, wd = o / 4, mis = o % 4;  // compile-time
            const uint32_t h0 = mis ? (w[wd] >> 16) : (w[wd] & 0xffffu);
            const float d = h2f(h0) * wsc;
            p.d1[j] = d * 16777216.f;
            if constexpr (OFS) {
                // m (4-byte aligned blocks), as an f16 B value of the extra k-step
                p.c1[j] = 0.f;
                const uint32_t mh = __builtin_bit_cast(uint16_t, (_Float16)(h2f(w[wd] >> 16) * wsc));
                if (j & 1) p.mw[j >> 1] |= mh << 16;
                else p.mw[j >> 1] = mh;
            } else {
                p.c1[j] = (Q5 ? -16.f : -8.f) * d;
            }
            const int qo = o + (OFS ? 4 : 2) + (Q5 ? 4 : 0);  // byte of qs[0]
            auto dword_at = [&](int byte) -> uint32_t {
                return (byte % 4) ? __builtin_amdgcn_alignbyte(w[byte / 4 + 1], w[byte / 4], byte % 4) : w[byte / 4];
            };
#pragma unroll
            for (int i = 0; i < 4; i++) p.q[4 * j + i] = dword_at(qo + 4 * i);
            if constexpr (Q5) {
                const uint32_t qh = dword_at(o + (OFS ? 4 : 2));
                p.e[2 * j] = (qh & 0x3333u) | ((qh & 0xccccu) << 14);
                p.e[2 * j + 1] = ((qh >> 16) & 0x3333u) | (((qh >> 16) & 0xccccu) << 14);
            }
        }
    }
    // dword d of k-step s: f16 slots hold values (0, 2), (1, 3), (4, 6), (5, 7) of the 8
    __device__ static uint32_t dw(const Prep &p, int s, int d) {
        const int j = s >> 2, sub = s & 3, hi = sub >> 1;
        uint32_t q = p.q[4 * j + 2 * (sub & 1) + (d >> 1)];
        if (d & 1) q >>= 8;
        uint32_t v = q & (hi ? 0x00f000f0u : 0x000f000fu);
        if constexpr (Q5) {
            // value index i = 8(sub & 1) + (d & 1) + 4(d >> 1) within its 16: its
            // fifth bit (bit i of e) goes to bit 4 (low nibbles) or 8 (high), the
            // bit of value i + 2 (bit i + 16 of e) to bit 20 or 24
            const int i = 8 * (sub & 1) + (d & 1) + 4 * (d >> 1), to = hi ? 8 : 4;
            const uint32_t e = p.e[2 * j + hi];
            v |= (to >= i ? e << (to - i) : e >> (i - to)) & (hi ? 0x01000100u : 0x00100010u);
        }
        return scale2(v, hi ? p.d1[j] * 0.0625f : p.d1[j], p.c1[j]);
    }
    // dword d of the extra k-step's B operand (OFS): the m of blocks 2d, 2d+1, then zeros
    __device__ static uint32_t odw(const Prep &p, int d) { return d < 2 ? p.mw[d] : 0u; }
};
template <> struct GB<TYPE_Q4_0> : GBL<TYPE_Q4_0> {};
template <> struct GB<TYPE_Q4_1> : GBL<TYPE_Q4_1> {};
template <> struct GB<TYPE_Q5_0> : GBL<TYPE_Q5_0> {};
template <> struct GB<TYPE_Q5_1> : GBL<TYPE_Q5_1> {};

// Q2_K (scales[16], qs[64], d, dmin: 84 B, 4-byte aligned).  Value 128h + 32j + l
// (l < 32) is bits 2j, 2j+1 of qs[32h + l], in sub-block 8h + 2j + l/16, whose
// scale byte holds the 4-bit scale (low) and min (high): w = d*sc*q - dmin*mn.
// Lane half h holds qs[32h..32h+31] and scales[8h..8h+7].  The 2-bit codes stay in
// place (bits 2j, 2j+1 of a byte), so the scale is pre-multiplied by 2^(24-2j).
template <>
struct GB<TYPE_Q2_K> {
    static constexpr int BYTES = 84;
    static constexpr int NL = 5;
    struct Raw { u32x4a4 q[2]; uint32_t sc[2], dd; };
    struct Prep { float d1[8], c1[8]; uint32_t q[8]; };
    __device__ static void load_part(const uint8_t *blk, int h, Raw &r, int i) {
        if (i < 2) r.q[i] = gld16(align4_global(reinterpret_cast<uintptr_t>(blk + 16 + 32 * h + 16 * i)));
        else if (i < 4) r.sc[i - 2] = gld4(align4_global(reinterpret_cast<uintptr_t>(blk + 8 * h + 4 * (i - 2))));
        else r.dd = gld4(align4_global(reinterpret_cast<uintptr_t>(blk + 80)));  // d | dmin
    }
    __device__ static void prep(const Raw &r, float wsc, Prep &p) {
        const float d = h2f(r.dd & 0xffffu) * wsc, dmin = h2f(r.dd >> 16) * wsc;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t sc = (r.sc[i >> 2] >> (8 * (i & 3))) & 0xffu;
            p.d1[i] = d * (float)(sc & 0xfu) * __builtin_amdgcn_ldexpf(1.f, 24 - 2 * (i >> 1));
            p.c1[i] = -(dmin * (float)(sc >> 4));
        }
#pragma unroll
        for (int i = 0; i < 2; i++) { p.q[4 * i] = r.q[i].x; p.q[4 * i + 1] = r.q[i].y; p.q[4 * i + 2] = r.q[i].z; p.q[4 * i + 3] = r.q[i].w; }
    }
    // k-step s: shift j = s/4, qs bytes 8(s%4)..+7, sub-block 2j + (s%4)/2 = s/2
    __device__ static uint32_t dw(const Prep &p, int s, int d) {
        const int j = s >> 2;
        uint32_t q = p.q[2 * (s & 3) + (d >> 1)];
        if (d & 1) q >>= 8;
        return scale2(q & (0x00030003u << (2 * j)), p.d1[s >> 1], p.c1[s >> 1]);
    }
};

// Q3_K (hmask[32], qs[64], scales[12], d: 110 B, only 2-byte aligned).  Value
// 128h + 32j + l (l < 32): low bits 2j, 2j+1 of qs[32h + l], minus 4 unless bit
// 4h + j of hmask[l] is set, times d * (scale_{8h+2j+l/16} - 32), the 6-bit scale
// i having its low 4 bits in scales[i%8] (nibble i/8) and its top 2 in
// scales[8 + i%4] (bits 2(i/4)).  Lane half h holds qs[32h..32h+31], all of
// hmask (bits 4h..4h+3 of each byte) and all 12 scale bytes.  Fields are read as
// the aligned dwords that hold them (the last re-read when the field is 4-byte
// aligned, so no dword outside the block is touched) and funnel-shifted, as for
// Q6_K; the code u = low + 4*high sits at bits 2j..2j+2 of its byte, the scale is
// pre-multiplied by 2^(24-2j) and the -4 goes into c1.
template <>
struct GB<TYPE_Q3_K> {
    static constexpr int BYTES = 110;
    static constexpr int NL = 11;
    struct Raw { u32x4a4 ql[2], hm[2]; uint32_t qlt, hmt, sc[4], dw; };
    struct Prep { float d1[8], c1[8]; uint32_t l[8], hm[8]; };
    __device__ static gbytes_c al4(const uint8_t *p) { return align4_global(reinterpret_cast<uintptr_t>(p)); }
    __device__ static void load_part(const uint8_t *blk, int h, Raw &r, int i) {
        const bool mis = (reinterpret_cast<uintptr_t>(blk) & 3u) != 0;
        const gbytes_c ql = al4(blk + 32 + 32 * h), hm = al4(blk), sc = al4(blk + 96);
        if (i < 2) r.ql[i] = gld16(ql + 16 * i);
        else if (i < 4) r.hm[i - 2] = gld16(hm + 16 * (i - 2));
        else if (i == 4) r.qlt = gld4(ql + (mis ? 32 : 28));
        else if (i == 5) r.hmt = gld4(hm + (mis ? 32 : 28));
        else if (i < 9) r.sc[i - 6] = gld4(sc + 4 * (i - 6));
        else if (i == 9) r.sc[3] = gld4(sc + (mis ? 12 : 8));
        else r.dw = ld2_a2(blk + 108);
    }
    __device__ static void prep(const Raw &r, uint32_t mis, int h, float wsc, Prep &p) {
        uint32_t w[9], x[9];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            w[4 * i] = r.ql[i].x; w[4 * i + 1] = r.ql[i].y; w[4 * i + 2] = r.ql[i].z; w[4 * i + 3] = r.ql[i].w;
            x[4 * i] = r.hm[i].x; x[4 * i + 1] = r.hm[i].y; x[4 * i + 2] = r.hm[i].z; x[4 * i + 3] = r.hm[i].w;
        }
        w[8] = r.qlt;
        x[8] = r.hmt;
        const uint32_t sh = 4u * (uint32_t)h;  // bits 4h..4h+3 of every hmask byte to bits 0..3
#pragma unroll
        for (int i = 0; i < 8; i++) {
            p.l[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], mis);
            p.hm[i] = __builtin_amdgcn_alignbyte(x[i + 1], x[i], mis) >> sh;
        }
        const uint32_t s0 = __builtin_amdgcn_alignbyte(r.sc[1], r.sc[0], mis),
                       s1 = __builtin_amdgcn_alignbyte(r.sc[2], r.sc[1], mis),
                       s2 = __builtin_amdgcn_alignbyte(r.sc[3], r.sc[2], mis);
        const float d = h2f(r.dw) * wsc;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            // scale 8h + i: low nibble h of byte i, top bits 2(2h + i/4) of byte 8 + i%4
            const uint32_t lo = (((i < 4 ? s0 : s1) >> (8 * (i & 3))) >> sh) & 0xfu;
            const uint32_t hi2 = (s2 >> (8 * (i & 3) + 4 * h + 2 * (i >> 2))) & 3u;
            const float d1 = d * (float)((int)(lo | (hi2 << 4)) - 32);
            p.d1[i] = d1 * __builtin_amdgcn_ldexpf(1.f, 24 - 2 * (i >> 1));
            p.c1[i] = -4.f * d1;
        }
    }
    // k-step s: shift j = s/4, bytes 8(s%4)..+7 of the lane's qs and of hmask, sub-block s/2
    __device__ static uint32_t dw(const Prep &p, int s, int d) {
        const int j = s >> 2;
        uint32_t l = p.l[2 * (s & 3) + (d >> 1)], hq = p.hm[2 * (s & 3) + (d >> 1)];
        if (d & 1) { l >>= 8; hq >>= 8; }
        // the high bit (bit j of the hmask byte) to bit 2j + 2, above the low pair
        const uint32_t v = (l & (0x00030003u << (2 * j))) | ((hq << (j + 2)) & (0x00040004u << (2 * j)));
        return scale2(v, p.d1[s >> 1], p.c1[s >> 1]);
    }
};

template <int TYPE>
__device__ __forceinline__ void gb_prep(const typename GB<TYPE>::Raw &r, int h, const uint8_t *blk, float wsc,
                                        typename GB<TYPE>::Prep &p) {
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(blk) & 3u);
    if constexpr (TYPE == TYPE_Q6_K) { (void)h; GB<TYPE>::prep(r, mis, wsc, p); }
    else if constexpr (TYPE == TYPE_Q3_K) GB<TYPE>::prep(r, mis, h, wsc, p);
    else if constexpr (TYPE == TYPE_Q8_0 || TYPE == TYPE_Q2_K || is_legacy(TYPE)) { (void)h; (void)mis; GB<TYPE>::prep(r, wsc, p); }
    else { (void)blk; (void)mis; GB<TYPE>::prep(r, h, wsc, p); }
}


// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
struct GemmGrid {
    int tiles_m, tiles_n, bps;  // bps: blocks of k per split
    int64_t split_stride;       // floats between the partial outputs of two splits (0: no split)
    int splits;
    const int8_t *rexp;         // per weight row: e_n (w operands carry 2^-e_n)
    const _Float16 *ofs;        // OFS types: per operand row and super-block, 16 f16 A values of the extra k-step
    uint32_t *cnt;              // k-sliced split: per column tile, slices done (null: k_split_sum adds them)
    float *y;                   // ... and the output the last slice of a tile writes
    const float *x;             // k-sliced, Q8_K rows: f32 x [m][k] each workgroup quantises itself
};

// whether a weight type adds an extra k-step per super-block (odw)
template <int TYPE>
constexpr bool gemm_ofs() { return gemm_offset_step(TYPE); }

// the extra k-step's A operand of lane half h for operand row r, super-block b
__device__ __forceinline__ half8 ofs_operand(const _Float16 *ofs, int64_t r, int64_t nsb, int64_t b, int h) {
    return *reinterpret_cast<const half8 *>(ofs + (r * nsb + b) * 16 + 8 * h);
}

// resident workgroups per CU the register budget allows
template <int TYPE, int MT>
constexpr int gemm_occupancy() {
    return (MT == 4 || gemm_heavy(TYPE) || (TYPE != TYPE_Q4_K && MT == 2)) ? 1 : 2;
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
    // OFS types: the extra k-step's A operands, loaded at a block's k-step 0 and
    // used at its k-step 14 (while p still holds the block)
    constexpr bool OFS = gemm_ofs<TYPE>();
    half8 oa[OFS ? MT : 1];

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
                    if constexpr (OFS) {
                        if (s == 0 && j == 0) oa[i] = ofs_operand(g.ofs, m0 + 32 * i + lr, nb, b, h);
                        if (s == 14) {
                            const half8 bm = __builtin_bit_cast(half8, make_uint4(B::odw(p[j], 0), B::odw(p[j], 1), 0u, 0u));
                            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(oa[i], bm, acc[i][j], 0, 0, 0);
                        }
                    }
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
                // nontemporal, as in the wide and tall tiles (Q4_K 14336x4096 M = 48 / 64
                // 30.1 / 32.1 -> 29.5 / 31.2 us, split partials included)
                if (m < M && n < N) __builtin_nontemporal_store(__builtin_amdgcn_ldexpf(acc[i][j][v], e + en[j]), y + m * N + n);
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
    constexpr bool OFS = gemm_ofs<TYPE>();
    half8 oa[OFS ? 8 : 1];
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
    constexpr int AH = gemm_heavy(TYPE) ? 1 : 2;
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
        half8 bm;  // OFS: the extra k-step's B operand (the block's m values)
        if constexpr (OFS) bm = __builtin_bit_cast(half8, make_uint4(B::odw(p, 0), B::odw(p, 1), 0u, 0u));
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
                if constexpr (OFS) {
                    // the extra k-step: A loaded at the block's first k-step, used at
                    // its k-step 14 (while p still holds the block)
                    if (ts == 0 && ks == 0) oa[i] = ofs_operand(g.ofs, m0 + 32 * i + lr, nb, u >> 1, h);
                    if (ts == 1 && ks == 6) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(oa[i], bm, acc[i], 0, 0, 0);
                }
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
            // nontemporal: the output tile is written once, at the end, by every
            // workgroup at about the same time (Q4_K 14336x4096 M = 512 83.1 -> 80.5 us,
            // M = 2048 308.6 -> 302.3 us; Q6_K M = 512 108.5 -> 105.6 us)
            if (m < M && n < N) __builtin_nontemporal_store(__builtin_amdgcn_ldexpf(acc[i][v], Es[r] + en), y + m * N + n);
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
//
// NW = 7 (224-column tiles, the staging's 32 load instructions spread over the
// seven waves) where 256-column tiles leave part of the chip idle: 14336 columns
// at 128 rows are 224 workgroups of eight waves but 256 of seven.
constexpr int WBM = 128, WBN = 256;

template <int TYPE, int NW = 8>
__global__ __launch_bounds__(64 * NW, 1) void k_gemm_w(const uint8_t *__restrict__ W, int64_t N, int64_t row_bytes,
                                                       const _Float16 *__restrict__ A, const int *__restrict__ erow,
                                                       int64_t K, int64_t M, float *__restrict__ out, GemmGrid g) {
    static_assert(NW == 7 || NW == 8, "wide tiles: seven or eight waves");
    constexpr int CN = 32 * NW;  // columns per workgroup
    using B = GB<TYPE>;
    __shared__ __align__(1024) uint8_t As0[WBM * TROW];
    __shared__ __align__(1024) uint8_t As1[WBM * TROW];
    __shared__ int Es[WBM];

    const int G = (int)gridDim.x, L = (int)blockIdx.x;
    const int T = (G & 7) == 0 ? (L & 7) * (G >> 3) + (L >> 3) : L;
    const int tm = T % g.tiles_m, tn = (T / g.tiles_m) % g.tiles_n, z = T / (g.tiles_m * g.tiles_n);
    const int nb = (int)(K / KB);
    const int b0 = z * g.bps, b1 = min(nb, b0 + g.bps);
    const int64_t m0 = (int64_t)tm * WBM, n0 = (int64_t)tn * CN;
    float *y = out + (int64_t)z * g.split_stride;

    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6), h = lane >> 5,
              lr = lane & 31;
    const int64_t wr = min(n0 + 32 * wave + lr, N - 1);
    const uint8_t *wrow = W + wr * row_bytes;
    const int en = g.rexp[wr];
    const float wsc = __builtin_amdgcn_ldexpf(1.f, -en);
    if (t < WBM) Es[t] = erow[min(m0 + t, M - 1)];

    // staging: 32 load instructions per stage, instruction q filling stage rows
    // 4q + [0, 4); wave w issues q = w + NW i (i = 0.., q < 32): i = 0..3 at the
    // four MFMA regions of k-step 0, and with seven waves waves 0..3 a fifth at
    // region 0 of k-step 1.  Lane l writes row 4q + l/16, slot l%16, holding
    // logical chunk (l%16) ^ (row & 15) = (l%16) ^ ((4q + l/16) & 15).
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
    auto a_dma = [&](int u, int buf, int i) {  // this wave's instruction i (q = wave + NW i), if q < 32
        const int q = wave + NW * i;
        if (q >= 32) return;  // (wave-uniform)
        const int soff = (4 * q * (int)K + (u >> 1) * KB + 64 * (u & 1)) * 2;
        uint8_t *dst = (buf ? As1 : As0) + 4 * q * TROW;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (__attribute__((address_space(3))) void *)dst, 16, voff[q & 3],
                                                 soff, 0, 0);
    };
    constexpr int NI = (32 + NW - 1) / NW;  // staging instructions per wave and stage (at most)
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
    constexpr bool OFS = gemm_ofs<TYPE>();
    half8 oa[OFS ? 4 : 1];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[i][v] = 0.f;

#pragma unroll
    for (int j = 0; j < NI; j++) a_dma(2 * b0, 0, j);
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
        half8 bm;  // OFS: the extra k-step's B operand (the block's m values)
        if constexpr (OFS) bm = __builtin_bit_cast(half8, make_uint4(B::odw(p, 0), B::odw(p, 1), 0u, 0u));
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
                if constexpr (OFS) {  // the extra k-step, as in k_gemm_t
                    if (ts == 0 && ks == 0) oa[i] = ofs_operand(g.ofs, m0 + 32 * i + lr, nb, u >> 1, h);
                    if (ts == 1 && ks == 6) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(oa[i], bm, acc[i], 0, 0, 0);
                }
                if (ks + AH < 8) an[i] = a_read(buf, ks + AH, i);
                else an[i] = a_read(buf ^ 1, ks + AH - 8, i);
                if (s < 15) {
                    if (i == 0 || i == 2) { bnxt[i] = B::dw(p, s + 1, i); bnxt[i + 1] = B::dw(p, s + 1, i + 1); }
                } else {
                    if (i == 0) w_prep(bn);
                    else if (i == 1 || i == 3) { bnxt[i - 1] = B::dw(p, 0, i - 1); bnxt[i] = B::dw(p, 0, i); }
                }
                if (ks == 0) a_dma(un, buf ^ 1, i);
                if (NI > 4 && ks == 1 && i == 0) a_dma(un, buf ^ 1, 4);
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
            // nontemporal: the output tile is written once, at the end, by every
            // workgroup at about the same time (Q4_K 14336x4096 M = 512 83.1 -> 80.5 us,
            // M = 2048 308.6 -> 302.3 us; Q6_K M = 512 108.5 -> 105.6 us)
            if (m < M && n < N) __builtin_nontemporal_store(__builtin_amdgcn_ldexpf(acc[i][v], Es[r] + en), y + m * N + n);
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
//
// With f32 x and Q8_K activations (FX) there is no pre-pass: each workgroup
// quantises the rows of its own slice (Q8_K codes and scales as the reference,
// one operand exponent per row and slice) straight into LDS while its weight
// bytes are in flight.  The operand slots are then XOR-swizzled within each 1 KB
// (block, row tile, k-step) chunk (ks_swz) so that a wave's stores of one row
// spread over the banks; the MFMA reads apply the same swizzle.
// ---------------------------------------------------------------------------
constexpr int KSN = 128;  // columns per k-sliced workgroup

// FX operand slot swizzle of block b, k-step s: slot (32 h + row) ^ ks_swz
__device__ __forceinline__ constexpr int ks_swz(int b, int s) { return ((s >> 1) | ((b & 3) << 3)) & 31; }

constexpr int KS_BLOCKS = 4;  // longest slice: 4 x 16 KB of LDS, two workgroups per CU
constexpr int KS_FUSED_SLICES = 8;  // most slices the k-sliced kernel adds itself
constexpr int KS_FUSED_MIN_TILES = 64;  // ... and fewest column tiles
constexpr int KS_SC1 = 16;          // buffer-load cache policy: sc1 (agent-scope coherent)
constexpr int KS_SUM_Q = 4;         // slices each thread loads per round of the in-kernel sum
constexpr int KS_RING = 2;          // weight blocks in flight per wave

// With Q8_K activations the k-sliced layout's operand rows carry one exponent per
// group of KS_BLOCKS blocks (erow[group][m]) rather than per row, so its pre-pass
// runs one wave per (row, group); a slice (1, 2 or 4 blocks, aligned) never spans
// two groups.
template <int TYPE>
constexpr bool ks_group_exponents() { return vec_dot_type(TYPE) == TYPE_Q8_K; }

// FX: the rows 0 .. min(M, 32 T) - 1 of blocks b0 .. b0 + cnt - 1 of x, quantised
// to Q8_K (q8k_lane16: 16 lanes per (row, block), 16 values each), become the
// operands f16(q d 2^-e) in the slice's LDS layout (operand-major, swizzled), e
// = the row's exponent over the slice's blocks (as k_ops_ks over a group), in
// Es.  A wave takes 4 / S rows per pass.  ks_load_slice issues every pass's
// loads (before the weight loads, so no wait for x is held up behind them);
// ks_quantise_slice stores.  Rows past M and blocks past the slice are neither
// loaded nor stored (their MFMA rows are never written out, their blocks never
// multiplied).
template <int S, int MR>  // MR: rows quantised (16, 32 or 64; at least M)
struct KsSlice {
    static constexpr int RPW = KS_BLOCKS / S;  // rows per wave and pass
    static constexpr int NP = MR / (4 * RPW);  // passes
    float v[NP][16];
};

template <int S, int MR>
__device__ __forceinline__ void ks_load_slice(KsSlice<S, MR> &xs, const float *__restrict__ x, int64_t K, int64_t M,
                                              int b0, int cnt, int wave, int lane) {
    using X = KsSlice<S, MR>;
    const int sub = lane & 15, bi = (lane >> 4) % S, ri = (lane >> 4) / S;
#pragma unroll
    for (int p = 0; p < X::NP; p++) {
        const int row = (p * 4 + wave) * X::RPW + ri;
        const bool live = row < M && bi < cnt;
        const float4 *src = reinterpret_cast<const float4 *>(
            x + (live ? (int64_t)row * K + (int64_t)(b0 + bi) * KB + 16 * sub : 0));
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = live ? src[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            xs.v[p][4 * i] = f.x; xs.v[p][4 * i + 1] = f.y; xs.v[p][4 * i + 2] = f.z; xs.v[p][4 * i + 3] = f.w;
        }
    }
}

template <int S, int T, int MR>
__device__ __forceinline__ void ks_quantise_slice(KsSlice<S, MR> &xs, int64_t M, int cnt, int wave, int lane,
                                                  uint8_t *As, int *Es) {
    using X = KsSlice<S, MR>;
    const int sub = lane & 15, bi = (lane >> 4) % S, ri = (lane >> 4) / S;
#pragma unroll
    for (int p = 0; p < X::NP; p++) {
        const int row = (p * 4 + wave) * X::RPW + ri;
        const bool live = row < M && bi < cnt;
        uint32_t packed[4];
        int sum;
        float d;
        q8k_lane16(xs.v[p], sub, packed, &sum, &d);
        float mx = live ? fabsf(d) : 0.f;
        if constexpr (S >= 2) mx = fmaxf(mx, __shfl_xor(mx, 16));
        if constexpr (S >= 4) mx = fmaxf(mx, __shfl_xor(mx, 32));
        const int e = mx > 0.f ? __builtin_amdgcn_frexp_expf(mx) - 8 : 0;
        if (bi == 0 && sub == 0 && row < M) Es[row] = e;
        if (!live) continue;
        const float sx = __builtin_amdgcn_ldexpf(d, -e);
        const float cc = -1152.f * sx;
        uint32_t w8[8];
        codes_to_f16(packed[0], sx, cc, &w8[0], &w8[1]);
        codes_to_f16(packed[1], sx, cc, &w8[2], &w8[3]);
        codes_to_f16(packed[2], sx, cc, &w8[4], &w8[5]);
        codes_to_f16(packed[3], sx, cc, &w8[6], &w8[7]);
#pragma unroll
        for (int q = 0; q < 2; q++) {
            const int p8 = 2 * sub + q, st = p8 & 15, hh = p8 >> 4;
            const int chunk = (T * bi + (row >> 5)) * 16 + st;
            const int slot = (32 * hh + (row & 31)) ^ ks_swz(bi, st);
            *reinterpret_cast<uint4 *>(As + chunk * 1024 + slot * 16) =
                make_uint4(w8[4 * q], w8[4 * q + 1], w8[4 * q + 2], w8[4 * q + 3]);
        }
    }
}

// slice shapes whose x fits the registers beside the weight bytes (64 floats a
// lane): MR quantised rows (16 for m <= 16, else 32 per row tile) times S blocks
constexpr int ks_fx_rows(int64_t m, int T) { return m <= 16 ? 16 : 32 * T; }
constexpr bool ks_fx_shape(int S, int MR) { return (S == 1 || S == 2 || S == 4) && MR * S <= 64; }
constexpr int KS_FX_MAX_TILES = 32;  // most column tiles (4096 columns) that quantise x in the kernel

// Slices added in the kernel (k_gemm_ks): the partial stores before
// this call are agent-scope (written through to memory, not held in this XCD's
// L2), so once they have completed (vmcnt(0)) a counter increment publishes them
// without an L2 write-back.  The workgroup that completes a column tile's count
// adds the tile's slices in slice order -- the order k_split_sum uses, so the bits
// are the same -- reading them with the same agent-scope (sc1) policy, writes y
// and puts the counter back to zero for the next call.  The host uses this only
// for N % 4 == 0 (16-byte partial rows) and at most KS_FUSED_SLICES slices.
// Every thread of the workgroup (NT) calls it.
template <int T, int NT>
__device__ __forceinline__ void ks_slice_sum(const float *out, int64_t split_stride, int slices, int tn, int t,
                                             int64_t M, int64_t N, const GemmGrid &g) {
    __shared__ uint32_t last;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (t == 0) last = __hip_atomic_fetch_add(g.cnt + tn, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (last != (uint32_t)(slices - 1)) return;
    // thread t: columns 4(t % 32) .. +3 of the tile, rows t / 32 + (NT / 32) j
    constexpr int RS = NT / 32;                      // rows apart
    constexpr int RQ = (32 * T + RS - 1) / RS;       // rows per thread, two at a time
    const int64_t col = (int64_t)tn * KSN + 4 * (t & 31);
    const int rows = (int)min<int64_t>(M, 32 * T);
    if (col < N) {
        const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(out), (short)0, (int)(split_stride * slices * (int64_t)sizeof(float)), 0x00020000);
#pragma unroll
        for (int r0 = 0; r0 < RQ; r0 += 2) {
            float4 sum[2];
            for (int q0 = 0; q0 < slices; q0 += KS_SUM_Q) {
                float4 v[2][KS_SUM_Q];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int r = (t >> 5) + RS * (r0 + j);
#pragma unroll
                    for (int q = 0; q < KS_SUM_Q; q++)
                        if (r < rows && q0 + q < slices)
                            v[j][q] = __builtin_bit_cast(
                                float4, __builtin_amdgcn_raw_buffer_load_b128(
                                            prs, (int)(((int64_t)(q0 + q) * split_stride + (int64_t)r * N + col) * 4),
                                            0, KS_SC1));
                }
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int q = 0; q < KS_SUM_Q; q++) {
                        if (q0 + q >= slices) continue;
                        if (q0 + q == 0) {
                            sum[j] = v[j][q];
                        } else {
                            sum[j].x += v[j][q].x; sum[j].y += v[j][q].y;
                            sum[j].z += v[j][q].z; sum[j].w += v[j][q].w;
                        }
                    }
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int r = (t >> 5) + RS * (r0 + j);
                if (r >= rows) continue;
                float *yo = g.y + (int64_t)r * N + col;
                // the output: nontemporal, as every tile's final stores
                __builtin_nontemporal_store(sum[j].x, yo); __builtin_nontemporal_store(sum[j].y, yo + 1);
                __builtin_nontemporal_store(sum[j].z, yo + 2); __builtin_nontemporal_store(sum[j].w, yo + 3);
            }
        }
    }
    if (t == 0) __hip_atomic_store(g.cnt + tn, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int TYPE, int S, int T, int FXR = 0>
__global__ __launch_bounds__(256, 2) void k_gemm_ks(const uint8_t *W, int64_t N, int64_t row_bytes,
                                                    const _Float16 *__restrict__ A, const int *__restrict__ erow,
                                                    int64_t K, int64_t M, float *__restrict__ out, GemmGrid g) {
    const int slices = g.splits;
    const int64_t split_stride = g.split_stride;
    using B = GB<TYPE>;
    static_assert(S >= 1 && S <= KS_BLOCKS && (T == 1 || T == 2), "slice length, row tiles");
    constexpr bool FX = FXR > 0;  // FXR: rows this kernel quantises from x
    static_assert(!FX || (ks_group_exponents<TYPE>() && ks_fx_shape(S, FXR) && FXR <= 32 * T), "FX: Q8_K, x in registers");
    __shared__ __align__(1024) uint8_t As[S * T * 16384];
    __shared__ int Es[FX ? 32 * T : 1];  // FX: the slice's operand exponent per row
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
    if constexpr (!FX) {
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
    }
    // FX: the slice's x, before the weights
    KsSlice<FX ? S : 1, FX ? FXR : 16> xs;
    if constexpr (FX) {
        ks_load_slice<S, FXR>(xs, g.x, K, M, b0, cnt, wave, lane);
        __builtin_amdgcn_sched_barrier(0);
    }
    // OFS types: the extra k-step's A operands of the slice, before the weights
    constexpr bool OFS = gemm_ofs<TYPE>();
    half8 oa[OFS ? S : 1][T];
    if constexpr (OFS) {
#pragma unroll
        for (int b = 0; b < S; b++)
#pragma unroll
            for (int u = 0; u < T; u++) oa[b][u] = ofs_operand(g.ofs, 32 * u + lr, nb, b0 + min(b, cnt - 1), h);
    }
    // weight loads block by block, in order (each block's wait then covers only
    // the blocks before it).  Q4_K / Q5_K keep KS_RING blocks ahead: block b + D
    // goes out as soon as block b's bytes are in its Prep, so the stream feeds the
    // compute instead of every workgroup's whole slice arriving at once (1.5-2 us
    // faster at 4096 x 14336, m = 16); the other types issue the whole slice at
    // once (Q6_K: 1.4 us slower with the ring)
    constexpr int D = (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) && KS_RING < S ? KS_RING : S;
    typename B::Raw raw[D];
#pragma unroll
    for (int b = 0; b < D; b++) {
#pragma unroll
        for (int q = 0; q < B::NL; q++) B::load_part(wrow + (int64_t)min(b, cnt - 1) * B::BYTES, h, raw[b], q);
        __builtin_amdgcn_sched_barrier(0);
    }
    // The activation loads are the oldest in flight.  The compiler tracks loads
    // to LDS and, before the barrier, waits for exactly those (vmcnt = the number
    // of weight load instructions issued after them, as it emitted them -- it may
    // merge neighbouring loads, so a count written here could be too high).
    if constexpr (FX) ks_quantise_slice<S, T, FXR>(xs, M, cnt, wave, lane, As, Es);
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
            gb_prep<TYPE>(raw[b % D], h, wrow + (int64_t)b * B::BYTES, wsc, p);
            if constexpr (D < S) {
                if (b + D < S) {
#pragma unroll
                    for (int q = 0; q < B::NL; q++)
                        B::load_part(wrow + (int64_t)min(b + D, cnt - 1) * B::BYTES, h, raw[b % D], q);
                }
            }
#pragma unroll
            for (int s = 0; s < 16; s++) {
                uint32_t bw[4];
#pragma unroll
                for (int d = 0; d < 4; d++) bw[d] = B::dw(p, s, d);
                const half8 bo = __builtin_bit_cast(half8, make_uint4(bw[0], bw[1], bw[2], bw[3]));
#pragma unroll
                for (int u = 0; u < T; u++) {
                    const half8 a = FX ? *reinterpret_cast<const half8 *>(As + ((b * T + u) * 16 + s) * 1024 +
                                                                          ((lane ^ ks_swz(b, s)) << 4))
                                       : *reinterpret_cast<const half8 *>(arow + ((b * T + u) * 16 + s) * 1024);
                    acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bo, acc[u], 0, 0, 0);
                }
            }
            if constexpr (OFS) {
                const half8 bo = __builtin_bit_cast(half8, make_uint4(B::odw(p, 0), B::odw(p, 1), 0u, 0u));
#pragma unroll
                for (int u = 0; u < T; u++) acc[u] = __builtin_amdgcn_mfma_f32_32x32x16_f16(oa[b][u], bo, acc[u], 0, 0, 0);
            }
        }
    }

    float *y = out + (int64_t)z * split_stride;
    const int64_t n = n0 + lr;
    // D layout of a 32x32 MFMA tile: lane holds column l%32, rows 8(v/4) + 4h + v%4.
    // Every row's exponent is loaded before the first store (rows past m read row
    // m - 1 and are never stored), so the loads overlap instead of each waiting
    // behind the stores before it.
    const int *ex_row = erow + (ks_group_exponents<TYPE>() ? (int64_t)(b0 / KS_BLOCKS) * M : 0);
    int ex[T][16];
#pragma unroll
    for (int u = 0; u < T; u++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = 32 * u + 8 * (v >> 2) + 4 * h + (v & 3);
            ex[u][v] = FX ? Es[r < M ? r : M - 1] : ex_row[r < M ? r : M - 1];
        }
#pragma unroll
    for (int u = 0; u < T; u++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int r = 32 * u + 8 * (v >> 2) + 4 * h + (v & 3);
            acc[u][v] = __builtin_amdgcn_ldexpf(acc[u][v], ex[u][v] + en);
            if (r < M && n < N) {
                if (g.cnt) __hip_atomic_store(y + (int64_t)r * N + n, acc[u][v], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                // y itself (no split): nontemporal (Q6_K 128256x4096 m = 32 184.3 -> 182.9 us);
                // split partials, which the split-sum launch reads right back, stay cached
                // (nontemporal: 1024x4096 m = 32 10.7 -> 11.1 us)
                else if (g.split_stride == 0) __builtin_nontemporal_store(acc[u][v], y + (int64_t)r * N + n);
                else y[(int64_t)r * N + n] = acc[u][v];
            }
        }
    if (!g.cnt) return;
    ks_slice_sum<T, 256>(out, split_stride, slices, tn, t, M, N, g);
}

struct Plan {
    int mt, tiles_m, tiles_n, splits, bps;  // bps: blocks of k per split
    int rt = 1;                             // k-sliced kernel: 32-row tiles per workgroup
};

// mt = 8 selects the tall kernel (256 x 128 tiles), MT_WIDE the wide one (128 x 256),
// MT_WIDE7 the wide one with seven waves (128 x 224)
constexpr int MT_WIDE = 16, MT_WIDE7 = 17, MT_KS = 32;  // MT_KS: the k-sliced kernel (m <= 64)
inline int tile_rows(const Plan &p) {
    return p.mt == MT_KS ? 32 * p.rt : p.mt == 8 ? TBM : (p.mt == MT_WIDE || p.mt == MT_WIDE7) ? WBM : 32 * p.mt;
}
// the pre-pass layout: 32-row tiles of operand-major rows, or 0 (row-major)
inline int operand_major(const Plan &p) { return p.mt == MT_KS ? p.rt : 0; }
template <int TYPE>
hipError_t launch_typed(const Plan &p, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t row_bytes,
                        const _Float16 *a, const int *erow, const _Float16 *ofs, int64_t k, int64_t m, float *out,
                        int64_t split_stride, uint32_t *cnt, float *y, const float *x, hipStream_t st) {
    const GemmGrid g{p.tiles_m, p.tiles_n, p.bps, split_stride, p.splits, rexp, ofs, cnt, y, x};
    const dim3 grid((unsigned)(p.tiles_m * p.tiles_n * p.splits));
    if constexpr (ks_group_exponents<TYPE>()) {
        if (x) {  // k-sliced, quantising x in the kernel (ks_fx_shape slices)
            const int mr = ks_fx_rows(m, p.rt);
            if (p.mt != MT_KS || !ks_fx_shape(p.bps, mr)) return hipErrorInvalidValue;
#define LBQ_KS_FX(S_, T_, MR_) k_gemm_ks<TYPE, S_, T_, MR_><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g)
            if (p.rt == 2) LBQ_KS_FX(1, 2, 64);
            else if (mr == 16 && p.bps == 4) LBQ_KS_FX(4, 1, 16);
            else if (mr == 16 && p.bps == 2) LBQ_KS_FX(2, 1, 16);
            else if (mr == 16) LBQ_KS_FX(1, 1, 16);
            else if (p.bps == 2) LBQ_KS_FX(2, 1, 32);
            else LBQ_KS_FX(1, 1, 32);
#undef LBQ_KS_FX
            return hipGetLastError();
        }
    } else if (x) {
        return hipErrorInvalidValue;
    }
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
    case MT_WIDE7: k_gemm_w<TYPE, 7><<<grid, 448, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
    case 1: k_gemm<TYPE, 1><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
    case 2: k_gemm<TYPE, 2><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g); break;
    default:
        if constexpr (!gemm_heavy(TYPE))
            k_gemm<TYPE, 4><<<grid, 256, 0, st>>>(w, n, row_bytes, a, erow, k, m, out, g);
        break;
    }
    return hipGetLastError();
}

}  // namespace lbq
