// lbq_gemv_fast.hpp -- batch-1 decode GEMV.
//
// Same arithmetic as the general GEMV (exact int32 sub-block sums of Q8_K/Q8_0
// codes x weight codes, f32 combine), organised for the m = 1 weight stream:
//   - eight lanes share each weight block's header and read its 16-byte code
//     pieces side by side, so a wave instruction reads whole 128-byte runs;
//   - the quantised activation sits in LDS in a padded layout (odd multiples of
//     16 bytes per block), so lanes reading different blocks hit different banks;
//   - waves are persistent, each owning a contiguous range of row groups with
//     the weight loads of the next one (Q6_K, Q8_0) or two (Q4_K, Q5_K) groups
//     in flight while a group is computed;
//   - with FUSED, the workgroup quantises x itself (Q8_K or Q8_0, bit-identical
//     to the standalone kernels) into LDS first; the loads of the first row
//     group are issued before the quantisation so their latency overlaps it;
//   - row sums use DPP lane permutes and readlane, not LDS shuffles.
#pragma once
#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {



// Q8_K of one 256-value block by one wave (lane holds values 4*lane..4*lane+3).
// Same selection and arithmetic as q8k_block_wave: the first value of largest |x|
// (NaN never chosen) sets iscale = -128/max; q = min(127, round(iscale*x)); d = 1/iscale.
__device__ __forceinline__ uint32_t q8k_block_wave_dpp(const float v[4], int lane, int *sum16, float *d_out) {
    // |x| as ordered bits; NaN -> 0 (never selected, like candle's `amax < |x|`)
    uint32_t a[4], am = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float f = fabsf(v[i]);
        a[i] = (f == f) ? __float_as_uint(f) : 0u;
        am = max(am, a[i]);
    }
    am = row_max_u32(am);
    const uint32_t wmax = max(max(rl(am, 0), rl(am, 16)), max(rl(am, 32), rl(am, 48)));
    uint32_t packed = 0;
    int s = 0;
    float d = 0.f;
    if (wmax != 0u) {
        // first index holding the maximum
        uint32_t key = 0xffffffffu;
#pragma unroll
        for (int i = 3; i >= 0; i--)
            if (a[i] == wmax) key = (uint32_t)(lane * 4 + i);
        key = row_min_u32(key);
        const uint32_t first = min(min(rl(key, 0), rl(key, 16)), min(rl(key, 32), rl(key, 48)));
        const int src_lane = (int)(first >> 2), src_i = (int)(first & 3);
        const float mine = src_i == 0 ? v[0] : src_i == 1 ? v[1] : src_i == 2 ? v[2] : v[3];
        const float mx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), src_lane));
        const float iscale = -128.f / mx;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            float r = fminf(roundf(iscale * v[i]), 127.f);
            r = fmaxf(r, -128.f);
            const int q = (int)r;
            s += q;
            packed |= ((uint32_t)q & 0xffu) << (8 * i);
        }
        d = 1.f / iscale;
    }
    *sum16 = quad_sum_i32(s);
    *d_out = d;
    return packed;
}

// LDS layout of a quantised activation block.
//   Q8_K: 304-byte blocks (19 x 16 B, odd, so lanes reading different blocks spread
//         over all banks): codes [0,256), bsums int16[16] @256, d f32 @288.
//   Q8_0: 48-byte blocks: codes [0,32), d f32 @32.
constexpr int XS_K = 304;
constexpr int XS_0 = 48;

// ---------------------------------------------------------------------------
// per-type register traits.  A piece is the unit a lane decodes (see the
// general GEMV); XW is the number of activation dwords a lane keeps per block.
// ---------------------------------------------------------------------------
template <int TYPE, int PPB>
struct Fast;

typedef short short2v __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_halves(uint32_t lo_word, uint32_t hi_word, int h) {
    const uint32_t a = (lo_word >> (16 * h)) & 0xffffu, b = (hi_word >> (16 * h)) & 0xffffu;
    return a | (b << 16);
}

// Q4_K / Q5_K: piece p (0..3) of a block is its 32-byte qs chunk c = p: the low
// nibbles of qs[32c + l] are values 64c + l (sub-block 2c), the high nibbles values
// 64c + 32 + l (sub-block 2c + 1), l < 32.  The four lanes of a block form a DPP
// quad; lane p loads header dword p and the quad shares the four through quad
// broadcasts.  Sixty-four weights per lane and piece keep the per-piece work (header
// broadcast, scale unpack, float combine) to one instance per two sub-blocks.
template <int TYPE>
struct FastK45 {  // Q4_K and Q5_K
    static constexpr int PPB = 4, VALS = 256, XW = 19;
    static constexpr int BYTES = TYPE == TYPE_Q4_K ? 144 : 176;
    static constexpr int NBUF = 3;  // three-buffer ring allowed (see k_gemv1)
    static constexpr int RAW = TYPE == TYPE_Q4_K ? 9 : 17;  // registers a loaded piece occupies
    struct Raw { uint32_t hw; uint4 qh0, qh1, qs0, qs1; };
    __device__ static Raw load(const uint8_t *blk, int p) {
        Raw r;
        r.hw = *reinterpret_cast<const uint32_t *>(blk + 4 * p);
        if (TYPE == TYPE_Q5_K) {
            r.qh0 = ld_u4(blk + 16);
            r.qh1 = ld_u4(blk + 32);
        }
        const uint8_t *qs = blk + (TYPE == TYPE_Q4_K ? 16 : 48) + 32 * p;
        r.qs0 = ld_u4(qs);
        r.qs1 = ld_u4(qs + 16);
        return r;
    }
    // activation registers for piece p: codes 64p .. 64p + 63 (xr[0..15]), the
    // code sums of its two 32-value sub-blocks as an int16 pair (xr[16], from the
    // bsums of its four 16-value runs; |sum| <= 4096) and the block's d (xr[18])
    __device__ static void xload_lds(const uint8_t *xb, int p, uint32_t *xr) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 a = *reinterpret_cast<const uint4 *>(xb + 64 * p + 16 * j);
            xr[4 * j] = a.x; xr[4 * j + 1] = a.y; xr[4 * j + 2] = a.z; xr[4 * j + 3] = a.w;
        }
        const uint2 s = *reinterpret_cast<const uint2 *>(xb + 256 + 8 * p);
        // (run 0, run 2) + (run 1, run 3), lane-wise 16-bit adds
        const uint32_t r02 = __builtin_amdgcn_perm(s.y, s.x, 0x05040100u), r13 = __builtin_amdgcn_perm(s.y, s.x, 0x07060302u);
        xr[16] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(short2v, r02) + __builtin_bit_cast(short2v, r13));
        xr[17] = 0u;
        xr[18] = *reinterpret_cast<const uint32_t *>(xb + 288);
    }
    // Piece p of one weight block against MR activation rows: the weight codes are
    // unpacked once; xl(m, xr) fills row m's activation registers; valid masks the
    // contribution of a clamped (duplicate) block.
    template <int MR, class XL>
    __device__ static void dotm(const Raw &r, int p, XL xl, float *acc, bool valid) {
        // Header dword i sits in lane i of every quad.  The 6-bit scales and mins of
        // sub-blocks 2p, 2p + 1 (get_scale_min_k4): for p < 2, sc = scales[j] & 63 and
        // m = scales[j + 4] & 63 (bytes 2p, 2p + 1 of dwords 1 and 2); for p >= 2,
        // sc = (scales[j + 4] & 15) | (scales[j - 4] >> 6) << 4 and
        // m = (scales[j + 4] >> 4) | (scales[j] >> 6) << 4 (dword 3 with the top bits
        // of dwords 1 and 2).  X and Y deliver dword 1 / 2 to lanes 0, 1 of the quad
        // and dword 3 to lanes 2, 3; shifts and masks depend on p only.
        const uint32_t h0 = qperm<0x00>(r.hw), s0 = qperm<0x55>(r.hw), s1 = qperm<0xAA>(r.hw);
        const uint32_t X = qperm<0xF5>(r.hw), Y = qperm<0xFA>(r.hw);
        const bool upper = p >= 2;
        const uint32_t bsh = 16u * (uint32_t)(p & 1);
        const uint32_t MA = upper ? 0x0f0fu : 0x3f3fu, MB = upper ? 0x3030u : 0u;
        const uint32_t sc2 = ((X >> bsh) & MA) | ((s0 >> (bsh + 2)) & MB);
        const uint32_t m2 = ((Y >> (bsh + (upper ? 4u : 0u))) & MA) | ((s1 >> (bsh + 2)) & MB);
        const uint32_t q[8] = {r.qs0.x, r.qs0.y, r.qs0.z, r.qs0.w, r.qs1.x, r.qs1.y, r.qs1.z, r.qs1.w};
        uint32_t lo[8], hi[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i] = q[i] & 0x0f0f0f0fu;
            hi[i] = (q[i] >> 4) & 0x0f0f0f0fu;
            if (TYPE == TYPE_Q5_K) {
                const uint32_t qh = i < 4 ? (i == 0 ? r.qh0.x : i == 1 ? r.qh0.y : i == 2 ? r.qh0.z : r.qh0.w)
                                          : (i == 4 ? r.qh1.x : i == 5 ? r.qh1.y : i == 6 ? r.qh1.z : r.qh1.w);
                lo[i] |= ((qh >> (2 * p)) & 0x01010101u) << 4;
                hi[i] |= ((qh >> (2 * p + 1)) & 0x01010101u) << 4;
            }
        }
        // a clamped (duplicate) block contributes through zero scales
        const float dw = valid ? h2f(h0 & 0xffffu) : 0.f, dmw = valid ? h2f(h0 >> 16) : 0.f;
        const int scl = (int)(sc2 & 0xffu), sch = (int)(sc2 >> 8);
        const short2v mins = __builtin_bit_cast(short2v, (m2 & 0xffu) | ((m2 >> 8) << 16));  // (m_lo, m_hi)
#pragma unroll
        for (int m = 0; m < MR; m++) {
            uint32_t xr[XW];
            xl(m, xr);
            int sl = 0, sh = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                sl = dot4(lo[i], xr[i], sl);
                sh = dot4(hi[i], xr[8 + i], sh);
            }
            const int isum = __mul24(scl, sl) + __mul24(sch, sh);
            const int msum = __builtin_amdgcn_sdot2(mins, __builtin_bit_cast(short2v, xr[16]), 0, false);
            const float dx = __uint_as_float(xr[18]);
            acc[m] = fmaf(dw * dx, (float)isum, acc[m]);
            acc[m] = fmaf(-(dmw * dx), (float)msum, acc[m]);
        }
    }
};
// Q4_K / Q5_K: piece p (0..7) of a block is qs bytes 16p..16p+15, i.e. values
// 64c + 16h + [0,16) (low nibbles) and 64c + 32 + 16h + [0,16) (high) with c = p/2,
// h = p%2.  The eight lanes of a block each load one dword of its 16-byte header
// (dword p%4) and share the four through DPP quad broadcasts, instead of each
// holding the whole header.
template <int TYPE>
struct FastK45T {  // Q4_K and Q5_K, eight lanes per block
    static constexpr int PPB = 8, VALS = 256, XW = 10;
    static constexpr int BYTES = TYPE == TYPE_Q4_K ? 144 : 176;
    static constexpr int NBUF = 3;
    static constexpr int RAW = TYPE == TYPE_Q4_K ? 5 : 9;
    struct Raw { uint32_t hw; uint4 qh, qs; };
    __device__ static Raw load(const uint8_t *blk, int p) {
        Raw r;
        r.hw = *reinterpret_cast<const uint32_t *>(blk + 4 * (p & 3));
        if (TYPE == TYPE_Q5_K) r.qh = ld_u4(blk + 16 + 16 * (p & 1));
        r.qs = ld_u4(blk + (TYPE == TYPE_Q4_K ? 16 : 48) + 16 * p);
        return r;
    }
    // activation registers for piece p of a block, from the LDS layout
    __device__ static void xload_lds(const uint8_t *xb, int p, uint32_t *xr) {
        const int c = p >> 1, h = p & 1;
        const uint4 a = *reinterpret_cast<const uint4 *>(xb + 64 * c + 16 * h);
        const uint4 b = *reinterpret_cast<const uint4 *>(xb + 64 * c + 32 + 16 * h);
        const uint2 s = *reinterpret_cast<const uint2 *>(xb + 256 + 8 * c);
        xr[0] = a.x; xr[1] = a.y; xr[2] = a.z; xr[3] = a.w;
        xr[4] = b.x; xr[5] = b.y; xr[6] = b.z; xr[7] = b.w;
        xr[8] = pack_halves(s.x, s.y, h);
        xr[9] = *reinterpret_cast<const uint32_t *>(xb + 288);
    }
    template <int MR, class XL>
    __device__ static void dotm(const Raw &r, int p, XL xl, float *acc, bool valid) {
        const int c = p >> 1;
        // header dword i sits in lane i of every quad (quad_perm [i,i,i,i])
        const uint32_t h0 = qperm<0x00>(r.hw), s0 = qperm<0x55>(r.hw);
        const uint32_t s1 = qperm<0xAA>(r.hw), s2 = qperm<0xFF>(r.hw);
        uint32_t sc2, m2;
        k4_scale_pair(s0, s1, s2, c, &sc2, &m2);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t lo[4], hi[4];
        if (TYPE == TYPE_Q4_K) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = q[i] & 0x0f0f0f0fu;
                hi[i] = (q[i] >> 4) & 0x0f0f0f0fu;
            }
        } else {
            const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                lo[i] = (q[i] & 0x0f0f0f0fu) | (((qh[i] >> (2 * c)) & 0x01010101u) << 4);
                hi[i] = ((q[i] >> 4) & 0x0f0f0f0fu) | (((qh[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            }
        }
        const float dw = h2f(h0 & 0xffffu), dmw = h2f(h0 >> 16);
        const int scl = (int)(sc2 & 0xffu), sch = (int)(sc2 >> 8), ml = (int)(m2 & 0xffu), mh = (int)(m2 >> 8);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            uint32_t xr[XW];
            xl(m, xr);
            int sl = 0, sh = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                sl = dot4(lo[i], xr[i], sl);
                sh = dot4(hi[i], xr[4 + i], sh);
            }
            const int isum = __mul24(scl, sl) + __mul24(sch, sh);
            const int msum = __mul24(ml, (int)(int16_t)(xr[8] & 0xffffu)) + __mul24(mh, (int)(int16_t)(xr[8] >> 16));
            const float dx = __uint_as_float(xr[9]);
            const float v = (dw * dx) * (float)isum - (dmw * dx) * (float)msum;
            acc[m] += valid ? v : 0.f;
        }
    }
};
template <> struct Fast<TYPE_Q4_K, 4> : FastK45<TYPE_Q4_K> {};
template <> struct Fast<TYPE_Q5_K, 4> : FastK45<TYPE_Q5_K> {};
template <> struct Fast<TYPE_Q4_K, 8> : FastK45T<TYPE_Q4_K> {};
template <> struct Fast<TYPE_Q5_K, 8> : FastK45T<TYPE_Q5_K> {};

// Q6_K piece p = (n, h) covers runs 128n+16h+32j (j < 4) with int8 scales 8n+h+2j.
template <>
struct Fast<TYPE_Q6_K, 4> {
    static constexpr int PPB = 4, VALS = 256, XW = 19, BYTES = 210;
    static constexpr int NBUF = 2, RAW = 15;
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
    // xr: 16 code dwords (run j at 4j), bsums packed (j=0,1) and (j=2,3), d
    __device__ static void xload_lds(const uint8_t *xb, int p, uint32_t *xr) {
        const int n = p >> 1, h = p & 1;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint4 a = *reinterpret_cast<const uint4 *>(xb + 128 * n + 16 * h + 32 * j);
            xr[4 * j] = a.x; xr[4 * j + 1] = a.y; xr[4 * j + 2] = a.z; xr[4 * j + 3] = a.w;
        }
        const uint4 s = *reinterpret_cast<const uint4 *>(xb + 256 + 16 * n);
        xr[16] = pack_halves(s.x, s.y, h);
        xr[17] = pack_halves(s.z, s.w, h);
        xr[18] = *reinterpret_cast<const uint32_t *>(xb + 288);
    }
    template <int MR, class XL>
    __device__ static void dotm(const Raw &r, int p, XL xl, float *acc, bool valid) {
        const int h = p & 1;
        const int sh = 8 * h;
        const int sc[4] = {(int)(int8_t)(r.s0 >> sh), (int)(int8_t)(r.s0 >> (sh + 16)), (int)(int8_t)(r.s1 >> sh),
                           (int)(int8_t)(r.s1 >> (sh + 16))};
        uint32_t v[4][4];  // 6-bit codes (0..63) of run j, four per dword
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t *qs = (j & 1) ? r.qb : r.qa;
            const int shq = (j >> 1) * 4, shh = 2 * j;
#pragma unroll
            for (int i = 0; i < 4; i++) v[j][i] = ((qs[i] >> shq) & 0x0f0f0f0fu) | (((r.qh[i] >> shh) & 0x03030303u) << 4);
        }
        const float dw = h2f(r.dbits);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            uint32_t xr[XW];
            xl(m, xr);
            const int bs[4] = {(int)(int16_t)(xr[16] & 0xffffu), (int)(int16_t)(xr[16] >> 16),
                               (int)(int16_t)(xr[17] & 0xffffu), (int)(int16_t)(xr[17] >> 16)};
            int isum = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                int s = 0;
#pragma unroll
                for (int i = 0; i < 4; i++) s = dot4(v[j][i], xr[4 * j + i], s);
                isum += sc[j] * (s - 32 * bs[j]);
            }
            const float val = (dw * __uint_as_float(xr[18])) * (float)isum;
            acc[m] += valid ? val : 0.f;
        }
    }
};

// Q8_0: one 34-byte block (32 values) per piece.
template <>
struct Fast<TYPE_Q8_0, 1> {
    static constexpr int PPB = 1, VALS = 32, XW = 9, BYTES = 34;
    static constexpr int NBUF = 2, RAW = 10;
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
    __device__ static void xload_lds(const uint8_t *xb, int, uint32_t *xr) {
        const uint4 a = *reinterpret_cast<const uint4 *>(xb);
        const uint4 b = *reinterpret_cast<const uint4 *>(xb + 16);
        xr[0] = a.x; xr[1] = a.y; xr[2] = a.z; xr[3] = a.w;
        xr[4] = b.x; xr[5] = b.y; xr[6] = b.z; xr[7] = b.w;
        xr[8] = *reinterpret_cast<const uint32_t *>(xb + 32);
    }
    template <int MR, class XL>
    __device__ static void dotm(const Raw &r, int, XL xl, float *acc, bool valid) {
        const bool odd = r.mis != 0;
        const float d = h2f(odd ? (r.w[0] >> 16) : (r.w[0] & 0xffffu));
        uint32_t q[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q[i] = odd ? r.w[i + 1] : __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
#pragma unroll
        for (int m = 0; m < MR; m++) {
            uint32_t xr[XW];
            xl(m, xr);
            int s = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) s = dot4(q[i], xr[i], s);
            const float v = ((float)s * d) * __uint_as_float(xr[8]);
            acc[m] += valid ? v : 0.f;
        }
    }
};

// ---------------------------------------------------------------------------
// Fused activation quantisation into LDS by the whole workgroup (m = 1).
// ---------------------------------------------------------------------------
// `between` runs after the x loads are issued and before any of them is used:
// loads issued there (the weight ring) queue behind x, so the in-order memory
// counter lets the quantisation start as soon as x has arrived.
//
// NORM (k-quants, nbx <= 32): x is first RMS-normalised as candle's RmsNorm does
// in f32 -- x / sqrt(sum(x^2) / k + eps) * alpha -- with the sum of squares taken
// over the whole workgroup (every workgroup holds all of x).
// Workgroup barrier.  FENCE: __syncthreads (its release fence also waits for
// every load to LDS still in flight); otherwise this wave's LDS writes complete,
// then a plain s_barrier, so loads to LDS issued by `between` stay in flight.
template <bool FENCE>
__device__ __forceinline__ void wg_barrier() {
    if constexpr (FENCE) {
        __syncthreads();
    } else {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
        __builtin_amdgcn_s_barrier();
    }
}

template <int TYPE, bool NORM, int XJ, int WPG, int NBMAX = 64, class Between = void, bool FENCE = true>
__device__ __forceinline__ void quantise_x_lds(const float *__restrict__ x, int nbx, uint8_t *sx, Between between,
                                               const float *__restrict__ alpha, float eps) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr bool vec = true;  // the host only fuses for 16-byte aligned x
    if constexpr (TYPE != TYPE_Q8_0 && !NORM && 2 * WPG >= NBMAX) {
        // 32 lanes per 256-value block, 8 consecutive values each (q8k_lane8): one
        // pass covers the row (nbx <= NBMAX <= 2 WPG), every lane quantises values
        // of its own.  With 16 lanes per block an eight-wave workgroup would leave
        // half its waves quantising clamped duplicates on the SIMDs the other half
        // runs on (Q4_K 14336 x 4096: 8.2 -> 7.8 us per launch).  Same bytes as
        // q8k_lane16.
        const int t = threadIdx.x, sub = t & 31, b = min(t >> 5, nbx - 1);
        const float4 *src = reinterpret_cast<const float4 *>(x + (int64_t)b * QK_K + 8 * sub);
        const float4 f0 = src[0], f1 = src[1];
        const float v[8] = {f0.x, f0.y, f0.z, f0.w, f1.x, f1.y, f1.z, f1.w};
        __builtin_amdgcn_sched_barrier(0);
        between();
        __builtin_amdgcn_sched_barrier(0);
        uint32_t packed[2];
        int sum;
        float d;
        q8k_lane8(v, sub, packed, &sum, &d);
        if ((t >> 5) < nbx) {
            uint8_t *xb = sx + b * XS_K;
            *reinterpret_cast<uint2 *>(xb + 8 * sub) = make_uint2(packed[0], packed[1]);
            if (!(sub & 1)) *reinterpret_cast<int16_t *>(xb + 256 + sub) = (int16_t)sum;  // entry sub / 2
            if (sub == 0) *reinterpret_cast<float *>(xb + 288) = d;
        }
    } else if constexpr (TYPE != TYPE_Q8_0) {
        // 16 lanes per 256-value block, 16 consecutive values per lane
        // (q8k_lane16), so a workgroup of WPG waves quantises BPP = 4 WPG blocks
        // per pass (nbx <= NBMAX <= 64, 32 with the norm); a lane's 16 codes are
        // exactly one bsums entry.
        constexpr int BPP = 4 * WPG, NBM = NBMAX < (NORM ? 32 : 64) ? NBMAX : (NORM ? 32 : 64);
        constexpr int MAXP = (NBM + BPP - 1) / BPP;
        const int t = threadIdx.x, sub = t & 15;
        const int np = (nbx + BPP - 1) / BPP;  // workgroup-uniform
        float v[MAXP][16], al[NORM ? MAXP : 1][16];
#pragma unroll
        for (int j = 0; j < MAXP; j++) {
            const int b = min(BPP * j + (t >> 4), nbx - 1);
            const float4 *src = reinterpret_cast<const float4 *>(x + (int64_t)b * QK_K + 16 * sub);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float4 f = src[i];
                v[j][4 * i] = f.x; v[j][4 * i + 1] = f.y; v[j][4 * i + 2] = f.z; v[j][4 * i + 3] = f.w;
            }
            if constexpr (NORM) {
                const float4 *wsrc = reinterpret_cast<const float4 *>(alpha + (int64_t)b * QK_K + 16 * sub);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 f = wsrc[i];
                    al[j][4 * i] = f.x; al[j][4 * i + 1] = f.y; al[j][4 * i + 2] = f.z; al[j][4 * i + 3] = f.w;
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        between();
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (NORM) {
            __shared__ float red[WPG];
            float ss = 0.f;
#pragma unroll
            for (int j = 0; j < MAXP; j++) {
                if (j < np && BPP * j + (t >> 4) < nbx) {  // clamped duplicates do not count
#pragma unroll
                    for (int i = 0; i < 16; i++) ss += v[j][i] * v[j][i];
                }
            }
            ss = row_sum_f32(ss);
            ss = __int_as_float(rl(__float_as_uint(ss), 0)) + __int_as_float(rl(__float_as_uint(ss), 16)) +
                 __int_as_float(rl(__float_as_uint(ss), 32)) + __int_as_float(rl(__float_as_uint(ss), 48));
            if (lane == 0) red[wave] = ss;
            wg_barrier<FENCE>();
            float tot = red[0];
#pragma unroll
            for (int w = 1; w < WPG; w++) tot += red[w];
            const float rms = sqrtf(tot / (float)(nbx * QK_K) + eps);
#pragma unroll
            for (int j = 0; j < MAXP; j++)
#pragma unroll
                for (int i = 0; i < 16; i++) v[j][i] = v[j][i] / rms * al[j][i];
        }
#pragma unroll
        for (int j = 0; j < MAXP; j++) {
            if (j == 0 || j < np) {  // pass 0 unconditional: its loads stay ahead of the ring
                uint32_t packed[4];
                int sum;
                float d;
                q8k_lane16(v[j], sub, packed, &sum, &d);
                const int b = BPP * j + (t >> 4);
                if (b < nbx) {
                    uint8_t *xb = sx + b * XS_K;
                    *reinterpret_cast<uint4 *>(xb + 16 * sub) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
                    *reinterpret_cast<int16_t *>(xb + 256 + 2 * sub) = (int16_t)sum;
                    if (sub == 0) *reinterpret_cast<float *>(xb + 288) = d;
                }
            }
        }
    } else {
        // 2 lanes per 32-value block, 16 consecutive values each; thread t handles
        // blocks t/2 + 32 WPG j, j < XJ (XJ = ceil(blocks / (32 WPG)) for the kernel's
        // largest row: every load is issued, so no more than the row needs).  The
        // block maximum is order-free and each code depends on its value and the
        // block's scale only, so any lane split gives the same bytes.
        constexpr int MAXJ = XJ;
        static_assert(MAXJ >= 1 && MAXJ <= 4, "x passes");
        const int sub = threadIdx.x & 1, bt = threadIdx.x >> 1;
        float v[MAXJ][16];
#pragma unroll
        for (int j = 0; j < MAXJ; j++) {
            const int b = min(bt + 32 * WPG * j, nbx - 1);
#pragma unroll
            for (int i = 0; i < 4; i++) load4f(x + (int64_t)b * QK8_0 + sub * 16 + 4 * i, vec, &v[j][4 * i]);
        }
        __builtin_amdgcn_sched_barrier(0);
        between();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < MAXJ; j++) {
            if (32 * WPG * j < nbx) {  // uniform across the workgroup: the shuffle stays convergent
                float amax = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[j][i]));
                amax = fmaxf(amax, __shfl_xor(amax, 1));
                const float d = amax / 127.f;
                const float id = d != 0.f ? 1.f / d : 0.f;
                uint32_t packed[4] = {0u, 0u, 0u, 0u};
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float r = roundf(v[j][i] * id);
                    const int q = (r != r) ? 0 : (int)fminf(fmaxf(r, -128.f), 127.f);
                    packed[i >> 2] |= ((uint32_t)q & 0xffu) << (8 * (i & 3));
                }
                const int b = min(bt + 32 * WPG * j, nbx - 1);  // clamped duplicates rewrite equal data
                uint8_t *xb = sx + b * XS_0;
                *reinterpret_cast<uint4 *>(xb + sub * 16) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
                if (sub == 0) *reinterpret_cast<float *>(xb + 32) = __half2float(__float2half_rn(d));
            }
        }
    }
    wg_barrier<FENCE>();
}

// MR rows of f32 x (row stride nbx * 256) quantised to Q8_K into MR consecutive
// LDS row images, as quantise_x_lds does for one row (same code, same bytes).
// IT passes of 16 blocks per row (nbx <= 16 * IT); every (row, pass) load is
// issued before `between` (the weight ring), so none of them waits behind the
// weight stream (memory loads complete in order).  With rows < MR the rows past
// `rows` repeat the last real one (computed, never stored); rows == 0 means MR.
template <int TYPE, int MR, int IT, class Between>
__device__ __forceinline__ void quantise_rows_lds(const float *__restrict__ x, int rows, int nbx, uint8_t *sx,
                                                  Between between) {
    static_assert(TYPE != TYPE_Q8_0 && MR * IT <= 8, "Q8_K rows, at most 8 (row, pass) items");
    // (the host fuses at most four items; eight are compiled for the 8-row shape)
    constexpr int NI = MR * IT;
    const int t = threadIdx.x, sub = t & 15;
    const int64_t k = (int64_t)nbx * QK_K;
    float v[NI][16];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int m = i / IT, j = i % IT;
        const int src = rows > 0 ? min(m, rows - 1) : m;
        const int b = min(16 * j + (t >> 4), nbx - 1);
        const float4 *p = reinterpret_cast<const float4 *>(x + (int64_t)src * k + (int64_t)b * QK_K + 16 * sub);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = p[q];
            v[i][4 * q] = f.x; v[i][4 * q + 1] = f.y; v[i][4 * q + 2] = f.z; v[i][4 * q + 3] = f.w;
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    between();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int m = i / IT, j = i % IT;
        if (j == 0 || 16 * j < nbx) {  // workgroup-uniform: the DPP reductions stay convergent
            uint32_t packed[4];
            int sum;
            float d;
            q8k_lane16(v[i], sub, packed, &sum, &d);
            const int b = 16 * j + (t >> 4);
            if (b < nbx) {
                uint8_t *xb = sx + ((int64_t)m * nbx + b) * XS_K;
                *reinterpret_cast<uint4 *>(xb + 16 * sub) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
                *reinterpret_cast<int16_t *>(xb + 256 + 2 * sub) = (int16_t)sum;
                if (sub == 0) *reinterpret_cast<float *>(xb + 288) = d;
            }
        }
    }
    __syncthreads();
}

// Pre-quantised activations (split global layout) -> the LDS layout.  Straight-line
// code for nbx <= 64 (k <= 16384, the fast path's limit): every load is issued
// before any store, with indices clamped into range instead of branches;
// `between` as for quantise_x_lds.
template <int TYPE, class Between>
__device__ __forceinline__ void copy_x_row_lds(const ActView &a, int nbx, uint8_t *sx, Between between) {
    constexpr int XS = TYPE == TYPE_Q8_0 ? XS_0 : XS_K;
    constexpr int CPB = TYPE == TYPE_Q8_0 ? 2 : 16;  // 16-byte code chunks per block
    constexpr int NC = TYPE == TYPE_Q8_0 ? 4 : 4;    // code chunks per thread (<= 1024 total)
    const int t = (int)threadIdx.x;
    const int ncode = nbx * CPB;
    uint4 v[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) v[j] = *reinterpret_cast<const uint4 *>(a.xq + (int64_t)min(t + 256 * j, ncode - 1) * 16);
    uint4 bsv = make_uint4(0u, 0u, 0u, 0u);
    if constexpr (TYPE != TYPE_Q8_0) bsv = *reinterpret_cast<const uint4 *>(a.xbs + (int64_t)min(t, 2 * nbx - 1) * 8);
    // block scales: nbx <= 512, so two per thread cover every block
    const float d0 = a.xd[min(t, nbx - 1)];
    const float d1 = a.xd[min(t + 256, nbx - 1)];
    __builtin_amdgcn_sched_barrier(0);
    between();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NC; j++) {
        const int i = min(t + 256 * j, ncode - 1);  // clamped duplicates rewrite equal data
        *reinterpret_cast<uint4 *>(sx + (i / CPB) * XS + 16 * (i % CPB)) = make_uint4(v[j].x, v[j].y, v[j].z, v[j].w);
    }
    if constexpr (TYPE != TYPE_Q8_0) {
        const int i = min(t, 2 * nbx - 1);
        *reinterpret_cast<uint4 *>(sx + (i >> 1) * XS + 256 + 16 * (i & 1)) = bsv;
    }
    *reinterpret_cast<float *>(sx + min(t, nbx - 1) * XS + (TYPE == TYPE_Q8_0 ? 32 : 288)) = d0;
    *reinterpret_cast<float *>(sx + min(t + 256, nbx - 1) * XS + (TYPE == TYPE_Q8_0 ? 32 : 288)) = d1;
}

// MR pre-quantised activation rows -> MR consecutive LDS row images of nbx
// blocks each; `between` runs once, inside the first row's copy.  With
// a.rows < MR the rows past a.rows repeat the last real one (they are computed
// and never stored).
template <int TYPE, int MR, class Between>
__device__ __forceinline__ void copy_x_lds(const ActView &a, int nbx, uint8_t *sx, Between between) {
    constexpr int XS = TYPE == TYPE_Q8_0 ? XS_0 : XS_K;
    copy_x_row_lds<TYPE>(a, nbx, sx, between);
#pragma unroll 1
    for (int m = 1; m < MR; m++) {
        const int src = a.rows > 0 ? min(m, a.rows - 1) : m;
        ActView r = a;
        r.xq = a.xq + (int64_t)src * a.k;
        r.xd = a.xd + (int64_t)src * a.nb;
        if constexpr (TYPE != TYPE_Q8_0) r.xbs = a.xbs + (int64_t)src * (a.k / 16);
        copy_x_row_lds<TYPE>(r, nbx, sx + (int64_t)m * nbx * XS, [] {});
    }
    __syncthreads();
}

// A row map held in scalar registers (named fields, no arrays: nothing is
// indexed).  Each field passes through an empty asm statement, so lookups
// select between values; a select between the kernel argument's fields would
// otherwise become a load from a selected address, whose wait would also wait
// for every load issued before it.  Lookups take wave-uniform rows and run on
// the scalar unit.
static_assert(GROUP_MAX == 4, "RowMapS has four segments");
struct RowMapS {
    uint64_t w0, w1, w2, w3, y0, y1, y2, y3;
    int32_t e0, e1, e2;
};
__device__ __forceinline__ uint64_t sreg(uint64_t v) {
    asm volatile("" : "+s"(v));
    return v;
}
__device__ __forceinline__ int32_t sreg32(int32_t v) {
    asm volatile("" : "+s"(v));
    return v;
}
__device__ __forceinline__ RowMapS map_regs(const RowMap &rm) {
    RowMapS r;
    r.w0 = sreg(reinterpret_cast<uint64_t>(rm.w[0]));
    r.w1 = sreg(reinterpret_cast<uint64_t>(rm.w[1]));
    r.w2 = sreg(reinterpret_cast<uint64_t>(rm.w[2]));
    r.w3 = sreg(reinterpret_cast<uint64_t>(rm.w[3]));
    r.y0 = sreg(reinterpret_cast<uint64_t>(rm.y[0]));
    r.y1 = sreg(reinterpret_cast<uint64_t>(rm.y[1]));
    r.y2 = sreg(reinterpret_cast<uint64_t>(rm.y[2]));
    r.y3 = sreg(reinterpret_cast<uint64_t>(rm.y[3]));
    r.e0 = sreg32(rm.end[0]);
    r.e1 = sreg32(rm.end[1]);
    r.e2 = sreg32(rm.end[2]);
    return r;
}
// (segment base pointer, first row of the segment) for a row of the space
__device__ __forceinline__ void map_seg(const RowMapS &rm, int32_t row, uint64_t a0, uint64_t a1, uint64_t a2,
                                        uint64_t a3, uint64_t *ptr, int32_t *base) {
    uint64_t p = a0;
    int32_t b = 0;
    if (row >= rm.e0) { p = a1; b = rm.e0; }
    if (row >= rm.e1) { p = a2; b = rm.e1; }
    if (row >= rm.e2) { p = a3; b = rm.e2; }
    *ptr = p;
    *base = b;
}
// Global-address-space views of looked-up pointers, so accesses through them
// stay global loads and stores.
typedef const __attribute__((address_space(1))) uint8_t *gbytes;
typedef __attribute__((address_space(1))) float *gfloats;

// ---------------------------------------------------------------------------
// The m = 1 kernel.  A row group is RPW rows; lane (r, li) decodes piece
// li % PPB of blocks li / PPB + BPI*i (i < IT) of row r.  Requires nb <= BPI*IT.
// ---------------------------------------------------------------------------
// Row maps: MAP_ONE is one weight, addressed directly; MAP_SEGMENTS holds
// several weights (rows looked up per group); MAP_SILU_PAIRS interleaves the
// rows of a gate (w[0]) and an up (w[1]) weight -- row 2i is gate row i, 2i + 1
// up row i -- and writes silu(gate_i) * up_i to y[0][i]: the gate/up half of
// an MLP in one launch, with no gate/up round trip.
enum : int { MAP_ONE = 0, MAP_SEGMENTS = 1, MAP_SILU_PAIRS = 2 };

// candle's silu for f32: v / (1 + exp(-v))
__device__ __forceinline__ float silu_f32(float v) { return v / (1.f + expf(-v)); }

// Pairwise lane-half sums for reducing several accumulators at once.
// swap32_sum(a, b): lanes 0..31 get a[l] + a[l + 32], lanes 32..63 get b[l - 32] + b[l]
// (v_permlane32_swap exchanges a's upper half with b's lower half).
__device__ __forceinline__ float swap32_sum(float a, float b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// swap16_sum(a, b): 16-lane rows 0, 1, 2, 3 get a.row0 + a.row1, b.row0 + b.row1,
// a.row2 + a.row3, b.row2 + b.row3 (v_permlane16_swap exchanges a's odd rows with
// b's even rows)
__device__ __forceinline__ float swap16_sum(float a, float b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int TYPE, int PPB, int RPW, int IT, int MR, bool FUSED, int MAP, bool NORM = false, int WPG = 4, int RING = 0,
          int RMAX = 0>
__global__ __launch_bounds__(64 * WPG) void k_gemv1(RowMap rm, int64_t row_bytes, int nb, const float *__restrict__ x,
                                                    ActView act, const float *__restrict__ alpha, float eps) {
    static_assert(WPG == 4 || (FUSED && WPG == 8), "waves per workgroup: 4, or 8 for the fused prologue");
    static_assert(!NORM || (FUSED && TYPE != TYPE_Q8_0), "the RMS norm runs in the quantising prologue");
    static_assert(MR == 1 || (MAP == MAP_ONE && !NORM && WPG == 4 && (!FUSED || TYPE != TYPE_Q8_0)),
                  "several activation rows: one weight; quantised in the prologue for Q8_K rows only");
    constexpr bool GROUPED = MAP == MAP_SEGMENTS, PAIRED = MAP == MAP_SILU_PAIRS;
    static_assert(!PAIRED || RPW <= 2, "a silu pair spans two row groups or one");
    static_assert(RMAX == 0 || (MAP == MAP_ONE && MR == 1 && RING >= 2), "static schedule: one weight, one row, a given ring");
    const int64_t n = rm.n;
    const uint8_t *__restrict__ W = rm.w[0];
    float *__restrict__ y = rm.y[0];
    RowMapS rs{};
    if constexpr (MAP != MAP_ONE) rs = map_regs(rm);
    // silu pairs: up row i is (w1 - w0) past gate row i (arithmetic, not a select
    // between fields, which the compiler would turn into an indexed copy)
    const uint64_t wdiff = rs.w1 - rs.w0;
    using F = Fast<TYPE, PPB>;
    using Raw = typename F::Raw;
    constexpr int LPR = 64 / RPW;
    constexpr int BPI = LPR / F::PPB;
    static_assert(BPI >= 1, "a row needs at least one whole block per sweep");
    // the wave index as a scalar, so row-group indices, row addresses and row-map
    // lookups run on the scalar unit
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane / LPR, li = lane % LPR;
    const int p = li % F::PPB, bs0 = li / F::PPB;
    // silu pairs are never split between waves: ranges are counted in pairs
    constexpr int GPU_ = PAIRED ? 2 / RPW : 1;  // row groups per unit
    const int64_t ng = PAIRED ? n / 2 : (n + RPW - 1) / RPW;
    const int64_t gw = (int64_t)blockIdx.x * WPG + wave, nw = (int64_t)gridDim.x * WPG;
    const int64_t per = ng / nw, rem = ng % nw;
    const int64_t g0 = (gw * per + (gw < rem ? gw : rem)) * GPU_, g1 = g0 + (per + (gw < rem ? 1 : 0)) * GPU_;

    // loads are unconditional (row and block clamped into range); compute masks.
    // Grouped: the group's rows are looked up once each (g is wave-uniform),
    // and each lane takes its own row's base.
    auto load_group = [&](int64_t g, Raw *buf) {
        const uint8_t *wr;
        if constexpr (GROUPED) {
            uint64_t rp = 0;
            int64_t roff = 0;
#pragma unroll
            for (int q = 0; q < RPW; q++) {
                const int32_t row = (int32_t)min(g * RPW + q, n - 1);
                uint64_t sp;
                int32_t sb;
                map_seg(rs, row, rs.w0, rs.w1, rs.w2, rs.w3, &sp, &sb);
                if (q == 0 || r == q) {
                    rp = sp;
                    roff = (int64_t)(row - sb) * row_bytes;
                }
            }
            wr = (const uint8_t *)((gbytes)rp + roff);
        } else if constexpr (PAIRED) {
            uint64_t rp = 0;
            int64_t roff = 0;
#pragma unroll
            for (int q = 0; q < RPW; q++) {
                const int64_t v = min(g * RPW + q, n - 1);
                if (q == 0 || r == q) {
                    rp = rs.w0 + (uint64_t)(v & 1) * wdiff;
                    roff = (v >> 1) * row_bytes;
                }
            }
            wr = (const uint8_t *)((gbytes)rp + roff);
        } else {
            wr = W + min(g * RPW + r, n - 1) * row_bytes;
        }
        // blocks of sweeps before the last are in range (the host launches the
        // smallest IT with nb <= BPI * IT); only the last sweep's block is clamped
        const uint8_t *lb = wr + bs0 * F::BYTES;
#pragma unroll
        for (int i = 0; i < IT - 1; i++) buf[i] = F::load(lb + i * BPI * F::BYTES, p);
        buf[IT - 1] = F::load(wr + (int64_t)min(bs0 + BPI * (IT - 1), nb - 1) * F::BYTES, p);
    };

    // group indices are clamped into the wave's range (a wave without groups
    // touches row group 0), so every load is unconditional
    const int64_t glast = g0 < g1 ? g1 - 1 : 0;
    auto gc = [&](int64_t g) { return g < glast ? g : glast; };
    // Ring of NBUF row-group buffers: NBUF - 1 groups are in flight while one is
    // computed, and the first NBUF - 1 are issued inside the x prologue, right
    // after its x loads, so the weight stream overlaps the prologue without the
    // prologue waiting for it.  Loads are clamped, not skipped (no branches
    // around loads).  Three buffers measured best: deeper rings, and issuing a
    // wave's whole stream up front, leave every wave waiting for its first rows
    // while the whole matrix is in flight, and bunch the compute at the end.
    // Deep rows (IT > 4) keep two buffers (registers).
    // Static schedule (RMAX > 0: the host guarantees at most RMAX groups per wave):
    // the group loop is unrolled at compile time, so no load past the wave's last
    // group is ever issued -- the dynamic loop below issues clamped duplicates of
    // the last group for every slot past it (up to three per wave), which cost
    // issue slots and L2 bandwidth -- and the ring depth is the host's: the first
    // RING - 1 groups ahead of the x prologue, one more after each computed group.
    // Q4_K Llama-3-8B layer step (per launch): q/o 4.5 -> 4.1, k/v 3.1 -> 2.8,
    // gate/up 7.8 -> 7.5 us (with the 32-lane quantiser).
    constexpr int NBUF3 = RING > 0 ? RING : (F::NBUF == 3 && IT <= (MR > 1 ? 2 : 4)) ? 3 : 2;
    // several activation rows: a two-deep ring where that keeps their activation
    // images in registers (below) and the three-deep one would not
    constexpr bool XFIT3 = MR * IT * F::XW <= 160 && NBUF3 * IT * F::RAW + MR * IT * F::XW <= 190;
    constexpr bool XFIT2 = MR * IT * F::XW <= 160 && 2 * IT * F::RAW + MR * IT * F::XW <= 190;
    constexpr int NBUF = (RING == 0 && MR > 1 && !XFIT3 && XFIT2) ? 2 : NBUF3;
    Raw ring[NBUF][IT];
    constexpr int PRE = (RMAX > 0 && RMAX < NBUF - 1) ? RMAX : NBUF - 1;  // groups issued before the prologue
    auto issue_ring = [&] {
#pragma unroll
        for (int k = 0; k < PRE; k++) load_group(gc(g0 + k), ring[k]);
    };

    extern __shared__ __align__(16) uint8_t sx[];
    constexpr int XS = TYPE == TYPE_Q8_0 ? XS_0 : XS_K;
    // Q8_0: at most 64 IT activation blocks (the sweeps cover the row), 32 WPG per pass
    constexpr int XJ = (64 * IT + 32 * WPG - 1) / (32 * WPG);
    if constexpr (FUSED && MR > 1) quantise_rows_lds<TYPE, MR, IT>(x, act.rows, nb, sx, issue_ring);
    else if constexpr (FUSED) quantise_x_lds<TYPE, NORM, (XJ < 4 ? XJ : 4), WPG, BPI * IT>(x, nb, sx, issue_ring, alpha, eps);
    else copy_x_lds<TYPE, MR>(act, nb, sx, issue_ring);

    // A lane decodes the same piece slots in every row, so when they fit its
    // activation registers are read from LDS once and kept for the whole row loop.
    constexpr bool XREG = MR * IT * F::XW <= (MR == 1 ? 80 : 160) && NBUF * IT * F::RAW + MR * IT * F::XW <= 190;
    uint32_t xk[XREG ? MR : 1][XREG ? IT : 1][F::XW];
    if constexpr (XREG) {
#pragma unroll
        for (int m = 0; m < MR; m++)
#pragma unroll
            for (int i = 0; i < IT; i++) F::xload_lds(sx + (m * nb + min(bs0 + BPI * i, nb - 1)) * XS, p, xk[m][i]);
    }

    float pend = 0.f;  // silu pairs: the gate sum waiting for its up sum (wave-uniform)
    const int nrows = act.rows > 0 ? act.rows : MR;  // several rows: the ones stored
    auto compute_group = [&](int64_t g, const Raw *buf, bool store) {
        float accm[MR];
#pragma unroll
        for (int m = 0; m < MR; m++) accm[m] = 0.f;
#pragma unroll
        for (int i = 0; i < IT; i++) {
            const int b = bs0 + BPI * i;
            auto xl = [&](int m, uint32_t *xr) {
                if constexpr (XREG) {
#pragma unroll
                    for (int w = 0; w < F::XW; w++) xr[w] = xk[m][i][w];
                } else {
                    // The LDS image does not change inside the row loop, so without this
                    // barrier the compiler hoists every row's and sweep's reads out of it
                    // and holds them all in registers (spilling): read them where used.
                    if constexpr (MR > 1) asm volatile("" ::: "memory");
                    F::xload_lds(sx + (m * nb + min(b, nb - 1)) * XS, p, xr);
                }
            };
            F::template dotm<MR>(buf[i], p, xl, accm, b < nb);
            // several rows: one piece's unpacked codes live at a time
            if constexpr (MR > 1) __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (MR > 1 && LPR == 64 && (MR == 2 || MR == 4 || MR == 8)) {
            // one weight row per wave, 2 / 4 / 8 activation rows: the MR 64-lane sums
            // by halving exchanges (lane halves, then 16-lane rows), so each 16-lane
            // row ends with two (MR = 8) or one of the sums to finish with the row
            // butterfly -- 20 VALU for eight rows instead of 88
            const int rowi = lane >> 4;
            float s0, s1 = 0.f;
            int m0, m1 = -1;
            if constexpr (MR == 8) {
                const float a0 = swap32_sum(accm[0], accm[4]), a1 = swap32_sum(accm[1], accm[5]);
                const float a2 = swap32_sum(accm[2], accm[6]), a3 = swap32_sum(accm[3], accm[7]);
                s0 = row_sum_f32(swap16_sum(a0, a2));  // rows: activation rows 0, 2, 4, 6
                s1 = row_sum_f32(swap16_sum(a1, a3));  // 1, 3, 5, 7
                m0 = 2 * rowi;
                m1 = 2 * rowi + 1;
            } else if constexpr (MR == 4) {
                const float a0 = swap32_sum(accm[0], accm[2]), a1 = swap32_sum(accm[1], accm[3]);
                s0 = row_sum_f32(swap16_sum(a0, a1));  // rows: activation rows 0, 1, 2, 3
                m0 = rowi;
            } else {
                const float a0 = swap32_sum(accm[0], accm[1]);
                s0 = row_sum_f32(swap16_sum(a0, a0));  // rows: 0, 0, 1, 1
                m0 = (rowi & 1) ? -1 : rowi >> 1;
            }
            const int64_t rq = g;  // RPW = 1
            if (store && (lane & 15) == 0 && rq < n) {
                if (m0 >= 0 && m0 < nrows) y[(int64_t)m0 * n + rq] = s0;
                if (m1 >= 0 && m1 < nrows) y[(int64_t)m1 * n + rq] = s1;
            }
            return;
        } else if constexpr (MR > 1) {
            // several activation rows (one weight, MAP_ONE): row q of the group,
            // activation row m goes to y[m][row]
#pragma unroll
            for (int m = 0; m < MR; m++) {
                const float a = row_sum_f32(accm[m]);
#pragma unroll
                for (int q = 0; q < RPW; q++) {
                    float s;
                    if constexpr (LPR == 64) {
                        s = __int_as_float(rl(__float_as_uint(a), 0)) + __int_as_float(rl(__float_as_uint(a), 16)) +
                            __int_as_float(rl(__float_as_uint(a), 32)) + __int_as_float(rl(__float_as_uint(a), 48));
                    } else if constexpr (LPR == 32) {
                        s = __int_as_float(rl(__float_as_uint(a), 32 * q)) +
                            __int_as_float(rl(__float_as_uint(a), 32 * q + 16));
                    } else {
                        s = __int_as_float(rl(__float_as_uint(a), 16 * q));
                    }
                    const int64_t rq = g * RPW + q;
                    if (store && lane == LPR * q && rq < n && m < nrows) y[(int64_t)m * n + rq] = s;
                }
            }
            return;
        }
        float acc = accm[0];
        acc = row_sum_f32(acc);
        // row group q of this wave spans 16-lane rows LPR/16*q .. ; lane LPR*q writes it
#pragma unroll
        for (int q = 0; q < RPW; q++) {
            float s;
            if constexpr (LPR == 64) {
                s = __int_as_float(rl(__float_as_uint(acc), 0)) + __int_as_float(rl(__float_as_uint(acc), 16)) +
                    __int_as_float(rl(__float_as_uint(acc), 32)) + __int_as_float(rl(__float_as_uint(acc), 48));
            } else if constexpr (LPR == 32) {
                s = __int_as_float(rl(__float_as_uint(acc), 32 * q)) + __int_as_float(rl(__float_as_uint(acc), 32 * q + 16));
            } else {
                s = __int_as_float(rl(__float_as_uint(acc), 16 * q));
            }
            const int64_t rq = g * RPW + q;
            if constexpr (PAIRED) {
                if ((rq & 1) == 0) {
                    pend = s;
                } else if (store && lane == LPR * q && rq < n) {
                    y[rq >> 1] = silu_f32(pend) * s;
                }
            } else if constexpr (GROUPED) {
                uint64_t yp;
                int32_t yb;
                map_seg(rs, (int32_t)min(rq, n - 1), rs.y0, rs.y1, rs.y2, rs.y3, &yp, &yb);
                if (store && lane == LPR * q && rq < n) *(float *)((gfloats)yp + (rq - yb)) = s;
            } else {
                if (store && lane == LPR * q && rq < n) y[rq] = s;
            }
        }
    };

    if constexpr (RMAX > 0) {
        // group i of the wave (i < RMAX); the load for group i + NBUF - 1 goes out
        // before group i is computed, if the wave can have that group at all
#pragma unroll
        for (int i = 0; i < RMAX; i++) {
            if (i + NBUF - 1 < RMAX && i + NBUF - 1 >= PRE) load_group(gc(g0 + i + NBUF - 1), ring[(i + NBUF - 1) % NBUF]);
            __builtin_amdgcn_sched_barrier(0);
            if (i == 0 || g0 + i < g1) compute_group(g0 + i, ring[i % NBUF], g0 + i < g1);  // wave-uniform
            __builtin_amdgcn_sched_barrier(0);
        }
        return;
    }
    // The first pass runs even for a wave without groups (it stores nothing):
    // the ring's first loads then have an unconditional use and stay where they
    // are issued, ahead of the prologue, instead of being sunk into the loop.
    for (int64_t g = g0;; g += NBUF) {
#pragma unroll
        for (int k = 0; k < NBUF; k++) {
            load_group(gc(g + k + NBUF - 1), ring[(k + NBUF - 1) % NBUF]);
            __builtin_amdgcn_sched_barrier(0);
            if (k == 0 || g + k < g1) compute_group(g + k, ring[k], g + k < g1);  // wave-uniform
            __builtin_amdgcn_sched_barrier(0);
        }
        if (g + NBUF >= g1) break;
    }
}

}  // namespace lbq
