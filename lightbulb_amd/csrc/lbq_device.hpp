// lbq_device.hpp -- device-side building blocks for the gfx950 quantized-linear kernels.
//
// GGUF block layouts (byte offsets inside one block, little endian), as fixed by
// the ggml block specification that candle-core 0.10.2 and ggml-quants 0.1.0
// implement (type sizes: /root/reference/src/quantization/mod.rs:108-126):
//   Q8_0  34 B / 32 values : f16 d @0, i8 qs[32] @2
//   Q4_K 144 B / 256 values: f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qs[128] @16
//   Q5_K 176 B / 256 values: f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qh[32] @16, u8 qs[128] @48
//   Q6_K 210 B / 256 values: u8 ql[128] @0, u8 qh[64] @128, i8 scales[16] @192, f16 d @208
//   Q8_K 292 B / 256 values: f32 d @0, i8 qs[256] @4, i16 bsums[16] @260
// Q4_K/Q5_K blocks are 16-byte multiples; Q6_K and Q8_0 blocks are only 2-byte
// aligned, so their fields are read as aligned dwords and funnel-shifted
// (v_alignbyte_b32) -- never as misaligned vector loads.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <type_traits>
#include <stdint.h>

namespace lbq {

// ---------------------------------------------------------------------------
// DPP helpers (gfx9 dpp_ctrl: quad_perm 0x00-0xFF, row_ror:n = 0x120+n)
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
// quad_perm broadcast with every lane active (no old value to preserve)
template <int CTRL>
__device__ __forceinline__ uint32_t qperm(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
// every lane of each 16-lane row gets the row's max / min / sum
__device__ __forceinline__ uint32_t row_max_u32(uint32_t v) {
    v = max(v, dpp_u32<0xB1>(v));   // quad_perm [1,0,3,2]
    v = max(v, dpp_u32<0x4E>(v));   // quad_perm [2,3,0,1]
    v = max(v, dpp_u32<0x124>(v));  // row_ror:4
    v = max(v, dpp_u32<0x128>(v));  // row_ror:8
    return v;
}
__device__ __forceinline__ uint32_t row_min_u32(uint32_t v) {
    v = min(v, dpp_u32<0xB1>(v));
    v = min(v, dpp_u32<0x4E>(v));
    v = min(v, dpp_u32<0x124>(v));
    v = min(v, dpp_u32<0x128>(v));
    return v;
}
__device__ __forceinline__ float row_sum_f32(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x124>(v);
    v += dpp_f32<0x128>(v);
    return v;
}
__device__ __forceinline__ int quad_sum_i32(int v) {
    v += (int)dpp_u32<0xB1>((uint32_t)v);
    v += (int)dpp_u32<0x4E>((uint32_t)v);
    return v;
}
__device__ __forceinline__ uint32_t rl(uint32_t v, int lane) { return (uint32_t)__builtin_amdgcn_readlane((int)v, lane); }

// Q8_K quantisation of one 256-value block by 16 aligned lanes, 16 consecutive
// values per lane (lane sub = lane % 16 holds values 16 sub .. 16 sub + 15).
// Candle's BlockQ8K::from_float: the first value of largest |x| (NaN never
// chosen) sets iscale = -128/max; q = min(127, round(iscale*x)); d = 1/iscale;
// an all-zero block gives d = 0 and zero codes.  Out: the lane's 16 codes packed
// little-endian, their sum (one bsums entry) and the block's d.
__device__ __forceinline__ void q8k_lane16(const float *v, int sub, uint32_t packed[4], int *sum_out, float *d_out) {
    // the lane's largest |x| and the sign of the first value holding it (the
    // reference scans in ascending order with a strict >, so ties keep the lower
    // index and a NaN, comparing false, is never chosen): the signed maximum and
    // minimum (maximumNumber / minimumNumber: any NaN, signalling included, is
    // passed over), then, only where both +am and -am occur, the first of them
    float mxp = v[0], mnn = v[0];
#pragma unroll
    for (int i = 1; i < 16; i++) {
        mxp = __builtin_fmaximum_numf(mxp, v[i]);
        mnn = __builtin_fminimum_numf(mnn, v[i]);
    }
    const float am = __builtin_fmaximum_numf(__builtin_fmaximum_numf(mxp, -mnn), 0.f);  // 0 if every value is NaN
    uint32_t neg = -mnn == am ? 1u : 0u;
    if (mxp == am && neg && am > 0.f) {  // +am and -am both present: the first one decides
#pragma unroll
        for (int i = 15; i >= 0; i--)
            if (fabsf(v[i]) == am) neg = __float_as_uint(v[i]) >> 31;
    }
    const uint32_t amb = __float_as_uint(am) & 0x7fffffffu;  // +0 for a zero lane
    const uint32_t bmax = row_max_u32(amb);  // non-negative: bits order as values
    uint32_t key = amb == bmax ? ((uint32_t)sub << 1) | neg : 0xffffffffu;
    key = row_min_u32(key);  // the first lane holding the block max, and that value's sign
    packed[0] = packed[1] = packed[2] = packed[3] = 0u;
    int sum = 0;
    float d = 0.f;
    if (bmax != 0u) {  // uniform within the 16-lane block
        const float mx = (key & 1u) ? -__uint_as_float(bmax) : __uint_as_float(bmax);
        const float iscale = -128.f / mx;
        // min(roundf(iscale * x), 127) as i8: for |t| <= 2^23, adding 0.5 - 2^-25
        // with t's sign and truncating rounds exactly the halves (and everything
        // above them) away from zero -- checked for every such float; fminf sends
        // NaN to 127 as the reference's min does.  Separate roundings: no fma
        // contraction.  With a finite iscale |iscale * x| <= 128 (1 + 2^-23), so no
        // code falls below -128; only a subnormal block maximum (iscale infinite)
        // needs the saturation of Rust's `as i8` (uniform within the block).
        auto codes = [&](auto lower) {
            int q[16];
#pragma unroll
            for (int i = 0; i < 16; i++) {
#pragma clang fp contract(off)
                const float tt = iscale * v[i];
                const float r = fminf(tt + copysignf(0x1.fffffep-2f, tt), 127.f);
                q[i] = decltype(lower)::value ? max(-128, (int)r) : (int)r;
            }
#pragma unroll
            for (int w = 0; w < 4; w++) {
                const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q[4 * w + 1], (uint32_t)q[4 * w], 0x0c0c0400u);
                const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q[4 * w + 3], (uint32_t)q[4 * w + 2], 0x0c0c0400u);
                packed[w] = lo | (hi << 16);
            }
        };
        if (fabsf(iscale) <= 3.4028235e38f) codes(std::false_type{});
        else codes(std::true_type{});
        // the bsums entry: the 16 codes summed four at a time (sdot4 with ones)
#pragma unroll
        for (int w = 0; w < 4; w++) sum = __builtin_amdgcn_sdot4((int)packed[w], 0x01010101, sum, false);
        d = 1.f / iscale;
    }
    *sum_out = sum;
    *d_out = d;
}

// max / min of each 32-lane half's two 16-lane rows (v_permlane16_swap exchanges
// a's odd rows with the even rows of its second operand: with both a, the two
// results hold each row and its partner row)
__device__ __forceinline__ uint32_t row_pair_max_u32(uint32_t a) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, a, false, false);
    return max((uint32_t)r[0], (uint32_t)r[1]);
}
__device__ __forceinline__ uint32_t row_pair_min_u32(uint32_t a) {
    const auto r = __builtin_amdgcn_permlane16_swap(a, a, false, false);
    return min((uint32_t)r[0], (uint32_t)r[1]);
}

// Q8_K quantisation of one 256-value block by 32 aligned lanes, 8 consecutive
// values per lane (lane sub = lane % 32 holds values 8 sub .. 8 sub + 7): the
// selection and arithmetic of q8k_lane16, so the same codes and d.  Out: the
// lane's 8 codes packed little-endian, the bsums entry sub / 2 (the codes of
// lanes sub and sub ^ 1; both lanes hold it) and the block's d.
__device__ __forceinline__ void q8k_lane8(const float *v, int sub, uint32_t packed[2], int *sum_out, float *d_out) {
    float mxp = v[0], mnn = v[0];
#pragma unroll
    for (int i = 1; i < 8; i++) {
        mxp = __builtin_fmaximum_numf(mxp, v[i]);
        mnn = __builtin_fminimum_numf(mnn, v[i]);
    }
    const float am = __builtin_fmaximum_numf(__builtin_fmaximum_numf(mxp, -mnn), 0.f);  // 0 if every value is NaN
    uint32_t neg = -mnn == am ? 1u : 0u;
    if (mxp == am && neg && am > 0.f) {  // +am and -am both present: the first one decides
#pragma unroll
        for (int i = 7; i >= 0; i--)
            if (fabsf(v[i]) == am) neg = __float_as_uint(v[i]) >> 31;
    }
    const uint32_t amb = __float_as_uint(am) & 0x7fffffffu;
    const uint32_t bmax = row_pair_max_u32(row_max_u32(amb));
    uint32_t key = amb == bmax ? ((uint32_t)sub << 1) | neg : 0xffffffffu;
    key = row_pair_min_u32(row_min_u32(key));  // the first lane holding the block max, and its sign
    packed[0] = packed[1] = 0u;
    int sum = 0;
    float d = 0.f;
    if (bmax != 0u) {  // uniform within the 32-lane block
        const float mx = (key & 1u) ? -__uint_as_float(bmax) : __uint_as_float(bmax);
        const float iscale = -128.f / mx;
        // codes exactly as q8k_lane16 forms them
        auto codes = [&](auto lower) {
            int q[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
#pragma clang fp contract(off)
                const float tt = iscale * v[i];
                const float r = fminf(tt + copysignf(0x1.fffffep-2f, tt), 127.f);
                q[i] = decltype(lower)::value ? max(-128, (int)r) : (int)r;
            }
#pragma unroll
            for (int w = 0; w < 2; w++) {
                const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q[4 * w + 1], (uint32_t)q[4 * w], 0x0c0c0400u);
                const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q[4 * w + 3], (uint32_t)q[4 * w + 2], 0x0c0c0400u);
                packed[w] = lo | (hi << 16);
            }
        };
        if (fabsf(iscale) <= 3.4028235e38f) codes(std::false_type{});
        else codes(std::true_type{});
        sum = __builtin_amdgcn_sdot4((int)packed[0], 0x01010101, 0, false);
        sum = __builtin_amdgcn_sdot4((int)packed[1], 0x01010101, sum, false);
        d = 1.f / iscale;
    }
    sum += (int)dpp_u32<0xB1>((uint32_t)sum);  // + lane sub ^ 1 (quad_perm [1,0,3,2])
    *sum_out = sum;
    *d_out = d;
}

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;

// Internal (split) layout of a quantised activation matrix [m][k]:
//   xq  int8  [m][k]          the Q8_K / Q8_0 integer codes
//   xd  f32   [m][k/QK]       the block scale (Q8_0: the f32 value of the stored f16)
//   xbs int16 [m][k/16]       Q8_K only: sums of 16 consecutive codes
struct ActView {
    const int8_t *xq;
    const float *xd;
    const int16_t *xbs;
    int64_t k;  // row length in values
    int nb;     // scale blocks per row (k/256 or k/32)
    const float *xs = nullptr;  // Q8_1: per-block s = d * sum(codes), widened from f16
    int rows = 0;               // multi-row GEMV: real rows of the MR it runs (0: all MR)
};

struct __attribute__((aligned(4))) u32x4a4 { uint32_t x, y, z, w; };

__device__ __forceinline__ float h2f(uint32_t bits16) { return __half2float(__ushort_as_half((unsigned short)bits16)); }
// a 16-bit dense weight (bits16 < 2^16) widened exactly to f32: IEEE half, or with
// BF a bfloat16, whose bits are the upper half of the f32 it stands for
template <bool BF>
__device__ __forceinline__ float w16(uint32_t bits16) {
    if constexpr (BF) return __uint_as_float(bits16 << 16);
    else return h2f(bits16);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

__device__ __forceinline__ uint4 ld_u4(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

// Weight blocks live in global memory.  Aligned dwords around a 2-byte aligned
// field are addressed through an explicit global pointer built from the integer
// address: a generic pointer rebuilt from an integer would make flat loads, and
// rounding the pointer itself (__builtin_align_down) lets the compiler assume the
// field is 4-byte aligned and merge neighbouring byte loads into the wrong dword.
typedef const __attribute__((address_space(1))) uint8_t *gbytes_c;
__device__ __forceinline__ gbytes_c align4_global(uintptr_t a) { return (gbytes_c)(a & ~(uintptr_t)3); }
typedef uint32_t u32x4v4 __attribute__((ext_vector_type(4), aligned(4)));  // 16 bytes, 4-byte aligned
__device__ __forceinline__ u32x4a4 gld16(gbytes_c p) {
    const u32x4v4 v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4v4 *>(p);
    return u32x4a4{v.x, v.y, v.z, v.w};
}
__device__ __forceinline__ uint32_t gld4(gbytes_c p) {
    return *reinterpret_cast<const __attribute__((address_space(1))) uint32_t *>(p);
}

// 16 / 4 bytes at a 2-byte aligned address as single unaligned global loads
// (dwordx4 / dword at the field's own address: the hardware's unaligned access
// mode, which the compiler itself relies on for under-aligned types on this
// target); they read exactly the field's bytes.
typedef uint32_t u32x4v2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32a2 __attribute__((aligned(2)));
__device__ __forceinline__ void ld16_u2(const uint8_t *p, uint32_t out[4]) {
    const u32x4v2 v = *reinterpret_cast<const __attribute__((address_space(1))) u32x4v2 *>(reinterpret_cast<uintptr_t>(p));
    out[0] = v.x; out[1] = v.y; out[2] = v.z; out[3] = v.w;
}
__device__ __forceinline__ uint32_t ld4_u2(const uint8_t *p) {
    return *reinterpret_cast<const __attribute__((address_space(1))) u32a2 *>(reinterpret_cast<uintptr_t>(p));
}

// 2 bytes (f16 bits) at a 2-byte aligned address.
__device__ __forceinline__ uint32_t ld2_a2(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t w = gld4(align4_global(a));
    return (a & 2u) ? (w >> 16) : (w & 0xffffu);
}

// Q4_K / Q5_K 6-bit scale+min pair for sub-blocks j = 2c and 2c+1 (c = 0..3),
// from the 12 scale bytes held in dwords s0 (bytes 0..3), s1 (4..7), s2 (8..11).
// ggml get_scale_min_k4: j<4: sc = s[j]&63, m = s[j+4]&63;
// j>=4: sc = (s[j+4]&15) | (s[j-4]>>6)<<4, m = (s[j+4]>>4) | (s[j]>>6)<<4.
// Returns sc(2c) | sc(2c+1)<<8 in *sc2 and the mins likewise in *m2.
__device__ __forceinline__ void k4_scale_pair(uint32_t s0, uint32_t s1, uint32_t s2, int c, uint32_t *sc2,
                                              uint32_t *m2) {
    const uint32_t sh = (uint32_t)(c & 1) * 16u;
    const uint32_t A = (s0 >> sh) & 0xffffu, B = (s1 >> sh) & 0xffffu, C = (s2 >> sh) & 0xffffu;
    if (c < 2) {
        *sc2 = A & 0x3f3fu;
        *m2 = B & 0x3f3fu;
    } else {
        *sc2 = (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
        *m2 = ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u);
    }
}

// ---------------------------------------------------------------------------
// Activation quantisation, shared by the standalone kernels and the GEMV prologue.
// ---------------------------------------------------------------------------

// Q8_K (candle BlockQ8K::from_float) of one 256-value block by one 64-lane wave;
// the lane holds values 4*lane .. 4*lane+3 in v.  The signed value of largest |x|
// (first on ties, NaN never chosen) gives iscale = -128/max; q = min(127, round(iscale*x));
// d = 1/iscale; amax == 0 gives d = 0 and all-zero codes.  Returns the 4 codes packed
// little-endian; *sum4 gets the sum of 16 codes on every lane of each aligned lane quad.
__device__ __forceinline__ uint32_t q8k_block_wave(const float v[4], int lane, int *sum16, float *d_out) {
    float bk = -1.f, bv = 0.f;
    int bi = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float a = fabsf(v[i]);
        const float key = (a == a) ? a : -1.f;
        if (key > bk) { bk = key; bv = v[i]; bi = lane * 4 + i; }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ok = __shfl_xor(bk, off);
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (ok > bk || (ok == bk && oi < bi)) { bk = ok; bv = ov; bi = oi; }
    }
    uint32_t packed = 0;
    int s = 0;
    float d = 0.f;
    if (bk > 0.f) {
        const float iscale = -128.f / bv;
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
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    *sum16 = s;
    *d_out = d;
    return packed;
}

// Q8_0 (candle BlockQ8_0::from_float) of one 32-value block by 8 aligned lanes; sub =
// lane % 8 holds values 4*sub .. 4*sub+3.  d = amax/127 (NaN ignored); q = round(x/d)
// with the unrounded d, saturating, NaN -> 0.  *dh gets f16(d), the stored scale.
__device__ __forceinline__ uint32_t q8_0_block8(const float v[4], __half *dh) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    *dh = __float2half_rn(d);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float r = roundf(v[i] * id);
        const int q = (r != r) ? 0 : (int)fminf(fmaxf(r, -128.f), 127.f);
        packed |= ((uint32_t)q & 0xffu) << (8 * i);
    }
    return packed;
}

__device__ __forceinline__ void load4f(const float *p, bool vec, float v[4]) {
    if (vec) {
        const float4 f = *reinterpret_cast<const float4 *>(p);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
        v[0] = p[0]; v[1] = p[1]; v[2] = p[2]; v[3] = p[3];
    }
}

}  // namespace lbq
