// lbq_act.hip -- activation quantisation (Q8_K, Q8_0) and block dequantisation kernels.
//
// Activation quantisation restates candle-core 0.10.2 k_quants.rs
// BlockQ8K::from_float and BlockQ8_0::from_float, the first step of
// QMatMul::forward on the reference CPU path.  Every code and scale must be
// bit-identical to the CPU: the kernels use IEEE division (HIP's default,
// correctly rounded), roundf (half away from zero, like Rust's f32::round) and
// the same selection of the maximum.
//
// Dequantisation restates GgmlType::to_float / ggml-quants dequantize
// (lightbulb: /root/reference/src/quantization/mod.rs:158-247): f16 scales are
// widened exactly, and d1 = d*sc, m1 = dmin*m, y = d1*q - m1 are each rounded
// to f32 separately -- contraction into FMA is disabled in these functions.
#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

// ---------------------------------------------------------------------------
// Q8_K: one 64-lane wave per 256-value block, 4 values per lane.
// candle: the signed value `max` of largest |x| (first on ties; NaN is never
// selected because `amax < NaN` is false) gives iscale = -128/max;
// q = min(127, round(iscale*x)) as i8; d = 1/iscale; bsums over 16 codes.
// ---------------------------------------------------------------------------
template <bool GGUF_OUT, bool VEC_IN>
__global__ __launch_bounds__(256) void k_quant_q8k(const float *__restrict__ x, int64_t nblocks, int8_t *__restrict__ xq,
                                                   float *__restrict__ xd, int16_t *__restrict__ xbs,
                                                   uint8_t *__restrict__ gguf) {
    const int lane = threadIdx.x & 63;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) return;  // whole wave exits together
    const float *src = x + blk * QK_K + lane * 4;
    float v[4];
    if (VEC_IN) {
        const float4 f = *reinterpret_cast<const float4 *>(src);
        v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
    } else {
        for (int i = 0; i < 4; i++) v[i] = src[i];
    }
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
    if (GGUF_OUT) {
        uint8_t *b = gguf + blk * 292;
        *reinterpret_cast<uint32_t *>(b + 4 + lane * 4) = packed;
        if ((lane & 3) == 0) *reinterpret_cast<int16_t *>(b + 260 + 2 * (lane >> 2)) = (int16_t)s;
        if (lane == 0) *reinterpret_cast<float *>(b) = d;
    } else {
        *reinterpret_cast<uint32_t *>(xq + blk * QK_K + lane * 4) = packed;
        if ((lane & 3) == 0) xbs[blk * 16 + (lane >> 2)] = (int16_t)s;
        if (lane == 0) xd[blk] = d;
    }
}

// ---------------------------------------------------------------------------
// Q8_0: 8 lanes per 32-value block, 8 blocks per wave.
// candle: d = amax/127 (amax over |x|, NaN ignored by f32::max); id = 1/d or 0;
// q = round(x*id) as i8 (saturating, NaN -> 0), using the unrounded d; the
// stored scale is f16(d), so the value the dot product uses is f32(f16(d)).
// ---------------------------------------------------------------------------
template <bool GGUF_OUT, bool VEC_IN>
__global__ __launch_bounds__(256) void k_quant_q8_0(const float *__restrict__ x, int64_t nblocks,
                                                    int8_t *__restrict__ xq, float *__restrict__ xd,
                                                    uint8_t *__restrict__ gguf) {
    const int tid = blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = (int64_t)tid >> 3;
    const int sub = threadIdx.x & 7;
    const bool ok = blk < nblocks;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (ok) {
        const float *src = x + blk * QK8_0 + sub * 4;
        if (VEC_IN) {
            const float4 f = *reinterpret_cast<const float4 *>(src);
            v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
        } else {
            for (int i = 0; i < 4; i++) v[i] = src[i];
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) amax = fmaxf(amax, fabsf(v[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    amax = fmaxf(amax, __shfl_xor(amax, 4));
    const float d = amax / 127.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    const __half dh = __float2half_rn(d);
    uint32_t packed = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float r = roundf(v[i] * id);
        int q = (r != r) ? 0 : (int)fminf(fmaxf(r, -128.f), 127.f);
        packed |= ((uint32_t)q & 0xffu) << (8 * i);
    }
    if (!ok) return;
    if (GGUF_OUT) {
        uint8_t *b = gguf + blk * 34;
        if (sub == 0) *reinterpret_cast<unsigned short *>(b) = __half_as_ushort(dh);
        *reinterpret_cast<unsigned short *>(b + 2 + sub * 4) = (unsigned short)(packed & 0xffffu);
        *reinterpret_cast<unsigned short *>(b + 4 + sub * 4) = (unsigned short)(packed >> 16);
    } else {
        *reinterpret_cast<uint32_t *>(xq + blk * QK8_0 + sub * 4) = packed;
        if (sub == 0) xd[blk] = __half2float(dh);
    }
}

// ---------------------------------------------------------------------------
// Dequantisation: one thread per run of 16 consecutive output values.
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)

// value index e = 16*g + i of a 256-value k-quant block, or of a 32-value Q8_0 block
template <int TYPE>
__device__ __forceinline__ void deq_group(const uint8_t *__restrict__ b, int g, float out[16]) {
    if constexpr (TYPE == TYPE_Q8_0) {
        const float d = h2f(ld2_a2(b));
        const uint8_t *qs = b + 2 + 16 * g;
        for (int i = 0; i < 16; i++) out[i] = (float)(int8_t)qs[i] * d;
    } else if constexpr (TYPE == TYPE_Q4_K || TYPE == TYPE_Q5_K) {
        const uint32_t dd = ld_u32(b);
        const float d = h2f(dd & 0xffffu), dmin = h2f(dd >> 16);
        const int c = g >> 2, r = g & 3, hi = r >> 1, h = r & 1;
        uint32_t sc2, m2;
        k4_scale_pair(ld_u32(b + 4), ld_u32(b + 8), ld_u32(b + 12), c, &sc2, &m2);
        const uint32_t sc = hi ? (sc2 >> 8) : (sc2 & 0xffu);
        const uint32_t mn = hi ? (m2 >> 8) : (m2 & 0xffu);
        const float d1 = d * (float)sc;
        const float m1 = dmin * (float)mn;
        const uint8_t *qs = b + (TYPE == TYPE_Q4_K ? 16 : 48) + 32 * c + 16 * h;
        for (int i = 0; i < 16; i++) {
            int q = hi ? (qs[i] >> 4) : (qs[i] & 0xF);
            if (TYPE == TYPE_Q5_K) q += ((b[16 + 16 * h + i] >> (2 * c + hi)) & 1) ? 16 : 0;
            out[i] = d1 * (float)q - m1;
        }
    } else if constexpr (TYPE == TYPE_Q6_K) {
        const float d = h2f(ld2_a2(b + 208));
        const int n = g >> 3, s = (g & 7) >> 1, h = g & 1;
        const float sc = (float)(int8_t)b[192 + g];
        const uint8_t *ql = b + 64 * n + 32 * (s & 1) + 16 * h;
        const uint8_t *qh = b + 128 + 32 * n + 16 * h;
        for (int i = 0; i < 16; i++) {
            const int lo = (s >> 1) ? (ql[i] >> 4) : (ql[i] & 0xF);
            const int q = (lo | (((qh[i] >> (2 * s)) & 3) << 4)) - 32;
            out[i] = d * sc * (float)q;
        }
    } else {  // Q8_K
        const float d = *reinterpret_cast<const float *>(b);
        const int8_t *qs = reinterpret_cast<const int8_t *>(b + 4 + 16 * g);
        for (int i = 0; i < 16; i++) out[i] = d * (float)qs[i];
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *__restrict__ blocks, int64_t ngroups,
                                                 float *__restrict__ y) {
    constexpr int BS = TYPE == TYPE_Q8_0 ? 32 : 256;
    constexpr int TS = TYPE == TYPE_Q8_0 ? 34 : TYPE == TYPE_Q4_K ? 144 : TYPE == TYPE_Q5_K ? 176 : TYPE == TYPE_Q6_K ? 210 : 292;
    constexpr int GPB = BS / 16;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= ngroups) return;
    const int64_t blk = t / GPB;
    const int g = (int)(t % GPB);
    float out[16];
    deq_group<TYPE>(blocks + blk * TS, g, out);
    float4 *dst = reinterpret_cast<float4 *>(y + t * 16);
    for (int i = 0; i < 4; i++) dst[i] = make_float4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
}

#pragma clang fp contract(on)

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_quant_act(int act_type, const float *x, int64_t m, int64_t k, int8_t *xq, float *xd, int16_t *xbs,
                            uint8_t *gguf, hipStream_t st) {
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    if (act_type == TYPE_Q8_K) {
        const int64_t nb = m * (k / QK_K);
        const dim3 grid((unsigned)((nb + 3) / 4));
        if (gguf) {
            if (vec) k_quant_q8k<true, true><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf);
            else k_quant_q8k<true, false><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf);
        } else {
            if (vec) k_quant_q8k<false, true><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf);
            else k_quant_q8k<false, false><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf);
        }
    } else {
        const int64_t nb = m * (k / QK8_0);
        const dim3 grid((unsigned)((nb * 8 + 255) / 256));
        if (gguf) {
            if (vec) k_quant_q8_0<true, true><<<grid, 256, 0, st>>>(x, nb, xq, xd, gguf);
            else k_quant_q8_0<true, false><<<grid, 256, 0, st>>>(x, nb, xq, xd, gguf);
        } else {
            if (vec) k_quant_q8_0<false, true><<<grid, 256, 0, st>>>(x, nb, xq, xd, gguf);
            else k_quant_q8_0<false, false><<<grid, 256, 0, st>>>(x, nb, xq, xd, gguf);
        }
    }
    return hipGetLastError();
}

hipError_t launch_dequant(int type, const uint8_t *blocks, int64_t nelem, float *y, hipStream_t st) {
    const int64_t ng = nelem / 16;
    const dim3 grid((unsigned)((ng + 255) / 256));
    switch (type) {
    case TYPE_Q8_0: k_dequant<TYPE_Q8_0><<<grid, 256, 0, st>>>(blocks, ng, y); break;
    case TYPE_Q4_K: k_dequant<TYPE_Q4_K><<<grid, 256, 0, st>>>(blocks, ng, y); break;
    case TYPE_Q5_K: k_dequant<TYPE_Q5_K><<<grid, 256, 0, st>>>(blocks, ng, y); break;
    case TYPE_Q6_K: k_dequant<TYPE_Q6_K><<<grid, 256, 0, st>>>(blocks, ng, y); break;
    case TYPE_Q8_K: k_dequant<TYPE_Q8_K><<<grid, 256, 0, st>>>(blocks, ng, y); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lbq
