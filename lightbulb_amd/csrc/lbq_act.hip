// lbq_act.hip -- activation quantisation (Q8_K, Q8_0, Q8_1) and block dequantisation kernels.
//
// Activation quantisation restates candle-core 0.10.2 k_quants.rs
// BlockQ8K::from_float, BlockQ8_0::from_float and BlockQ8_1::from_float, the first step of
// QMatMul::forward on the reference CPU path.  Every code and scale must be
// bit-identical to the CPU: the kernels use IEEE division (HIP's default,
// correctly rounded), roundf (half away from zero, like Rust's f32::round) and
// the same selection of the maximum.
//
// Dequantisation restates GgmlType::to_float / ggml-quants dequantize
// (lightbulb: /root/reference/src/quantization/mod.rs:158-247): f16 scales are
// widened exactly, and d1 = d*sc, m1 = dmin*m, y = d1*q - m1 are each rounded
// to f32 separately -- contraction into FMA is disabled in these functions.
#include <algorithm>

#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

// ---------------------------------------------------------------------------
// Q8_K: sixteen lanes per 256-value block (a DPP row), 16 values per lane, four
// blocks per wave (q8k_lane16: the selection and arithmetic every Q8_K quantiser
// here shares).  candle: the signed value `max` of largest |x| (first on ties;
// NaN is never selected because `amax < NaN` is false) gives iscale = -128/max;
// q = min(127, round(iscale*x)) as i8; d = 1/iscale; bsums over 16 codes -- a
// lane's own 16 codes.
// ---------------------------------------------------------------------------
// Zero the listed buffers (the matrix-core kernel's y, which its two-way split adds
// into): 16-byte stores where the buffer is 16-byte aligned, spread over the
// whole grid.
__device__ __forceinline__ void zero_fill(const ZeroList &zero) {
    const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x, nt = (int64_t)gridDim.x * 256;
    for (int z = 0; z < zero.count; z++) {
        float *p = zero.p[z];
        const int64_t n = zero.n[z];
        int64_t head = 0;
        if ((reinterpret_cast<uintptr_t>(p) & 15u) == 0) {
            head = n & ~int64_t(3);
            for (int64_t i = tid; 4 * i < head; i += nt) *reinterpret_cast<float4 *>(p + 4 * i) = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        for (int64_t i = head + tid; i < n; i += nt) p[i] = 0.f;
    }
}

template <bool GGUF_OUT, bool VEC_IN>
__global__ __launch_bounds__(256) void k_quant_q8k(const float *__restrict__ x, int64_t nblocks, int8_t *__restrict__ xq,
                                                   float *__restrict__ xd, int16_t *__restrict__ xbs,
                                                   uint8_t *__restrict__ gguf, ZeroList zero) {
    const int sub = threadIdx.x & 15;
    // workgroups past the blocks only zero (the grid may be widened for the zeroing)
    const bool quant = (int64_t)blockIdx.x * 16 < nblocks;
    // the 16 lanes of a row share the block (wave-uniform exits only at the end)
    const int64_t blk0 = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool ok = blk0 < nblocks;
    const int64_t blk = ok ? blk0 : nblocks - 1;
    float v[16];
    if (quant) {
#pragma unroll
        for (int i = 0; i < 4; i++) load4f(x + blk * QK_K + sub * 16 + 4 * i, VEC_IN, &v[4 * i]);
    }
    zero_fill(zero);  // after the x loads are issued: its stores do not delay them
    if (!quant) return;
    uint32_t packed[4];
    int s;
    float d;
    q8k_lane16(v, sub, packed, &s, &d);
    if (!ok) return;
    if (GGUF_OUT) {
        uint8_t *b = gguf + blk * 292;  // 4-byte aligned: dword stores
#pragma unroll
        for (int w = 0; w < 4; w++) *reinterpret_cast<uint32_t *>(b + 4 + 16 * sub + 4 * w) = packed[w];
        *reinterpret_cast<int16_t *>(b + 260 + 2 * sub) = (int16_t)s;
        if (sub == 0) *reinterpret_cast<float *>(b) = d;
    } else {
        *reinterpret_cast<uint4 *>(xq + blk * QK_K + 16 * sub) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
        xbs[blk * 16 + sub] = (int16_t)s;
        if (sub == 0) xd[blk] = d;
    }
}

// ---------------------------------------------------------------------------
// Q8_0 / Q8_1: 8 lanes per 32-value block, 8 blocks per wave.  Q8_1 adds
// s = f16(f16(sum of the codes) * d) with d the stored f16 scale (candle
// BlockQ8_1::from_float multiplies two f16 values: widened, multiplied in f32,
// rounded back).
// ---------------------------------------------------------------------------
template <bool GGUF_OUT, bool VEC_IN, bool S>
__global__ __launch_bounds__(256) void k_quant_q8_0(const float *__restrict__ x, int64_t nblocks,
                                                    int8_t *__restrict__ xq, float *__restrict__ xd,
                                                    float *__restrict__ xs, uint8_t *__restrict__ gguf, ZeroList zero) {
    const int tid = blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = (int64_t)tid >> 3;
    const int sub = threadIdx.x & 7;
    const bool ok = blk < nblocks;
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    if (ok) load4f(x + blk * QK8_0 + sub * 4, VEC_IN, v);
    zero_fill(zero);  // after the x loads are issued
    __half dh;
    const uint32_t packed = q8_0_block8(v, &dh);
    __half sh = __float2half_rn(0.f);
    if constexpr (S) {
        int sum = dot4(packed, 0x01010101u, 0);
        sum += __shfl_xor(sum, 1);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 4);
        sh = __float2half_rn(__half2float(__float2half_rn((float)sum)) * __half2float(dh));
    }
    if (!ok) return;
    if (GGUF_OUT) {
        if constexpr (S) {
            uint8_t *b = gguf + blk * 36;
            if (sub == 0) {
                *reinterpret_cast<unsigned short *>(b) = __half_as_ushort(dh);
                *reinterpret_cast<unsigned short *>(b + 2) = __half_as_ushort(sh);
            }
            *reinterpret_cast<uint32_t *>(b + 4 + sub * 4) = packed;
        } else {
            uint8_t *b = gguf + blk * 34;
            if (sub == 0) *reinterpret_cast<unsigned short *>(b) = __half_as_ushort(dh);
            *reinterpret_cast<unsigned short *>(b + 2 + sub * 4) = (unsigned short)(packed & 0xffffu);
            *reinterpret_cast<unsigned short *>(b + 4 + sub * 4) = (unsigned short)(packed >> 16);
        }
    } else {
        *reinterpret_cast<uint32_t *>(xq + blk * QK8_0 + sub * 4) = packed;
        if (sub == 0) {
            xd[blk] = __half2float(dh);
            if constexpr (S) xs[blk] = __half2float(sh);
        }
    }
}

// ---------------------------------------------------------------------------
// Dequantisation: one thread per run of 16 consecutive output values.
// ---------------------------------------------------------------------------
#pragma clang fp contract(off)

// value index e = 16*g + i of a 256-value k-quant block, or of a 32-value block
template <int TYPE>
__device__ __forceinline__ void deq_group(const uint8_t *__restrict__ b, int g, float out[16]) {
    if constexpr (TYPE == TYPE_Q8_0 || TYPE == TYPE_Q8_1) {
        const float d = h2f(ld2_a2(b));
        const uint8_t *qs = b + (TYPE == TYPE_Q8_0 ? 2 : 4) + 16 * g;
        for (int i = 0; i < 16; i++) out[i] = (float)(int8_t)qs[i] * d;
    } else if constexpr (TYPE == TYPE_Q2_K || TYPE == TYPE_Q3_K) {
        // group g = sub-block 8h + 2s + t: values 128h + 32s + 16t + [0,16), low
        // bits (qs[32h + 16t + i] >> 2s) & 3
        const int h = g >> 3, s = (g >> 1) & 3, t = g & 1;
        if constexpr (TYPE == TYPE_Q2_K) {
            const uint32_t dd = ld_u32(b + 80);
            const float d = h2f(dd & 0xffffu), dmin = h2f(dd >> 16);
            const uint32_t sc = b[g];
            const float dl = d * (float)(sc & 0xFu);
            const float ml = dmin * (float)(sc >> 4);
            const uint8_t *qs = b + 16 + 32 * h + 16 * t;
            for (int i = 0; i < 16; i++) out[i] = dl * (float)((qs[i] >> (2 * s)) & 3) - ml;
        } else {
            // 6-bit scale: low nibble of scales[g % 8] (nibble g / 8), top 2 bits of
            // scales[8 + g % 4] (bits 2 * (g / 4)); code - 4 unless bit 4h + s of
            // hmask[16t + i] is set
            const float d = h2f(ld2_a2(b + 108));
            const int lo = (b[96 + (g & 7)] >> (4 * (g >> 3))) & 0xF;
            const int hi = (b[104 + (g & 3)] >> (2 * (g >> 2))) & 3;
            const float dl = d * (float)((lo | (hi << 4)) - 32);
            const uint8_t *qs = b + 32 + 32 * h + 16 * t;
            const uint8_t *hm = b + 16 * t;
            for (int i = 0; i < 16; i++) {
                const int q = ((qs[i] >> (2 * s)) & 3) - (((hm[i] >> (4 * h + s)) & 1) ? 0 : 4);
                out[i] = dl * (float)q;
            }
        }
    } else if constexpr (is_legacy(TYPE)) {
        // value 16g + i: nibble g of qs[i]; Q5_* bit 4 from bit 16g + i of qh
        constexpr bool HAS_M = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;
        constexpr bool FIVE = TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1;
        constexpr int QH = HAS_M ? 4 : 2, QS = (HAS_M ? 4 : 2) + (FIVE ? 4 : 0);
        const float d = h2f(ld2_a2(b));
        const float m = HAS_M ? h2f(ld2_a2(b + 2)) : 0.f;
        const uint32_t qh = FIVE ? (ld2_a2(b + QH) | (ld2_a2(b + QH + 2) << 16)) >> (16 * g) : 0u;
        const uint8_t *qs = b + QS;
        for (int i = 0; i < 16; i++) {
            const int q = (int)((qs[i] >> (4 * g)) & 15u) | (int)(((qh >> i) & 1u) << 4);
            if constexpr (HAS_M) out[i] = (float)q * d + m;
            else out[i] = (float)(q - (FIVE ? 16 : 8)) * d;
        }
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
constexpr int type_bs() { return TYPE == TYPE_Q8_0 || TYPE == TYPE_Q8_1 || is_legacy(TYPE) ? 32 : 256; }
template <int TYPE>
constexpr int type_ts() {
    return TYPE == TYPE_Q4_0 ? 18 : TYPE == TYPE_Q4_1 ? 20 : TYPE == TYPE_Q5_0 ? 22 : TYPE == TYPE_Q5_1 ? 24
         : TYPE == TYPE_Q8_0 ? 34 : TYPE == TYPE_Q8_1 ? 36 : TYPE == TYPE_Q2_K ? 84 : TYPE == TYPE_Q3_K ? 110
         : TYPE == TYPE_Q4_K ? 144 : TYPE == TYPE_Q5_K ? 176 : TYPE == TYPE_Q6_K ? 210 : 292;
}

__device__ __forceinline__ void store16(float *dst, const float out[16]) {
    float4 *d4 = reinterpret_cast<float4 *>(dst);
    for (int i = 0; i < 4; i++) d4[i] = make_float4(out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]);
}

template <int TYPE>
__global__ __launch_bounds__(256) void k_dequant(const uint8_t *__restrict__ blocks, int64_t ngroups,
                                                 float *__restrict__ y) {
    constexpr int GPB = type_bs<TYPE>() / 16;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= ngroups) return;
    const int64_t blk = t / GPB;
    const int g = (int)(t % GPB);
    float out[16];
    deq_group<TYPE>(blocks + blk * type_ts<TYPE>(), g, out);
    store16(y + t * 16, out);
}

// Embedding rows: thread t handles group g = t % gpr (16 values) of output row
// i = t / gpr, read from weight row ids[i].
template <int TYPE>
__global__ __launch_bounds__(256) void k_embed_rows(const uint8_t *__restrict__ w, int64_t n, int64_t row_bytes,
                                                    const int32_t *__restrict__ ids, int64_t count, int64_t gpr,
                                                    float *__restrict__ y) {
    constexpr int GPB = type_bs<TYPE>() / 16;
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= count * gpr) return;
    const int64_t i = t / gpr, g = t % gpr;
    const int64_t id = ids[i];
    float out[16];
    if (id < 0 || id >= n) {
        for (int j = 0; j < 16; j++) out[j] = __int_as_float(0x7fc00000);
    } else {
        deq_group<TYPE>(w + id * row_bytes + (g / GPB) * type_ts<TYPE>(), (int)(g % GPB), out);
    }
    store16(y + t * 16, out);
}

// F32 / F16 / BF16 tensors: y[i] = x[i] (bits) / the exact f16 or bf16 -> f32 widening
template <bool F16, bool BF = false>
__global__ __launch_bounds__(256) void k_dense_f32(const uint8_t *__restrict__ x, int64_t n, float *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    if constexpr (F16) y[i] = w16<BF>(reinterpret_cast<const unsigned short *>(x)[i]);
    else y[i] = reinterpret_cast<const float *>(x)[i];
}

// Embedding rows of an F32 / F16 / BF16 table (16 values per thread, widened
// exactly); ids outside [0, n) give NaN rows, as k_embed_rows.
template <bool F16, bool BF = false>
__global__ __launch_bounds__(256) void k_embed_dense(const uint8_t *__restrict__ w, int64_t n, int64_t k,
                                                     const int32_t *__restrict__ ids, int64_t count, int64_t gpr,
                                                     float *__restrict__ y) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (t >= count * gpr) return;
    const int64_t i = t / gpr, g = t % gpr;
    const int64_t id = ids[i];
    float out[16];
    if (id < 0 || id >= n) {
        for (int j = 0; j < 16; j++) out[j] = __int_as_float(0x7fc00000);
    } else if constexpr (F16) {
        const unsigned short *src = reinterpret_cast<const unsigned short *>(w) + id * k + 16 * g;
        for (int j = 0; j < 16; j++) out[j] = w16<BF>(src[j]);
    } else {
        const float *src = reinterpret_cast<const float *>(w) + id * k + 16 * g;
        for (int j = 0; j < 16; j++) out[j] = src[j];
    }
    store16(y + t * 16, out);
}

#pragma clang fp contract(on)

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
hipError_t launch_quant_act(int act_type, const float *x, int64_t m, int64_t k, int8_t *xq, float *xd, int16_t *xbs,
                            float *xs, uint8_t *gguf, hipStream_t st, const ZeroList *zero) {
    const ZeroList zl = zero ? *zero : ZeroList{};
    if (zl.count && act_type != TYPE_Q8_K && act_type != TYPE_Q8_0 && act_type != TYPE_Q8_1) return hipErrorInvalidValue;
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    if (act_type == TYPE_Q8_K) {
        const int64_t nb = m * (k / QK_K);
        int64_t zn = 0;
        for (int z = 0; z < zl.count; z++) zn += zl.n[z];
        // at least one workgroup per 16 K floats to zero (4 stores of 16 bytes per lane), at most 1024
        const dim3 grid((unsigned)std::max<int64_t>((nb + 15) / 16, std::min<int64_t>((zn + 16383) / 16384, 1024)));
        if (gguf) {
            if (vec) k_quant_q8k<true, true><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf, zl);
            else k_quant_q8k<true, false><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf, zl);
        } else {
            if (vec) k_quant_q8k<false, true><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf, zl);
            else k_quant_q8k<false, false><<<grid, 256, 0, st>>>(x, nb, xq, xd, xbs, gguf, zl);
        }
    } else if (act_type == TYPE_Q8_0 || act_type == TYPE_Q8_1) {
        const int64_t nb = m * (k / QK8_0);
        int64_t zn = 0;
        for (int z = 0; z < zl.count; z++) zn += zl.n[z];
        // (workgroups past the blocks only zero, as for Q8_K)
        const dim3 grid((unsigned)std::max<int64_t>((nb * 8 + 255) / 256, std::min<int64_t>((zn + 16383) / 16384, 1024)));
#define LBQ_Q8(G, V)                                                                                       \
    if (act_type == TYPE_Q8_1) k_quant_q8_0<G, V, true><<<grid, 256, 0, st>>>(x, nb, xq, xd, xs, gguf, zl); \
    else k_quant_q8_0<G, V, false><<<grid, 256, 0, st>>>(x, nb, xq, xd, xs, gguf, zl);
        if (gguf) {
            if (vec) { LBQ_Q8(true, true) } else { LBQ_Q8(true, false) }
        } else {
            if (vec) { LBQ_Q8(false, true) } else { LBQ_Q8(false, false) }
        }
#undef LBQ_Q8
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

#define LBQ_BLOCK_TYPES(X) \
    X(TYPE_Q4_0) X(TYPE_Q4_1) X(TYPE_Q5_0) X(TYPE_Q5_1) X(TYPE_Q8_0) X(TYPE_Q8_1) X(TYPE_Q2_K) X(TYPE_Q3_K) \
    X(TYPE_Q4_K) X(TYPE_Q5_K) X(TYPE_Q6_K) X(TYPE_Q8_K)

hipError_t launch_dequant(int type, const uint8_t *blocks, int64_t nelem, float *y, hipStream_t st) {
    if (is_dense(type)) {
        const dim3 grid((unsigned)((nelem + 255) / 256));
        if (type == TYPE_F16) k_dense_f32<true><<<grid, 256, 0, st>>>(blocks, nelem, y);
        else if (type == TYPE_BF16) k_dense_f32<true, true><<<grid, 256, 0, st>>>(blocks, nelem, y);
        else k_dense_f32<false><<<grid, 256, 0, st>>>(blocks, nelem, y);
        return hipGetLastError();
    }
    const int64_t ng = nelem / 16;
    const dim3 grid((unsigned)((ng + 255) / 256));
    switch (type) {
#define LBQ_DEQ(T) \
    case T: k_dequant<T><<<grid, 256, 0, st>>>(blocks, ng, y); break;
        LBQ_BLOCK_TYPES(LBQ_DEQ)
#undef LBQ_DEQ
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_embedding(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const int32_t *ids,
                            int64_t count, float *y, hipStream_t st) {
    const int64_t gpr = k / 16;
    const dim3 grid((unsigned)((count * gpr + 255) / 256));
    switch (type) {
    case TYPE_F16: k_embed_dense<true><<<grid, 256, 0, st>>>(w, n, k, ids, count, gpr, y); break;
    case TYPE_BF16: k_embed_dense<true, true><<<grid, 256, 0, st>>>(w, n, k, ids, count, gpr, y); break;
    case TYPE_F32: k_embed_dense<false><<<grid, 256, 0, st>>>(w, n, k, ids, count, gpr, y); break;
#define LBQ_EMB(T) \
    case T: k_embed_rows<T><<<grid, 256, 0, st>>>(w, n, row_bytes, ids, count, gpr, y); break;
        LBQ_BLOCK_TYPES(LBQ_EMB)
#undef LBQ_EMB
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// candle's RmsNorm (f32): y = x / sqrt(sum(x^2) / k + eps) * w, one workgroup per row
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float eps,
                                                 int64_t k, float *__restrict__ y) {
    __shared__ float red[4];
    const int64_t m = blockIdx.x;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float *xr = x + m * k;
    float ss = 0.f;
    for (int64_t i = t; i < k; i += 256) ss += xr[i] * xr[i];
    ss = row_sum_f32(ss);
    ss = __int_as_float(rl(__float_as_uint(ss), 0)) + __int_as_float(rl(__float_as_uint(ss), 16)) +
         __int_as_float(rl(__float_as_uint(ss), 32)) + __int_as_float(rl(__float_as_uint(ss), 48));
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float rms = sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)k + eps);
    for (int64_t i = t; i < k; i += 256) y[m * k + i] = xr[i] / rms * w[i];
}

// candle's RmsNorm (f32) of each row and the Q8_K quantisation of the result in
// one launch (the call-site entry points at m > 1): one workgroup per row, 16
// lanes per 256-value block and 16 values per lane (q8k_lane16, as every Q8_K
// quantiser here), P passes of 16 blocks; the normalised row never reaches
// memory.  The norm is x / sqrt(sum(x^2) / k + eps) * w in that order, the sum
// over the lanes' own values, then DPP rows, then the four waves.  Also zeroes
// the listed outputs (ZeroList), as k_quant_q8k does; workgroups past the rows
// only zero (the grid may be widened for the zeroing).
template <int P>
__global__ __launch_bounds__(256) void k_rmsnorm_q8k(const float *__restrict__ x, const float *__restrict__ w, float eps,
                                                     int64_t rows, int64_t k, int8_t *__restrict__ xq,
                                                     float *__restrict__ xd, int16_t *__restrict__ xbs, ZeroList zero) {
    __shared__ float red[4];
    const int64_t m = blockIdx.x;
    if (m >= rows) {  // workgroup-uniform
        zero_fill(zero);
        return;
    }
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, sub = t & 15;
    const int nbx = (int)(k / QK_K);
    const float *xr = x + m * k;
    float v[P][16], al[P][16];
#pragma unroll
    for (int j = 0; j < P; j++) {
        const int b = min(16 * j + (t >> 4), nbx - 1);
        const float4 *src = reinterpret_cast<const float4 *>(xr + (int64_t)b * QK_K + 16 * sub);
        const float4 *wsrc = reinterpret_cast<const float4 *>(w + (int64_t)b * QK_K + 16 * sub);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 f = src[i], g = wsrc[i];
            v[j][4 * i] = f.x; v[j][4 * i + 1] = f.y; v[j][4 * i + 2] = f.z; v[j][4 * i + 3] = f.w;
            al[j][4 * i] = g.x; al[j][4 * i + 1] = g.y; al[j][4 * i + 2] = g.z; al[j][4 * i + 3] = g.w;
        }
    }
    zero_fill(zero);  // after the loads are issued
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < P; j++)
        if (16 * j + (t >> 4) < nbx)  // clamped duplicates do not count
#pragma unroll
            for (int i = 0; i < 16; i++) ss += v[j][i] * v[j][i];
    ss = row_sum_f32(ss);
    ss = __int_as_float(rl(__float_as_uint(ss), 0)) + __int_as_float(rl(__float_as_uint(ss), 16)) +
         __int_as_float(rl(__float_as_uint(ss), 32)) + __int_as_float(rl(__float_as_uint(ss), 48));
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float rms = sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)k + eps);
#pragma unroll
    for (int j = 0; j < P; j++) {
        if (j > 0 && 16 * j >= nbx) continue;  // workgroup-uniform
#pragma unroll
        for (int i = 0; i < 16; i++) v[j][i] = v[j][i] / rms * al[j][i];
        uint32_t packed[4];
        int sum;
        float d;
        q8k_lane16(v[j], sub, packed, &sum, &d);
        const int b = 16 * j + (t >> 4);
        if (b < nbx) {
            const int64_t blk = m * nbx + b;
            *reinterpret_cast<uint4 *>(xq + blk * QK_K + 16 * sub) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            xbs[blk * 16 + sub] = (int16_t)sum;
            if (sub == 0) xd[blk] = d;
        }
    }
}

hipError_t launch_rmsnorm_q8k(const float *x, const float *w, float eps, int64_t m, int64_t k, int8_t *xq, float *xd,
                              int16_t *xbs, hipStream_t st, const ZeroList *zero) {
    const ZeroList zl = zero ? *zero : ZeroList{};
    if (k % QK_K || k / QK_K > 64 || ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) & 15u))
        return hipErrorInvalidValue;
    if (m <= 0) return hipSuccess;
    const int nbx = (int)(k / QK_K);
    int64_t zn = 0;
    for (int z = 0; z < zl.count; z++) zn += zl.n[z];
    // at least one workgroup per 16 K floats to zero, at most 1024 (as launch_quant_act)
    const dim3 grid((unsigned)std::max<int64_t>(m, std::min<int64_t>((zn + 16383) / 16384, 1024)));
    if (nbx <= 16) k_rmsnorm_q8k<1><<<grid, 256, 0, st>>>(x, w, eps, m, k, xq, xd, xbs, zl);
    else if (nbx <= 32) k_rmsnorm_q8k<2><<<grid, 256, 0, st>>>(x, w, eps, m, k, xq, xd, xbs, zl);
    else if (nbx <= 48) k_rmsnorm_q8k<3><<<grid, 256, 0, st>>>(x, w, eps, m, k, xq, xd, xbs, zl);
    else k_rmsnorm_q8k<4><<<grid, 256, 0, st>>>(x, w, eps, m, k, xq, xd, xbs, zl);
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int64_t m, int64_t k, float *y, hipStream_t st) {
    if (m <= 0) return hipSuccess;
    k_rmsnorm<<<(unsigned)m, 256, 0, st>>>(x, w, eps, k, y);
    return hipGetLastError();
}

// out = silu(g) * u with candle's f32 silu, v / (1 + exp(-v)) (the gate/up
// product of mlp_wrapper.rs:190-194 when it is not fused into the GEMV)
__global__ __launch_bounds__(256) void k_silu_mul(const float *__restrict__ g, const float *__restrict__ u, int64_t count,
                                                  float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= count) return;
    const float v = g[i];
    out[i] = v / (1.f + expf(-v)) * u[i];
}

hipError_t launch_silu_mul(const float *g, const float *u, int64_t count, float *out, hipStream_t st) {
    if (count <= 0) return hipSuccess;
    k_silu_mul<<<(unsigned)((count + 255) / 256), 256, 0, st>>>(g, u, count, out);
    return hipGetLastError();
}

}  // namespace lbq
