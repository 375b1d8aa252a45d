// lbq_wquant.hip -- f32 weights -> GGUF blocks on the device.
//
// lightbulb's quantize_tensor (/root/reference/src/quantization/mod.rs:257-327)
// calls ggml-quants 0.1.0, a port of ggml's reference quantisers
// (quantize_row_q8_0/q4_K/q5_K/q6_K_ref with make_qkx2_quants / make_qx_quants,
// and the 32-value quantize_row_q4_0/q4_1/q5_0/q5_1_ref).
// This file restates those published algorithms for the device so multi-GB
// weight sets can be built in HBM.  Built with -ffp-contract=off: every
// product and sum is rounded separately, in the source order, so the blocks
// match a CPU build of the same algorithm bit for bit.
#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

__device__ __forceinline__ int nearest_int(float fval) {
    const float val = fval + 12582912.f;
    return (__float_as_int(val) & 0x007fffff) - 0x00400000;
}

__device__ __forceinline__ uint32_t f2h_bits(float f) { return __half_as_ushort(__float2half_rn(f)); }

// ggml make_qkx2_quants(n = 32, weights, use_mad = false)
template <int NMAX>
__device__ float make_qkx2_32(const float *x, const float *weights, uint8_t *L, float *the_min, float rmin,
                              float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
#pragma unroll
        for (int i = 0; i < 32; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = (float)NMAX / (max - min);
    float scale = 1.f / iscale;
    float best_mad = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        const int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : l > NMAX ? NMAX : l);
        float diff = scale * (float)L[i] + min - x[i];
        diff = diff * diff;
        best_mad += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)NMAX) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        uint8_t Laux[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : l > NMAX ? NMAX : l;
            Laux[i] = (uint8_t)l;
            const float w = weights[i];
            sum_l += w * (float)l;
            sum_l2 += w * (float)l * (float)l;
            sum_xl += w * (float)l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float mad = 0;
#pragma unroll
            for (int i = 0; i < 32; ++i) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = diff * diff;
                mad += weights[i] * diff;
            }
            if (mad < best_mad) {
#pragma unroll
                for (int i = 0; i < 32; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

// Q4_K (NMAX 15) / Q5_K (NMAX 31): 8 lanes per super-block, lane j owns sub-block j.
template <int NMAX>
__global__ __launch_bounds__(256) void k_quant_w_k45(const float *__restrict__ w, int64_t nblocks,
                                                     uint8_t *__restrict__ out) {
    constexpr int TS = NMAX == 15 ? 144 : 176;
    __shared__ uint8_t Ls[32][QK_K];
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = t >> 3;
    const int j = threadIdx.x & 7, bl = threadIdx.x >> 3;
    const bool ok = blk < nblocks;
    float x[32], weights[32];
    uint8_t L[32];
    const float *src = w + (ok ? blk : 0) * QK_K + 32 * j;
#pragma unroll
    for (int l = 0; l < 32; ++l) x[l] = ok ? src[l] : 0.f;
    float sum_x2 = 0;
#pragma unroll
    for (int l = 0; l < 32; ++l) sum_x2 += x[l] * x[l];
    const float av_x = sqrtf(sum_x2 / 32.f);
#pragma unroll
    for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[l]);
    float mn;
    const float sc = NMAX == 15 ? make_qkx2_32<15>(x, weights, L, &mn, -1.f, 0.1f, 20)
                                : make_qkx2_32<31>(x, weights, L, &mn, -0.5f, 0.1f, 15);
    // max over the 8 sub-blocks (ggml: strict > from 0)
    float max_scale = sc > 0.f ? sc : 0.f, max_min = mn > 0.f ? mn : 0.f;
#pragma unroll
    for (int off = 1; off < 8; off <<= 1) {
        const float a = __shfl_xor(max_scale, off), b = __shfl_xor(max_min, off);
        max_scale = a > max_scale ? a : max_scale;
        max_min = b > max_min ? b : max_min;
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    int ls = nearest_int(inv_scale * sc) & 255;  // ggml stores into uint8_t first
    int lm = nearest_int(inv_min * mn) & 255;
    ls = ls > 63 ? 63 : ls;
    lm = lm > 63 ? 63 : lm;
    const uint32_t dh = f2h_bits(max_scale / 63.f);
    const uint32_t dminh = f2h_bits(max_min / 63.f);
    const int ls_hi = __shfl_xor(ls, 4), lm_hi = __shfl_xor(lm, 4);
    uint8_t *ob = out + (ok ? blk : 0) * TS;
    if (ok) {
        if (j < 4) {
            ob[4 + j] = (uint8_t)((ls & 63) | ((ls_hi >> 4) << 6));
            ob[4 + j + 4] = (uint8_t)((lm & 63) | ((lm_hi >> 4) << 6));
        } else {
            ob[4 + j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
        }
        if (j == 0) {
            ob[0] = (uint8_t)(dh & 0xff);
            ob[1] = (uint8_t)(dh >> 8);
            ob[2] = (uint8_t)(dminh & 0xff);
            ob[3] = (uint8_t)(dminh >> 8);
        }
    }
    const float d = h2f(dh) * (float)ls;
    if (d != 0.f) {
        const float dm = h2f(dminh) * (float)lm;
#pragma unroll
        for (int ii = 0; ii < 32; ++ii) {
            const int l = nearest_int((x[ii] + dm) / d);
            L[ii] = (uint8_t)(l < 0 ? 0 : l > NMAX ? NMAX : l);
        }
    }
#pragma unroll
    for (int ii = 0; ii < 32; ++ii) Ls[bl][32 * j + ii] = L[ii];
    __syncthreads();
    if (!ok) return;
    const uint8_t *Lb = Ls[bl];
    uint8_t *q = ob + (NMAX == 15 ? 16 : 48);
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) {
        const int i = 16 * j + ii, c = i >> 5, l = i & 31;
        q[i] = (uint8_t)((Lb[64 * c + l] & 15) | ((Lb[64 * c + 32 + l] & 15) << 4));
    }
    if (NMAX == 31) {
        uint8_t *qh = ob + 16;
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int l = 4 * j + ii;
            uint32_t v = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                v |= (uint32_t)(Lb[64 * c + l] >> 4) << (2 * c);
                v |= (uint32_t)(Lb[64 * c + 32 + l] >> 4) << (2 * c + 1);
            }
            qh[l] = (uint8_t)v;
        }
    }
}

// ggml make_qx_quants(n = 16, nmax = 32, rmse_type = 1, qw = NULL)
__device__ float make_qx_16(const float *x, uint8_t *L) {
    constexpr int nmax = 32;
    float max = 0, amax = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < 1e-15f) {
#pragma unroll
        for (int i = 0; i < 16; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -(float)nmax / max;
    float sumlx = 0, suml2 = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
        L[i] = (uint8_t)(l + nmax);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -9; is <= 9; ++is) {
        if (is == 0) continue;
        iscale = -((float)nmax + 0.1f * (float)is) / max;
        sumlx = suml2 = 0;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                int l = nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
                L[i] = (uint8_t)(nmax + l);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

// Q6_K: 16 lanes per super-block, lane t owns values 16t..16t+15.
__global__ __launch_bounds__(256) void k_quant_w_q6k(const float *__restrict__ w, int64_t nblocks,
                                                     uint8_t *__restrict__ out) {
    __shared__ uint8_t Ls[16][QK_K];
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t blk = t >> 4;
    const int ib = threadIdx.x & 15, bl = threadIdx.x >> 4;
    const bool ok = blk < nblocks;
    float x[16];
    uint8_t L[16];
    const float *src = w + (ok ? blk : 0) * QK_K + 16 * ib;
#pragma unroll
    for (int l = 0; l < 16; ++l) x[l] = ok ? src[l] : 0.f;
    const float scale = make_qx_16(x, L);
    // first sub-block of largest |scale| (ggml: strict > from 0)
    float ba = (scale == scale) ? fabsf(scale) : -1.f, bs = scale;
    int bi = ib;
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
        const float oa = __shfl_xor(ba, off), os = __shfl_xor(bs, off);
        const int oi = __shfl_xor(bi, off);
        if (oa > ba || (oa == ba && oi < bi)) {
            ba = oa;
            bs = os;
            bi = oi;
        }
    }
    uint8_t *ob = out + (ok ? blk : 0) * 210;
    const bool zero_block = !(ba >= 1e-15f);
    uint32_t dh = 0;
    int scq = 0;
    if (!zero_block) {
        const float iscale = -128.f / bs;
        dh = f2h_bits(1.f / iscale);
        const int v = nearest_int(iscale * scale);
        scq = (int)(int8_t)(v > 127 ? 127 : v);
        const float d = h2f(dh) * (float)scq;
        if (d != 0.f) {
#pragma unroll
            for (int ii = 0; ii < 16; ++ii) {
                int l = nearest_int(x[ii] / d);
                l = l < -32 ? -32 : l > 31 ? 31 : l;
                L[ii] = (uint8_t)(l + 32);
            }
        }
    }
#pragma unroll
    for (int ii = 0; ii < 16; ++ii) Ls[bl][16 * ib + ii] = L[ii];
    __syncthreads();
    if (!ok) return;
    if (zero_block) {
        // ggml: memset(block, 0); d = f16(0)
        for (int i = 0; i < 14; ++i) {
            const int idx = 14 * ib + i;
            if (idx < 210) ob[idx] = 0;
        }
        return;
    }
    const uint8_t *Lb = Ls[bl];
#pragma unroll
    for (int ii = 0; ii < 8; ++ii) {
        const int i = 8 * ib + ii, n = i >> 6, l = i & 63;
        ob[i] = (uint8_t)((Lb[128 * n + l] & 15) | ((Lb[128 * n + l + 64] & 15) << 4));
    }
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        const int i = 4 * ib + ii, n = i >> 5, l = i & 31;
        const uint8_t *Ln = Lb + 128 * n;
        ob[128 + i] = (uint8_t)((Ln[l] >> 4) | ((Ln[l + 32] >> 4) << 2) | ((Ln[l + 64] >> 4) << 4) |
                                ((Ln[l + 96] >> 4) << 6));
    }
    ob[192 + ib] = (uint8_t)scq;
    if (ib == 0) {
        ob[208] = (uint8_t)(dh & 0xff);
        ob[209] = (uint8_t)(dh >> 8);
    }
}

// ggml quantize_row_q4_0/q4_1/q5_0/q5_1_ref: one thread per 32-value block.
//   _0: d = max / -8 (-16), max the signed value of largest |x| (first on ties),
//       q = min(15 (31), (int8)(x*id + 8.5 (16.5)));
//   _1: d = (max - min) / 15 (31), m = min, q = (int8)((x - min)*id + 0.5),
//       clamped to 15 for Q4_1 only;
// id = 1/d (0 when d = 0); codes are truncated toward zero, as C's cast does.
template <int TYPE>
__global__ __launch_bounds__(256) void k_quant_w_legacy(const float *__restrict__ w, int64_t nblocks,
                                                        uint8_t *__restrict__ out) {
    constexpr bool HAS_M = TYPE == TYPE_Q4_1 || TYPE == TYPE_Q5_1;
    constexpr bool FIVE = TYPE == TYPE_Q5_0 || TYPE == TYPE_Q5_1;
    constexpr int BYTES = 18 + (HAS_M ? 2 : 0) + (FIVE ? 4 : 0);
    const int64_t blk = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (blk >= nblocks) return;
    const float *x = w + blk * 32;
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; j++) v[j] = x[j];
    float d, mn = 0.f;
    if constexpr (HAS_M) {
        float lo = v[0], hi = v[0];
#pragma unroll
        for (int j = 1; j < 32; j++) {
            if (v[j] < lo) lo = v[j];
            if (v[j] > hi) hi = v[j];
        }
        d = (hi - lo) / (FIVE ? 31.f : 15.f);
        mn = lo;
    } else {
        float amax = 0.f, mx = 0.f;
#pragma unroll
        for (int j = 0; j < 32; j++)
            if (amax < fabsf(v[j])) { amax = fabsf(v[j]); mx = v[j]; }
        d = mx / (FIVE ? -16.f : -8.f);
        // An all-zero block has d = 0 / -8 = -0, stored as f16 0x8000.  The
        // compiler would fold the (power-of-two) quotient and the f16 conversion
        // into one v_fma_mix with a +0 addend, which turns -0 into +0; keep the
        // f32 quotient as its own value.
        asm volatile("" : "+v"(d));
    }
    const float id = d != 0.f ? 1.f / d : 0.f;
    uint32_t qh = 0;
    uint8_t qs[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        int a, b;
        if constexpr (HAS_M) {
            a = (int)((v[j] - mn) * id + 0.5f);
            b = (int)((v[j + 16] - mn) * id + 0.5f);
            if constexpr (!FIVE) { a = a < 15 ? a : 15; b = b < 15 ? b : 15; }
        } else {
            constexpr float BIAS = FIVE ? 16.5f : 8.5f;
            constexpr int TOP = FIVE ? 31 : 15;
            a = (int)(v[j] * id + BIAS);
            b = (int)(v[j + 16] * id + BIAS);
            a = a < TOP ? a : TOP;
            b = b < TOP ? b : TOP;
        }
        qs[j] = (uint8_t)((a & 15) | ((b & 15) << 4));
        if constexpr (FIVE) qh |= ((uint32_t)(a >> 4) & 1u) << j | ((uint32_t)(b >> 4) & 1u) << (j + 16);
    }
    // 2-byte stores: 18- and 22-byte blocks sit at even, not always 4-aligned, offsets
    unsigned short *o = reinterpret_cast<unsigned short *>(out + blk * BYTES);
    int h = 0;
    o[h++] = (unsigned short)f2h_bits(d);
    if constexpr (HAS_M) o[h++] = (unsigned short)f2h_bits(mn);
    if constexpr (FIVE) {
        o[h++] = (unsigned short)(qh & 0xffffu);
        o[h++] = (unsigned short)(qh >> 16);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) o[h + j] = (unsigned short)(qs[2 * j] | (qs[2 * j + 1] << 8));
}

hipError_t launch_quant_weights(int type, const float *w, int64_t nelem, uint8_t *out, hipStream_t st) {
    switch (type) {
    case TYPE_Q8_0: return launch_quant_act(TYPE_Q8_0, w, 1, nelem, nullptr, nullptr, nullptr, nullptr, out, st);
    case TYPE_Q4_K: {
        const int64_t nb = nelem / QK_K;
        k_quant_w_k45<15><<<dim3((unsigned)((nb * 8 + 255) / 256)), 256, 0, st>>>(w, nb, out);
        break;
    }
    case TYPE_Q5_K: {
        const int64_t nb = nelem / QK_K;
        k_quant_w_k45<31><<<dim3((unsigned)((nb * 8 + 255) / 256)), 256, 0, st>>>(w, nb, out);
        break;
    }
    case TYPE_Q6_K: {
        const int64_t nb = nelem / QK_K;
        k_quant_w_q6k<<<dim3((unsigned)((nb * 16 + 255) / 256)), 256, 0, st>>>(w, nb, out);
        break;
    }
    case TYPE_Q4_0: case TYPE_Q4_1: case TYPE_Q5_0: case TYPE_Q5_1: {
        const int64_t nb = nelem / 32;
        const dim3 grid((unsigned)((nb + 255) / 256));
        if (type == TYPE_Q4_0) k_quant_w_legacy<TYPE_Q4_0><<<grid, 256, 0, st>>>(w, nb, out);
        else if (type == TYPE_Q4_1) k_quant_w_legacy<TYPE_Q4_1><<<grid, 256, 0, st>>>(w, nb, out);
        else if (type == TYPE_Q5_0) k_quant_w_legacy<TYPE_Q5_0><<<grid, 256, 0, st>>>(w, nb, out);
        else k_quant_w_legacy<TYPE_Q5_1><<<grid, 256, 0, st>>>(w, nb, out);
        break;
    }
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lbq
