/*
 * lbq_oracle.c -- CPU restatement of the reference's quantized-linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library under lightbulb_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker or as the
 * timed CPU baseline -- never as a product code path.
 *
 * What it restates
 * ----------------
 * lightbulb's GGUF serving route sends every projection and the LM head
 * through QuantizableLinear::Quantized(QMatMul)::forward
 * (/root/reference/src/model/quantizable_linear.rs:63-69).  The arithmetic
 * behind QMatMul lives in the third-party crate candle-core 0.10.2
 * (/root/reference/Cargo.lock:717-746, reached through candlelight d70a03f,
 * Cargo.lock:956-967), which is not vendored.  Its CPU algorithm is the
 * public ggml/candle k-quants algorithm, restated here from the published
 * block specification:
 *   - activation quantisation to Q8_K (k-quant weights) or Q8_0 (Q8_0
 *     weights): candle k_quants.rs BlockQ8K::from_float / BlockQ8_0::from_float
 *   - the generic (non-SIMD) integer vec_dot for Q8_0.Q8_0, Q4_K.Q8_K,
 *     Q5_K.Q8_K, Q6_K.Q8_K and Q3_K.Q8_K with its 8-lane partial sums,
 *     Q2_K.Q8_K (one integer sum per block, minus dmin * sum(bsum * m)), and for the
 *     32-value legacy blocks Q4_0.Q8_0, Q5_0.Q8_0, Q4_1.Q8_1, Q5_1.Q8_1
 *     (activation quantisation to Q8_1: BlockQ8_1::from_float)
 *   - the k_quants::matmul driver: quantise all M rows, then for each row a
 *     parallel loop over N output columns (rayon, chunks of 128..512)
 *   - dequantisation (GgmlType::to_float; lightbulb's own dequantize_tensor,
 *     /root/reference/src/quantization/mod.rs:158-247) with every float op
 *     rounded separately (Rust never contracts a*b-c into an FMA); this file
 *     must be compiled with -ffp-contract=off
 *   - weight quantisers (ggml quantize_row_*_ref, make_qkx2_quants,
 *     make_qx_quants) used to build fixtures; lightbulb's quantize_tensor
 *     (/root/reference/src/quantization/mod.rs:257-327) calls the
 *     ggml-quants 0.1.0 port of the same routines.
 * Type ids, block sizes and byte sizes follow the GgmlDType table,
 * /root/reference/src/quantization/mod.rs:58-126.
 *
 * Parity pins: see the module docstring of oracle/__init__.py (which checks
 * pin which function).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "lbq_oracle.h"

#define QK_K 256
#define QK8_0 32

typedef struct { uint16_t d; int8_t qs[QK8_0]; } blk_q8_0;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[QK_K / 2]; } blk_q4_k;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[QK_K / 8]; uint8_t qs[QK_K / 2]; } blk_q5_k;
typedef struct { uint8_t ql[QK_K / 2]; uint8_t qh[QK_K / 4]; int8_t scales[QK_K / 16]; uint16_t d; } blk_q6_k;
typedef struct { float d; int8_t qs[QK_K]; int16_t bsums[QK_K / 16]; } blk_q8_k;
typedef struct { uint8_t scales[QK_K / 16]; uint8_t qs[QK_K / 4]; uint16_t d, dmin; } blk_q2_k;
typedef struct { uint8_t hmask[QK_K / 8]; uint8_t qs[QK_K / 4]; uint8_t scales[12]; uint16_t d; } blk_q3_k;
/* 32-value blocks (ggml legacy types) */
typedef struct { uint16_t d; uint8_t qs[16]; } blk_q4_0;
typedef struct { uint16_t d, m; uint8_t qs[16]; } blk_q4_1;
typedef struct { uint16_t d; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_0;
typedef struct { uint16_t d, m; uint8_t qh[4]; uint8_t qs[16]; } blk_q5_1;
typedef struct { uint16_t d, s; int8_t qs[32]; } blk_q8_1;

_Static_assert(sizeof(blk_q8_0) == 34, "q8_0 size");
_Static_assert(sizeof(blk_q4_k) == 144, "q4_k size");
_Static_assert(sizeof(blk_q5_k) == 176, "q5_k size");
_Static_assert(sizeof(blk_q6_k) == 210, "q6_k size");
_Static_assert(sizeof(blk_q2_k) == 84, "q2_k size");
_Static_assert(sizeof(blk_q3_k) == 110, "q3_k size");
_Static_assert(sizeof(blk_q8_k) == 292, "q8_k size");
_Static_assert(sizeof(blk_q4_0) == 18, "q4_0 size");
_Static_assert(sizeof(blk_q4_1) == 20, "q4_1 size");
_Static_assert(sizeof(blk_q5_0) == 22, "q5_0 size");
_Static_assert(sizeof(blk_q5_1) == 24, "q5_1 size");
_Static_assert(sizeof(blk_q8_1) == 36, "q8_1 size");

/* ------------------------------------------------------------------ */
/* type table: reference src/quantization/mod.rs:58-126                */
/* ------------------------------------------------------------------ */
int oracle_block_size(uint32_t type) {
    switch (type) {
    case ORACLE_Q8_0: case ORACLE_Q4_0: case ORACLE_Q4_1: case ORACLE_Q5_0: case ORACLE_Q5_1: case ORACLE_Q8_1: return 32;
    case ORACLE_Q2_K: case ORACLE_Q3_K: case ORACLE_Q4_K: case ORACLE_Q5_K: case ORACLE_Q6_K: case ORACLE_Q8_K: return 256;
    default: return 0;
    }
}

int oracle_type_size(uint32_t type) {
    switch (type) {
    case ORACLE_Q8_0: return 34;
    case ORACLE_Q4_0: return 18;
    case ORACLE_Q4_1: return 20;
    case ORACLE_Q5_0: return 22;
    case ORACLE_Q5_1: return 24;
    case ORACLE_Q8_1: return 36;
    case ORACLE_Q2_K: return 84;
    case ORACLE_Q3_K: return 110;
    case ORACLE_Q4_K: return 144;
    case ORACLE_Q5_K: return 176;
    case ORACLE_Q6_K: return 210;
    case ORACLE_Q8_K: return 292;
    default: return 0;
    }
}

/* ------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32 (the `half` crate's semantics: exact     */
/* widening, round-to-nearest-even narrowing with overflow to inf).    */
/* ------------------------------------------------------------------ */
float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    float f;
    if (exp == 0) {
        /* zero or subnormal: value = man * 2^-24, exact in binary32 */
        f = (float)man * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    if (exp == 31) bits = sign | 0x7f800000u | (man << 13);
    else bits = sign | ((exp + 112u) << 23) | (man << 13);
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN stays NaN */
    if (ax >= 0x47800000u) return (uint16_t)(sign | 0x7c00u);                           /* >= 2^16: inf */
    if (ax < 0x38800000u) {
        /* result is a binary16 subnormal (or rounds up to the smallest normal) */
        uint32_t e = ax >> 23;
        if (e < 102) return (uint16_t)sign; /* below half of the smallest subnormal */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e; /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e16 = (ax >> 23) - 112u;
    uint32_t h = (e16 << 10) | ((ax >> 13) & 0x3ffu);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++; /* carry may reach inf: correct */
    return (uint16_t)(sign | h);
}

/* Rust `f32::round` (half away from zero) followed by a saturating `as i8`. */
static int8_t round_sat_i8(float v) {
    float r = roundf(v);
    if (r != r) return 0;
    if (r > 127.f) return 127;
    if (r < -128.f) return -128;
    return (int8_t)r;
}

/* ggml nearest_int: round-half-even via the 1.5*2^23 trick (|v| < 2^22). */
static int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, 4);
    return (i & 0x007fffff) - 0x00400000;
}

/* ------------------------------------------------------------------ */
/* 6-bit scale/min unpack shared by Q4_K and Q5_K (ggml get_scale_min_k4) */
/* ------------------------------------------------------------------ */
static void get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4));
    }
}

void oracle_unpack_scales_k4(const uint8_t scales[12], uint8_t sc[8], uint8_t mn[8]) {
    for (int j = 0; j < 8; j++) get_scale_min_k4(j, scales, &sc[j], &mn[j]);
}

/* ------------------------------------------------------------------ */
/* Dequantisation (GgmlType::to_float).  Association as in the Rust   */
/* source: d1 = d*sc; m1 = dmin*m; y = d1*q - m1; no FMA.             */
/* ------------------------------------------------------------------ */
static void deq_q8_0(const blk_q8_0 *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    for (int i = 0; i < QK8_0; i++) y[i] = (float)b->qs[i] * d;
}

static void deq_q4_k(const blk_q4_k *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    const float min = oracle_f16_to_f32(b->dmin);
    const uint8_t *q = b->qs;
    int is = 0;
    for (int j = 0; j < QK_K; j += 64) {
        uint8_t sc, m;
        get_scale_min_k4(is + 0, b->scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = min * (float)m;
        get_scale_min_k4(is + 1, b->scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; l++) *y++ = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; l++) *y++ = d2 * (float)(q[l] >> 4) - m2;
        q += 32;
        is += 2;
    }
}

static void deq_q5_k(const blk_q5_k *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    const float min = oracle_f16_to_f32(b->dmin);
    const uint8_t *ql = b->qs;
    const uint8_t *qh = b->qh;
    int is = 0;
    uint8_t u1 = 1, u2 = 2;
    for (int j = 0; j < QK_K; j += 64) {
        uint8_t sc, m;
        get_scale_min_k4(is + 0, b->scales, &sc, &m);
        const float d1 = d * (float)sc, m1 = min * (float)m;
        get_scale_min_k4(is + 1, b->scales, &sc, &m);
        const float d2 = d * (float)sc, m2 = min * (float)m;
        for (int l = 0; l < 32; l++) *y++ = d1 * (float)((ql[l] & 0xF) + (qh[l] & u1 ? 16 : 0)) - m1;
        for (int l = 0; l < 32; l++) *y++ = d2 * (float)((ql[l] >> 4) + (qh[l] & u2 ? 16 : 0)) - m2;
        ql += 32;
        is += 2;
        u1 <<= 2;
        u2 <<= 2;
    }
}

static void deq_q6_k(const blk_q6_k *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    const uint8_t *ql = b->ql;
    const uint8_t *qh = b->qh;
    const int8_t *sc = b->scales;
    for (int n = 0; n < QK_K; n += 128) {
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
            const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
            y[l + 0] = d * (float)sc[is + 0] * (float)q1;
            y[l + 32] = d * (float)sc[is + 2] * (float)q2;
            y[l + 64] = d * (float)sc[is + 4] * (float)q3;
            y[l + 96] = d * (float)sc[is + 6] * (float)q4;
        }
        y += 128;
        ql += 64;
        qh += 32;
        sc += 8;
    }
}

static void deq_q8_k(const blk_q8_k *b, float *y) {
    for (int i = 0; i < QK_K; i++) y[i] = b->d * (float)b->qs[i];
}

/* Q2_K (candle BlockQ2K::to_float): element 128h + 32s + 16t + l (h < 2, s < 4,
 * t < 2, l < 16) is code (qs[32h + 16t + l] >> 2s) & 3 of sub-block j = 8h + 2s + t,
 * whose scale byte holds the 4-bit scale (low) and min (high):
 * y = (d * sc) * q - (dmin * m). */
static void deq_q2_k(const blk_q2_k *b, float *y) {
    const float d = oracle_f16_to_f32(b->d), dmin = oracle_f16_to_f32(b->dmin);
    for (int h = 0; h < 2; h++)
        for (int s = 0; s < 4; s++)
            for (int t = 0; t < 2; t++) {
                const uint8_t sc = b->scales[8 * h + 2 * s + t];
                const float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                for (int l = 0; l < 16; l++) {
                    const int q = (b->qs[32 * h + 16 * t + l] >> (2 * s)) & 3;
                    *y++ = dl * (float)q - ml;
                }
            }
}

/* Q3_K 6-bit sub-block scales (ggml's aux rearrangement of the 12 bytes):
 * scale j = low 4 bits from scales[j % 8] (nibble j / 8) | 2 high bits from
 * scales[8 + j % 4] (bits 2*(j / 4)), minus 32. */
static int q3k_scale(const uint8_t sc[12], int j) {
    const int lo = (sc[j % 8] >> (4 * (j / 8))) & 0xF;
    const int hi = (sc[8 + j % 4] >> (2 * (j / 4))) & 3;
    return (lo | (hi << 4)) - 32;
}

/* Q3_K (candle BlockQ3K::to_float): element 128h + 32s + 16t + l has low bits
 * (qs[32h + 16t + l] >> 2s) & 3, minus 4 unless bit 4h + s of hmask[16t + l] is
 * set; sub-block j = 8h + 2s + t: y = (d * scale_j) * q. */
static void deq_q3_k(const blk_q3_k *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    for (int h = 0; h < 2; h++)
        for (int s = 0; s < 4; s++)
            for (int t = 0; t < 2; t++) {
                const float dl = d * (float)q3k_scale(b->scales, 8 * h + 2 * s + t);
                for (int l = 0; l < 16; l++) {
                    const int lo = (b->qs[32 * h + 16 * t + l] >> (2 * s)) & 3;
                    const int q = lo - ((b->hmask[16 * t + l] >> (4 * h + s)) & 1 ? 0 : 4);
                    *y++ = dl * (float)q;
                }
            }
}

/* 32-value blocks (candle k_quants to_float): element j from the low nibble of
 * qs[j], element j + 16 from its high nibble; Q5 fifth bits from the u32 qh,
 * bit j (element j) and bit j + 16 (element j + 16). */
static uint32_t qh_u32(const uint8_t qh[4]) {
    return (uint32_t)qh[0] | ((uint32_t)qh[1] << 8) | ((uint32_t)qh[2] << 16) | ((uint32_t)qh[3] << 24);
}

static void deq_q4_0(const blk_q4_0 *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    for (int j = 0; j < 16; j++) {
        y[j] = (float)((int)(b->qs[j] & 0xF) - 8) * d;
        y[j + 16] = (float)((int)(b->qs[j] >> 4) - 8) * d;
    }
}

static void deq_q4_1(const blk_q4_1 *b, float *y) {
    const float d = oracle_f16_to_f32(b->d), m = oracle_f16_to_f32(b->m);
    for (int j = 0; j < 16; j++) {
        y[j] = (float)(b->qs[j] & 0xF) * d + m;
        y[j + 16] = (float)(b->qs[j] >> 4) * d + m;
    }
}

static void deq_q5_0(const blk_q5_0 *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    const uint32_t qh = qh_u32(b->qh);
    for (int j = 0; j < 16; j++) {
        const uint32_t h0 = ((qh >> j) << 4) & 0x10, h1 = (qh >> (j + 12)) & 0x10;
        y[j] = (float)((int)((b->qs[j] & 0xF) | h0) - 16) * d;
        y[j + 16] = (float)((int)((b->qs[j] >> 4) | h1) - 16) * d;
    }
}

static void deq_q5_1(const blk_q5_1 *b, float *y) {
    const float d = oracle_f16_to_f32(b->d), m = oracle_f16_to_f32(b->m);
    const uint32_t qh = qh_u32(b->qh);
    for (int j = 0; j < 16; j++) {
        const uint32_t h0 = ((qh >> j) << 4) & 0x10, h1 = (qh >> (j + 12)) & 0x10;
        y[j] = (float)((b->qs[j] & 0xF) | h0) * d + m;
        y[j + 16] = (float)((b->qs[j] >> 4) | h1) * d + m;
    }
}

static void deq_q8_1(const blk_q8_1 *b, float *y) {
    const float d = oracle_f16_to_f32(b->d);
    for (int j = 0; j < 32; j++) y[j] = (float)b->qs[j] * d;
}

int oracle_dequantize(uint32_t type, const void *blocks, int64_t nblocks, float *out) {
    const uint8_t *p = (const uint8_t *)blocks;
    const int ts = oracle_type_size(type), bs = oracle_block_size(type);
    if (!ts) return -1;
    for (int64_t i = 0; i < nblocks; i++) {
        const void *b = p + i * ts;
        float *y = out + i * bs;
        switch (type) {
        case ORACLE_Q8_0: deq_q8_0((const blk_q8_0 *)b, y); break;
        case ORACLE_Q4_K: deq_q4_k((const blk_q4_k *)b, y); break;
        case ORACLE_Q5_K: deq_q5_k((const blk_q5_k *)b, y); break;
        case ORACLE_Q6_K: deq_q6_k((const blk_q6_k *)b, y); break;
        case ORACLE_Q8_K: deq_q8_k((const blk_q8_k *)b, y); break;
        case ORACLE_Q4_0: deq_q4_0((const blk_q4_0 *)b, y); break;
        case ORACLE_Q4_1: deq_q4_1((const blk_q4_1 *)b, y); break;
        case ORACLE_Q5_0: deq_q5_0((const blk_q5_0 *)b, y); break;
        case ORACLE_Q5_1: deq_q5_1((const blk_q5_1 *)b, y); break;
        case ORACLE_Q8_1: deq_q8_1((const blk_q8_1 *)b, y); break;
        case ORACLE_Q2_K: deq_q2_k((const blk_q2_k *)b, y); break;
        case ORACLE_Q3_K: deq_q3_k((const blk_q3_k *)b, y); break;
        }
    }
    return 0;
}

/* ------------------------------------------------------------------ */
/* Activation quantisation                                              */
/* ------------------------------------------------------------------ */
/* candle k_quants.rs BlockQ8K::from_float: the signed value of largest |x|
 * (first one on ties, NaN never selected) sets iscale = -128/max;
 * q = min(127, round(iscale*x)); d = 1/iscale; bsums = sums of 16. */
static void quant_row_q8_k(const float *x, blk_q8_k *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, x += QK_K, y++) {
        float max = 0.f, amax = 0.f;
        for (int j = 0; j < QK_K; j++) {
            const float ax = fabsf(x[j]);
            if (amax < ax) {
                amax = ax;
                max = x[j];
            }
        }
        if (amax == 0.f) {
            y->d = 0.f;
            memset(y->qs, 0, sizeof(y->qs));
            memset(y->bsums, 0, sizeof(y->bsums));
            continue;
        }
        const float iscale = -128.f / max;
        for (int j = 0; j < QK_K; j++) {
            float v = roundf(iscale * x[j]);
            v = fminf(v, 127.f); /* NaN -> 127, like Rust's f32::min */
            y->qs[j] = round_sat_i8(v);
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int sum = 0;
            for (int l = 0; l < 16; l++) sum += y->qs[j * 16 + l];
            y->bsums[j] = (int16_t)sum;
        }
        y->d = 1.f / iscale;
    }
}

/* candle k_quants.rs BlockQ8_0::from_float: d = amax/127 (amax ignores NaN),
 * id = 1/d (0 if d==0), q = round(x*id) computed from the unrounded d,
 * stored scale = f16(d). */
static void quant_row_q8_0(const float *x, blk_q8_0 *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, x += QK8_0, y++) {
        float amax = 0.f;
        for (int j = 0; j < QK8_0; j++) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        y->d = oracle_f32_to_f16(d);
        for (int j = 0; j < QK8_0; j++) y->qs[j] = round_sat_i8(x[j] * id);
    }
}

/* candle BlockQ8_1::from_float: as Q8_0 (d = amax/127, q = round(x / d) with
 * the unrounded d, stored f16(d)), plus s = f16(sum of the codes) * f16(d) taken
 * in f16 (the half crate multiplies in f32 and rounds back). */
static void quant_row_q8_1(const float *x, blk_q8_1 *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, x += 32, y++) {
        float amax = 0.f;
        for (int j = 0; j < 32; j++) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax / 127.f;
        const float id = d != 0.f ? 1.f / d : 0.f;
        y->d = oracle_f32_to_f16(d);
        int sum = 0;
        for (int j = 0; j < 32; j++) {
            y->qs[j] = round_sat_i8(x[j] * id);
            sum += y->qs[j];
        }
        y->s = oracle_f32_to_f16(oracle_f16_to_f32(oracle_f32_to_f16((float)sum)) * oracle_f16_to_f32(y->d));
    }
}

int oracle_quantize_act(uint32_t type, const float *x, int64_t m, int64_t k, void *out) {
    if (type == ORACLE_Q8_1) {
        if (k % 32) return -1;
        quant_row_q8_1(x, (blk_q8_1 *)out, m * (k / 32));
        return 0;
    }
    if (type == ORACLE_Q8_K) {
        if (k % QK_K) return -1;
        quant_row_q8_k(x, (blk_q8_k *)out, m * (k / QK_K));
        return 0;
    }
    if (type == ORACLE_Q8_0) {
        if (k % QK8_0) return -1;
        quant_row_q8_0(x, (blk_q8_0 *)out, m * (k / QK8_0));
        return 0;
    }
    return -1;
}

/* ------------------------------------------------------------------ */
/* vec_dot: the generic (non-SIMD) candle/ggml bodies.  n = K.          */
/* ------------------------------------------------------------------ */
static float vec_dot_q8_0(int64_t n, const blk_q8_0 *xs, const blk_q8_0 *ys) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / QK8_0; i++) {
        int sumi = 0;
        for (int j = 0; j < QK8_0; j++) sumi += (int)xs[i].qs[j] * (int)ys[i].qs[j];
        sumf += (float)sumi * oracle_f16_to_f32(xs[i].d) * oracle_f16_to_f32(ys[i].d);
    }
    return sumf;
}

static float vec_dot_q4_k(int64_t n, const blk_q4_k *xs, const blk_q8_k *ys) {
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8] = {0};
    int32_t aux32[8];
    float sumf = 0.f;
    for (int64_t i = 0; i < n / QK_K; i++) {
        const blk_q4_k *x = &xs[i];
        const blk_q8_k *y = &ys[i];
        const uint8_t *q4 = x->qs;
        int8_t *a = aux8;
        for (int j = 0; j < QK_K / 64; j++) {
            for (int l = 0; l < 32; l++) a[l] = (int8_t)(q4[l] & 0xF);
            a += 32;
            for (int l = 0; l < 32; l++) a[l] = (int8_t)(q4[l] >> 4);
            a += 32;
            q4 += 32;
        }
        uint8_t sc[8], mn[8];
        oracle_unpack_scales_k4(x->scales, sc, mn);
        int sumi = 0;
        for (int j = 0; j < QK_K / 16; j++) sumi += (int)y->bsums[j] * (int)mn[j / 2];
        memset(aux32, 0, sizeof(aux32));
        const int8_t *q8 = y->qs;
        a = aux8;
        for (int j = 0; j < 8; j++) {
            const int32_t scale = sc[j];
            for (int t = 0; t < 4; t++) {
                for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; l++) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = oracle_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        const float dmin = oracle_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float s = 0.f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}

static float vec_dot_q5_k(int64_t n, const blk_q5_k *xs, const blk_q8_k *ys) {
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8] = {0};
    int32_t aux32[8];
    float sumf = 0.f;
    for (int64_t i = 0; i < n / QK_K; i++) {
        const blk_q5_k *x = &xs[i];
        const blk_q8_k *y = &ys[i];
        const uint8_t *q5 = x->qs;
        const uint8_t *hm = x->qh;
        int8_t *a = aux8;
        uint8_t m = 1;
        for (int j = 0; j < QK_K / 64; j++) {
            for (int l = 0; l < 32; l++) a[l] = (int8_t)((q5[l] & 0xF) + (hm[l] & m ? 16 : 0));
            a += 32;
            m <<= 1;
            for (int l = 0; l < 32; l++) a[l] = (int8_t)((q5[l] >> 4) + (hm[l] & m ? 16 : 0));
            a += 32;
            m <<= 1;
            q5 += 32;
        }
        uint8_t sc[8], mn[8];
        oracle_unpack_scales_k4(x->scales, sc, mn);
        int sumi = 0;
        for (int j = 0; j < QK_K / 16; j++) sumi += (int)y->bsums[j] * (int)mn[j / 2];
        memset(aux32, 0, sizeof(aux32));
        const int8_t *q8 = y->qs;
        a = aux8;
        for (int j = 0; j < 8; j++) {
            const int32_t scale = sc[j];
            for (int t = 0; t < 4; t++) {
                for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; l++) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = oracle_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
        const float dmin = oracle_f16_to_f32(x->dmin) * y->d;
        sumf -= dmin * (float)sumi;
    }
    float s = 0.f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return sumf + s;
}

static float vec_dot_q6_k(int64_t n, const blk_q6_k *xs, const blk_q8_k *ys) {
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8] = {0};
    int32_t aux32[8];
    for (int64_t i = 0; i < n / QK_K; i++) {
        const blk_q6_k *x = &xs[i];
        const blk_q8_k *y = &ys[i];
        const uint8_t *q4 = x->ql;
        const uint8_t *qh = x->qh;
        int8_t *a = aux8;
        for (int j = 0; j < QK_K; j += 128) {
            for (int l = 0; l < 32; l++) {
                a[l + 0] = (int8_t)((int)((q4[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32);
                a[l + 32] = (int8_t)((int)((q4[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32);
                a[l + 64] = (int8_t)((int)((q4[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32);
                a[l + 96] = (int8_t)((int)((q4[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32);
            }
            a += 128;
            q4 += 64;
            qh += 32;
        }
        memset(aux32, 0, sizeof(aux32));
        const int8_t *q8 = y->qs;
        a = aux8;
        for (int j = 0; j < QK_K / 16; j++) {
            const int32_t scale = x->scales[j];
            for (int t = 0; t < 2; t++) {
                for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; l++) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = oracle_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
    }
    float s = 0.f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

/* the generic candle/ggml bodies of the 32-block vec_dots */
/* ggml/candle generic Q2_K.Q8_K: per block an exact integer sum of
 * sc_j * (codes . x) over the 16 sub-blocks and summs = sum(bsum_j * m_j);
 * sumf += (y.d * d) * isum - (y.d * dmin) * summs. */
static float vec_dot_q2_k(int64_t n, const blk_q2_k *xs, const blk_q8_k *ys) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / QK_K; i++) {
        const blk_q2_k *x = &xs[i];
        const blk_q8_k *y = &ys[i];
        int summs = 0;
        for (int j = 0; j < 16; j++) summs += (int)y->bsums[j] * (int)(x->scales[j] >> 4);
        const float dall = y->d * oracle_f16_to_f32(x->d);
        const float dmin = y->d * oracle_f16_to_f32(x->dmin);
        int isum = 0, is = 0;
        const uint8_t *q2 = x->qs;
        const int8_t *q8 = y->qs;
        for (int h = 0; h < 2; h++) {
            for (int s = 0; s < 4; s++) {
                for (int t = 0; t < 2; t++) {
                    const int d = x->scales[is++] & 0xF;
                    int isuml = 0;
                    for (int l = 0; l < 16; l++) isuml += (int)q8[16 * t + l] * ((q2[16 * t + l] >> (2 * s)) & 3);
                    isum += d * isuml;
                }
                q8 += 32;
            }
            q2 += 32;
        }
        sumf += dall * (float)isum - dmin * (float)summs;
    }
    return sumf;
}

/* ggml/candle generic Q3_K.Q8_K: codes in [-4, 3] expanded to aux8, then the
 * same 8-lane int32 sums scaled per sub-block as Q6_K. */
static float vec_dot_q3_k(int64_t n, const blk_q3_k *xs, const blk_q8_k *ys) {
    int8_t aux8[QK_K];
    int16_t aux16[8];
    float sums[8] = {0};
    int32_t aux32[8];
    for (int64_t i = 0; i < n / QK_K; i++) {
        const blk_q3_k *x = &xs[i];
        const blk_q8_k *y = &ys[i];
        const uint8_t *q3 = x->qs;
        int8_t *a = aux8;
        uint8_t m = 1;
        for (int h = 0; h < 2; h++) {
            for (int s = 0; s < 4; s++) {
                for (int l = 0; l < 32; l++) a[l] = (int8_t)((q3[l] >> (2 * s)) & 3);
                for (int l = 0; l < 32; l++) a[l] = (int8_t)(a[l] - ((x->hmask[l] & m) ? 0 : 4));
                a += 32;
                m = (uint8_t)(m << 1);
            }
            q3 += 32;
        }
        memset(aux32, 0, sizeof(aux32));
        const int8_t *q8 = y->qs;
        a = aux8;
        for (int j = 0; j < QK_K / 16; j++) {
            const int32_t scale = q3k_scale(x->scales, j);
            for (int t = 0; t < 2; t++) {
                for (int l = 0; l < 8; l++) aux16[l] = (int16_t)(q8[l] * a[l]);
                for (int l = 0; l < 8; l++) aux32[l] += scale * aux16[l];
                q8 += 8;
                a += 8;
            }
        }
        const float d = oracle_f16_to_f32(x->d) * y->d;
        for (int l = 0; l < 8; l++) sums[l] += d * (float)aux32[l];
    }
    float s = 0.f;
    for (int l = 0; l < 8; l++) s += sums[l];
    return s;
}

static float vec_dot_q4_0(int64_t n, const blk_q4_0 *xs, const blk_q8_0 *ys) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / 32; i++) {
        int sumi = 0;
        for (int j = 0; j < 16; j++) {
            const int v0 = (int)(xs[i].qs[j] & 0xF) - 8, v1 = (int)(xs[i].qs[j] >> 4) - 8;
            sumi += v0 * (int)ys[i].qs[j] + v1 * (int)ys[i].qs[j + 16];
        }
        sumf += (float)sumi * oracle_f16_to_f32(xs[i].d) * oracle_f16_to_f32(ys[i].d);
    }
    return sumf;
}

static float vec_dot_q4_1(int64_t n, const blk_q4_1 *xs, const blk_q8_1 *ys) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / 32; i++) {
        int sumi = 0;
        for (int j = 0; j < 16; j++) {
            const int v0 = xs[i].qs[j] & 0xF, v1 = xs[i].qs[j] >> 4;
            sumi += v0 * (int)ys[i].qs[j] + v1 * (int)ys[i].qs[j + 16];
        }
        sumf += (oracle_f16_to_f32(xs[i].d) * oracle_f16_to_f32(ys[i].d)) * (float)sumi +
                oracle_f16_to_f32(xs[i].m) * oracle_f16_to_f32(ys[i].s);
    }
    return sumf;
}

static float vec_dot_q5_0(int64_t n, const blk_q5_0 *xs, const blk_q8_0 *ys) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / 32; i++) {
        const uint32_t qh = qh_u32(xs[i].qh);
        int sumi = 0;
        for (int j = 0; j < 16; j++) {
            const uint32_t h0 = ((qh >> j) << 4) & 0x10, h1 = (qh >> (j + 12)) & 0x10;
            const int v0 = (int)((xs[i].qs[j] & 0xF) | h0) - 16, v1 = (int)((xs[i].qs[j] >> 4) | h1) - 16;
            sumi += v0 * (int)ys[i].qs[j] + v1 * (int)ys[i].qs[j + 16];
        }
        sumf += (oracle_f16_to_f32(xs[i].d) * oracle_f16_to_f32(ys[i].d)) * (float)sumi;
    }
    return sumf;
}

static float vec_dot_q5_1(int64_t n, const blk_q5_1 *xs, const blk_q8_1 *ys) {
    float sumf = 0.f;
    for (int64_t i = 0; i < n / 32; i++) {
        const uint32_t qh = qh_u32(xs[i].qh);
        int sumi = 0;
        for (int j = 0; j < 16; j++) {
            const uint32_t h0 = ((qh >> j) << 4) & 0x10, h1 = (qh >> (j + 12)) & 0x10;
            const int v0 = (int)((xs[i].qs[j] & 0xF) | h0), v1 = (int)((xs[i].qs[j] >> 4) | h1);
            sumi += v0 * (int)ys[i].qs[j] + v1 * (int)ys[i].qs[j + 16];
        }
        sumf += (oracle_f16_to_f32(xs[i].d) * oracle_f16_to_f32(ys[i].d)) * (float)sumi +
                oracle_f16_to_f32(xs[i].m) * oracle_f16_to_f32(ys[i].s);
    }
    return sumf;
}

uint32_t oracle_vec_dot_type(uint32_t type) {
    switch (type) {
    case ORACLE_Q8_0: case ORACLE_Q4_0: case ORACLE_Q5_0: return ORACLE_Q8_0;
    case ORACLE_Q4_1: case ORACLE_Q5_1: return ORACLE_Q8_1;
    case ORACLE_Q2_K: case ORACLE_Q3_K: case ORACLE_Q4_K: case ORACLE_Q5_K: case ORACLE_Q6_K: return ORACLE_Q8_K;
    default: return 0;
    }
}

int oracle_vec_dot(uint32_t type, int64_t k, const void *wrow, const void *xrow, float *out) {
    switch (type) {
    case ORACLE_Q4_0: *out = vec_dot_q4_0(k, (const blk_q4_0 *)wrow, (const blk_q8_0 *)xrow); return 0;
    case ORACLE_Q4_1: *out = vec_dot_q4_1(k, (const blk_q4_1 *)wrow, (const blk_q8_1 *)xrow); return 0;
    case ORACLE_Q5_0: *out = vec_dot_q5_0(k, (const blk_q5_0 *)wrow, (const blk_q8_0 *)xrow); return 0;
    case ORACLE_Q5_1: *out = vec_dot_q5_1(k, (const blk_q5_1 *)wrow, (const blk_q8_1 *)xrow); return 0;
    case ORACLE_Q8_0: *out = vec_dot_q8_0(k, (const blk_q8_0 *)wrow, (const blk_q8_0 *)xrow); return 0;
    case ORACLE_Q4_K: *out = vec_dot_q4_k(k, (const blk_q4_k *)wrow, (const blk_q8_k *)xrow); return 0;
    case ORACLE_Q5_K: *out = vec_dot_q5_k(k, (const blk_q5_k *)wrow, (const blk_q8_k *)xrow); return 0;
    case ORACLE_Q6_K: *out = vec_dot_q6_k(k, (const blk_q6_k *)wrow, (const blk_q8_k *)xrow); return 0;
    case ORACLE_Q2_K: *out = vec_dot_q2_k(k, (const blk_q2_k *)wrow, (const blk_q8_k *)xrow); return 0;
    case ORACLE_Q3_K: *out = vec_dot_q3_k(k, (const blk_q3_k *)wrow, (const blk_q8_k *)xrow); return 0;
    default: return -1;
    }
}

/* ------------------------------------------------------------------ */
/* k_quants::matmul driver: quantise the M activation rows, then for    */
/* each row split the N output columns over threads in chunks (rayon    */
/* with_min_len(128).with_max_len(512)); here a shared chunk counter.   */
/* ------------------------------------------------------------------ */
typedef struct {
    uint32_t type;
    const uint8_t *w;
    int64_t n, k;
    const uint8_t *xq;
    float *y;
    int64_t row;
    int64_t chunk;
    volatile int64_t next;
    pthread_mutex_t mu;
} mm_job;

static void *mm_worker(void *arg) {
    mm_job *j = (mm_job *)arg;
    const int64_t w_row_bytes = (j->k / oracle_block_size(j->type)) * oracle_type_size(j->type);
    const uint32_t vt = oracle_vec_dot_type(j->type);
    const int64_t x_row_bytes = (j->k / oracle_block_size(vt)) * oracle_type_size(vt);
    const uint8_t *xrow = j->xq + j->row * x_row_bytes;
    float *dst = j->y + j->row * j->n;
    for (;;) {
        pthread_mutex_lock(&j->mu);
        const int64_t c0 = j->next;
        j->next = c0 + j->chunk;
        pthread_mutex_unlock(&j->mu);
        if (c0 >= j->n) break;
        const int64_t c1 = c0 + j->chunk < j->n ? c0 + j->chunk : j->n;
        for (int64_t col = c0; col < c1; col++) oracle_vec_dot(j->type, j->k, j->w + col * w_row_bytes, xrow, &dst[col]);
    }
    return NULL;
}

int oracle_qmatmul(uint32_t type, const void *w, int64_t n, int64_t k, const float *x, int64_t m, float *y, int nthreads) {
    const uint32_t vt = oracle_vec_dot_type(type);
    if (!vt) return -1;
    if (k % oracle_block_size(type)) return -1;
    if (m == 0 || n == 0) return 0;
    const int64_t x_row_bytes = (k / oracle_block_size(vt)) * oracle_type_size(vt);
    uint8_t *xq = (uint8_t *)malloc((size_t)(m * x_row_bytes));
    if (!xq) return -2;
    oracle_quantize_act(vt, x, m, k, xq);
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    pthread_t th[256];
    for (int64_t row = 0; row < m; row++) {
        mm_job job;
        job.type = type;
        job.w = (const uint8_t *)w;
        job.n = n;
        job.k = k;
        job.xq = xq;
        job.y = y;
        job.row = row;
        job.chunk = 256; /* inside rayon's [128, 512] bounds */
        job.next = 0;
        pthread_mutex_init(&job.mu, NULL);
        if (nthreads == 1) {
            mm_worker(&job);
        } else {
            for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, mm_worker, &job);
            for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
        }
        pthread_mutex_destroy(&job.mu);
    }
    free(xq);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Weight quantisers (ggml quantize_row_{q8_0,q4_K,q5_K,q6_K}_ref).     */
/* Fixture generation only: the kernels consume whatever valid blocks   */
/* they are given, so these are not on the parity-critical path.        */
/* ------------------------------------------------------------------ */
static float make_qkx2_quants(int n, int nmax, const float *x, const float *weights, uint8_t *L, float *the_min,
                              uint8_t *Laux, float rmin, float rdelta, int nstep) {
    float min = x[0], max = x[0];
    float sum_w = weights[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < min) min = x[i];
        if (x[i] > max) max = x[i];
        const float w = weights[i];
        sum_w += w;
        sum_x += w * x[i];
    }
    if (min > 0) min = 0;
    if (max == min) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *the_min = -min;
        return 0.f;
    }
    float iscale = (float)nmax / (max - min);
    float scale = 1.f / iscale;
    float best_mad = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * (x[i] - min));
        L[i] = (uint8_t)(l < 0 ? 0 : l > nmax ? nmax : l);
        float diff = scale * (float)L[i] + min - x[i];
        diff = diff * diff;
        best_mad += weights[i] * diff;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (max - min);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * (x[i] - min));
            l = l < 0 ? 0 : l > nmax ? nmax : l;
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
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * (float)Laux[i] + this_min - x[i];
                diff = diff * diff;
                mad += weights[i] * diff;
            }
            if (mad < best_mad) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best_mad = mad;
                scale = this_scale;
                min = this_min;
            }
        }
    }
    *the_min = -min;
    return scale;
}

static void quantize_q4_k_or_q5_k(const float *x, uint8_t *blk, int nmax) {
    /* nmax = 15 (Q4_K) or 31 (Q5_K) */
    uint8_t L[QK_K], Laux[32];
    float weights[32], mins[8], scales[8];
    uint8_t *bscales = blk + 4;
    memset(blk, 0, nmax == 15 ? 144 : 176);
    float max_scale = 0, max_min = 0;
    for (int j = 0; j < 8; ++j) {
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += x[32 * j + l] * x[32 * j + l];
        const float av_x = sqrtf(sum_x2 / 32.f);
        for (int l = 0; l < 32; ++l) weights[l] = av_x + fabsf(x[32 * j + l]);
        if (nmax == 15)
            scales[j] = make_qkx2_quants(32, 15, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -1.f, 0.1f, 20);
        else
            scales[j] = make_qkx2_quants(32, 31, x + 32 * j, weights, L + 32 * j, &mins[j], Laux, -0.5f, 0.1f, 15);
        if (scales[j] > max_scale) max_scale = scales[j];
        if (mins[j] > max_min) max_min = mins[j];
    }
    const float inv_scale = max_scale > 0 ? 63.f / max_scale : 0.f;
    const float inv_min = max_min > 0 ? 63.f / max_min : 0.f;
    for (int j = 0; j < 8; ++j) {
        int ls = nearest_int(inv_scale * scales[j]) & 255; /* ggml stores into uint8_t first */
        int lm = nearest_int(inv_min * mins[j]) & 255;
        ls = ls > 63 ? 63 : ls;
        lm = lm > 63 ? 63 : lm;
        if (j < 4) {
            bscales[j] = (uint8_t)ls;
            bscales[j + 4] = (uint8_t)lm;
        } else {
            bscales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
            bscales[j - 4] |= (uint8_t)((ls >> 4) << 6);
            bscales[j - 0] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t dh = oracle_f32_to_f16(max_scale / 63.f);
    const uint16_t dminh = oracle_f32_to_f16(max_min / 63.f);
    memcpy(blk + 0, &dh, 2);
    memcpy(blk + 2, &dminh, 2);
    for (int j = 0; j < 8; ++j) {
        uint8_t sc, m;
        get_scale_min_k4(j, bscales, &sc, &m);
        const float d = oracle_f16_to_f32(dh) * (float)sc;
        if (d == 0.f) continue;
        const float dm = oracle_f16_to_f32(dminh) * (float)m;
        for (int ii = 0; ii < 32; ++ii) {
            int l = nearest_int((x[32 * j + ii] + dm) / d);
            L[32 * j + ii] = (uint8_t)(l < 0 ? 0 : l > nmax ? nmax : l);
        }
    }
    if (nmax == 15) {
        uint8_t *q = blk + 16;
        for (int j = 0; j < QK_K; j += 64) {
            for (int l = 0; l < 32; ++l) q[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
            q += 32;
        }
    } else {
        uint8_t *qh = blk + 16;
        uint8_t *ql = blk + 48;
        uint8_t m1 = 1, m2 = 2;
        for (int n = 0; n < QK_K; n += 64) {
            for (int j = 0; j < 32; ++j) {
                int l1 = L[n + j];
                if (l1 > 15) {
                    l1 -= 16;
                    qh[j] |= m1;
                }
                int l2 = L[n + j + 32];
                if (l2 > 15) {
                    l2 -= 16;
                    qh[j] |= m2;
                }
                ql[j] = (uint8_t)(l1 | (l2 << 4));
            }
            m1 <<= 2;
            m2 <<= 2;
            ql += 32;
        }
    }
}

static float make_qx_quants_rmse1(int n, int nmax, const float *x, int8_t *L) {
    float max = 0, amax = 0;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    if (amax < 1e-15f) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.f;
    }
    float iscale = -(float)nmax / max;
    float sumlx = 0, suml2 = 0;
    for (int i = 0; i < n; ++i) {
        int l = nearest_int(iscale * x[i]);
        l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
        L[i] = (int8_t)(l + nmax);
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
        for (int i = 0; i < n; ++i) {
            int l = nearest_int(iscale * x[i]);
            l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0 && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i) {
                int l = nearest_int(iscale * x[i]);
                l = l < -nmax ? -nmax : l > nmax - 1 ? nmax - 1 : l;
                L[i] = (int8_t)(nmax + l);
            }
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

static void quantize_q6_k(const float *x, blk_q6_k *y) {
    int8_t L[QK_K];
    float scales[QK_K / 16];
    float max_scale = 0, max_abs_scale = 0;
    for (int ib = 0; ib < QK_K / 16; ++ib) {
        const float scale = make_qx_quants_rmse1(16, 32, x + 16 * ib, L + 16 * ib);
        scales[ib] = scale;
        const float abs_scale = fabsf(scale);
        if (abs_scale > max_abs_scale) {
            max_abs_scale = abs_scale;
            max_scale = scale;
        }
    }
    memset(y, 0, sizeof(*y));
    if (max_abs_scale < 1e-15f) return;
    const float iscale = -128.f / max_scale;
    y->d = oracle_f32_to_f16(1.f / iscale);
    for (int ib = 0; ib < QK_K / 16; ++ib) {
        int v = nearest_int(iscale * scales[ib]);
        y->scales[ib] = (int8_t)(v > 127 ? 127 : v);
    }
    for (int j = 0; j < QK_K / 16; ++j) {
        const float d = oracle_f16_to_f32(y->d) * (float)y->scales[j];
        if (d == 0.f) continue;
        for (int ii = 0; ii < 16; ++ii) {
            int l = nearest_int(x[16 * j + ii] / d);
            l = l < -32 ? -32 : l > 31 ? 31 : l;
            L[16 * j + ii] = (int8_t)(l + 32);
        }
    }
    uint8_t *ql = y->ql;
    uint8_t *qh = y->qh;
    for (int j = 0; j < QK_K; j += 128) {
        for (int l = 0; l < 32; ++l) {
            const uint8_t q1 = L[j + l + 0] & 0xF;
            const uint8_t q2 = L[j + l + 32] & 0xF;
            const uint8_t q3 = L[j + l + 64] & 0xF;
            const uint8_t q4 = L[j + l + 96] & 0xF;
            ql[l + 0] = (uint8_t)(q1 | (q3 << 4));
            ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
            qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                              ((L[j + l + 96] >> 4) << 6));
        }
        ql += 64;
        qh += 32;
    }
}

/* ggml quantize_row_q4_0/q4_1/q5_0/q5_1 reference quantisers (fixtures) */
static void quantize_q4_0(const float *x, blk_q4_0 *y) {
    float amax = 0.f, max = 0.f;
    for (int j = 0; j < 32; j++) {
        const float v = x[j];
        if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
    }
    const float d = max / -8.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    y->d = oracle_f32_to_f16(d);
    for (int j = 0; j < 16; j++) {
        int8_t a = (int8_t)(x[j] * id + 8.5f), b2 = (int8_t)(x[j + 16] * id + 8.5f);
        const uint8_t xi0 = (uint8_t)(a < 15 ? a : 15), xi1 = (uint8_t)(b2 < 15 ? b2 : 15);
        y->qs[j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}

static void minmax32(const float *x, float *mn, float *mx) {
    float lo = x[0], hi = x[0];
    for (int j = 1; j < 32; j++) {
        if (x[j] < lo) lo = x[j];
        if (x[j] > hi) hi = x[j];
    }
    *mn = lo;
    *mx = hi;
}

static void quantize_q4_1(const float *x, blk_q4_1 *y) {
    float min, max;
    minmax32(x, &min, &max);
    const float d = (max - min) / 15.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    y->d = oracle_f32_to_f16(d);
    y->m = oracle_f32_to_f16(min);
    for (int j = 0; j < 16; j++) {
        int8_t a = (int8_t)((x[j] - min) * id + 0.5f), b2 = (int8_t)((x[j + 16] - min) * id + 0.5f);
        const uint8_t xi0 = (uint8_t)(a < 15 ? a : 15), xi1 = (uint8_t)(b2 < 15 ? b2 : 15);
        y->qs[j] = (uint8_t)(xi0 | (xi1 << 4));
    }
}

static void quantize_q5_0(const float *x, blk_q5_0 *y) {
    float amax = 0.f, max = 0.f;
    for (int j = 0; j < 32; j++) {
        const float v = x[j];
        if (amax < fabsf(v)) { amax = fabsf(v); max = v; }
    }
    const float d = max / -16.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    y->d = oracle_f32_to_f16(d);
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        int8_t a = (int8_t)(x[j] * id + 16.5f), b2 = (int8_t)(x[j + 16] * id + 16.5f);
        const uint8_t xi0 = (uint8_t)(a < 31 ? a : 31), xi1 = (uint8_t)(b2 < 31 ? b2 : 31);
        y->qs[j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
        qh |= ((uint32_t)(xi0 & 0x10) >> 4) << j;
        qh |= ((uint32_t)(xi1 & 0x10) >> 4) << (j + 16);
    }
    memcpy(y->qh, &qh, 4);
}

static void quantize_q5_1(const float *x, blk_q5_1 *y) {
    float min, max;
    minmax32(x, &min, &max);
    const float d = (max - min) / 31.f;
    const float id = d != 0.f ? 1.f / d : 0.f;
    y->d = oracle_f32_to_f16(d);
    y->m = oracle_f32_to_f16(min);
    uint32_t qh = 0;
    for (int j = 0; j < 16; j++) {
        const uint8_t xi0 = (uint8_t)(int8_t)((x[j] - min) * id + 0.5f), xi1 = (uint8_t)(int8_t)((x[j + 16] - min) * id + 0.5f);
        y->qs[j] = (uint8_t)((xi0 & 0x0F) | ((xi1 & 0x0F) << 4));
        qh |= ((uint32_t)(xi0 & 0x10) >> 4) << j;
        qh |= ((uint32_t)(xi1 & 0x10) >> 4) << (j + 16);
    }
    memcpy(y->qh, &qh, 4);
}

int oracle_quantize_weights(uint32_t type, const float *w, int64_t nelem, void *out) {
    const int bs = oracle_block_size(type);
    if (!bs || nelem % bs) return -1;
    const int64_t nb = nelem / bs;
    uint8_t *o = (uint8_t *)out;
    switch (type) {
    case ORACLE_Q8_0: quant_row_q8_0(w, (blk_q8_0 *)out, nb); return 0;
    case ORACLE_Q4_K:
        for (int64_t i = 0; i < nb; i++) quantize_q4_k_or_q5_k(w + i * QK_K, o + i * 144, 15);
        return 0;
    case ORACLE_Q5_K:
        for (int64_t i = 0; i < nb; i++) quantize_q4_k_or_q5_k(w + i * QK_K, o + i * 176, 31);
        return 0;
    case ORACLE_Q6_K:
        for (int64_t i = 0; i < nb; i++) quantize_q6_k(w + i * QK_K, (blk_q6_k *)(o + i * 210));
        return 0;
    case ORACLE_Q4_0: for (int64_t i = 0; i < nb; i++) quantize_q4_0(w + i * 32, (blk_q4_0 *)(o + i * 18)); return 0;
    case ORACLE_Q4_1: for (int64_t i = 0; i < nb; i++) quantize_q4_1(w + i * 32, (blk_q4_1 *)(o + i * 20)); return 0;
    case ORACLE_Q5_0: for (int64_t i = 0; i < nb; i++) quantize_q5_0(w + i * 32, (blk_q5_0 *)(o + i * 22)); return 0;
    case ORACLE_Q5_1: for (int64_t i = 0; i < nb; i++) quantize_q5_1(w + i * 32, (blk_q5_1 *)(o + i * 24)); return 0;
    default: return -1;
    }
}
