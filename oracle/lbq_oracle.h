/* lbq_oracle.h -- CPU restatement of the reference quantized-linear path.
 * TEST INFRASTRUCTURE ONLY (see lbq_oracle.c): never linked by the product. */
#ifndef LBQ_ORACLE_H
#define LBQ_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids, /root/reference/src/quantization/mod.rs:58-75 */
enum {
    ORACLE_Q4_0 = 2, ORACLE_Q4_1 = 3, ORACLE_Q5_0 = 6, ORACLE_Q5_1 = 7, ORACLE_Q8_0 = 8, ORACLE_Q8_1 = 9,
    ORACLE_Q2_K = 10, ORACLE_Q3_K = 11, ORACLE_Q4_K = 12, ORACLE_Q5_K = 13, ORACLE_Q6_K = 14, ORACLE_Q8_K = 15
};
/* the activation type a weight type's vec_dot takes (0 if none) */
uint32_t oracle_vec_dot_type(uint32_t type);

int oracle_block_size(uint32_t type);
int oracle_type_size(uint32_t type);
float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);
void oracle_unpack_scales_k4(const uint8_t scales[12], uint8_t sc[8], uint8_t mn[8]);

/* out: nblocks*block_size floats */
int oracle_dequantize(uint32_t type, const void *blocks, int64_t nblocks, float *out);
/* type: ORACLE_Q8_K, ORACLE_Q8_0 or ORACLE_Q8_1; x is [m][k] f32; out is m*(k/QK) blocks */
int oracle_quantize_act(uint32_t type, const float *x, int64_t m, int64_t k, void *out);
/* one output element: dot of a weight row (k/QK blocks) with a quantised activation row */
int oracle_vec_dot(uint32_t type, int64_t k, const void *wrow, const void *xrow, float *out);
/* y[m][n] = x[m][k] . W[n][k]^T, candle's CPU algorithm, over nthreads threads */
int oracle_qmatmul(uint32_t type, const void *w, int64_t n, int64_t k, const float *x, int64_t m, float *y,
                   int nthreads);
/* f32 -> GGUF blocks (ggml reference quantisers), nelem % block_size == 0 */
int oracle_quantize_weights(uint32_t type, const float *w, int64_t nelem, void *out);

#ifdef __cplusplus
}
#endif
#endif
