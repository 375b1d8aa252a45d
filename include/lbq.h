/*
 * lbq.h -- C ABI of the MI355X quantized-linear library (liblbq.so).
 *
 * This is the drop-in boundary for lightbulb's GGUF quantized-linear path.
 * lightbulb calls QuantizableLinear::Quantized(QMatMul)::forward for every
 * attention/MLP projection and the LM head
 * (/root/reference/src/model/quantizable_linear.rs:36-43, 63-69).  A Rust shim
 * keeps that surface and binds the functions below through `extern "C"`; the
 * binding is plain pointers, 64-bit sizes and an opaque stream pointer, in
 * the style of the reference's only FFI precedent
 * (/root/reference/src/backend/marlin_ffi.rs:84-215), plus status codes.
 *
 * Conventions
 *   - Every function returns 0 (LBQ_OK) or a negative lbq_status, never
 *     aborts; lbq_last_error() gives a thread-local message for the last
 *     failure on the calling thread.
 *   - Pointers named d_* are device pointers (HBM).  `stream` is a
 *     hipStream_t passed as void* (NULL = the null stream); work is ordered
 *     on it and the call does not synchronise unless stated.
 *   - Weights are GGUF blocks in their on-disk byte layout: row-major
 *     [n][k / block_size] blocks, rows contiguous along k
 *     (GGUF ne0 = k; /root/reference/src/gguf/parser.rs:180-199).
 *   - A context owns per-device scratch (quantised activations, the batched
 *     GEMM's workspace, grown on demand, and 64 KiB of its tile counters).  Calls that share a context must be
 *     ordered on one stream (the reference runs every forward on one model
 *     thread, src/engine/model_runner.rs:236,383).  Weight handles are
 *     immutable and may be read concurrently.
 */
#ifndef LBQ_H
#define LBQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lbq_ctx lbq_ctx;
typedef struct lbq_weight lbq_weight;

enum lbq_status {
    LBQ_OK = 0,
    LBQ_ERR_INVALID_ARG = -1,      /* null pointer, negative size, misaligned pointer */
    LBQ_ERR_UNSUPPORTED_TYPE = -2, /* ggml type id not served by this path */
    LBQ_ERR_SHAPE = -3,            /* k not a multiple of the block size, byte count mismatch */
    LBQ_ERR_OOM = -4,              /* device allocation failed */
    LBQ_ERR_HIP = -5,              /* a HIP runtime call failed */
    LBQ_ERR_LIMIT = -6,            /* size beyond a documented maximum */
    LBQ_ERR_FORMAT = -7,           /* malformed or unsupported GGUF container */
    LBQ_ERR_NOT_FOUND = -8,        /* no tensor or metadata key of that name */
    LBQ_ERR_IO = -9                /* a file could not be opened or mapped */
};

/* GGUF/ggml type ids: /root/reference/src/quantization/mod.rs:58-75 (GgmlDType),
 * plus BF16 (30), which candle-core's GgmlDType carries and the reference's own
 * table does not: candle's GGUF reader hands a BF16 tensor to QMatMul::from_qtensor
 * (custom_transformer.rs:358-363), which serves it as its dense variant. */
enum lbq_ggml_type {
    LBQ_TYPE_F32 = 0,  /* dense: an f32 matmul (candle's dense QMatMul variant), k % 8 == 0 */
    LBQ_TYPE_F16 = 1,  /* dense: widened exactly to f32, then as F32 */
    LBQ_TYPE_Q4_0 = 2, /* 32-value blocks, Q8_0 activations */
    LBQ_TYPE_Q4_1 = 3, /* 32-value blocks, Q8_1 activations */
    LBQ_TYPE_Q5_0 = 6, /* 32-value blocks, Q8_0 activations */
    LBQ_TYPE_Q5_1 = 7, /* 32-value blocks, Q8_1 activations */
    LBQ_TYPE_Q8_0 = 8,
    LBQ_TYPE_Q8_1 = 9, /* activation-only type (vec-dot partner of Q4_1/Q5_1) */
    LBQ_TYPE_Q2_K = 10,
    LBQ_TYPE_Q3_K = 11,
    LBQ_TYPE_Q4_K = 12,
    LBQ_TYPE_Q5_K = 13,
    LBQ_TYPE_Q6_K = 14,
    LBQ_TYPE_Q8_K = 15, /* activation-only type (vec-dot partner of the k-quants) */
    LBQ_TYPE_BF16 = 30  /* dense: widened exactly to f32 (bits << 16), then as F32 */
};

/* Thread-local description of the last error on this thread ("" if none). */
const char *lbq_last_error(void);

/* GgmlDType::block_size / type_size (/root/reference/src/quantization/mod.rs:99-126)
 * for the types above (BF16: candle's 1 and 2); 0 for any other id.  lbq_type_size
 * returns the table's value, so GGUF extents computed from it agree with the
 * reference's extract_tensor_bytes (src/quantization/gguf_ops.rs:19-59); for Q2_K
 * that is 82.  (lbq_gguf_tensor_bytes, the mirror of extract_tensor_bytes, still
 * refuses BF16 tensors as the reference's GgmlDType::from_u32 does.) */
int lbq_type_block_size(uint32_t ggml_type);
int lbq_type_size(uint32_t ggml_type);

/* Bytes of one block as it sits in device memory and as the kernels read it
 * (candle's BlockQ2K: scales[16], qs[64], d, dmin): equal to lbq_type_size except
 * for Q2_K, whose block is 84 bytes.  Weight handles take
 * n * (k / block_size) * lbq_type_block_bytes bytes.  No counterpart in the
 * reference, whose table (mod.rs:118) is 2 bytes short for Q2_K. */
int lbq_type_block_bytes(uint32_t ggml_type);

/* Open a context on HIP device `device`.  Replaces the device selection at
 * /root/reference/src/model/parallel_model_manager.rs:239-248. */
int lbq_init(int device, lbq_ctx **out_ctx);
int lbq_ctx_destroy(lbq_ctx *ctx);

/* Upload GGUF blocks (host bytes, on-disk layout, unchanged) to the device
 * and return an immutable weight handle.  Replaces QMatMul::from_qtensor
 * (called at /root/reference/src/model/custom_attention.rs:195-206,
 * mlp_wrapper.rs:127-135, custom_transformer.rs:360-363) together with the
 * upload done by Content::tensor (src/gguf/mod.rs:274-282).
 * nbytes must equal n * (k / block_size) * lbq_type_block_bytes. */
int lbq_weight_create(lbq_ctx *ctx, uint32_t ggml_type, int64_t n, int64_t k, const void *host_blocks,
                      size_t nbytes, lbq_weight **out_w);

/* As lbq_weight_create, but borrows blocks that are already device resident
 * (no copy; the caller keeps the memory alive until lbq_weight_destroy).  Like
 * lbq_weight_create it derives per-row fp16 operand exponents for the batched
 * MFMA GEMM (m > 8) from the block scales, so the blocks must already hold their
 * final contents: the call synchronises the device (whatever writes the blocks,
 * on any stream, completes first) and allocates n bytes for the exponents.  If
 * the caller rewrites the blocks while the handle lives, lbq_weight_refresh must
 * follow before the next forward, or results at m > 8 are wrong (overflowing or
 * underflowing fp16 operands, no error). */
int lbq_weight_wrap_device(lbq_ctx *ctx, uint32_t ggml_type, int64_t n, int64_t k, const void *d_blocks,
                           size_t nbytes, lbq_weight **out_w);

/* Recompute a weight's derived state (the per-row operand exponents above) from
 * its current blocks, stream-ordered on `stream`.  No counterpart in the
 * reference, whose QTensor is immutable; for callers that fill or change the
 * device blocks of a wrapped handle after wrapping it.  A no-op for types and
 * k the MFMA GEMM does not serve (dense weights, k % 256 != 0). */
int lbq_weight_refresh(lbq_weight *w, void *stream);

int lbq_weight_destroy(lbq_weight *w);

/* Shape and type of a weight handle (QTensor::dtype / QTensor::shape). */
int lbq_weight_info(const lbq_weight *w, uint32_t *ggml_type, int64_t *n, int64_t *k);

/* y[m][n] = x[m][k] . W^T in f32 -- QMatMul::forward (candle-core 0.10.2,
 * reached through /root/reference/src/model/quantizable_linear.rs:67).
 * x and y are contiguous f32 device buffers that must not overlap
 * (LBQ_ERR_INVALID_ARG otherwise; the reference returns a new tensor); any
 * leading dims of the reference's [.., k] tensor are flattened into m.  The
 * activation is quantised to Q8_K (k-quant weights), Q8_1 (Q4_1/Q5_1) or Q8_0
 * (the other 32-value types) exactly as the reference CPU path does.
 * Arithmetic by (type, m):
 *   - m <= 8, Q4_K/Q5_K weights of 1024 rows or more up to m = 32 (and
 *     m = 33..64 up to 8192 rows, as two 32-row halves), Q6_K weights with
 *     k > 8192 on the same shapes, Q8_0 weights of 1024 rows or more
 *     (k % 256 == 0) up to m = 32 (m = 33..64 as halves at k <= 8192 up to 8192
 *     rows), and Q4_0/Q4_1/Q5_0/Q5_1 weights of 1024 rows or more (k % 256 == 0)
 *     up to m = 16: each output from integer sub-block dot
 *     products as in the reference (f32 combine; only the summation order
 *     differs, ~1e-7 relative);
 *   - m > 8 otherwise, for every quantised type when k % 256 == 0 (Q4_0, Q4_1,
 *     Q5_0, Q5_1, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K): MFMA on fp16 roundings of
 *     the same activation and weight values (about 4e-4 relative on a row);
 *   - m > 8 with k % 256 != 0: the integer GEMV over chunks of 8 rows.
 * Where the matrix-core decode kernel (m = 2..64) splits a 32-row
 * tile between two workgroups, their halves are added into y with f32 atomic
 * adds when y is plain device memory (hipMalloc; checked once per allocation),
 * else through partial sums in the workspace; either way y = a + b for the two
 * halves, the same bits for finite normal-range halves.  Dense F32/F16/BF16
 * weights are candle's dense variant: no quantisation, an f32 matmul.  m == 0 is
 * a no-op. */
int lbq_qmatmul_f32(lbq_ctx *ctx, const lbq_weight *w, const float *d_x, int64_t m, float *d_y, void *stream);

/* lbq_qmatmul_f32's result (the same kernels, the same bits), allocating
 * nothing: no hipMalloc, hipFree or allocating library call.
 * No counterpart in the reference; for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid it.  The quantised activations and the batched GEMM's workspace live
 * in a fixed array of LBQ_NOALLOC_SCRATCH_BYTES per device (its last 64 KiB
 * are the GEMM's tile counters, zeroed by lbq_init and left zero by every
 * call), resolved by lbq_init and held until the process ends.  A call that needs more (roughly
 * m * k * 2 bytes of fp16 operands plus split-k partials above m = 8; every
 * Llama-3-8B projection fits up to m = 512, down_proj up to m = 2048) returns
 * LBQ_ERR_LIMIT before launching anything.  All contexts on a device share the
 * one array, which keeps the last call's contents: calls that overlap on one
 * device (on different streams or threads) race and must be ordered by the
 * caller. */
#define LBQ_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int lbq_qmatmul_f32_noalloc(lbq_ctx *ctx, const lbq_weight *w, const float *d_x, int64_t m, float *d_y,
                            void *stream);

/* Several weights applied to one x: ys[i][m][n_i] = x . W_i^T, exactly as
 * `count` separate lbq_qmatmul_f32 calls compute them (bit-identical), with x
 * quantised once and, at m = 1, every weight's rows streamed by one launch.
 * Replaces the runs of QMatMul::forward calls on the same input at the q/k/v
 * projections (/root/reference/src/model/custom_attention.rs:265-267) and the
 * gate/up projections (/root/reference/src/model/mlp_wrapper.rs:190,193).
 * 1 <= count <= LBQ_GROUP_MAX; all weights share the ggml type and k. */
#define LBQ_GROUP_MAX 4
int lbq_qmatmul_group_f32(lbq_ctx *ctx, const lbq_weight *const *ws, int count, const float *d_x, int64_t m,
                          float *const *d_ys, void *stream);

/* The gate/up half of the reference's MLP forward (/root/reference/src/model/
 * mlp_wrapper.rs:190-194: `silu(gate_proj.forward(x)) * up_proj.forward(x)`):
 * d_out[m][n] = silu(x . Wg^T) * (x . Wu^T), silu(v) = v / (1 + exp(-v)) in f32.
 * The two products are computed exactly as lbq_qmatmul_f32 computes them.  At
 * m = 1, and for Q4_K / Q5_K weights of more than 8192 rows (and more than 32
 * rows per CU) at m = 5..32 -- m = 2..32 when k > 8192 -- (after one activation
 * quantisation), both weights stream through one launch and the product is
 * formed in its epilogue, so neither product is written out; otherwise
 * the grouped path fills context memory and one elementwise launch combines it
 * (the m = 2..32 pair launch gives the same bits as that).  gate and up share the
 * ggml type, n and k. */
int lbq_gate_up_silu_f32(lbq_ctx *ctx, const lbq_weight *w_gate, const lbq_weight *w_up, const float *d_x, int64_t m,
                         float *d_out, void *stream);

/* The RMS norm that precedes those projections (input_layernorm before q/k/v,
 * post_attention_layernorm before gate/up: /root/reference/src/model/
 * custom_transformer_block.rs:329 and the MLP path; candle's RmsNorm in f32:
 * x_norm = x / sqrt(sum(x^2) / k + eps) * norm_w), then the grouped projections or
 * the gate/up product of x_norm.  At m = 1 (k-quants, k <= 8192, x and norm_w
 * 16-byte aligned) the norm and the Q8_K quantisation run in the GEMV prologue
 * -- one launch, x_norm never written.  At m > 1, where every weight reads
 * pre-quantised Q8_K activations (k-quants, k % 256 == 0 up to 16384, x and
 * norm_w 16-byte aligned; m <= 8, or Q4_K/Q5_K weights on the matrix-core batch
 * decode), the norm runs inside the one Q8_K quantisation launch, x_norm again
 * never written; otherwise x_norm goes to context memory first.
 * lbq_rmsnorm_f32 is the norm alone. */
int lbq_rmsnorm_f32(const float *d_x, const float *d_w, float eps, int64_t m, int64_t k, float *d_y, void *stream);
int lbq_rmsnorm_qmatmul_group_f32(lbq_ctx *ctx, const lbq_weight *const *ws, int count, const float *d_x,
                                  const float *d_norm_w, float eps, int64_t m, float *const *d_ys, void *stream);
int lbq_rmsnorm_gate_up_silu_f32(lbq_ctx *ctx, const lbq_weight *w_gate, const lbq_weight *w_up, const float *d_x,
                                 const float *d_norm_w, float eps, int64_t m, float *d_out, void *stream);

/* Quantised-activation handle: the two halves of QMatMul::forward as separate
 * calls.  candle's k_quants::matmul first quantises every row of x into
 * vec-dot blocks and then runs vec_dot for all output columns; splitting the
 * two lets call sites that feed one x to several weights -- q/k/v at
 * /root/reference/src/model/custom_attention.rs:265-267, gate/up at
 * mlp_wrapper.rs:190,193 -- quantise x once.  act_type is LBQ_TYPE_Q8_K for
 * k-quant weights, LBQ_TYPE_Q8_0 for Q8_0/Q4_0/Q5_0 weights and LBQ_TYPE_Q8_1
 * for Q4_1/Q5_1 weights.  The handle owns device memory for m rows of k values. */
typedef struct lbq_act lbq_act;
int lbq_act_create(lbq_ctx *ctx, uint32_t act_type, int64_t m, int64_t k, lbq_act **out_act);
int lbq_act_quantize(lbq_act *act, const float *d_x, void *stream);
int lbq_act_destroy(lbq_act *act);
/* y[m][n] from a quantised activation; act's k and vec-dot type must match w. */
int lbq_qmatmul_act_f32(lbq_ctx *ctx, const lbq_weight *w, const lbq_act *act, float *d_y, void *stream);

/* Dequantise the whole weight to f32 [n][k] -- QTensor::dequantize (used at
 * /root/reference/src/model/custom_transformer.rs:323,347 and
 * custom_transformer_block.rs:229,231).  Bit-exact with the reference. */
int lbq_dequantize_f32(lbq_ctx *ctx, const lbq_weight *w, float *d_y, void *stream);

/* Dequantise nelem values of raw device blocks -- dequantize_tensor
 * (/root/reference/src/quantization/mod.rs:158-247), extended to every block type
 * above, and F32 / F16 / BF16 tensors (QTensor::dequantize of the norm weights,
 * custom_transformer_block.rs:229-231, which GGUF files store as F32).
 * nelem must be a multiple of the block size. */
int lbq_dequantize_blocks_f32(uint32_t ggml_type, const void *d_blocks, int64_t nelem, float *d_y, void *stream);

/* Embedding lookup without the dense table: d_out[i][:] = row d_ids[i] of the
 * dequantised weight (f32 [count][k], bit-exact with QTensor::dequantize followed
 * by Embedding::forward's index_select -- custom_transformer.rs:321-323, the
 * token embedding, which the reference dequantises whole at load).  d_ids holds
 * count int32 ids; an id outside [0, n) yields a row of NaN (the reference's
 * index_select raises; the device cannot, so the row is poisoned instead).
 * k must be a multiple of 16; d_out 16-byte aligned. */
int lbq_embedding_f32(lbq_ctx *ctx, const lbq_weight *w, const int32_t *d_ids, int64_t count, float *d_out,
                      void *stream);

/* Quantise activations x[m][k] to GGUF blocks of `act_type` (LBQ_TYPE_Q8_K:
 * 292-byte blocks; LBQ_TYPE_Q8_0: 34-byte blocks; LBQ_TYPE_Q8_1: 36-byte
 * blocks) -- the activation quantisation inside QMatMul::forward (candle
 * BlockQ8K / BlockQ8_0 / BlockQ8_1 ::from_float).  Exposed so the step can be
 * checked on its own. */
int lbq_quantize_act(uint32_t act_type, const float *d_x, int64_t m, int64_t k, void *d_out_blocks, void *stream);

/* Quantise f32 weights (nelem values, row-major, rows along k) to GGUF blocks
 * of `ggml_type` -- quantize_tensor (/root/reference/src/quantization/mod.rs:257-327),
 * extended to Q5_K/Q6_K and Q4_1/Q5_0/Q5_1.  Runs on the device. */
int lbq_quantize_weights_f32(uint32_t ggml_type, const float *d_w, int64_t nelem, void *d_out_blocks, void *stream);

/* ---------------------------------------------------------------------------
 * GGUF container (v3, little-endian) and the direct GGUF -> device upload.
 * lbq_gguf_open maps the file and parses it as the reference's parse_gguf does
 * (/root/reference/src/gguf/parser.rs:136-213, reached from Content::read,
 * src/gguf/mod.rs:62-92): magic, version 3 only, metadata (types 0..12, arrays),
 * tensor infos, data section at the infos' end rounded up to general.alignment
 * (UInt32; default 32).  Every read is bounds-checked: a malformed file gives
 * LBQ_ERR_FORMAT with the reference's message, never a fault.  Parsing and the
 * byte accessors are host-only.  Strings returned point into the handle and live
 * until lbq_gguf_close.
 * ------------------------------------------------------------------------- */
typedef struct lbq_gguf lbq_gguf;
int lbq_gguf_open(const char *path, lbq_gguf **out);
int lbq_gguf_close(lbq_gguf *g);
/* GGUFHeader fields (parser.rs:112-121) and the file size; any pointer may be NULL. */
int lbq_gguf_header(const lbq_gguf *g, uint32_t *version, int64_t *tensor_count, int64_t *metadata_count,
                    uint64_t *alignment, uint64_t *tensor_data_offset, uint64_t *file_size);
/* TensorInfo of tensor `index` in file order (parser.rs:103-109): name, ggml type,
 * dims (ne0 first; dims must hold n_dims <= 8 values), offset within the data section. */
int lbq_gguf_tensor_info(const lbq_gguf *g, int64_t index, const char **name, uint32_t *ggml_type, uint32_t *n_dims,
                         uint64_t *dims, uint64_t *offset);
int lbq_gguf_find_tensor(const lbq_gguf *g, const char *name, int64_t *index);
/* A tensor's bytes in the mapped file, as extract_tensor_bytes
 * (src/quantization/gguf_ops.rs:19-59): ceil(numel / block_size) * type_size
 * bytes at data_offset + offset, for every GgmlDType (quantization/mod.rs:58-127). */
int lbq_gguf_tensor_bytes(const lbq_gguf *g, const char *name, const void **data, size_t *nbytes);
/* Metadata (parser.rs:24-81): key and MetadataValueType by index; typed reads by
 * key (integers of any width and bool; f32/f64; strings; array element type and
 * length).  A missing key gives LBQ_ERR_NOT_FOUND, a type mismatch LBQ_ERR_FORMAT. */
int lbq_gguf_meta_key(const lbq_gguf *g, int64_t index, const char **key, uint32_t *value_type);
int lbq_gguf_meta_int(const lbq_gguf *g, const char *key, int64_t *out);
int lbq_gguf_meta_float(const lbq_gguf *g, const char *key, double *out);
int lbq_gguf_meta_string(const lbq_gguf *g, const char *key, const char **data, size_t *len);
int lbq_gguf_meta_array(const lbq_gguf *g, const char *key, uint32_t *elem_type, uint64_t *len);
/* Copy a tensor's blocks into device memory through pinned staging (synchronous):
 * ceil(numel / block_size) * lbq_type_block_bytes bytes -- the extent above except
 * for Q2_K, whose GgmlDType entry (82 bytes) is shorter than its 84-byte block. */
int lbq_gguf_copy_tensor(const lbq_gguf *g, const char *name, void *d_dst, size_t dst_bytes);
/* A weight handle straight from the file: the tensor (2-D, ne0 = k, ne1 = n, a
 * served type) goes through pinned staging into device memory the handle owns.
 * Replaces Content::tensor -> QMatMul::from_qtensor (src/gguf/mod.rs:274-282 and
 * the call sites listed at lbq_weight_create). */
int lbq_weight_from_gguf(lbq_ctx *ctx, const lbq_gguf *g, const char *name, lbq_weight **out_w);

#ifdef __cplusplus
}
#endif
#endif /* LBQ_H */
