// lbq_internal.hpp -- launcher declarations shared between the kernel translation
// units and the C ABI (lbq_api.cpp).  Host-side only types; no torch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbq {

enum : int {
    TYPE_F32 = 0, TYPE_F16 = 1,
    TYPE_Q4_0 = 2, TYPE_Q4_1 = 3, TYPE_Q5_0 = 6, TYPE_Q5_1 = 7, TYPE_Q8_0 = 8, TYPE_Q8_1 = 9,
    TYPE_Q2_K = 10, TYPE_Q3_K = 11, TYPE_Q4_K = 12, TYPE_Q5_K = 13, TYPE_Q6_K = 14, TYPE_Q8_K = 15,
    TYPE_BF16 = 30  // candle's GgmlDType::BF16 (the GGUF id); not in the reference's own table
};

// 32-value weight blocks that pair with Q8_0 / Q8_1 activations.
constexpr bool is_legacy(int t) { return t == TYPE_Q4_0 || t == TYPE_Q4_1 || t == TYPE_Q5_0 || t == TYPE_Q5_1; }
// 256-value weight blocks that pair with Q8_K activations.
constexpr bool is_kquant(int t) {
    return t == TYPE_Q2_K || t == TYPE_Q3_K || t == TYPE_Q4_K || t == TYPE_Q5_K || t == TYPE_Q6_K;
}
// weight types with the register-resident decode GEMV decoders (the m = 1 fast path)
constexpr bool has_fast_gemv(int t) { return t == TYPE_Q4_K || t == TYPE_Q5_K || t == TYPE_Q6_K || t == TYPE_Q8_0; }
// weight types the MFMA GEMM serves at m > 8: every quantised weight type
constexpr bool has_mfma_gemm(int t) { return is_kquant(t) || is_legacy(t) || t == TYPE_Q8_0; }
// ... at this k: the GEMM steps through k in 256-value super-blocks (32-value
// types: 8 blocks); other k run the decode GEMV over row chunks of 8
constexpr bool gemm_serves(int t, int64_t k) { return has_mfma_gemm(t) && k % 256 == 0; }
// types whose per-lane weight state (raw bytes + expanded operands) is large: one
// workgroup per CU for the 32-row-tile kernels, no 128-row k_gemm tiles, one
// k-step of A read-ahead in the tall kernel; the k-sliced kernel up to 64 rows
// types whose GEMM adds an extra k-step per super-block for the reference's
// m * s term (Q8_1 activations' stored block sums)
constexpr bool gemm_offset_step(int t) { return t == TYPE_Q4_1 || t == TYPE_Q5_1; }
constexpr bool gemm_heavy(int t) {
    return t == TYPE_Q6_K || t == TYPE_Q8_0 || t == TYPE_Q3_K || t == TYPE_Q5_0 || t == TYPE_Q5_1;
}
// activation type of QMatMul's vec_dot for a weight type (candle GgmlType::VecDotType)
constexpr int vec_dot_type(int t) {
    return is_kquant(t) ? TYPE_Q8_K : (t == TYPE_Q4_1 || t == TYPE_Q5_1) ? TYPE_Q8_1 : TYPE_Q8_0;
}

struct ActView;

// Launch-plan overrides for tuning runs, read from the environment once, when a
// context is created (lbq_init), never on a forward call.  Any setting computes
// the same result; only the kernel shape changes.  Zero / false: the measured
// default plan.
//   LBQ_GEMM_KS64, LBQ_GEMM_NO_KS, LBQ_GEMM_KS=<blocks>, LBQ_GEMM_NO_TALL,
//   LBQ_GEMM_BIG=wide|tall, LBQ_GEMM_SPLITS=<n>,
//   LBQ_GEMM_WIDE7=0|1                              batched GEMM plan
//   LBQ_GEMV1_NOFUSE, LBQ_GEMV1_CFG=<ppb>,<rpw>, LBQ_GEMV1_WPC=<waves per CU>,
//   LBQ_GEMV1_WPG=<waves per workgroup>, LBQ_GEMV="rpw,it,wpc,fused",
//   LBQ_GEMV_ROWS_OFF, LBQ_GEMV1_DYNAMIC            decode GEMV plan
//   LBQ_GEMV_MX_OFF, LBQ_GEMV_MX_WIDE_OFF (m = 9..32 only),
//   LBQ_GEMV_MX_SPLITS=<workgroups per tile>, LBQ_GEMV_MX_WAVES=4|8, LBQ_GEMV_MX_ALL,
//   LBQ_GEMV_MX_PAIR_OFF, LBQ_GEMV_MX_HALVES_OFF   matrix-core batch decode plan
struct Tuning {
    bool gemm_ks64 = false, gemm_no_ks = false, gemm_no_tall = false;
    int gemm_ks = 0;      // k-sliced tiles: blocks per slice (0: planned)
    int gemm_big = 0;     // 1: wide tiles, 2: tall tiles (0: planned)
    int gemm_splits = 0;  // split-k count (0: planned)
    int gemm_wide7 = 0;   // seven-wave wide tiles: 1 always where n allows, -1 never (0: planned)
    bool gemm_split_launch = false;  // k-sliced slices added by the separate launch, never in the kernel
    bool gemm_prepass = false;       // k-sliced operands always from the separate pre-pass
    bool gemv1_nofuse = false, gemv_rows_off = false;
    int gemv1_ppb = 0, gemv1_rpw = 0;  // m = 1 shape (0: planned)
    int gemv1_wpc = 0, gemv1_wpg = 0;
    bool gemv1_dynamic = false;  // m = 1: never the static (compile-time group count) schedule
    bool gemv_mx_off = false;  // batch decode never on the matrix cores
    bool gemv_mx_wide_off = false;  // m = 9..32 never on the integer matrix-core kernel
    int gemv_mx_splits = 0, gemv_mx_waves = 0;  // matrix-core batch decode: workgroups per tile, waves (0: planned)
    bool gemv_mx_all = false;  // matrix-core batch decode wherever it can run (m = 2..32, Q4_K / Q5_K / Q6_K)
    bool gemv_mx_pair_off = false;  // gate/up pairs at m = 2..32 as two launches and a product launch
    bool gemv_mx_halves_off = false;  // m = 33..64 never on the integer matrix-core kernel
    int gemv_cfg[4] = {0, 0, 0, 0};  // general GEMV "rpw,it,wpc,fused" (gemv_cfg[0] == 0: planned)
};
Tuning tuning_from_env();
// The plan overrides of the context the calling thread is inside (set by the C
// ABI entry points for the duration of a call), or the defaults.
const Tuning &tuning();
struct TuningScope {
    explicit TuningScope(const Tuning *t);
    ~TuningScope();
    const Tuning *prev;
};

// The rows of up to GROUP_MAX weights of one type and k, seen as one row space
// (weights applied to the same x: q|k|v, gate|up).  Segment s holds rows
// [end[s-1], end[s]) of the space, its blocks at w[s] and its outputs at y[s];
// entries past the last segment have end = INT32_MAX.  A plain single weight is
// the one-segment map.  A row space has fewer than 2^31 - 1 rows.
constexpr int GROUP_MAX = 4;
// tile counters of the k-sliced GEMM's in-kernel slice sum (column tiles per launch)
constexpr int KS_COUNTERS = 16384;
constexpr int64_t MAX_ROWS = 0x7ffffffe;
struct RowMap {
    const uint8_t *w[GROUP_MAX];
    float *y[GROUP_MAX];
    int32_t end[GROUP_MAX];
    int64_t n;  // rows in all segments
};
RowMap single_row_map(const uint8_t *w, int64_t n, float *y);

// f32 ranges a Q8_K quantisation launch also sets to zero (the outputs that the
// matrix-core decode kernel then adds its two split halves into)
struct ZeroList {
    float *p[4] = {nullptr, nullptr, nullptr, nullptr};
    int64_t n[4] = {0, 0, 0, 0};
    int count = 0;
};

// Quantise x[m][k] to Q8_K (act_type 15), Q8_0 (8) or Q8_1 (9).  Writes the split
// internal layout (codes xq, scales xd, Q8_K sub-block sums xbs, Q8_1 block sums
// xs) when gguf == nullptr, else GGUF blocks to gguf.  Q8_K: the same launch
// zeroes the ranges of `zero` (if any).
hipError_t launch_quant_act(int act_type, const float *x, int64_t m, int64_t k, int8_t *xq, float *xd,
                            int16_t *xbs, float *xs, uint8_t *gguf, hipStream_t st, const ZeroList *zero = nullptr);

// candle's RmsNorm of x[m][k] (f32, weight w) and the Q8_K quantisation of the
// result into the split layout, one launch; zeroes the listed buffers as
// launch_quant_act does.  k a multiple of 256 up to 16384, x and w 16-byte aligned.
hipError_t launch_rmsnorm_q8k(const float *x, const float *w, float eps, int64_t m, int64_t k, int8_t *xq, float *xd,
                              int16_t *xbs, hipStream_t st, const ZeroList *zero = nullptr);

// Dequantise nelem values (multiple of the block size) of `type` blocks to f32
// (F32 / F16: any nelem, a copy / an exact widening).
hipError_t launch_dequant(int type, const uint8_t *blocks, int64_t nelem, float *y, hipStream_t st);

// y[i][:] = the dequantised row ids[i] of an [n][k] weight (rows row_bytes apart),
// i < count; an id outside [0, n) gives a row of NaN.  k is a multiple of 16.
hipError_t launch_embedding(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const int32_t *ids,
                            int64_t count, float *y, hipStream_t st);

// y[m][n] += nothing: y is overwritten.  Weight rows are row_bytes apart.
// Requires m <= 8 (decode GEMV) -- the kernels keep one accumulator per row of x.
hipError_t launch_gemv(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act,
                       int m, float *y, hipStream_t st);

// Batch decode on the matrix cores (i8 MFMA, exact integer sums) for pre-quantised
// Q8_K rows: Q4_K / Q5_K, k % 256 == 0, k <= 16384, 5 <= m <= 8, where it is the
// faster kernel (n >= 4096, or k > 8192).
bool gemv_mx_serves(int type, int64_t n, int64_t k, int m);
// device memory launch_gemv_mx needs at ws (0: none); counters: KS_COUNTERS
// zeroed words (each launch leaves them zero)
size_t gemv_mx_workspace_bytes(int type, int64_t n, int64_t k, int m);
// true where the launch splits each tile over two workgroups: given a y that is
// already zero (y_zeroed), their halves are then added into it atomically (two
// addends: the same bits in either order) instead of through the workspace
bool gemv_mx_adds(int type, int64_t n, int64_t k, int m);
hipError_t launch_gemv_mx(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act, int m,
                          float *y, float *ws, uint32_t *counters, hipStream_t st, bool y_zeroed = false);
// a grouped call's weights (2..4, same type and k, each served by the kernel with
// at most two workgroups per tile, and the same wave count) in one launch, with the
// bits of their own launches; every two-way split y must already be zero
// (hipErrorNotSupported: launch them one by one)
hipError_t launch_gemv_mx_group(int type, int count, const uint8_t *const *w, const int64_t *n, int64_t k,
                                int64_t row_bytes, const ActView &act, int m, float *const *y, hipStream_t st);
// gate/up pair at m = 2..32: out[i][r] = silu(x_i . gate_r) * (x_i . up_r) in one
// launch, with the bits of the two single-weight launches and the product launch
bool gemv_mx_pair_serves(int type, int64_t n, int64_t k, int m);
hipError_t launch_gemv_mx_pair(int type, const uint8_t *w_gate, const uint8_t *w_up, int64_t n, int64_t k,
                               int64_t row_bytes, const ActView &act, int m, float *out, hipStream_t st);

// True when the decode GEMV quantises x itself (m = 1, k within the fast path,
// x 16-byte aligned).
bool gemv_fuses_quant(int type, int64_t n, int64_t k, int m, const float *x);

// Decode GEMV that quantises raw f32 x [m][k] in its prologue (act supplies k and
// the scale-block count only).  x == nullptr means act holds quantised codes.
hipError_t launch_gemv_x(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act,
                         const float *x, int m, float *y, hipStream_t st);

// m = 1 over a multi-weight row map in one launch, quantising x in the prologue
// (x != nullptr).  hipErrorNotSupported when k is outside the single-row fast
// path or x is not given; the caller then runs the weights one by one.
// With norm_w, x is first RMS-normalised in the prologue (k-quants, k <= 8192).
hipError_t launch_gemv_group(int type, const RowMap &rm, int64_t k, int64_t row_bytes, const ActView &act,
                             const float *x, hipStream_t st, const float *norm_w = nullptr, float eps = 0.f);

// m = 1 gate/up pair (same type, n, k): out[i] = silu(x . gate_i) * (x . up_i)
// in one launch that quantises x in its prologue.  hipErrorNotSupported when the
// single-row fast path does not cover k (or x is not 16-byte aligned); the
// caller then computes gate and up and combines them with launch_silu_mul.
hipError_t launch_gemv_silu_pair(int type, const uint8_t *w_gate, const uint8_t *w_up, int64_t n, int64_t k,
                                 int64_t row_bytes, const float *x, float *out, hipStream_t st,
                                 const float *norm_w = nullptr, float eps = 0.f);
// candle's RmsNorm in f32, one workgroup per row: y = x / sqrt(sum(x^2)/k + eps) * w
hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int64_t m, int64_t k, float *y, hipStream_t st);
// out[i] = silu(g[i]) * u[i], count values
hipError_t launch_silu_mul(const float *g, const float *u, int64_t count, float *out, hipStream_t st);

// Batched path (m > 8): weights dequantised in registers into MFMA operands.
// Needs gemm_workspace_bytes(type, n, k, m) bytes of device memory at ws (fp16
// activation operands and, for shapes that split k, the partial sums).  For
// k-quants it is a pre-pass that writes the operand rows -- from raw f32 x
// (quantised to Q8_K on the way) when x != nullptr, else from act's codes --
// and the GEMM proper, which weights of one type, k and m can share a pre-pass
// for (the operand rows do not depend on n).
size_t gemm_workspace_bytes(int type, int64_t n, int64_t k, int64_t m);
bool gemm_prepass_fuses_quant(int type, int64_t k, const float *x);
hipError_t gemm_prepass(int type, int64_t k, const ActView &act, const float *x, int64_t m, void *ws, hipStream_t st);
// rexp: the weight's per-row operand exponents (launch_row_exponents).
// counters: KS_COUNTERS zeroed words the k-sliced kernel uses to add its own
// slices (the last workgroup of a column tile sums them and puts the word back
// to zero); nullptr keeps the separate slice-sum launch.
// x: f32 activations the k-sliced kernel quantises itself (gemm_quantises_in_kernel;
// no pre-pass then), or nullptr for the operands gemm_prepass left in ws.
hipError_t gemm_main(int type, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t k, int64_t row_bytes, int64_t m,
                     float *y, void *ws, uint32_t *counters, const float *x, hipStream_t st);
// whether the GEMM for (type, n, k, m) quantises f32 x itself (the k-sliced
// kernel with Q8_K activations, on slices whose x fits its registers)
bool gemm_quantises_in_kernel(int type, int64_t n, int64_t k, int64_t m, const float *x);
hipError_t launch_gemm(int type, const uint8_t *w, const int8_t *rexp, int64_t n, int64_t k, int64_t row_bytes,
                       const ActView &act, const float *x, int64_t m, float *y, void *ws, uint32_t *counters,
                       hipStream_t st);
// Per-row operand exponents of a weight the MFMA GEMM serves (gemm_serves):
// rexp[i] = e such that every value row i's blocks can produce is below
// 2^(15 + e), so the GEMM's fp16 weight operands, scaled by 2^-e, stay clear
// of the fp16 subnormal range.  n bytes at rexp.
hipError_t launch_row_exponents(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, int8_t *rexp,
                                hipStream_t st);

// Dense F32 / F16 weights (candle's dense QMatMul variant): y[m][n] = x . W^T in
// f32, W [n][k] in its file layout widened on the fly; k % 8 == 0.
constexpr bool is_dense(int t) { return t == TYPE_F32 || t == TYPE_F16 || t == TYPE_BF16; }
hipError_t launch_dense(int type, const uint8_t *w, int64_t n, int64_t k, const float *x, int64_t m, float *y,
                        hipStream_t st);

// Compute units of the current device (cached after the first call).
int num_cus();

// f32 weights -> GGUF blocks on the device (ggml reference quantisers).
hipError_t launch_quant_weights(int type, const float *w, int64_t nelem, uint8_t *out, hipStream_t st);

}  // namespace lbq
