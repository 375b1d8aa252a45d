// lbq_api.cpp -- the C ABI (include/lbq.h): argument checking, device scratch,
// and dispatch between the decode GEMV (m <= 8) and the MFMA GEMM (m > 8).
//
// Error behaviour mirrors candle's QMatMul surface as the reference sees it: a
// failure is returned (candle::Result propagated with `?` through
// QuantizableLinear::forward, /root/reference/src/model/quantizable_linear.rs:63-69),
// never an abort.  Here that is a negative status plus a thread-local message.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/lbq.h"
#include "lbq_device.hpp"
#include "lbq_internal.hpp"

static_assert(LBQ_GROUP_MAX == lbq::GROUP_MAX, "one group limit for the ABI and the kernels");

// Scratch of lbq_qmatmul_f32_noalloc: one array per device (each GPU holds its
// own copy while the process lives).  Host code never uses the array's name as
// an address: lbq_init resolves it once per device with hipGetSymbolAddress.
// Calls that overlap on one device share it and race.
static __device__ __align__(256) uint8_t scratch[LBQ_NOALLOC_SCRATCH_BYTES];
// its last bytes hold the k-sliced GEMM's tile counters, the rest the buffers
constexpr size_t NOALLOC_COUNTER_BYTES = sizeof(uint32_t) * lbq::KS_COUNTERS;
constexpr size_t NOALLOC_FIXED_BYTES = LBQ_NOALLOC_SCRATCH_BYTES - NOALLOC_COUNTER_BYTES;

struct lbq_ctx {
    int device;
    uint8_t *noalloc_scratch;  // this device's `scratch`, from hipGetSymbolAddress
    lbq::Tuning tune;     // launch-plan overrides, read from the environment at lbq_init
    std::mutex mu;        // guards scratch growth
    uint8_t *scratch;     // quantised activations (split layout)
    size_t scratch_bytes;
    uint8_t *ws;          // batched GEMM workspace (fp16 activations, split-k partials)
    size_t ws_bytes;
    uint8_t *tmp;         // gate and up outputs when their product is not fused
    size_t tmp_bytes;
    uint32_t *tile_counters;  // KS_COUNTERS zeroed words of the k-sliced GEMM (each launch leaves them zero)
};

struct lbq_weight {
    lbq_ctx *ctx;
    int type;
    int64_t n, k;
    int64_t row_bytes;
    size_t nbytes;
    const uint8_t *d_blocks;
    bool owned;
    int8_t *d_rexp;  // per-row operand exponents of the MFMA GEMM (types it serves), else null
};

struct lbq_act {
    lbq_ctx *ctx;
    int act_type;
    int64_t m, k;
    uint8_t *buf;
    lbq::ActView view;
};

namespace lbq {
namespace {
thread_local const Tuning *t_tuning = nullptr;
const Tuning k_default_tuning{};
int env_int(const char *name) {
    const char *e = getenv(name);
    return e ? atoi(e) : 0;
}
}  // namespace

Tuning tuning_from_env() {
    Tuning t;
    t.gemm_ks64 = getenv("LBQ_GEMM_KS64") != nullptr;
    t.gemm_no_ks = getenv("LBQ_GEMM_NO_KS") != nullptr;
    t.gemm_no_tall = getenv("LBQ_GEMM_NO_TALL") != nullptr;
    t.gemm_ks = std::max(0, env_int("LBQ_GEMM_KS"));
    if (const char *e = getenv("LBQ_GEMM_BIG")) t.gemm_big = e[0] == 't' ? 2 : 1;
    t.gemm_splits = std::max(0, env_int("LBQ_GEMM_SPLITS"));
    if (const char *e = getenv("LBQ_GEMM_WIDE7")) t.gemm_wide7 = e[0] == '0' ? -1 : 1;
    t.gemm_split_launch = getenv("LBQ_GEMM_SPLIT_LAUNCH") != nullptr;
    t.gemm_prepass = getenv("LBQ_GEMM_PREPASS") != nullptr;
    t.gemv1_nofuse = getenv("LBQ_GEMV1_NOFUSE") != nullptr;
    t.gemv_rows_off = getenv("LBQ_GEMV_ROWS_OFF") != nullptr;
    if (const char *e = getenv("LBQ_GEMV1_CFG")) {
        int q = 0, r = 0;
        if (sscanf(e, "%d,%d", &q, &r) == 2 && q > 0 && r > 0) { t.gemv1_ppb = q; t.gemv1_rpw = r; }
    }
    t.gemv1_wpc = std::max(0, env_int("LBQ_GEMV1_WPC"));
    t.gemv1_wpg = std::max(0, env_int("LBQ_GEMV1_WPG"));
    t.gemv1_dynamic = getenv("LBQ_GEMV1_DYNAMIC") != nullptr;
    t.gemv_mx_off = getenv("LBQ_GEMV_MX_OFF") != nullptr;
    t.gemv_mx_wide_off = getenv("LBQ_GEMV_MX_WIDE_OFF") != nullptr;
    t.gemv_mx_splits = env_int("LBQ_GEMV_MX_SPLITS");
    t.gemv_mx_waves = env_int("LBQ_GEMV_MX_WAVES");
    t.gemv_mx_all = getenv("LBQ_GEMV_MX_ALL") != nullptr;
    t.gemv_mx_pair_off = getenv("LBQ_GEMV_MX_PAIR_OFF") != nullptr;
    t.gemv_mx_halves_off = getenv("LBQ_GEMV_MX_HALVES_OFF") != nullptr;
    if (const char *e = getenv("LBQ_GEMV")) {
        int v[4] = {0, 0, 0, 0};
        if (sscanf(e, "%d,%d,%d,%d", &v[0], &v[1], &v[2], &v[3]) >= 3 && v[0] > 0 && v[1] > 0 && v[2] > 0)
            for (int i = 0; i < 4; i++) t.gemv_cfg[i] = v[i];
    }
    return t;
}

const Tuning &tuning() { return t_tuning ? *t_tuning : k_default_tuning; }
TuningScope::TuningScope(const Tuning *t) : prev(t_tuning) { t_tuning = t; }
TuningScope::~TuningScope() { t_tuning = prev; }

int num_cus() {
    static int cus = 0;
    if (!cus) {
        int dev = 0;
        hipDeviceProp_t p;
        if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess) cus = p.multiProcessorCount;
        if (cus <= 0) cus = 256;
    }
    return cus;
}
}  // namespace lbq

namespace {

thread_local std::string g_err;

int fail(int status, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return status;
}

int hip_fail(hipError_t e, const char *what) {
    return fail(LBQ_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

bool weight_type_ok(uint32_t t) {
    return t == LBQ_TYPE_Q8_0 || lbq::is_kquant((int)t) || lbq::is_legacy((int)t) || lbq::is_dense((int)t);
}

bool act_type_ok(uint32_t t) { return t == LBQ_TYPE_Q8_K || t == LBQ_TYPE_Q8_0 || t == LBQ_TYPE_Q8_1; }

// Restores the caller's current device on scope exit.
struct DeviceGuard {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// Split activation layout for m rows of length k quantised to act_type: codes,
// f32 scales, then the Q8_K 16-value sums (int16) or the Q8_1 block sums (f32).
struct ActLayout {
    size_t q_off, d_off, bs_off, total;
    int nb;
    int act_type;
};

ActLayout act_layout(int act_type, int64_t m, int64_t k) {
    ActLayout L;
    const int bs = act_type == LBQ_TYPE_Q8_K ? 256 : 32;
    L.nb = (int)(k / bs);
    L.act_type = act_type;
    L.q_off = 0;
    L.d_off = align_up((size_t)(m * k), 256);
    L.bs_off = align_up(L.d_off + (size_t)(m * L.nb) * sizeof(float), 256);
    size_t tail = 0;
    if (act_type == LBQ_TYPE_Q8_K) tail = (size_t)(m * (k / 16)) * sizeof(int16_t);
    else if (act_type == LBQ_TYPE_Q8_1) tail = (size_t)(m * L.nb) * sizeof(float);
    L.total = align_up(L.bs_off + tail, 256);
    return L;
}

// Grows a context buffer to at least `bytes` (what: message tag).
int ensure_buffer(uint8_t **buf, size_t *have, size_t bytes, const char *what) {
    if (*have >= bytes) return LBQ_OK;
    const size_t want = align_up(bytes > *have * 2 ? bytes : *have * 2, 1 << 20);
    if (*buf) {
        // in-flight kernels on any stream may still read the old buffer
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize");
        (void)hipFree(*buf);
        *buf = nullptr;
        *have = 0;
    }
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) return fail(LBQ_ERR_OOM, "hipMalloc(%zu) for %s: %s", want, what, hipGetErrorString(e));
    *buf = static_cast<uint8_t *>(p);
    *have = want;
    return LBQ_OK;
}

int ensure_scratch(lbq_ctx *ctx, size_t bytes) {
    return ensure_buffer(&ctx->scratch, &ctx->scratch_bytes, bytes, "activation scratch");
}

lbq::ActView view_of(uint8_t *base, const ActLayout &L, int64_t k) {
    const bool q8k = L.act_type == LBQ_TYPE_Q8_K, q81 = L.act_type == LBQ_TYPE_Q8_1;
    return lbq::ActView{reinterpret_cast<const int8_t *>(base + L.q_off), reinterpret_cast<const float *>(base + L.d_off),
                        q8k ? reinterpret_cast<const int16_t *>(base + L.bs_off) : nullptr, k, L.nb,
                        q81 ? reinterpret_cast<const float *>(base + L.bs_off) : nullptr};
}

// An RMS norm to apply to x before its quantisation (the call-site entry points)
struct NormArg {
    const float *w;
    float eps;
};

// The activation quantisation of x -- or, with nm, of candle's RmsNorm of x (Q8_K
// activations only) -- into the split layout of av, zeroing the ranges of `zero`
// in the same launch
hipError_t quant_into(int act_type, const float *d_x, int64_t m, int64_t k, const lbq::ActView &av, hipStream_t st,
                      const lbq::ZeroList *zero = nullptr, const NormArg *nm = nullptr) {
    if (nm) {
        if (act_type != lbq::TYPE_Q8_K) return hipErrorInvalidValue;
        return lbq::launch_rmsnorm_q8k(d_x, nm->w, nm->eps, m, k, const_cast<int8_t *>(av.xq), const_cast<float *>(av.xd),
                                       const_cast<int16_t *>(av.xbs), st, zero);
    }
    return lbq::launch_quant_act(act_type, d_x, m, k, const_cast<int8_t *>(av.xq), const_cast<float *>(av.xd),
                                 const_cast<int16_t *>(av.xbs), const_cast<float *>(av.xs), nullptr, st, zero);
}

// Device memory of one forward call: the quantised activations, then the batched
// GEMM's workspace.  Either the context's buffers, grown on demand (the caller
// holds ctx->mu), or one fixed region (the allocation-free entry point): the
// activations at its start, the workspace after them, both checked against its
// size before any launch.
struct Scratch {
    lbq_ctx *ctx = nullptr;
    uint8_t *fixed = nullptr;
    size_t fixed_bytes = 0;
    uint32_t *fixed_counters = nullptr;  // fixed region: its tile counters
    size_t act_used = 0;  // fixed region: bytes taken by the activations

    uint32_t *counters() const { return fixed ? fixed_counters : ctx->tile_counters; }

    int limit(size_t need) const {
        return fail(LBQ_ERR_LIMIT,
                    "the call needs %zu bytes of scratch; the allocation-free entry point has %zu per device", need,
                    fixed_bytes);
    }
    int act(size_t bytes, uint8_t **out) {
        if (!fixed) {
            const int s = ensure_scratch(ctx, bytes);
            *out = ctx->scratch;
            return s;
        }
        if (bytes > fixed_bytes) return limit(bytes);
        act_used = align_up(bytes, 256);
        *out = fixed;
        return LBQ_OK;
    }
    int ws(size_t bytes, uint8_t **out) {
        if (!fixed) {
            const int s = ensure_buffer(&ctx->ws, &ctx->ws_bytes, bytes, "GEMM workspace");
            *out = ctx->ws;
            return s;
        }
        if (act_used + bytes > fixed_bytes) return limit(act_used + bytes);
        *out = fixed + act_used;
        return LBQ_OK;
    }
};

// Batch decode on the matrix cores for this weight and row count
static bool uses_mx(const lbq_weight *w, int64_t m) { return m <= 64 && lbq::gemv_mx_serves(w->type, w->n, w->k, (int)m); }
// ... with its two split halves added into y, which the quantisation launch zeroes
static bool mx_adds(const lbq_weight *w, int64_t m) { return uses_mx(w, m) && lbq::gemv_mx_adds(w->type, w->n, w->k, (int)m); }

// Whether y[0, count) lies in plain device memory (hipMalloc: device resident, not
// managed, no allocation flags), where the matrix-core kernel's f32 atomic adds
// are defined; host-pinned, managed and fine-grained memory are not (the adds are
// built with -munsafe-fp-atomics).  Queried once per allocation: ranges found to
// qualify are remembered (at most 64, oldest dropped first).
static bool y_is_plain_device(const float *y, int64_t count) {
    static std::mutex mu;
    static std::vector<std::pair<uintptr_t, size_t>> known;
    const uintptr_t p = reinterpret_cast<uintptr_t>(y);
    const size_t bytes = (size_t)count * sizeof(float);
    {
        std::lock_guard<std::mutex> lock(mu);
        for (const auto &r : known)
            if (p >= r.first && p - r.first + bytes <= r.second) return true;
    }
    hipPointerAttribute_t a{};
    if (hipPointerGetAttributes(&a, y) != hipSuccess) {
        (void)hipGetLastError();  // an unknown pointer: not plain device memory
        return false;
    }
    if (a.type != hipMemoryTypeDevice || a.isManaged || a.allocationFlags != 0) return false;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, const_cast<float *>(y)) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    const uintptr_t b = reinterpret_cast<uintptr_t>(base);
    if (p < b || p - b + bytes > size) return false;
    std::lock_guard<std::mutex> lock(mu);
    if (known.size() >= 64) known.erase(known.begin());
    known.emplace_back(b, size);
    return true;
}

// adds y (m rows of w) to the quantisation launch's zero list where the
// matrix-core kernel adds into it; returns whether it did.  Outputs that are not
// plain device memory take the kernel's other protocol (partials and a tile
// counter in the workspace, the same bits).
static bool zero_for_mx(lbq::ZeroList &zl, const lbq_weight *w, int64_t m, float *y) {
    if (!mx_adds(w, m) || zl.count >= 4 || !y_is_plain_device(y, m * w->n)) return false;
    zl.p[zl.count] = y;
    zl.n[zl.count] = m * w->n;
    zl.count++;
    return true;
}

// The dot half of QMatMul::forward: decode GEMV for m <= 8 (the i8 matrix-core
// kernel at m = 5..8 where it serves), MFMA GEMM above.
int run_dot(Scratch &sc, const lbq_weight *w, const lbq::ActView &av, int64_t m, float *d_y, hipStream_t st,
            bool y_zeroed = false) {
    hipError_t e;
    if (uses_mx(w, m)) {
        const bool add = y_zeroed && mx_adds(w, m);
        const size_t wsb = add ? 0 : lbq::gemv_mx_workspace_bytes(w->type, w->n, w->k, (int)m);
        uint8_t *ws = nullptr;
        if (wsb) {
            int s = sc.ws(wsb, &ws);
            if (s) return s;
        }
        e = lbq::launch_gemv_mx(w->type, w->d_blocks, w->n, w->k, w->row_bytes, av, (int)m, d_y,
                                reinterpret_cast<float *>(ws), sc.counters(), st, add);
    } else if (m <= 8) {
        e = lbq::launch_gemv(w->type, w->d_blocks, w->n, w->k, w->row_bytes, av, (int)m, d_y, st);
    } else {
        const size_t wsb = lbq::gemm_workspace_bytes(w->type, w->n, w->k, m);
        uint8_t *ws = nullptr;
        if (wsb) {
            int s = sc.ws(wsb, &ws);
            if (s) return s;
        }
        e = lbq::launch_gemm(w->type, w->d_blocks, w->d_rexp, w->n, w->k, w->row_bytes, av, nullptr, m, d_y, ws,
                             sc.counters(), st);
    }
    if (e != hipSuccess) return hip_fail(e, "quantized matmul launch");
    return LBQ_OK;
}

// QMatMul::forward after the argument checks, on the caller's device; `mu`
// (the context's lock, null for the fixed region) is taken before any buffer is
// touched.
int forward(lbq_ctx *ctx, const lbq_weight *w, const float *d_x, int64_t m, float *d_y, hipStream_t st, Scratch &sc,
            std::mutex *mu) {
    const int act_type = lbq::vec_dot_type(w->type);
    if (lbq::is_dense(w->type)) {
        // candle's dense variant: an f32 matmul, no activation quantisation
        hipError_t e = lbq::launch_dense(w->type, w->d_blocks, w->n, w->k, d_x, m, d_y, st);
        return e == hipSuccess ? LBQ_OK : hip_fail(e, "dense matmul launch");
    }
    const ActLayout L = act_layout(act_type, m, w->k);
    if (m <= 8 && !uses_mx(w, m) && lbq::gemv_fuses_quant(w->type, w->n, w->k, (int)m, d_x)) {
        // decode: the GEMV quantises x in its own prologue -- one launch, no scratch
        const lbq::ActView av{nullptr, nullptr, nullptr, w->k, L.nb};
        hipError_t e = lbq::launch_gemv_x(w->type, w->d_blocks, w->n, w->k, w->row_bytes, av, d_x, (int)m, d_y, st);
        if (e != hipSuccess) return hip_fail(e, "quantized matmul launch");
        return LBQ_OK;
    }
    std::unique_lock<std::mutex> lock;
    if (mu) lock = std::unique_lock<std::mutex>(*mu);
    (void)ctx;
    if (m > 8 && !uses_mx(w, m) && lbq::gemm_prepass_fuses_quant(w->type, w->k, d_x)) {
        // batched: the operand pre-pass quantises x itself
        uint8_t *ws = nullptr;
        int s = sc.ws(lbq::gemm_workspace_bytes(w->type, w->n, w->k, m), &ws);
        if (s) return s;
        const lbq::ActView none{nullptr, nullptr, nullptr, w->k, L.nb};
        hipError_t e = lbq::launch_gemm(w->type, w->d_blocks, w->d_rexp, w->n, w->k, w->row_bytes, none, d_x, m, d_y, ws,
                                        sc.counters(), st);
        if (e != hipSuccess) return hip_fail(e, "quantized matmul launch");
        return LBQ_OK;
    }
    uint8_t *abuf = nullptr;
    int s = sc.act(L.total, &abuf);
    if (s) return s;
    lbq::ZeroList zl;
    const bool zeroed = zero_for_mx(zl, w, m, d_y);
    {  // reserve the GEMM's (or the matrix-core decode's) workspace too before anything is launched
        uint8_t *ws = nullptr;
        const size_t wsb = zeroed        ? 0
                           : uses_mx(w, m) ? lbq::gemv_mx_workspace_bytes(w->type, w->n, w->k, (int)m)
                           : m > 8       ? lbq::gemm_workspace_bytes(w->type, w->n, w->k, m)
                                         : 0;
        if (wsb && (s = sc.ws(wsb, &ws))) return s;
    }
    const lbq::ActView av = view_of(abuf, L, w->k);
    hipError_t e = quant_into(act_type, d_x, m, w->k, av, st, &zl);
    if (e != hipSuccess) return hip_fail(e, "activation quantisation launch");
    return run_dot(sc, w, av, m, d_y, st, zeroed);
}

// whether the f32 ranges [a, a + na) and [b, b + nb) share an element
static bool overlaps(const float *a, int64_t na, const float *b, int64_t nb) {
    const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
    return pa < pb + (uintptr_t)nb * sizeof(float) && pb < pa + (uintptr_t)na * sizeof(float);
}

int check_weight_args(uint32_t type, int64_t n, int64_t k, size_t nbytes) {
    if (!weight_type_ok(type)) return fail(LBQ_ERR_UNSUPPORTED_TYPE, "ggml type %u is not served (F32=0, F16=1, Q4_0=2, Q4_1=3, Q5_0=6, Q5_1=7, Q8_0=8, Q2_K=10, Q3_K=11, Q4_K=12, Q5_K=13, Q6_K=14, BF16=30)", type);
    const int bs = lbq_type_block_size(type);
    if (n <= 0 || k <= 0) return fail(LBQ_ERR_SHAPE, "weight shape (%lld, %lld) must be positive", (long long)n, (long long)k);
    if (k % bs) return fail(LBQ_ERR_SHAPE, "k = %lld is not a multiple of the %d-value block", (long long)k, bs);
    if (lbq::is_dense((int)type) && k % 8)
        return fail(LBQ_ERR_SHAPE, "k = %lld: dense weights need k to be a multiple of 8", (long long)k);
    if (k / bs > (1 << 24)) return fail(LBQ_ERR_LIMIT, "k = %lld exceeds the supported maximum", (long long)k);
    if (n > lbq::MAX_ROWS) return fail(LBQ_ERR_LIMIT, "n = %lld exceeds the supported maximum", (long long)n);
    const size_t want = (size_t)n * (size_t)(k / bs) * (size_t)lbq_type_block_bytes(type);
    if (nbytes != want)
        return fail(LBQ_ERR_SHAPE, "byte count %zu does not match n*(k/%d)*%d = %zu", nbytes, bs, lbq_type_block_bytes(type),
                    want);
    return LBQ_OK;
}

int make_weight(lbq_ctx *ctx, uint32_t type, int64_t n, int64_t k, const uint8_t *dev, size_t nbytes, bool owned,
                lbq_weight **out) {
    lbq_weight *w = new (std::nothrow) lbq_weight;
    if (!w) return fail(LBQ_ERR_OOM, "host allocation failed");
    w->ctx = ctx;
    w->type = (int)type;
    w->n = n;
    w->k = k;
    w->row_bytes = (k / lbq_type_block_size(type)) * lbq_type_block_bytes(type);
    w->nbytes = nbytes;
    w->d_blocks = dev;
    w->owned = owned;
    w->d_rexp = nullptr;
    if (lbq::gemm_serves((int)type, k)) {
        // the batched GEMM's per-row operand exponents, once per weight (load time):
        // wait for whatever wrote the blocks on any stream, then one small launch
        DeviceGuard g(ctx->device);
        hipError_t e = g.err != hipSuccess ? g.err : hipDeviceSynchronize();
        void *p = nullptr;
        if (e == hipSuccess) e = hipMalloc(&p, (size_t)n);
        if (e == hipSuccess) e = lbq::launch_row_exponents((int)type, dev, n, k, w->row_bytes, static_cast<int8_t *>(p), nullptr);
        if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess) {
            if (p) (void)hipFree(p);
            delete w;
            return hip_fail(e, "per-row exponents of the weight");
        }
        w->d_rexp = static_cast<int8_t *>(p);
    }
    *out = w;
    return LBQ_OK;
}

}  // namespace

// shared with lbq_gguf.cpp
int lbq_fail_status(int status, const char *msg) { return fail(status, "%s", msg); }
int lbq_ctx_device(const lbq_ctx *ctx) { return ctx->device; }
int lbq_make_owned_weight(lbq_ctx *ctx, uint32_t type, int64_t n, int64_t k, void *d_blocks, size_t nbytes,
                          lbq_weight **out) {
    const int s = check_weight_args(type, n, k, nbytes);
    if (s) return s;
    return make_weight(ctx, type, n, k, static_cast<const uint8_t *>(d_blocks), nbytes, true, out);
}

namespace {
// Per device: the address of `scratch` there, resolved once with the device current.
std::mutex g_noalloc_mu;
uint8_t *g_noalloc_ptr[64];

int noalloc_scratch_of(int device, uint8_t **out) {
    if (device >= 64) return fail(LBQ_ERR_LIMIT, "device %d: the allocation-free scratch covers devices 0..63", device);
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
        // the tile counters at the array's end start at zero; each launch that
        // uses them leaves them zero again
        e = hipMemset(static_cast<uint8_t *>(p) + NOALLOC_FIXED_BYTES, 0, NOALLOC_COUNTER_BYTES);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) return hip_fail(e, "clearing the allocation-free tile counters");
        g_noalloc_ptr[device] = static_cast<uint8_t *>(p);
    }
    *out = g_noalloc_ptr[device];
    return LBQ_OK;
}
}  // namespace

extern "C" {

const char *lbq_last_error(void) { return g_err.c_str(); }

int lbq_type_block_size(uint32_t t) {
    switch (t) {
    case LBQ_TYPE_F32: case LBQ_TYPE_F16: case LBQ_TYPE_BF16: return 1;
    case LBQ_TYPE_Q4_0: case LBQ_TYPE_Q4_1: case LBQ_TYPE_Q5_0: case LBQ_TYPE_Q5_1: case LBQ_TYPE_Q8_0: case LBQ_TYPE_Q8_1:
        return 32;
    case LBQ_TYPE_Q2_K: case LBQ_TYPE_Q3_K: case LBQ_TYPE_Q4_K: case LBQ_TYPE_Q5_K: case LBQ_TYPE_Q6_K: case LBQ_TYPE_Q8_K:
        return 256;
    default: return 0;
    }
}

int lbq_type_size(uint32_t t) {
    switch (t) {
    case LBQ_TYPE_F32: return 4;
    case LBQ_TYPE_F16: case LBQ_TYPE_BF16: return 2;
    case LBQ_TYPE_Q4_0: return 18;
    case LBQ_TYPE_Q4_1: return 20;
    case LBQ_TYPE_Q5_0: return 22;
    case LBQ_TYPE_Q5_1: return 24;
    case LBQ_TYPE_Q8_0: return 34;
    case LBQ_TYPE_Q8_1: return 36;
    case LBQ_TYPE_Q2_K: return 82;  // as GgmlDType::type_size; the block itself is 84 bytes
    case LBQ_TYPE_Q3_K: return 110;
    case LBQ_TYPE_Q4_K: return 144;
    case LBQ_TYPE_Q5_K: return 176;
    case LBQ_TYPE_Q6_K: return 210;
    case LBQ_TYPE_Q8_K: return 292;
    default: return 0;
    }
}

int lbq_type_block_bytes(uint32_t t) { return t == LBQ_TYPE_Q2_K ? 84 : lbq_type_size(t); }


int lbq_init(int device, lbq_ctx **out_ctx) {
    if (!out_ctx) return fail(LBQ_ERR_INVALID_ARG, "out_ctx is null");
    *out_ctx = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if (device < 0 || device >= count) return fail(LBQ_ERR_INVALID_ARG, "device %d out of range (%d devices)", device, count);
    DeviceGuard g(device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    uint8_t *noalloc = nullptr;
    const int s = noalloc_scratch_of(device, &noalloc);
    if (s) return s;
    lbq_ctx *c = new (std::nothrow) lbq_ctx;
    if (!c) return fail(LBQ_ERR_OOM, "host allocation failed");
    c->device = device;
    c->noalloc_scratch = noalloc;
    c->tune = lbq::tuning_from_env();
    c->scratch = nullptr;
    c->scratch_bytes = 0;
    c->ws = nullptr;
    c->ws_bytes = 0;
    c->tmp = nullptr;
    c->tmp_bytes = 0;
    c->tile_counters = nullptr;
    e = hipMalloc(&c->tile_counters, NOALLOC_COUNTER_BYTES);
    if (e == hipSuccess) e = hipMemset(c->tile_counters, 0, NOALLOC_COUNTER_BYTES);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e != hipSuccess) {
        if (c->tile_counters) (void)hipFree(c->tile_counters);
        delete c;
        return hip_fail(e, "tile counter allocation");
    }
    *out_ctx = c;
    return LBQ_OK;
}

int lbq_ctx_destroy(lbq_ctx *ctx) {
    if (!ctx) return LBQ_OK;
    DeviceGuard g(ctx->device);
    (void)hipDeviceSynchronize();
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->ws) (void)hipFree(ctx->ws);
    if (ctx->tmp) (void)hipFree(ctx->tmp);
    if (ctx->tile_counters) (void)hipFree(ctx->tile_counters);
    delete ctx;
    return LBQ_OK;
}

int lbq_weight_create(lbq_ctx *ctx, uint32_t type, int64_t n, int64_t k, const void *host_blocks, size_t nbytes,
                      lbq_weight **out_w) {
    if (!ctx || !host_blocks || !out_w) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_weight_create");
    *out_w = nullptr;
    int s = check_weight_args(type, n, k, nbytes);
    if (s) return s;
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    void *d = nullptr;
    hipError_t e = hipMalloc(&d, nbytes);
    if (e != hipSuccess) return fail(LBQ_ERR_OOM, "hipMalloc(%zu) for weight blocks: %s", nbytes, hipGetErrorString(e));
    e = hipMemcpy(d, host_blocks, nbytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return hip_fail(e, "hipMemcpy H2D of weight blocks");
    }
    s = make_weight(ctx, type, n, k, static_cast<const uint8_t *>(d), nbytes, true, out_w);
    if (s) (void)hipFree(d);
    return s;
}

int lbq_weight_wrap_device(lbq_ctx *ctx, uint32_t type, int64_t n, int64_t k, const void *d_blocks, size_t nbytes,
                           lbq_weight **out_w) {
    if (!ctx || !d_blocks || !out_w) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_weight_wrap_device");
    *out_w = nullptr;
    int s = check_weight_args(type, n, k, nbytes);
    if (s) return s;
    if (reinterpret_cast<uintptr_t>(d_blocks) & 15u)
        return fail(LBQ_ERR_INVALID_ARG, "device weight blocks must be 16-byte aligned");
    return make_weight(ctx, type, n, k, static_cast<const uint8_t *>(d_blocks), nbytes, false, out_w);
}

int lbq_weight_destroy(lbq_weight *w) {
    if (!w) return LBQ_OK;
    if (w->owned || w->d_rexp) {
        DeviceGuard g(w->ctx->device);
        if (w->owned) (void)hipFree(const_cast<uint8_t *>(w->d_blocks));
        if (w->d_rexp) (void)hipFree(w->d_rexp);
    }
    delete w;
    return LBQ_OK;
}

int lbq_weight_refresh(lbq_weight *w, void *stream) {
    if (!w) return fail(LBQ_ERR_INVALID_ARG, "null weight");
    if (!w->d_rexp) return LBQ_OK;  // no derived state for this type and k
    DeviceGuard g(w->ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipError_t e = lbq::launch_row_exponents(w->type, w->d_blocks, w->n, w->k, w->row_bytes, w->d_rexp,
                                             static_cast<hipStream_t>(stream));
    return e == hipSuccess ? LBQ_OK : hip_fail(e, "per-row exponents of the weight");
}

int lbq_weight_info(const lbq_weight *w, uint32_t *type, int64_t *n, int64_t *k) {
    if (!w) return fail(LBQ_ERR_INVALID_ARG, "null weight");
    if (type) *type = (uint32_t)w->type;
    if (n) *n = w->n;
    if (k) *k = w->k;
    return LBQ_OK;
}

int lbq_qmatmul_f32(lbq_ctx *ctx, const lbq_weight *w, const float *d_x, int64_t m, float *d_y, void *stream) {
    if (!ctx || !w) return fail(LBQ_ERR_INVALID_ARG, "null context or weight");
    if (m < 0) return fail(LBQ_ERR_INVALID_ARG, "m = %lld is negative", (long long)m);
    if (m == 0) return LBQ_OK;
    if (!d_x || !d_y) return fail(LBQ_ERR_INVALID_ARG, "null activation or output pointer");
    if ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_y)) & 3u)
        return fail(LBQ_ERR_INVALID_ARG, "x and y must be 4-byte aligned f32 buffers");
    if (m > (int64_t)1 << 24) return fail(LBQ_ERR_LIMIT, "m = %lld exceeds the supported maximum", (long long)m);
    if (overlaps(d_x, m * w->k, d_y, m * w->n)) return fail(LBQ_ERR_INVALID_ARG, "x and y overlap");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    Scratch sc;
    sc.ctx = ctx;
    return forward(ctx, w, d_x, m, d_y, static_cast<hipStream_t>(stream), sc, &ctx->mu);
}

int lbq_qmatmul_f32_noalloc(lbq_ctx *ctx, const lbq_weight *w, const float *d_x, int64_t m, float *d_y,
                            void *stream) {
    if (!ctx || !w) return fail(LBQ_ERR_INVALID_ARG, "null context or weight");
    if (m < 0) return fail(LBQ_ERR_INVALID_ARG, "m = %lld is negative", (long long)m);
    if (m == 0) return LBQ_OK;
    if (!d_x || !d_y) return fail(LBQ_ERR_INVALID_ARG, "null activation or output pointer");
    if ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_y)) & 3u)
        return fail(LBQ_ERR_INVALID_ARG, "x and y must be 4-byte aligned f32 buffers");
    if (m > (int64_t)1 << 24) return fail(LBQ_ERR_LIMIT, "m = %lld exceeds the supported maximum", (long long)m);
    if (overlaps(d_x, m * w->k, d_y, m * w->n)) return fail(LBQ_ERR_INVALID_ARG, "x and y overlap");
    if (!ctx->noalloc_scratch) return fail(LBQ_ERR_INVALID_ARG, "context has no allocation-free scratch");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    // every buffer the kernels need comes from this device's `scratch` (through
    // the address lbq_init resolved); nothing is allocated and nothing needs
    // clearing: each kernel writes every scratch byte it later reads, and the
    // tile counters at the array's end were zeroed at lbq_init and are left zero
    // by every launch
    Scratch sc;
    sc.ctx = ctx;
    sc.fixed = ctx->noalloc_scratch;
    sc.fixed_bytes = NOALLOC_FIXED_BYTES;
    sc.fixed_counters = reinterpret_cast<uint32_t *>(ctx->noalloc_scratch + NOALLOC_FIXED_BYTES);
    return forward(ctx, w, d_x, m, d_y, static_cast<hipStream_t>(stream), sc, nullptr);
}

namespace {
int group_f32(lbq_ctx *ctx, const lbq_weight *const *ws, int count, const float *d_x, int64_t m, float *const *d_ys,
              void *stream, const NormArg *nm);
}  // namespace

int lbq_qmatmul_group_f32(lbq_ctx *ctx, const lbq_weight *const *ws, int count, const float *d_x, int64_t m,
                          float *const *d_ys, void *stream) {
    return group_f32(ctx, ws, count, d_x, m, d_ys, stream, nullptr);
}

namespace {
// lbq_qmatmul_group_f32; with nm, of candle's RmsNorm of x, normalised and quantised
// in one launch (the caller has checked that every weight takes pre-quantised
// Q8_K activations: rmsnorm_fuses)
int group_f32(lbq_ctx *ctx, const lbq_weight *const *ws, int count, const float *d_x, int64_t m, float *const *d_ys,
              void *stream, const NormArg *nm) {
    if (!ctx || !ws || !d_ys) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_qmatmul_group_f32");
    if (count < 1 || count > LBQ_GROUP_MAX) return fail(LBQ_ERR_LIMIT, "count = %d outside 1..%d", count, LBQ_GROUP_MAX);
    if (m < 0) return fail(LBQ_ERR_INVALID_ARG, "m = %lld is negative", (long long)m);
    for (int i = 0; i < count; i++) {
        if (!ws[i] || !d_ys[i]) return fail(LBQ_ERR_INVALID_ARG, "null weight or output %d", i);
        if (reinterpret_cast<uintptr_t>(d_ys[i]) & 3u) return fail(LBQ_ERR_INVALID_ARG, "output %d must be a 4-byte aligned f32 buffer", i);
        if (ws[i]->type != ws[0]->type || ws[i]->k != ws[0]->k)
            return fail(LBQ_ERR_SHAPE, "weight %d (type %d, k = %lld) differs from weight 0 (type %d, k = %lld)", i, ws[i]->type,
                        (long long)ws[i]->k, ws[0]->type, (long long)ws[0]->k);
    }
    if (m == 0) return LBQ_OK;
    if (!d_x) return fail(LBQ_ERR_INVALID_ARG, "null activation pointer");
    if (reinterpret_cast<uintptr_t>(d_x) & 3u) return fail(LBQ_ERR_INVALID_ARG, "x must be a 4-byte aligned f32 buffer");
    if (m > (int64_t)1 << 24) return fail(LBQ_ERR_LIMIT, "m = %lld exceeds the supported maximum", (long long)m);
    for (int i = 0; i < count; i++)
        if (overlaps(d_x, m * ws[0]->k, d_ys[i], m * ws[i]->n)) return fail(LBQ_ERR_INVALID_ARG, "x and output %d overlap", i);
    const lbq_weight *w0 = ws[0];
    const int act_type = lbq::vec_dot_type(w0->type);
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (lbq::is_dense(w0->type)) {
        for (int i = 0; i < count; i++) {
            hipError_t e = lbq::launch_dense(ws[i]->type, ws[i]->d_blocks, ws[i]->n, ws[i]->k, d_x, m, d_ys[i], st);
            if (e != hipSuccess) return hip_fail(e, "dense matmul launch");
        }
        return LBQ_OK;
    }
    const ActLayout L = act_layout(act_type, m, w0->k);
    // m = 1: every weight's rows in one launch (one row space)
    lbq::RowMap rm = lbq::single_row_map(w0->d_blocks, w0->n, d_ys[0]);
    int64_t rows = 0;
    for (int i = 0; i < count; i++) {
        rm.w[i] = ws[i]->d_blocks;
        rm.y[i] = d_ys[i];
        rows += ws[i]->n;
        rm.end[i] = (int32_t)std::min<int64_t>(rows, lbq::MAX_ROWS);
    }
    rm.n = rows;
    const bool one_launch = rows <= lbq::MAX_ROWS;  // else weight by weight
    if (!nm && one_launch && m == 1 && lbq::gemv_fuses_quant(w0->type, rows, w0->k, 1, d_x)) {
        const lbq::ActView av{nullptr, nullptr, nullptr, w0->k, L.nb};
        hipError_t e = lbq::launch_gemv_group(w0->type, rm, w0->k, w0->row_bytes, av, d_x, st);
        if (e != hipErrorNotSupported) return e == hipSuccess ? LBQ_OK : hip_fail(e, "grouped matmul launch");
    }
    std::lock_guard<std::mutex> lock(ctx->mu);
    bool all_mx = true;  // every weight on the integer matrix-core kernel: x quantised once below
    for (int i = 0; i < count; i++) all_mx = all_mx && uses_mx(ws[i], m);
    if (m > 8 && !all_mx && lbq::gemm_serves(w0->type, w0->k)) {
        if (nm) return fail(LBQ_ERR_INVALID_ARG, "internal: the fused norm needs pre-quantised activations");
        // batched: one operand pre-pass (quantising x itself when it can) shared
        // by every weight's GEMM; weights on the integer matrix-core kernel share
        // one Q8_K quantisation of x and run after the GEMMs (their split partials
        // reuse the workspace the pre-pass operands occupy)
        size_t wsb = 0;
        bool mx[LBQ_GROUP_MAX], any_mx = false;
        for (int i = 0; i < count; i++) {
            mx[i] = uses_mx(ws[i], m);
            any_mx = any_mx || mx[i];
            wsb = std::max(wsb, mx[i] ? lbq::gemv_mx_workspace_bytes(w0->type, ws[i]->n, w0->k, (int)m)
                                      : lbq::gemm_workspace_bytes(w0->type, ws[i]->n, w0->k, m));
        }
        int s = ensure_buffer(&ctx->ws, &ctx->ws_bytes, wsb, "GEMM workspace");
        if (s) return s;
        bool in_kernel[LBQ_GROUP_MAX], all_in_kernel = true;
        for (int i = 0; i < count; i++) {
            in_kernel[i] = !mx[i] && lbq::gemm_quantises_in_kernel(w0->type, ws[i]->n, w0->k, m, d_x);
            all_in_kernel = all_in_kernel && (mx[i] || in_kernel[i]);
        }
        const bool fused_prepass = !all_in_kernel && lbq::gemm_prepass_fuses_quant(w0->type, w0->k, d_x);
        lbq::ZeroList zl;
        bool zeroed[LBQ_GROUP_MAX];
        for (int i = 0; i < count; i++) zeroed[i] = mx[i] && zero_for_mx(zl, ws[i], m, d_ys[i]);
        if ((any_mx || (!all_in_kernel && !fused_prepass)) && (s = ensure_scratch(ctx, L.total))) return s;
        const lbq::ActView av = ctx->scratch ? view_of(ctx->scratch, L, w0->k) : lbq::ActView{nullptr, nullptr, nullptr, w0->k, L.nb};
        bool quantised = false;
        hipError_t e = hipSuccess;
        if (all_in_kernel) {
            // every GEMM weight's k-sliced kernel quantises x itself
        } else if (fused_prepass) {
            const lbq::ActView none{nullptr, nullptr, nullptr, w0->k, L.nb};
            e = lbq::gemm_prepass(w0->type, w0->k, none, d_x, m, ctx->ws, st);
        } else {
            e = quant_into(act_type, d_x, m, w0->k, av, st, &zl);
            quantised = true;
            if (e == hipSuccess) e = lbq::gemm_prepass(w0->type, w0->k, av, nullptr, m, ctx->ws, st);
        }
        if (e != hipSuccess) return hip_fail(e, "operand pre-pass launch");
        for (int i = 0; i < count; i++) {
            if (mx[i]) continue;
            e = lbq::gemm_main(w0->type, ws[i]->d_blocks, ws[i]->d_rexp, ws[i]->n, w0->k, w0->row_bytes, m, d_ys[i],
                               ctx->ws, ctx->tile_counters, in_kernel[i] ? d_x : nullptr, st);
            if (e != hipSuccess) return hip_fail(e, "grouped matmul launch");
        }
        if (!any_mx) return LBQ_OK;
        if (!quantised && (e = quant_into(act_type, d_x, m, w0->k, av, st, &zl)) != hipSuccess)
            return hip_fail(e, "activation quantisation launch");
        for (int i = 0; i < count; i++) {
            if (!mx[i]) continue;
            Scratch sc;
            sc.ctx = ctx;
            if ((s = run_dot(sc, ws[i], av, m, d_ys[i], st, zeroed[i]))) return s;
        }
        return LBQ_OK;
    }
    // otherwise x is quantised once into the context's scratch and shared by
    // one launch per weight
    int s = ensure_scratch(ctx, L.total);
    if (s) return s;
    const lbq::ActView av = view_of(ctx->scratch, L, w0->k);
    lbq::ZeroList zl;
    bool zeroed[LBQ_GROUP_MAX];
    for (int i = 0; i < count; i++) zeroed[i] = zero_for_mx(zl, ws[i], m, d_ys[i]);
    hipError_t e = quant_into(act_type, d_x, m, w0->k, av, st, &zl, nm);
    if (e != hipSuccess) return hip_fail(e, "activation quantisation launch");
    bool one = count >= 2;  // every weight on the matrix-core kernel: one launch for all
    for (int i = 0; i < count; i++) one = one && uses_mx(ws[i], m) && (!mx_adds(ws[i], m) || zeroed[i]);
    if (one) {
        const uint8_t *wp[LBQ_GROUP_MAX];
        int64_t ns[LBQ_GROUP_MAX];
        for (int i = 0; i < count; i++) {
            wp[i] = ws[i]->d_blocks;
            ns[i] = ws[i]->n;
        }
        e = lbq::launch_gemv_mx_group(w0->type, count, wp, ns, w0->k, w0->row_bytes, av, (int)m, d_ys, st);
        if (e == hipSuccess) return LBQ_OK;
        if (e != hipErrorNotSupported) return hip_fail(e, "grouped matmul launch");
    }
    for (int i = 0; i < count; i++) {
        Scratch sc;
        sc.ctx = ctx;
        s = run_dot(sc, ws[i], av, m, d_ys[i], st, zeroed[i]);
        if (s) return s;
    }
    return LBQ_OK;
}

// lbq_gate_up_silu_f32; with nm, of candle's RmsNorm of x (as group_f32)
int gate_up_f32(lbq_ctx *ctx, const lbq_weight *w_gate, const lbq_weight *w_up, const float *d_x, int64_t m,
                float *d_out, void *stream, const NormArg *nm) {
    if (!ctx || !w_gate || !w_up || !d_out) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_gate_up_silu_f32");
    if (w_gate->type != w_up->type || w_gate->n != w_up->n || w_gate->k != w_up->k)
        return fail(LBQ_ERR_SHAPE, "gate (type %d, %lld x %lld) and up (type %d, %lld x %lld) differ", w_gate->type,
                    (long long)w_gate->n, (long long)w_gate->k, w_up->type, (long long)w_up->n, (long long)w_up->k);
    if (m < 0) return fail(LBQ_ERR_INVALID_ARG, "m = %lld is negative", (long long)m);
    if (m == 0) return LBQ_OK;
    if (!d_x) return fail(LBQ_ERR_INVALID_ARG, "null activation pointer");
    if ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_out)) & 3u)
        return fail(LBQ_ERR_INVALID_ARG, "x and out must be 4-byte aligned f32 buffers");
    if (m > (int64_t)1 << 24) return fail(LBQ_ERR_LIMIT, "m = %lld exceeds the supported maximum", (long long)m);
    if (w_gate->n > lbq::MAX_ROWS / 2) return fail(LBQ_ERR_LIMIT, "n = %lld exceeds the supported maximum", (long long)w_gate->n);
    if (overlaps(d_x, m * w_gate->k, d_out, m * w_gate->n)) return fail(LBQ_ERR_INVALID_ARG, "x and out overlap");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!nm && m == 1 && lbq::gemv_fuses_quant(w_gate->type, 2 * w_gate->n, w_gate->k, 1, d_x)) {
        // one launch: both weights' rows interleaved, the product in the epilogue
        hipError_t e = lbq::launch_gemv_silu_pair(w_gate->type, w_gate->d_blocks, w_up->d_blocks, w_gate->n, w_gate->k,
                                                  w_gate->row_bytes, d_x, d_out, st);
        if (e != hipErrorNotSupported) return e == hipSuccess ? LBQ_OK : hip_fail(e, "gate/up launch");
    }
    if (m >= 2 && lbq::gemv_mx_pair_serves(w_gate->type, w_gate->n, w_gate->k, (int)m)) {
        // one Q8_K quantisation, then both weights and the product in one launch
        std::lock_guard<std::mutex> lock(ctx->mu);
        const ActLayout L = act_layout(lbq::vec_dot_type(w_gate->type), m, w_gate->k);
        int s = ensure_scratch(ctx, L.total);
        if (s) return s;
        const lbq::ActView av = view_of(ctx->scratch, L, w_gate->k);
        hipError_t e = quant_into(L.act_type, d_x, m, w_gate->k, av, st, nullptr, nm);
        if (e == hipSuccess)
            e = lbq::launch_gemv_mx_pair(w_gate->type, w_gate->d_blocks, w_up->d_blocks, w_gate->n, w_gate->k,
                                         w_gate->row_bytes, av, (int)m, d_out, st);
        return e == hipSuccess ? LBQ_OK : hip_fail(e, "gate/up launch");
    }
    // otherwise gate and up through the grouped path into context memory, then
    // one elementwise launch
    const size_t half = ((size_t)m * (size_t)w_gate->n * sizeof(float) + 255) / 256 * 256;
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        int s = ensure_buffer(&ctx->tmp, &ctx->tmp_bytes, 2 * half, "gate/up outputs");
        if (s) return s;
    }
    float *gy = reinterpret_cast<float *>(ctx->tmp), *uy = reinterpret_cast<float *>(ctx->tmp + half);
    const lbq_weight *pair[2] = {w_gate, w_up};
    float *outs[2] = {gy, uy};
    int s = group_f32(ctx, pair, 2, d_x, m, outs, stream, nm);
    if (s) return s;
    hipError_t e = lbq::launch_silu_mul(gy, uy, m * w_gate->n, d_out, st);
    if (e != hipSuccess) return hip_fail(e, "silu-mul launch");
    return LBQ_OK;
}
}  // namespace

int lbq_gate_up_silu_f32(lbq_ctx *ctx, const lbq_weight *w_gate, const lbq_weight *w_up, const float *d_x, int64_t m,
                         float *d_out, void *stream) {
    return gate_up_f32(ctx, w_gate, w_up, d_x, m, d_out, stream, nullptr);
}

int lbq_rmsnorm_f32(const float *d_x, const float *d_w, float eps, int64_t m, int64_t k, float *d_y, void *stream) {
    if (!d_x || !d_w || !d_y) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_rmsnorm_f32");
    if (m < 0 || k <= 0) return fail(LBQ_ERR_SHAPE, "rmsnorm shape (%lld, %lld) invalid", (long long)m, (long long)k);
    if ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_w) | reinterpret_cast<uintptr_t>(d_y)) & 3u)
        return fail(LBQ_ERR_INVALID_ARG, "x, w and y must be 4-byte aligned f32 buffers");
    if (m > (int64_t)1 << 24) return fail(LBQ_ERR_LIMIT, "m = %lld exceeds the supported maximum", (long long)m);
    hipError_t e = lbq::launch_rmsnorm(d_x, d_w, eps, m, k, d_y, static_cast<hipStream_t>(stream));
    return e == hipSuccess ? LBQ_OK : hip_fail(e, "rmsnorm launch");
}

namespace {
// x_norm = rmsnorm(x) in the context's gate/up memory (first m*k floats of tmp,
// after `skip` bytes); the caller holds no lock
int norm_into_tmp(lbq_ctx *ctx, const float *d_x, const float *d_w, float eps, int64_t m, int64_t k, size_t skip,
                  hipStream_t st, float **out) {
    const size_t need = skip + (size_t)m * (size_t)k * sizeof(float);
    {
        std::lock_guard<std::mutex> lock(ctx->mu);
        int s = ensure_buffer(&ctx->tmp, &ctx->tmp_bytes, need, "normalised activations");
        if (s) return s;
    }
    *out = reinterpret_cast<float *>(ctx->tmp + skip);
    hipError_t e = lbq::launch_rmsnorm(d_x, d_w, eps, m, k, *out, st);
    return e == hipSuccess ? LBQ_OK : hip_fail(e, "rmsnorm launch");
}

// Whether the RMS norm can run in the Q8_K quantisation launch (launch_rmsnorm_q8k)
// instead of a launch of its own: Q8_K activations, k up to 64 blocks, 16-byte
// aligned x and norm weight, and every weight on a path that reads pre-quantised
// activations (m <= 8, or the integer matrix-core kernel) -- not the fp16 GEMM's
// pre-pass or in-kernel quantisation, which read f32 x.
bool rmsnorm_fuses(const lbq_weight *const *ws, int count, const float *d_x, const float *d_w, int64_t m) {
    const lbq_weight *w0 = ws[0];
    if (lbq::is_dense(w0->type) || lbq::vec_dot_type(w0->type) != lbq::TYPE_Q8_K) return false;
    if (w0->k % 256 || w0->k / 256 > 64) return false;
    if ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_w)) & 15u) return false;
    if (m <= 8) return true;
    for (int i = 0; i < count; i++)
        if (!uses_mx(ws[i], m)) return false;
    return true;
}
}  // namespace

int lbq_rmsnorm_qmatmul_group_f32(lbq_ctx *ctx, const lbq_weight *const *ws, int count, const float *d_x,
                                  const float *d_norm_w, float eps, int64_t m, float *const *d_ys, void *stream) {
    if (!ctx || !ws || !d_ys || !d_norm_w) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_rmsnorm_qmatmul_group_f32");
    if (count < 1 || count > LBQ_GROUP_MAX) return fail(LBQ_ERR_LIMIT, "count = %d outside 1..%d", count, LBQ_GROUP_MAX);
    for (int i = 0; i < count; i++) {
        if (!ws[i] || !d_ys[i]) return fail(LBQ_ERR_INVALID_ARG, "null weight or output %d", i);
        if (ws[i]->type != ws[0]->type || ws[i]->k != ws[0]->k)
            return fail(LBQ_ERR_SHAPE, "weight %d differs from weight 0 in type or k", i);
    }
    if (m < 0) return fail(LBQ_ERR_INVALID_ARG, "m = %lld is negative", (long long)m);
    if (m == 0) return LBQ_OK;
    if (!d_x || ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_norm_w)) & 3u))
        return fail(LBQ_ERR_INVALID_ARG, "x and the norm weight must be 4-byte aligned f32 buffers");
    for (int i = 0; i < count; i++)
        if (overlaps(d_x, m * ws[0]->k, d_ys[i], m * ws[i]->n)) return fail(LBQ_ERR_INVALID_ARG, "x and output %d overlap", i);
    const lbq_weight *w0 = ws[0];
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    hipStream_t st = static_cast<hipStream_t>(stream);
    int64_t rows = 0;
    for (int i = 0; i < count; i++) rows += ws[i]->n;
    if (m == 1 && rows <= lbq::MAX_ROWS && !((reinterpret_cast<uintptr_t>(d_norm_w)) & 15u) &&
        lbq::gemv_fuses_quant(w0->type, rows, w0->k, 1, d_x)) {
        // one launch: the norm and the quantisation in the GEMV prologue
        lbq::RowMap rm = lbq::single_row_map(w0->d_blocks, w0->n, d_ys[0]);
        int64_t r = 0;
        for (int i = 0; i < count; i++) {
            rm.w[i] = ws[i]->d_blocks;
            rm.y[i] = d_ys[i];
            r += ws[i]->n;
            rm.end[i] = (int32_t)r;
        }
        rm.n = rows;
        const int act_type = lbq::vec_dot_type(w0->type);
        const lbq::ActView none{nullptr, nullptr, nullptr, w0->k, act_layout(act_type, 1, w0->k).nb};
        hipError_t e = lbq::launch_gemv_group(w0->type, rm, w0->k, w0->row_bytes, none, d_x, st, d_norm_w, eps);
        if (e != hipErrorNotSupported) return e == hipSuccess ? LBQ_OK : hip_fail(e, "grouped matmul launch");
    }
    if (rmsnorm_fuses(ws, count, d_x, d_norm_w, m)) {  // the norm in the quantisation launch
        const NormArg nm{d_norm_w, eps};
        return group_f32(ctx, ws, count, d_x, m, d_ys, stream, &nm);
    }
    float *xn;
    int s = norm_into_tmp(ctx, d_x, d_norm_w, eps, m, w0->k, 0, st, &xn);
    if (s) return s;
    return lbq_qmatmul_group_f32(ctx, ws, count, xn, m, d_ys, stream);
}

int lbq_rmsnorm_gate_up_silu_f32(lbq_ctx *ctx, const lbq_weight *w_gate, const lbq_weight *w_up, const float *d_x,
                                 const float *d_norm_w, float eps, int64_t m, float *d_out, void *stream) {
    if (!ctx || !w_gate || !w_up || !d_out || !d_norm_w)
        return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_rmsnorm_gate_up_silu_f32");
    if (w_gate->type != w_up->type || w_gate->n != w_up->n || w_gate->k != w_up->k)
        return fail(LBQ_ERR_SHAPE, "gate and up differ in type or shape");
    if (m < 0) return fail(LBQ_ERR_INVALID_ARG, "m = %lld is negative", (long long)m);
    if (m == 0) return LBQ_OK;
    if (!d_x || ((reinterpret_cast<uintptr_t>(d_x) | reinterpret_cast<uintptr_t>(d_norm_w) |
                  reinterpret_cast<uintptr_t>(d_out)) & 3u))
        return fail(LBQ_ERR_INVALID_ARG, "x, the norm weight and out must be 4-byte aligned f32 buffers");
    if (w_gate->n > lbq::MAX_ROWS / 2) return fail(LBQ_ERR_LIMIT, "n = %lld exceeds the supported maximum", (long long)w_gate->n);
    if (overlaps(d_x, m * w_gate->k, d_out, m * w_gate->n)) return fail(LBQ_ERR_INVALID_ARG, "x and out overlap");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (m == 1 && !((reinterpret_cast<uintptr_t>(d_norm_w)) & 15u) &&
        lbq::gemv_fuses_quant(w_gate->type, 2 * w_gate->n, w_gate->k, 1, d_x)) {
        hipError_t e = lbq::launch_gemv_silu_pair(w_gate->type, w_gate->d_blocks, w_up->d_blocks, w_gate->n,
                                                  w_gate->k, w_gate->row_bytes, d_x, d_out, st, d_norm_w, eps);
        if (e != hipErrorNotSupported) return e == hipSuccess ? LBQ_OK : hip_fail(e, "gate/up launch");
    }
    const lbq_weight *pair[2] = {w_gate, w_up};
    if (rmsnorm_fuses(pair, 2, d_x, d_norm_w, m)) {  // the norm in the quantisation launch
        const NormArg nm{d_norm_w, eps};
        return gate_up_f32(ctx, w_gate, w_up, d_x, m, d_out, stream, &nm);
    }
    // the normalised x sits after the gate/up halves lbq_gate_up_silu_f32 uses
    const size_t half = ((size_t)m * (size_t)w_gate->n * sizeof(float) + 255) / 256 * 256;
    float *xn;
    int s = norm_into_tmp(ctx, d_x, d_norm_w, eps, m, w_gate->k, 2 * half, st, &xn);
    if (s) return s;
    return lbq_gate_up_silu_f32(ctx, w_gate, w_up, xn, m, d_out, stream);
}

int lbq_act_create(lbq_ctx *ctx, uint32_t act_type, int64_t m, int64_t k, lbq_act **out_act) {
    if (!ctx || !out_act) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_act_create");
    *out_act = nullptr;
    if (!act_type_ok(act_type))
        return fail(LBQ_ERR_UNSUPPORTED_TYPE, "activation type %u must be Q8_K (15), Q8_0 (8) or Q8_1 (9)", act_type);
    const int bs = lbq_type_block_size(act_type);
    if (m <= 0 || k <= 0 || k % bs) return fail(LBQ_ERR_SHAPE, "activation shape (%lld, %lld) invalid for %d-value blocks", (long long)m, (long long)k, bs);
    if (m > (int64_t)1 << 24 || k / bs > (1 << 24)) return fail(LBQ_ERR_LIMIT, "activation shape exceeds the supported maximum");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    const ActLayout L = act_layout((int)act_type, m, k);
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, L.total);
    if (e != hipSuccess) return fail(LBQ_ERR_OOM, "hipMalloc(%zu) for activations: %s", L.total, hipGetErrorString(e));
    lbq_act *a = new (std::nothrow) lbq_act;
    if (!a) {
        (void)hipFree(p);
        return fail(LBQ_ERR_OOM, "host allocation failed");
    }
    a->ctx = ctx;
    a->act_type = (int)act_type;
    a->m = m;
    a->k = k;
    a->buf = static_cast<uint8_t *>(p);
    a->view = view_of(a->buf, L, k);
    *out_act = a;
    return LBQ_OK;
}

int lbq_act_quantize(lbq_act *a, const float *d_x, void *stream) {
    if (!a || !d_x) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_act_quantize");
    if (reinterpret_cast<uintptr_t>(d_x) & 3u) return fail(LBQ_ERR_INVALID_ARG, "x must be a 4-byte aligned f32 buffer");
    DeviceGuard g(a->ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    hipError_t e = quant_into(a->act_type, d_x, a->m, a->k, a->view, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "activation quantisation launch");
    return LBQ_OK;
}

int lbq_act_destroy(lbq_act *a) {
    if (!a) return LBQ_OK;
    DeviceGuard g(a->ctx->device);
    (void)hipFree(a->buf);
    delete a;
    return LBQ_OK;
}

int lbq_qmatmul_act_f32(lbq_ctx *ctx, const lbq_weight *w, const lbq_act *a, float *d_y, void *stream) {
    if (!ctx || !w || !a || !d_y) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_qmatmul_act_f32");
    if (reinterpret_cast<uintptr_t>(d_y) & 3u) return fail(LBQ_ERR_INVALID_ARG, "y must be a 4-byte aligned f32 buffer");
    if (lbq::is_dense(w->type))
        return fail(LBQ_ERR_UNSUPPORTED_TYPE, "dense weight (type %d) takes f32 activations: use lbq_qmatmul_f32", w->type);
    const int want = lbq::vec_dot_type(w->type);
    if (a->act_type != want) return fail(LBQ_ERR_UNSUPPORTED_TYPE, "weight type %d needs activation type %d, got %d", w->type, want, a->act_type);
    if (a->k != w->k) return fail(LBQ_ERR_SHAPE, "activation k = %lld, weight k = %lld", (long long)a->k, (long long)w->k);
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    std::lock_guard<std::mutex> lock(ctx->mu);
    Scratch sc;
    sc.ctx = ctx;
    return run_dot(sc, w, a->view, a->m, d_y, static_cast<hipStream_t>(stream));
}

int lbq_dequantize_f32(lbq_ctx *ctx, const lbq_weight *w, float *d_y, void *stream) {
    if (!ctx || !w || !d_y) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_dequantize_f32");
    if (reinterpret_cast<uintptr_t>(d_y) & 15u) return fail(LBQ_ERR_INVALID_ARG, "output must be 16-byte aligned");
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    hipError_t e = lbq::launch_dequant(w->type, w->d_blocks, w->n * w->k, d_y, static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    return LBQ_OK;
}

int lbq_dequantize_blocks_f32(uint32_t type, const void *d_blocks, int64_t nelem, float *d_y, void *stream) {
    if (!d_blocks || !d_y) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_dequantize_blocks_f32");
    if (!weight_type_ok(type) && !act_type_ok(type) && type != LBQ_TYPE_F32 && type != LBQ_TYPE_F16)
        return fail(LBQ_ERR_UNSUPPORTED_TYPE, "ggml type %u is not served", type);
    const int bs = lbq_type_block_size(type);
    if (nelem < 0 || nelem % bs) return fail(LBQ_ERR_SHAPE, "nelem = %lld is not a multiple of %d", (long long)nelem, bs);
    if ((reinterpret_cast<uintptr_t>(d_blocks) & 3u) || (reinterpret_cast<uintptr_t>(d_y) & 15u))
        return fail(LBQ_ERR_INVALID_ARG, "blocks must be 4-byte aligned and output 16-byte aligned");
    if (nelem == 0) return LBQ_OK;
    hipError_t e = lbq::launch_dequant((int)type, static_cast<const uint8_t *>(d_blocks), nelem, d_y,
                                       static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "dequantize launch");
    return LBQ_OK;
}

int lbq_embedding_f32(lbq_ctx *ctx, const lbq_weight *w, const int32_t *d_ids, int64_t count, float *d_out,
                      void *stream) {
    if (!ctx || !w) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_embedding_f32");
    if (count < 0) return fail(LBQ_ERR_INVALID_ARG, "count = %lld is negative", (long long)count);
    if (w->k % 16) return fail(LBQ_ERR_SHAPE, "k = %lld is not a multiple of 16", (long long)w->k);
    if (count == 0) return LBQ_OK;
    if (!d_ids || !d_out) return fail(LBQ_ERR_INVALID_ARG, "null ids or output pointer");
    if ((reinterpret_cast<uintptr_t>(d_ids) & 3u) || (reinterpret_cast<uintptr_t>(d_out) & 15u))
        return fail(LBQ_ERR_INVALID_ARG, "ids must be 4-byte and the output 16-byte aligned");
    if (count > ((int64_t)1 << 40) / w->k) return fail(LBQ_ERR_LIMIT, "count = %lld exceeds the supported maximum", (long long)count);
    DeviceGuard g(ctx->device);
    if (g.err != hipSuccess) return hip_fail(g.err, "hipSetDevice");
    lbq::TuningScope tsc(&ctx->tune);
    hipError_t e = lbq::launch_embedding(w->type, w->d_blocks, w->n, w->k, w->row_bytes, d_ids, count, d_out,
                                         static_cast<hipStream_t>(stream));
    return e == hipSuccess ? LBQ_OK : hip_fail(e, "embedding launch");
}

int lbq_quantize_act(uint32_t act_type, const float *d_x, int64_t m, int64_t k, void *d_out_blocks, void *stream) {
    if (!d_x || !d_out_blocks) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_quantize_act");
    if (!act_type_ok(act_type))
        return fail(LBQ_ERR_UNSUPPORTED_TYPE, "activation type %u must be Q8_K (15), Q8_0 (8) or Q8_1 (9)", act_type);
    const int bs = lbq_type_block_size(act_type);
    if (m < 0 || k <= 0 || k % bs) return fail(LBQ_ERR_SHAPE, "k = %lld is not a positive multiple of %d", (long long)k, bs);
    if ((reinterpret_cast<uintptr_t>(d_x) & 3u) || (reinterpret_cast<uintptr_t>(d_out_blocks) & 3u))
        return fail(LBQ_ERR_INVALID_ARG, "x and the output blocks must be 4-byte aligned");
    if (m == 0) return LBQ_OK;
    hipError_t e = lbq::launch_quant_act((int)act_type, d_x, m, k, nullptr, nullptr, nullptr, nullptr,
                                         static_cast<uint8_t *>(d_out_blocks), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "activation quantisation launch");
    return LBQ_OK;
}

int lbq_quantize_weights_f32(uint32_t type, const float *d_w, int64_t nelem, void *d_out_blocks, void *stream) {
    if (!d_w || !d_out_blocks) return fail(LBQ_ERR_INVALID_ARG, "null argument to lbq_quantize_weights_f32");
    if (!weight_type_ok(type) || type == LBQ_TYPE_Q2_K || type == LBQ_TYPE_Q3_K || lbq::is_dense((int)type))
        return fail(LBQ_ERR_UNSUPPORTED_TYPE, "no weight quantiser for ggml type %u", type);
    const int bs = lbq_type_block_size(type);
    if (nelem < 0 || nelem % bs) return fail(LBQ_ERR_SHAPE, "nelem = %lld is not a multiple of %d", (long long)nelem, bs);
    if ((reinterpret_cast<uintptr_t>(d_w) & 3u) || (reinterpret_cast<uintptr_t>(d_out_blocks) & 3u))
        return fail(LBQ_ERR_INVALID_ARG, "weights and output blocks must be 4-byte aligned");
    if (nelem == 0) return LBQ_OK;
    hipError_t e = lbq::launch_quant_weights((int)type, d_w, nelem, static_cast<uint8_t *>(d_out_blocks),
                                             static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "weight quantisation launch");
    return LBQ_OK;
}

}  // extern "C"
