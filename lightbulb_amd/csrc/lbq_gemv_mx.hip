// Batch decode on the matrix cores: y[m][n] = x[m][k] . W[n][k]^T for 2 <= m <= 8
// (the shapes gemv_mx_serves admits),
// Q8_K activation rows against Q4_K / Q5_K weights, in the reference's integer
// arithmetic (candle-core 0.10.2 k_quants.rs, BlockQ4K / BlockQ5K vec_dot with
// BlockQ8K: integer sub-block sums scaled by the 6-bit scales, mins against the
// Q8_K bsums, combined with d, dmin and the activation's d in f32).
//
// Per 32-value sub-block s of a block, the integer dot of every (activation row,
// weight row) pair is one v_mfma_i32_32x32x32_i8: A = the Q8_K codes of the
// activation rows (A rows past m repeat row m - 1 and are never stored), B = 32
// weight rows' 5-bit (Q5_K) or 4-bit (Q4_K) codes, both as int8, so the int32
// sums are exact.  Each lane owns one weight row (lane % 32), so the sub-block's
// 6-bit scale is one value per lane: isum += sc_s * dot_s.  The mins term
// sum_s m_s * bsum_s (bsum_s: the activation codes summed over sub-block s, from
// the Q8_K 16-value sums) is one v_mfma_f32_32x32x16_f16 per block with each
// bsum split as 64*hi + lo (|hi| <= 64, 0 <= lo < 64) against (64*m_s, m_s):
// every operand and partial sum is an integer below 2^24, so it is exact too.
// The block then adds d*dx*isum - dmin*dx*msum in f32, as the decode GEMV does.
// Where the multi-row decode kernel re-does its 16 sdot4 per 64 weights for every
// activation row, the matrix core does all rows at once: its VALU work per weight
// does not grow with m.
//
// Workgroup: 32 weight rows, four (or, with at most one workgroup per CU, eight)
// waves splitting the row's blocks into contiguous ranges; the partial tiles are
// added in wave order in LDS.
//
// Activations go through a wave-private LDS stage.  Per block, the wave's eight
// activation rows (2 KB of codes, 256 B of 16-value sums; rows past m repeat row
// m - 1) arrive by three loads in which every lane fetches its own 16-byte chunk
// -- two blocks ahead, into registers -- and are written to the stage one block
// ahead; the A operands are LDS reads.  A block then costs three activation loads
// (not nine) and 24 activation registers (not 72), for three waves per SIMD.
// Rows are 256 bytes apart in the stage, so chunk c of row r sits in slot
// c ^ (r & 15): the 16 distinct chunks an A read touches fall in different banks.
// Weights: one block ahead in registers (a deeper ring measured slower: it costs
// waves per SIMD).
#include <hip/hip_runtime.h>

#include "lbq_device.hpp"
#include "lbq_internal.hpp"

namespace lbq {

typedef int i32x4v __attribute__((ext_vector_type(4)));
typedef int i32x16v __attribute__((ext_vector_type(16)));
typedef float f32x16v __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8v __attribute__((ext_vector_type(8)));

constexpr int MX_STAGE = 8 * 256 + 256;  // codes of 8 activation rows, then their 16-value sums

template <int TYPE>
struct MxW {
    uint4 hd, qh, qs[4];  // block header (d, dmin, scales), the lane half's qh, its four 16-byte qs quarters
};
template <int TYPE>
__device__ __forceinline__ void mx_load_w(const uint8_t *blk, int h, MxW<TYPE> &r) {
    constexpr int QS = TYPE == TYPE_Q4_K ? 16 : 48;
    r.hd = ld_u4(blk);
    if constexpr (TYPE == TYPE_Q5_K) r.qh = ld_u4(blk + 16 + 16 * h);
#pragma unroll
    for (int c = 0; c < 4; c++) r.qs[c] = ld_u4(blk + QS + 32 * c + 16 * h);
}

// One block: xa = the 8 sub-blocks' A operands, xbv = the lane half's four pairs
// of 16-value sums; accumulators e = 0..3 are C rows 4h + e.
template <int TYPE, bool JIT>
__device__ __forceinline__ void mx_block(const MxW<TYPE> &r, const uint8_t *st, const int *ro, int h, const float *sdx,
                                         float *acc) {
    // A operands: all nine stage reads up front, or (JIT, fewer registers) each
    // right before its MFMA
    i32x4v xa[8];
    if constexpr (!JIT) {
#pragma unroll
        for (int s = 0; s < 8; s++) xa[s] = *reinterpret_cast<const i32x4v *>(st + ro[s]);
    }
    constexpr int E = 4;
    const uint32_t hw0 = r.hd.x, hw1 = r.hd.y, hw2 = r.hd.z, hw3 = r.hd.w;
    // get_scale_min_k4 for the 8 sub-blocks, as packed bytes: j < 4 from bytes j,
    // j + 4; j >= 4 from the nibbles of bytes j + 4 and the top bits of j - 4, j
    const uint32_t sc03 = hw1 & 0x3f3f3f3fu, m03 = hw2 & 0x3f3f3f3fu;
    const uint32_t sc47 = (hw3 & 0x0f0f0f0fu) | ((hw1 >> 2) & 0x30303030u);
    const uint32_t m47 = ((hw3 >> 4) & 0x0f0f0f0fu) | ((hw2 >> 2) & 0x30303030u);
    const uint32_t qh[4] = {r.qh.x, r.qh.y, r.qh.z, r.qh.w};
    int isum[E];
#pragma unroll
    for (int e = 0; e < E; e++) isum[e] = 0;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        // sub-block s = 2c + hn: nibble hn of qs quarter c, fifth bit s of qh
        const uint4 q = r.qs[s >> 1];
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
        i32x4v bw;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            uint32_t v = (qw[w] >> (4 * (s & 1))) & 0x0f0f0f0fu;
            if constexpr (TYPE == TYPE_Q5_K) v |= ((qh[w] >> s) & 0x01010101u) << 4;
            bw[w] = (int)v;
        }
        const i32x16v zero = {};
        if constexpr (JIT) xa[s] = *reinterpret_cast<const i32x4v *>(st + ro[s]);
        const i32x16v o = __builtin_amdgcn_mfma_i32_32x32x32_i8(xa[s], bw, zero, 0, 0, 0);
        const int sc = (int)(((s < 4 ? sc03 : sc47) >> (8 * (s & 3))) & 0xffu);
#pragma unroll
        for (int e = 0; e < E; e++) isum[e] += __mul24(sc, o[e]);
    }
    // mins: sub-blocks 4h + t of the lane half (k slots 8h + 2t, 8h + 2t + 1)
    const uint32_t mm = h ? m47 : m03;
    const i32x4v xbv = *reinterpret_cast<const i32x4v *>(st + ro[8]);
    const uint32_t xbw[4] = {(uint32_t)xbv.x, (uint32_t)xbv.y, (uint32_t)xbv.z, (uint32_t)xbv.w};
    f16x8v a, b;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int bs = (int)(int16_t)(xbw[t] & 0xffffu) + ((int)xbw[t] >> 16);  // the sub-block's code sum
        a[2 * t] = (_Float16)(bs >> 6);
        a[2 * t + 1] = (_Float16)(bs & 63);
        const int mv = (int)((mm >> (8 * t)) & 0xffu);
        b[2 * t] = (_Float16)(64 * mv);
        b[2 * t + 1] = (_Float16)mv;
    }
    const f32x16v zf = {};
    const f32x16v ms = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, zf, 0, 0, 0);
    const float d = h2f(hw0 & 0xffffu), dmin = h2f(hw0 >> 16);
#pragma unroll
    for (int e = 0; e < E; e++) {
        const float dx = sdx[4 * h + e];
        acc[e] = fmaf(d * dx, (float)isum[e], acc[e]);
        acc[e] = fmaf(-(dmin * dx), ms[e], acc[e]);
    }
}

struct MxX {
    i32x4v c[2], s;  // codes (rows 4q + lane/16, chunk lane%16), sums (row (lane%16)/2, half lane%2)
};

template <int TYPE, int MX_WAVES>
__global__ __launch_bounds__(64 * MX_WAVES) void k_gemv_mx(const uint8_t *__restrict__ W, int64_t row_bytes, int n,
                                                         int nb, ActView act, int m, float *__restrict__ y) {
    constexpr int E = 4;
    extern __shared__ __align__(16) float sdx[];  // [nb][8]: dx of block b, activation row i (0 past m)
    __shared__ float red[MX_WAVES][E][64];
    __shared__ __align__(16) uint8_t xs[MX_WAVES][MX_STAGE];
    const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int j = lane & 31, h = lane >> 5;
    const int row0 = blockIdx.x * 32;
    const int64_t k = act.k;
    const uint8_t *wr = W + (int64_t)min(row0 + j, n - 1) * row_bytes;
    const int b0 = wave * nb / MX_WAVES, b1 = (wave + 1) * nb / MX_WAVES;
    constexpr int BYTES = TYPE == TYPE_Q4_K ? 144 : 176;
    uint8_t *st = xs[wave];
    // this lane's share of a block's activations: two code chunks and a sums chunk
    const int8_t *xc[2];
    int wo[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int r = 4 * q + (lane >> 4), c = lane & 15;
        xc[q] = act.xq + (int64_t)min(r, m - 1) * k + 16 * c;
        wo[q] = r * 256 + 16 * (c ^ (r & 15));
    }
    const int16_t *xsum = act.xbs + (int64_t)min((lane & 15) >> 1, m - 1) * (k / 16) + 8 * (lane & 1);
    const int so = 2048 + 16 * (lane & 15);  // lanes 16..63 load copies and write nothing
    auto load_x = [&](int b, MxX &x) {
#pragma unroll
        for (int q = 0; q < 2; q++) x.c[q] = *reinterpret_cast<const i32x4v *>(xc[q] + 256 * b);
        x.s = *reinterpret_cast<const i32x4v *>(xsum + 16 * b);
    };
    auto write_x = [&](const MxX &x) {
#pragma unroll
        for (int q = 0; q < 2; q++) *reinterpret_cast<i32x4v *>(st + wo[q]) = x.c[q];
        if (lane < 16) *reinterpret_cast<i32x4v *>(st + so) = x.s;
    };
    // A-operand reads: row ra (A rows past m read row m - 1), chunk 2s + h
    const int ra = min(j, m - 1);
    int ro[9];
#pragma unroll
    for (int s = 0; s < 8; s++) ro[s] = ra * 256 + 16 * ((2 * s + h) ^ (ra & 15));
    ro[8] = 2048 + ra * 32 + 16 * h;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; e++) acc[e] = 0.f;
    // Loads are unconditional, their block clamped to the wave's last one (the
    // tail re-reads it and never uses the copy).  A wave with no blocks (nb < 4)
    // loads nothing.
    const bool any = b0 < b1;
    const int bl = b1 - 1;
    MxW<TYPE> rw[2];
    MxX xr[2];
    auto load_w = [&](int b, MxW<TYPE> &dst) { mx_load_w<TYPE>(wr + (int64_t)b * BYTES, h, dst); };
    if (any) {
        load_x(b0, xr[0]);
        load_x(min(b0 + 1, bl), xr[1]);
        load_w(b0, rw[0]);
        write_x(xr[0]);
    }
    for (int q = t; q < nb * 8; q += 64 * MX_WAVES) {
        const int b = q >> 3, i = q & 7;
        sdx[q] = i < m ? act.xd[(int64_t)i * nb + b] : 0.f;
    }
    __syncthreads();  // sdx (each wave's first stage is its own)
    if (any) {
        for (int b = b0;; b += 2) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
                // xr[1 - q] holds block b + q + 1 (loaded a block ago); xr[q] takes b + q + 2
                load_x(min(b + q + 2, bl), xr[q]);
                load_w(min(b + q + 1, bl), rw[1 - q]);
                mx_block<TYPE, (MX_WAVES > 4)>(rw[q], st, ro, h, sdx + 8 * (b + q), acc);
                if (b + q == bl) break;
                write_x(xr[1 - q]);  // after this block's stage reads (the MFMAs consumed them)
            }
            if (b + 2 > bl) break;
        }
    }
#pragma unroll
    for (int e = 0; e < E; e++) red[wave][e][lane] = acc[e];
    __syncthreads();
    // wave w < 4 stores accumulator w (C row 4h + w), the partials added in wave order
    if (wave < E) {
        const int e = wave;
        float s = red[0][e][lane];
#pragma unroll
        for (int w = 1; w < MX_WAVES; w++) s += red[w][e][lane];
        const int i = 4 * h + e;
        if (i < m && row0 + j < n) y[(int64_t)i * n + row0 + j] = s;
    }
}

bool gemv_mx_serves(int type, int64_t n, int64_t k, int m) {
    // Measured against the decode kernels (x quantised by the same separate pass
    // unless noted): Q5_K 14336 x 4096 m = 8 22.8 -> 18.2 us, Q4_K 14336 x 4096
    // 21.4 -> 16.8, 4096 x 4096 13.4 -> 12.5, 2048 x 4096 12.5 -> 11.9, 3072 x
    // 4096 m = 6 12.9 -> 11.9; with 1024 rows (32 eight-wave workgroups) 11.5 ->
    // 11.8, so fewer than 2048 rows keep the multi-row kernel.  At m <= 4
    // that kernel quantises x in its own prologue and stays ahead (m = 2: 12.8 vs
    // 17.9 us) -- except at k > 8192, where it cannot hold the activation rows and
    // the general GEMV runs: Q4_K 4096 x 14336 m = 2 / 3 / 4 / 8 22.2 / 26.3 /
    // 30.2 / 52.8 -> 21.0 / 20.9 / 20.8 / 21.0 us.  A Q6_K version (sixteen
    // 16-value groups per block, one v_mfma_i32_32x32x16_i8 each, the -32 offset
    // through the bsums) was correct but slower (14336 x 4096 m = 8 24.4 -> 30.1
    // us: fourteen 8-byte weight loads per block and lane) and was not kept.
    if (tuning().gemv_mx_off) return false;
    if (type != TYPE_Q4_K && type != TYPE_Q5_K) return false;
    if (k % 256 || k / 256 > 64 || m < 2 || m > 8 || n <= 0 || n > (int64_t)MAX_ROWS) return false;
    if (k / 256 > 32) return true;  // the multi-row decode kernel cannot hold these rows
    return m >= 5 && n >= 2048;
}

hipError_t launch_gemv_mx(int type, const uint8_t *w, int64_t n, int64_t k, int64_t row_bytes, const ActView &act, int m,
                          float *y, hipStream_t st) {
    if (!gemv_mx_serves(type, n, k, m)) return hipErrorNotSupported;
    const int nb = (int)(k / 256);
    if (act.k != k || act.nb != nb || !act.xq || !act.xd || !act.xbs) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)((n + 31) / 32);
    const size_t lds = (size_t)nb * 8 * sizeof(float);
    // Up to one workgroup per CU: eight waves split a row's blocks (2 per wave at
    // k = 4096), A operands read just in time to stay within four waves per SIMD
    // (4096 x 14336 m = 4: 21.8 -> 19.5 us; 4096 x 4096 m = 8: 12.9 -> 12.4).  With
    // more workgroups, four waves (14336 x 4096 m = 8: 16.9 at four, 18.7 at eight).
    const bool w8 = (int64_t)grid <= (int64_t)num_cus();
    if (type == TYPE_Q4_K) {
        if (w8) k_gemv_mx<TYPE_Q4_K, 8><<<grid, 64 * 8, lds, st>>>(w, row_bytes, (int)n, nb, act, m, y);
        else k_gemv_mx<TYPE_Q4_K, 4><<<grid, 64 * 4, lds, st>>>(w, row_bytes, (int)n, nb, act, m, y);
    } else {
        if (w8) k_gemv_mx<TYPE_Q5_K, 8><<<grid, 64 * 8, lds, st>>>(w, row_bytes, (int)n, nb, act, m, y);
        else k_gemv_mx<TYPE_Q5_K, 4><<<grid, 64 * 4, lds, st>>>(w, row_bytes, (int)n, nb, act, m, y);
    }
    return hipGetLastError();
}

}  // namespace lbq
