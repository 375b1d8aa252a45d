// lbq_probe.hip -- measurement-only kernels for bench.py (liblbq_probe.so), not
// part of the C ABI in include/lbq.h.
//
// lbq_probe_read: a read-only stream over [p, p + bytes) (whole KiB; a tail below
// 1 KiB is left out): every wave reads its own contiguous range in 1 KiB steps
// (64 lanes x 16 B), four steps in flight, and
// folds the words into one value that is written only if it matches a sentinel
// (so the loads cannot be dropped and nothing else reaches memory).  The same
// bytes the decode GEMV streams, with nothing but the loads: the time a launch
// of that size takes on this harness is the floor the GEMV's own time is
// compared with.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ __launch_bounds__(256) void k_probe_read(const uint4 *__restrict__ src, int64_t n16, unsigned *out) {
    const int64_t nw = (int64_t)gridDim.x * 4, w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t steps = n16 / 64;  // whole 1 KiB steps (a tail below 1 KiB is not read)
    const int64_t per = (steps + nw - 1) / nw;
    const int64_t s0 = w * per, s1 = s0 + per < steps ? s0 + per : steps;
    unsigned acc = 0;
    int64_t s = s0;
    for (; s + 4 <= s1; s += 4) {
        uint4 v[4];
#pragma unroll
        for (int d = 0; d < 4; d++) v[d] = src[(s + d) * 64 + lane];
#pragma unroll
        for (int d = 0; d < 4; d++) acc ^= v[d].x + v[d].y * 3u + v[d].z * 5u + v[d].w * 7u;
    }
    for (; s < s1; s++) {
        const uint4 v = src[s * 64 + lane];
        acc ^= v.x + v.y + v.z + v.w;
    }
    if (acc == 0x9e3779b9u) out[0] = acc;
}

}  // namespace

extern "C" int lbq_probe_read(const void *p, int64_t bytes, void *out, int grid, void *stream) {
    if (!p || !out || bytes < 16 || (reinterpret_cast<uintptr_t>(p) & 15u) || grid < 1) return -1;
    k_probe_read<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<const uint4 *>(p), bytes / 16,
                                                                       static_cast<unsigned *>(out));
    return hipGetLastError() == hipSuccess ? 0 : -7;
}
