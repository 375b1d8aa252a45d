// lbq_device.hpp -- device-side building blocks for the gfx950 quantized-linear kernels.
//
// GGUF block layouts (byte offsets inside one block, little endian), as fixed by
// the ggml block specification that candle-core 0.10.2 and ggml-quants 0.1.0
// implement (type sizes: /root/reference/src/quantization/mod.rs:108-126):
//   Q8_0  34 B / 32 values : f16 d @0, i8 qs[32] @2
//   Q4_K 144 B / 256 values: f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qs[128] @16
//   Q5_K 176 B / 256 values: f16 d @0, f16 dmin @2, u8 scales[12] @4, u8 qh[32] @16, u8 qs[128] @48
//   Q6_K 210 B / 256 values: u8 ql[128] @0, u8 qh[64] @128, i8 scales[16] @192, f16 d @208
//   Q8_K 292 B / 256 values: f32 d @0, i8 qs[256] @4, i16 bsums[16] @260
// Q4_K/Q5_K blocks are 16-byte multiples; Q6_K and Q8_0 blocks are only 2-byte
// aligned, so their fields are read as aligned dwords and funnel-shifted
// (v_alignbyte_b32) -- never as misaligned vector loads.
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lbq {

constexpr int QK_K = 256;
constexpr int QK8_0 = 32;

// Internal (split) layout of a quantised activation matrix [m][k]:
//   xq  int8  [m][k]          the Q8_K / Q8_0 integer codes
//   xd  f32   [m][k/QK]       the block scale (Q8_0: the f32 value of the stored f16)
//   xbs int16 [m][k/16]       Q8_K only: sums of 16 consecutive codes
struct ActView {
    const int8_t *xq;
    const float *xd;
    const int16_t *xbs;
    int64_t k;  // row length in values
    int nb;     // scale blocks per row (k/256 or k/32)
};

struct __attribute__((aligned(4))) u32x4a4 { uint32_t x, y, z, w; };

__device__ __forceinline__ float h2f(uint32_t bits16) { return __half2float(__ushort_as_half((unsigned short)bits16)); }

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t ld_u32(const uint8_t *p) { return *reinterpret_cast<const uint32_t *>(p); }

__device__ __forceinline__ uint4 ld_u4(const uint8_t *p) { return *reinterpret_cast<const uint4 *>(p); }

typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));

// Streaming (non-temporal) 16-byte load: weight bytes are read once per launch.
__device__ __forceinline__ uint4 ld_u4_nt(const uint8_t *p) {
    const u32x4v v = __builtin_nontemporal_load(reinterpret_cast<const u32x4v *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// 16 bytes starting at a 2-byte aligned address p.  Reads only aligned dwords that
// hold at least one byte of [p, p+16), so it never touches a dword outside the
// caller's buffer.
__device__ __forceinline__ void ld16_a2(const uint8_t *p, uint32_t out[4]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t mis = (uint32_t)(a & 3u);
    const uint8_t *base = reinterpret_cast<const uint8_t *>(a & ~(uintptr_t)3);
    const u32x4a4 v = *reinterpret_cast<const u32x4a4 *>(base);
    const uint32_t t = *reinterpret_cast<const uint32_t *>(base + (mis ? 16 : 12));
    out[0] = __builtin_amdgcn_alignbyte(v.y, v.x, mis);
    out[1] = __builtin_amdgcn_alignbyte(v.z, v.y, mis);
    out[2] = __builtin_amdgcn_alignbyte(v.w, v.z, mis);
    out[3] = __builtin_amdgcn_alignbyte(t, v.w, mis);
}

// 4 bytes at a 2-byte aligned address.
__device__ __forceinline__ uint32_t ld4_a2(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t mis = (uint32_t)(a & 3u);
    const uint8_t *base = reinterpret_cast<const uint8_t *>(a & ~(uintptr_t)3);
    const uint32_t lo = *reinterpret_cast<const uint32_t *>(base);
    const uint32_t hi = *reinterpret_cast<const uint32_t *>(base + (mis ? 4 : 0));
    return __builtin_amdgcn_alignbyte(hi, lo, mis);
}

// 2 bytes (f16 bits) at a 2-byte aligned address.
__device__ __forceinline__ uint32_t ld2_a2(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t w = *reinterpret_cast<const uint32_t *>(a & ~(uintptr_t)3);
    return (a & 2u) ? (w >> 16) : (w & 0xffffu);
}

// Q4_K / Q5_K 6-bit scale+min pair for sub-blocks j = 2c and 2c+1 (c = 0..3),
// from the 12 scale bytes held in dwords s0 (bytes 0..3), s1 (4..7), s2 (8..11).
// ggml get_scale_min_k4: j<4: sc = s[j]&63, m = s[j+4]&63;
// j>=4: sc = (s[j+4]&15) | (s[j-4]>>6)<<4, m = (s[j+4]>>4) | (s[j]>>6)<<4.
// Returns sc(2c) | sc(2c+1)<<8 in *sc2 and the mins likewise in *m2.
__device__ __forceinline__ void k4_scale_pair(uint32_t s0, uint32_t s1, uint32_t s2, int c, uint32_t *sc2,
                                              uint32_t *m2) {
    const uint32_t sh = (uint32_t)(c & 1) * 16u;
    const uint32_t A = (s0 >> sh) & 0xffffu, B = (s1 >> sh) & 0xffffu, C = (s2 >> sh) & 0xffffu;
    if (c < 2) {
        *sc2 = A & 0x3f3fu;
        *m2 = B & 0x3f3fu;
    } else {
        *sc2 = (C & 0x0f0fu) | ((A >> 2) & 0x3030u);
        *m2 = ((C >> 4) & 0x0f0fu) | ((B >> 2) & 0x3030u);
    }
}

}  // namespace lbq
