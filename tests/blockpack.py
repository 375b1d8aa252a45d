"""Independent GGUF block *encoders*, written from the block specification.

The oracle and the HIP kernels only decode blocks.  These packers go the other
way -- from chosen integer fields (d, dmin, 6-bit scales and mins, codes) to
bytes -- so a known-answer test can state the expected value of every output
element from the fields alone.  A transposed index or a wrong bit plane in a
decoder then fails, because encoder and decoder were written separately.

Spec (ggml block layouts, as used by candle-core 0.10.2 / ggml-quants 0.1.0):
  Q4_K: d f16, dmin f16, scales[12], qs[128]; value 64c+l (l<32) is the low
        nibble of qs[32c+l], value 64c+32+l the high nibble; sub-block j = v//32
        has 6-bit scale sc[j] and min m[j]: x = d*sc*q - dmin*m.
        scales bytes: for j<4: byte j holds sc[j] (bits 0-5) and sc[j+4]>>4
        (bits 6-7); byte j+4 holds m[j] and m[j+4]>>4 likewise; byte j+8 holds
        sc[j+4]&15 (bits 0-3) and m[j+4]&15 (bits 4-7).
  Q5_K: as Q4_K plus qh[32] between scales and qs: bit 2c of qh[l] is bit 4 of
        value 64c+l, bit 2c+1 of qh[l] is bit 4 of value 64c+32+l.
  Q6_K: ql[128], qh[64], int8 scales[16], d f16.  Value v = 128n + 32s + l
        (n<2, s<4, l<32) has 6-bit code L = q+32: its low 4 bits are nibble s//2
        of ql[64n + 32(s%2) + l], its top 2 bits are bits 2s..2s+1 of qh[32n+l];
        scale index v//16: x = d*scale*q.
  Q8_0: d f16, qs[32] int8: x = d*q.
  Q8_K: d f32, qs[256] int8, bsums[16] int16.
  Q2_K: scales[16] (scale | min << 4), qs[64], d f16, dmin f16: x = (d*sc)*q - dmin*m.
  Q3_K: hmask[32], qs[64], scales[12] (6-bit, -32 offset), d f16: x = (d*sc)*q, q in -4..3.
  32-value legacy blocks: value j (j<16) is the low nibble of qs[j], value
  j+16 its high nibble; Q5_* take bit 4 of value v from bit v of the little-
  endian u32 qh.
  Q4_0: d f16, qs[16]: x = d*(q-8).     Q4_1: d f16, m f16, qs[16]: x = d*q + m.
  Q5_0: d f16, qh[4], qs[16]: x = d*(q-16).  Q5_1: d, m f16, qh[4], qs[16]: x = d*q + m.
  Q8_1: d f16, s f16, qs[32] int8 (s = d * sum(qs), kept in f16).
"""
from __future__ import annotations

import numpy as np


def f16_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float16).view(np.uint16)[0])


def f16_val(bits: int) -> np.float32:
    return np.array([bits], dtype=np.uint16).view(np.float16).astype(np.float32)[0]


def pack_q4k(d: int, dmin: int, sc, mn, q) -> bytes:
    sc = [int(v) for v in sc]
    mn = [int(v) for v in mn]
    q = [int(v) for v in q]
    assert len(sc) == len(mn) == 8 and len(q) == 256
    assert all(0 <= v < 64 for v in sc + mn) and all(0 <= v < 16 for v in q)
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    qs = [0] * 128
    for v in range(256):
        c, r = divmod(v, 64)
        if r < 32:
            qs[32 * c + r] |= q[v]
        else:
            qs[32 * c + r - 32] |= q[v] << 4
    return (d.to_bytes(2, "little") + dmin.to_bytes(2, "little") + bytes(s) + bytes(qs))


def pack_q5k(d: int, dmin: int, sc, mn, q) -> bytes:
    q = [int(v) for v in q]
    assert all(0 <= v < 32 for v in q)
    base = pack_q4k(d, dmin, sc, mn, [v & 15 for v in q])
    qh = [0] * 32
    for v in range(256):
        c, r = divmod(v, 64)
        if q[v] & 16:
            if r < 32:
                qh[r] |= 1 << (2 * c)
            else:
                qh[r - 32] |= 1 << (2 * c + 1)
    return base[:16] + bytes(qh) + base[16:]


def pack_q6k(d: int, scales, q) -> bytes:
    scales = [int(v) for v in scales]
    q = [int(v) for v in q]
    assert len(scales) == 16 and len(q) == 256
    assert all(-128 <= v < 128 for v in scales) and all(-32 <= v < 32 for v in q)
    ql = [0] * 128
    qh = [0] * 64
    for v in range(256):
        L = q[v] + 32
        n, rest = divmod(v, 128)
        s, l = divmod(rest, 32)
        ql[64 * n + 32 * (s % 2) + l] |= (L & 15) << (4 * (s // 2))
        qh[32 * n + l] |= (L >> 4) << (2 * s)
    return bytes(ql) + bytes(qh) + bytes(v & 255 for v in scales) + d.to_bytes(2, "little")


def pack_q8_0(d: int, q) -> bytes:
    q = [int(v) for v in q]
    assert len(q) == 32
    return d.to_bytes(2, "little") + bytes(v & 255 for v in q)


def pack_q8k(d: float, q) -> bytes:
    q = np.asarray(q, dtype=np.int8)
    assert q.size == 256
    bsums = q.astype(np.int32).reshape(16, 16).sum(axis=1).astype(np.int16)
    return np.array([d], dtype=np.float32).tobytes() + q.tobytes() + bsums.tobytes()


def _k_low2_qs(L) -> bytes:
    """ggml's Q2_K/Q3_K 2-bit packing: for each 128-value half, value
    128h + 32s + l goes to bits 2s of qs[32h + l]."""
    qs = [0] * 64
    for h in range(2):
        for l in range(32):
            qs[32 * h + l] = sum((int(L[128 * h + 32 * s + l]) & 3) << (2 * s) for s in range(4))
    return bytes(qs)


def pack_q2k(d: int, dmin: int, sc, mn, q) -> bytes:
    """sc, mn: 16 4-bit scales/mins; q: 256 codes 0..3 (ggml quantize_row_q2_K
    layout: scales[16] = sc | mn << 4, qs[64], d, dmin)."""
    scales = bytes((int(sc[j]) & 15) | ((int(mn[j]) & 15) << 4) for j in range(16))
    return scales + _k_low2_qs(q) + d.to_bytes(2, "little") + dmin.to_bytes(2, "little")


def pack_q3k(d: int, sc, q) -> bytes:
    """sc: 16 signed 6-bit scales (-32..31); q: 256 codes -4..3.  ggml
    quantize_row_q3_K layout: hmask[32] (bit j/32 of hmask[j%32] set when code
    j >= 0), qs[64] (the low 2 bits of code+4), scales[12], d."""
    L = [int(v) + 4 for v in q]
    hmask = [0] * 32
    for j in range(256):
        if L[j] > 3:
            hmask[j % 32] |= 1 << (j // 32)
    scales = [0] * 12
    for j in range(16):
        l = int(sc[j]) + 32
        if j < 8:
            scales[j] = l & 0xF
        else:
            scales[j - 8] |= (l & 0xF) << 4
        scales[8 + j % 4] |= (l >> 4) << (2 * (j // 4))
    return bytes(hmask) + _k_low2_qs(L) + bytes(scales) + d.to_bytes(2, "little")


# ---- expected values, straight from the fields (every op rounded to f32) ----
def expect_q4k(d, dmin, sc, mn, q) -> np.ndarray:
    D, M = f16_val(d), f16_val(dmin)
    out = np.empty(256, dtype=np.float32)
    for v in range(256):
        j = v // 32
        d1 = np.float32(D * np.float32(sc[j]))
        m1 = np.float32(M * np.float32(mn[j]))
        out[v] = np.float32(np.float32(d1 * np.float32(q[v])) - m1)
    return out


def expect_q6k(d, scales, q) -> np.ndarray:
    D = f16_val(d)
    out = np.empty(256, dtype=np.float32)
    for v in range(256):
        out[v] = np.float32(np.float32(D * np.float32(scales[v // 16])) * np.float32(q[v]))
    return out


def expect_q2k(d, dmin, sc, mn, q) -> np.ndarray:
    D, M = f16_val(d), f16_val(dmin)
    out = np.empty(256, dtype=np.float32)
    for v in range(256):
        j = v // 16
        dl = np.float32(D * np.float32(sc[j]))
        ml = np.float32(M * np.float32(mn[j]))
        out[v] = np.float32(np.float32(dl * np.float32(q[v])) - ml)
    return out


def expect_q3k(d, sc, q) -> np.ndarray:
    D = f16_val(d)
    return np.array([np.float32(np.float32(D * np.float32(sc[v // 16])) * np.float32(q[v])) for v in range(256)],
                    dtype=np.float32)


# ---- unpack Q8_K / Q8_0 blocks produced by the quantisers ----
def unpack_q8k(raw: np.ndarray):
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, 292)
    d = raw[:, 0:4].copy().view(np.float32).reshape(-1)
    qs = raw[:, 4:260].copy().view(np.int8)
    bsums = raw[:, 260:292].copy().view(np.int16)
    return d, qs, bsums


def unpack_q8_0(raw: np.ndarray):
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, 34)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    qs = raw[:, 2:34].copy().view(np.int8)
    return d, qs


def _nib_pack(q) -> bytes:
    q = [int(v) for v in q]
    return bytes((q[j] & 15) | ((q[j + 16] & 15) << 4) for j in range(16))


def _qh_pack(q) -> bytes:
    h = 0
    for v in range(32):
        h |= ((int(q[v]) >> 4) & 1) << v
    return h.to_bytes(4, "little")


def pack_q4_0(d: int, q) -> bytes:
    return d.to_bytes(2, "little") + _nib_pack(q)


def pack_q4_1(d: int, m: int, q) -> bytes:
    return d.to_bytes(2, "little") + m.to_bytes(2, "little") + _nib_pack(q)


def pack_q5_0(d: int, q) -> bytes:
    return d.to_bytes(2, "little") + _qh_pack(q) + _nib_pack(q)


def pack_q5_1(d: int, m: int, q) -> bytes:
    return d.to_bytes(2, "little") + m.to_bytes(2, "little") + _qh_pack(q) + _nib_pack(q)


def unpack_legacy(t: int, raw: np.ndarray):
    """(d, m, codes) per block of the 32-value weight types; codes unsigned
    (0..15 or 0..31), m = 0 for Q4_0/Q5_0 (whose offset is -8 / -16)."""
    ts = {2: 18, 3: 20, 6: 22, 7: 24}[t]
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, ts)
    f16 = lambda c: raw[:, c:c + 2].copy().view(np.float16).astype(np.float64).reshape(-1)
    d = f16(0)
    m = f16(2) if t in (3, 7) else np.zeros(raw.shape[0])
    qs = raw[:, ts - 16:].astype(np.int64)
    q = np.concatenate([qs & 15, qs >> 4], axis=1)
    if t in (6, 7):
        off = 2 if t == 6 else 4
        h = raw[:, off:off + 4].copy().view("<u4").astype(np.int64).reshape(-1)
        q = q | (((h[:, None] >> np.arange(32)) & 1) << 4)
    return d, m, q


def unpack_q8_1(raw: np.ndarray):
    raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1, 36)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    s = raw[:, 2:4].copy().view(np.float16).astype(np.float32).reshape(-1)
    return d, s, raw[:, 4:36].copy().view(np.int8)


def random_blocks(rng: np.random.Generator, t: int, nblocks: int, d_scale: float = 1e-3) -> np.ndarray:
    """Random bytes in every field, with finite, moderate f16 scales."""
    ts = {2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210}[t]
    raw = rng.integers(0, 256, size=(nblocks, ts), dtype=np.uint8)
    def f16col(n):
        return (rng.standard_normal(n) * d_scale).astype(np.float16).view(np.uint8).reshape(n, 2)
    if t in (12, 13, 3, 7):
        raw[:, 0:2] = f16col(nblocks)
        raw[:, 2:4] = f16col(nblocks)
    elif t == 14:
        raw[:, 208:210] = f16col(nblocks)
    elif t == 10:
        raw[:, 80:82] = f16col(nblocks)
        raw[:, 82:84] = f16col(nblocks)
    elif t == 11:
        raw[:, 108:110] = f16col(nblocks)
    else:
        raw[:, 0:2] = f16col(nblocks)
    return raw.reshape(-1)
