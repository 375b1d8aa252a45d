"""Pins for the CPU oracle (oracle/), before it is trusted as the parity checker.

The reference is Rust and cannot be built here, and it holds no golden vectors
for QMatMul (its only quantisation tests are round-trip bounds,
/root/reference/src/quantization/mod.rs:333-369).  So each oracle function is
pinned by something that does not restate its formula:
independent bit-packers (tests/blockpack.py), exhaustive IEEE checks against
numpy, closed-form special cases, invariants, and float64 brute force.
"""
import numpy as np
import pytest

import blockpack as bp

Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 8, 12, 13, 14, 15


# ---------------------------------------------------------------- type table
def test_dtype_properties(oracle):
    # reference test_dtype_properties (src/quantization/mod.rs:114-120) plus the table :99-126
    from lightbulb_amd.quantized import GgmlDType
    assert GgmlDType.Q4_0.block_size() == 32
    assert GgmlDType.Q4K.block_size() == 256
    assert GgmlDType.Q4_0.type_name() == "Q4_0"
    assert GgmlDType.from_u32(12) == GgmlDType.Q4K
    assert GgmlDType.from_u32(4) is None
    for t, bs, ts in [(Q8_0, 32, 34), (Q4_K, 256, 144), (Q5_K, 256, 176), (Q6_K, 256, 210), (Q8_K, 256, 292)]:
        assert oracle.block_size(t) == bs and oracle.type_size(t) == ts
        assert GgmlDType(t).block_size() == bs and GgmlDType(t).type_size() == ts


# ---------------------------------------------------------------- f16
def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_round_nearest_even(oracle):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([65504, 65519.99, 65520, 70000, 6.1e-5, 5.96e-8, 2.98e-8, 2.99e-8, 1e-9, 0.0, -0.0,
                  np.inf, -np.inf], dtype=np.float32),
        # exact binary16 ties: halfway between neighbours
        (np.arange(1, 2000, dtype=np.float32) * np.float32(2 ** -10) + np.float32(2 ** -11)) + np.float32(1.0),
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- dequantize KATs
def _check_q4k_like(oracle, t, rng, sc, mn, q):
    d, dmin = bp.f16_bits(float(rng.uniform(1e-4, 2e-2))), bp.f16_bits(float(rng.uniform(1e-4, 2e-2)))
    raw = (bp.pack_q4k if t == Q4_K else bp.pack_q5k)(d, dmin, sc, mn, q)
    got = oracle.dequantize(t, np.frombuffer(raw, dtype=np.uint8))
    exp = bp.expect_q4k(d, dmin, sc, mn, q)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
def test_dequant_k4_known_answers(oracle, t):
    rng = np.random.default_rng(2)
    qmax = 16 if t == Q4_K else 32
    # every scale-unpack branch at its extremes (j<4 and j>=4, 6-bit max and high bits set)
    for sc_val, mn_val in [(63, 63), (48, 17), (16, 32), (1, 0), (0, 63)]:
        sc = [sc_val] * 8
        mn = [mn_val] * 8
        _check_q4k_like(oracle, t, rng, sc, mn, rng.integers(0, qmax, 256))
    # distinct scales per sub-block, every code value present in every sub-block
    codes = np.tile(np.arange(qmax), 256 // qmax)
    _check_q4k_like(oracle, t, rng, list(range(40, 48)), list(range(55, 63)), codes)
    for _ in range(50):
        _check_q4k_like(oracle, t, rng, rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, qmax, 256))


def test_dequant_q6k_known_answers(oracle):
    rng = np.random.default_rng(3)
    cases = [(np.full(16, 127), np.tile(np.arange(-32, 32), 4)), (np.full(16, -128), np.full(256, -32)),
             (np.arange(-8, 8), np.full(256, 31))]
    cases += [(rng.integers(-128, 128, 16), rng.integers(-32, 32, 256)) for _ in range(50)]
    for scales, q in cases:
        d = bp.f16_bits(float(rng.uniform(1e-5, 1e-3)))
        raw = bp.pack_q6k(d, scales, q)
        got = oracle.dequantize(Q6_K, np.frombuffer(raw, dtype=np.uint8))
        exp = bp.expect_q6k(d, scales, q)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


def test_dequant_q8_0_and_q8k_known_answers(oracle):
    rng = np.random.default_rng(4)
    for _ in range(20):
        d = bp.f16_bits(float(rng.uniform(-1, 1)))
        q = rng.integers(-128, 128, 32)
        got = oracle.dequantize(Q8_0, np.frombuffer(bp.pack_q8_0(d, q), dtype=np.uint8))
        exp = (q.astype(np.float32) * bp.f16_val(d)).astype(np.float32)
        assert np.array_equal(got, exp)
        dk = np.float32(rng.uniform(-1, 1))
        qk = rng.integers(-128, 128, 256)
        got = oracle.dequantize(Q8_K, np.frombuffer(bp.pack_q8k(dk, qk), dtype=np.uint8))
        assert np.array_equal(got, (dk * qk.astype(np.float32)).astype(np.float32))


def test_dequant_all_zero_block(oracle):
    for t, ts, bs in [(Q8_0, 34, 32), (Q4_K, 144, 256), (Q5_K, 176, 256), (Q6_K, 210, 256)]:
        out = oracle.dequantize(t, np.zeros(ts, dtype=np.uint8))
        assert out.shape == (bs,) and not out.any()


def test_round_trip_q8_0_reference_bound(oracle):
    # reference test_round_trip_q8_0 (src/quantization/mod.rs:99-112): i/256 ramp, |err| < 0.01
    data = (np.arange(256, dtype=np.float32) / 256.0).astype(np.float32)
    deq = oracle.dequantize(Q8_0, oracle.quantize_weights(Q8_0, data))
    assert deq.shape == data.shape
    assert np.max(np.abs(deq - data)) < 0.01


def test_round_trip_k_quants_bounds(oracle):
    # the same ramp through the k-quant weight quantisers; bounds follow from the code widths
    data = (np.arange(256, dtype=np.float32) / 256.0).astype(np.float32)
    for t, bound in [(Q4_K, 0.1), (Q5_K, 0.05), (Q6_K, 0.02)]:
        deq = oracle.dequantize(t, oracle.quantize_weights(t, data))
        assert np.max(np.abs(deq - data)) < bound, t


# ---------------------------------------------------------------- Q8_K activation quantisation
def test_q8k_single_nonzero_is_minus_128(oracle):
    for pos, v in [(0, 3.0), (77, -0.125), (255, 1e-20), (130, 12345.678)]:
        x = np.zeros(256, dtype=np.float32)
        x[pos] = v
        d, qs, bs = bp.unpack_q8k(oracle.quantize_act(Q8_K, x))
        assert qs[0, pos] == -128
        assert np.count_nonzero(qs) == 1
        assert bs[0, pos // 16] == -128 and np.count_nonzero(bs) == 1
        iscale = np.float32(-128.0) / np.float32(v)
        assert d[0] == np.float32(np.float32(1.0) / iscale)


def test_q8k_all_zero_and_sign_and_ties(oracle):
    d, qs, bs = bp.unpack_q8k(oracle.quantize_act(Q8_K, np.zeros(256, dtype=np.float32)))
    assert d[0] == 0 and not qs.any() and not bs.any()
    # equal |x| with opposite signs: the FIRST one sets the sign of the scale
    x = np.zeros(256, dtype=np.float32)
    x[3], x[7] = -2.0, 2.0
    d, qs, _ = bp.unpack_q8k(oracle.quantize_act(Q8_K, x))
    assert qs[0, 3] == -128 and qs[0, 7] == 127  # +128 saturates at 127
    assert d[0] == np.float32(1.0) / np.float32(64.0)  # max = -2 -> iscale = 64
    # assumption A-1: candle rounds with f32::round (half away from zero)
    x = np.zeros(256, dtype=np.float32)
    x[0] = -128.0  # iscale = 1
    x[1:6] = [2.5, -2.5, 3.5, 0.5, -0.5]
    _, qs, _ = bp.unpack_q8k(oracle.quantize_act(Q8_K, x))
    assert list(qs[0, :6]) == [-128, 3, -3, 4, 1, -1]


def test_q8k_nan_is_never_the_max(oracle):
    x = np.zeros(256, dtype=np.float32)
    x[5] = np.nan
    x[9] = -4.0
    d, qs, _ = bp.unpack_q8k(oracle.quantize_act(Q8_K, x))
    assert qs[0, 9] == -128
    assert qs[0, 5] == 127  # round(NaN).min(127) = 127 in Rust
    assert d[0] == np.float32(1.0) / np.float32(32.0)


def test_q8k_invariants_random(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 1024)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    d, qs, bs = bp.unpack_q8k(oracle.quantize_act(Q8_K, x))
    assert np.array_equal(bs.astype(np.int32), qs.astype(np.int32).reshape(-1, 16, 16).sum(axis=2))
    xb = x.reshape(-1, 256)
    recon = d[:, None] * qs.astype(np.float32)
    # |x - d q| <= |d|/2 (one code step at the +127 saturation edge)
    err = np.abs(xb - recon)
    assert np.all(err <= np.abs(d)[:, None] * 1.0 + 1e-6)
    assert np.mean(err <= np.abs(d)[:, None] * 0.5 + 1e-7) > 0.99
    assert np.all(qs.min(axis=1) == -128)  # the max element always maps to -128


# ---------------------------------------------------------------- Q8_0 activation quantisation
def test_q8_0_known_answers(oracle):
    x = np.zeros(32, dtype=np.float32)
    x[:5] = [127.0, 63.5, -63.5, 0.5, -127.0]  # d = 1, id = 1: half away from zero
    d, qs = bp.unpack_q8_0(oracle.quantize_act(Q8_0, x))
    assert d[0] == 1.0 and list(qs[0, :5]) == [127, 64, -64, 1, -127]
    d, qs = bp.unpack_q8_0(oracle.quantize_act(Q8_0, np.zeros(32, dtype=np.float32)))
    assert d[0] == 0 and not qs.any()
    rng = np.random.default_rng(6)
    x = rng.standard_normal((4, 256)).astype(np.float32)
    d, qs = bp.unpack_q8_0(oracle.quantize_act(Q8_0, x))
    amax = np.abs(x.reshape(-1, 32)).max(axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    assert np.all(np.abs(qs).max(axis=1) == 127)


# ---------------------------------------------------------------- vec_dot / qmatmul against float64
def _brute(oracle, t, w_raw, n, k, x):
    """float64 sum over dequantised weights x dequantised activations: the exact value
    the integer path represents (dequantisation is pinned above)."""
    wd = oracle.dequantize(t, w_raw).astype(np.float64).reshape(n, k)
    at = oracle.VEC_DOT_TYPE[t]
    xq = oracle.quantize_act(at, x)
    xd = oracle.dequantize(at, xq.reshape(-1)).astype(np.float64).reshape(x.shape[0], k)
    return xd @ wd.T


@pytest.mark.parametrize("t", [Q8_0, 10, 11, Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("k", [256, 512, 768])
def test_qmatmul_matches_float64_brute_force(oracle, t, k):
    rng = np.random.default_rng(100 + t + k)
    n, m = 48, 3
    bs = oracle.block_size(t)
    w_raw = bp.random_blocks(rng, t, n * k // bs)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = oracle.qmatmul(t, w_raw, n, k, x)
    ref = _brute(oracle, t, w_raw, n, k, x)
    rel = np.abs(y - ref) / (np.abs(ref).max(axis=1, keepdims=True) + 1e-30)
    assert rel.max() < 1e-5
    # the same through vec_dot one element at a time
    at = oracle.VEC_DOT_TYPE[t]
    xq = oracle.quantize_act(at, x)
    rb = k // bs * oracle.type_size(t)
    for r, c in [(0, 0), (2, 47), (1, 13)]:
        assert oracle.vec_dot(t, k, w_raw[c * rb:(c + 1) * rb], xq[r]) == y[r, c]


def test_qmatmul_threads_and_shape(oracle):
    rng = np.random.default_rng(7)
    n, k = 600, 512
    w_raw = bp.random_blocks(rng, Q4_K, n * k // 256)
    x = rng.standard_normal((5, k)).astype(np.float32)
    y1 = oracle.qmatmul(Q4_K, w_raw, n, k, x, nthreads=1)
    y4 = oracle.qmatmul(Q4_K, w_raw, n, k, x, nthreads=4)
    assert np.array_equal(y1, y4)  # each element is one vec_dot: thread split cannot change it
    # rows are independent: row 3 alone equals row 3 of the batch
    assert np.array_equal(oracle.qmatmul(Q4_K, w_raw, n, k, x[3:4]), y1[3:4])


def test_weight_quantisers_valid(oracle):
    # parity unpinned: the ggml quantisers' exact choices are not reproducible without the
    # reference; check the blocks they make are well-formed and reconstruct the weights.
    rng = np.random.default_rng(8)
    w = (rng.standard_normal(64 * 256) * 0.02).astype(np.float32)
    for t, tol in [(Q8_0, 0.01), (Q4_K, 0.12), (Q5_K, 0.06), (Q6_K, 0.03)]:
        raw = oracle.quantize_weights(t, w)
        assert raw.size == w.size // oracle.block_size(t) * oracle.type_size(t)
        deq = oracle.dequantize(t, raw)
        rel = np.linalg.norm(deq - w) / np.linalg.norm(w)
        assert rel < tol, (t, rel)


# ---------------------------------------------------------------- 32-value legacy blocks
LEGACY = [2, 3, 6, 7]  # Q4_0, Q4_1, Q5_0, Q5_1


@pytest.mark.parametrize("t", LEGACY)
def test_dequant_legacy_known_answers(oracle, t):
    # every code value in both nibble halves (and, for Q5_*, both qh halves),
    # through an independent packer: x = d*(q - off) or d*q + m, in f32
    rng = np.random.default_rng(200 + t)
    five = t in (6, 7)
    top = 32 if five else 16
    blobs, want = [], []
    for rep in range(4):
        q = rng.permutation(np.arange(32) % top)
        d = bp.f16_bits(float(rng.uniform(0.01, 2.0)) * (1 if rep % 2 else -1))
        m = bp.f16_bits(float(rng.uniform(-3, 3)))
        if t == 2:
            blobs.append(bp.pack_q4_0(d, q))
            want.append((q.astype(np.float32) - np.float32(8)) * bp.f16_val(d))
        elif t == 3:
            blobs.append(bp.pack_q4_1(d, m, q))
            want.append(q.astype(np.float32) * bp.f16_val(d) + bp.f16_val(m))
        elif t == 6:
            blobs.append(bp.pack_q5_0(d, q))
            want.append((q.astype(np.float32) - np.float32(16)) * bp.f16_val(d))
        else:
            blobs.append(bp.pack_q5_1(d, m, q))
            want.append(q.astype(np.float32) * bp.f16_val(d) + bp.f16_val(m))
    got = oracle.dequantize(t, np.frombuffer(b"".join(blobs), dtype=np.uint8))
    assert np.array_equal(got, np.concatenate(want).astype(np.float32))


def test_q8_1_known_answers(oracle):
    # as Q8_0 (d = amax/127 kept in f16, codes from the unrounded d), plus
    # s = f16(f16(sum q) * d) -- candle's half-precision product
    rng = np.random.default_rng(210)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    x[0, :32] = 0.0
    x[1, 5] = -40.0
    d, s, qs = bp.unpack_q8_1(oracle.quantize_act(9, x))
    d8, q8 = bp.unpack_q8_0(oracle.quantize_act(8, x))
    assert np.array_equal(d, d8) and np.array_equal(qs, q8)   # the Q8_0 half is Q8_0's
    assert d[0] == 0 and not qs[0].any() and s[0] == 0
    assert qs[2, 5] == -127
    sums = qs.astype(np.int64).sum(axis=1).astype(np.float32)
    want_s = (sums.astype(np.float16).astype(np.float32) * d).astype(np.float16).astype(np.float32)
    assert np.array_equal(s, want_s)


@pytest.mark.parametrize("t", LEGACY)
@pytest.mark.parametrize("k", [32, 256, 544])
def test_legacy_vec_dot_float64(oracle, t, k):
    # sum over blocks of d_w*d_x*sum(q_w*q_x) (q_w with its -8/-16 offset), plus
    # m_w*s_x for the _1 types, in float64 from independently unpacked fields
    rng = np.random.default_rng(220 + t + k)
    n, m = 20, 3
    w_raw = bp.random_blocks(rng, t, n * k // 32, d_scale=0.05)
    x = (rng.standard_normal((m, k)) * 2).astype(np.float32)
    y = oracle.qmatmul(t, w_raw, n, k, x)
    dw, mw, qw = bp.unpack_legacy(t, w_raw)
    off = {2: 8, 3: 0, 6: 16, 7: 0}[t]
    at = oracle.VEC_DOT_TYPE[t]
    xq = oracle.quantize_act(at, x)
    if at == 9:
        dx, sx, qx = bp.unpack_q8_1(xq.reshape(-1))
    else:
        dx, qx = bp.unpack_q8_0(xq.reshape(-1))
        sx = np.zeros_like(dx)
    nb = k // 32
    dw, mw, qw = dw.reshape(n, nb), mw.reshape(n, nb), (qw - off).reshape(n, nb, 32)
    dx, sx, qx = (a.astype(np.float64).reshape(m, nb) for a in (dx, sx)), None, qx.astype(np.int64).reshape(m, nb, 32)
    dx, sx = list(dx)
    ref = np.zeros((m, n))
    for r in range(m):
        isum = (qw * qx[r][None]).sum(axis=2)                    # [n, nb] exact integers
        ref[r] = (dw * dx[r][None] * isum + mw * sx[r][None]).sum(axis=1)
    scale = np.abs(ref).max(axis=1, keepdims=True) + 1e-30
    assert (np.abs(y - ref) / scale).max() < 1e-5
    xr = xq[1]
    rb = k // 32 * oracle.type_size(t)
    assert oracle.vec_dot(t, k, w_raw[3 * rb:4 * rb], xr) == y[1, 3]


def test_legacy_weight_quantisers_valid(oracle):
    # parity unpinned (ggml quantize_row_q4_0/q4_1/q5_0/q5_1 reference choices):
    # the blocks are well-formed and reconstruct the weights
    rng = np.random.default_rng(230)
    w = (rng.standard_normal(64 * 32) * 0.02).astype(np.float32)
    for t, tol in [(2, 0.15), (3, 0.12), (6, 0.08), (7, 0.06)]:
        raw = oracle.quantize_weights(t, w)
        assert raw.size == w.size // 32 * oracle.type_size(t)
        rel = np.linalg.norm(oracle.dequantize(t, raw) - w) / np.linalg.norm(w)
        assert rel < tol, (t, rel)


# ---------------------------------------------------------------- Q2_K / Q3_K
def test_dequant_q2k_known_answers(oracle):
    # every 4-bit scale and min value, every code in every 2-bit plane, through a
    # packer that follows ggml's quantize_row_q2_K layout
    rng = np.random.default_rng(240)
    blobs, want = [], []
    for rep in range(4):
        sc = rng.permutation(16)
        mn = rng.permutation(16)
        q = rng.integers(0, 4, 256)
        q[:4] = [0, 1, 2, 3]
        d = bp.f16_bits(float(rng.uniform(0.01, 1.0)))
        dmin = bp.f16_bits(float(rng.uniform(0.0, 1.0)) * (-1 if rep == 3 else 1))
        blobs.append(bp.pack_q2k(d, dmin, sc, mn, q))
        want.append(bp.expect_q2k(d, dmin, sc, mn, q))
    got = oracle.dequantize(10, np.frombuffer(b"".join(blobs), dtype=np.uint8))
    assert np.array_equal(got, np.concatenate(want))


def test_dequant_q3k_known_answers(oracle):
    # all 64 six-bit scales over the blocks (both halves of the high-bit byte
    # layout), codes -4..3 in every hmask bit plane
    rng = np.random.default_rng(250)
    blobs, want = [], []
    scales = rng.permutation(np.arange(-32, 32))
    for rep in range(4):
        sc = scales[16 * rep:16 * rep + 16]
        q = rng.integers(-4, 4, 256)
        q[:8] = np.arange(-4, 4)
        d = bp.f16_bits(float(rng.uniform(0.01, 1.0)) * (-1 if rep == 2 else 1))
        blobs.append(bp.pack_q3k(d, sc, q))
        want.append(bp.expect_q3k(d, sc, q))
    got = oracle.dequantize(11, np.frombuffer(b"".join(blobs), dtype=np.uint8))
    assert np.array_equal(got, np.concatenate(want))


@pytest.mark.parametrize("t", [10, 11])
def test_k23_integer_sum_closed_form(oracle, t):
    # one block, x quantised to a single non-zero code: the dot is exactly
    # d_x * (that value's dequantised weight), so the vec_dot must reproduce
    # the dequantised weight at each probed position (to f32 rounding)
    rng = np.random.default_rng(260 + t)
    raw = bp.random_blocks(rng, t, 1, d_scale=0.05)
    wd = oracle.dequantize(t, raw).astype(np.float64)
    for pos in (0, 15, 16, 37, 128, 200, 255):
        x = np.zeros((1, 256), dtype=np.float32)
        x[0, pos] = -3.0                                  # code -128, d_x = 3/128
        xq = oracle.quantize_act(Q8_K, x)
        got = oracle.vec_dot(t, 256, raw, xq[0])
        ref = wd[pos] * (-3.0)
        assert abs(got - ref) <= 1e-6 * max(1.0, abs(ref)), (pos, got, ref)
