"""Non-finite and tiny values through the device path, against the oracle.

* NaN in x: the reference's activation quantisation never picks a NaN as the
  block maximum and `min(round(NaN), 127)` stores code 127 (Q8_K) / `as i8`
  stores 0 (Q8_0), so QMatMul::forward stays finite.  Checked bitwise on the
  quantised blocks and through forward at m = 1 (fused prologue), m = 4
  (standalone quantiser + multi-row GEMV) and m = 32 / 512 (MFMA operands).
* NaN / Inf f16 d and dmin in weight blocks: dequantisation equal to the oracle
  bit for bit on every value that is not NaN and NaN exactly where the oracle
  is NaN; forward non-finite exactly on the output columns of rows holding such
  a block (NaN wherever the block's scale is NaN), finite and close elsewhere.
* Tiny block scales (|d| ~ 1e-6, f16 subnormals included) through the MFMA
  path at m = 32 and 512: its fp16 weight operands carry a per-row power-of-two
  scale, so they keep full precision; held to the same guard as normal scales.
"""
import numpy as np
import pytest
import torch

import blockpack as bp
from test_gpu_parity import Q4_K, Q5_K, Q6_K, Q8_0, Q8_K, assert_rows_close, gpu_qmatmul, tight_bound, to_dev

Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K = 2, 3, 6, 7, 10, 11
ALL = [Q4_K, Q5_K, Q6_K, Q8_0, Q4_0, Q4_1, Q5_0, Q5_1, Q2_K, Q3_K]

pytestmark = pytest.mark.gpu

# byte offsets of the f16 scales (and mins / offsets) in a block
HDR = {Q4_K: (0, 2), Q5_K: (0, 2), Q6_K: (208,), Q8_0: (0,), Q4_0: (0,), Q4_1: (0, 2), Q5_0: (0,), Q5_1: (0, 2),
       Q2_K: (80, 82), Q3_K: (108,)}
BYTES = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_0: 34, Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q2_K: 84, Q3_K: 110}


def _nan_rows(rng, m, k):
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, 5] = np.nan                       # one NaN in a block
    x[min(1, m - 1), 256:512] = np.nan     # a whole NaN block
    x[m - 1, rng.integers(0, k, 7)] = np.nan
    return x


@pytest.mark.parametrize("act", [Q8_K, Q8_0])
def test_quantize_act_nan_bitwise(oracle, lbq, dev, act):
    from lightbulb_amd.quantized import quantize_activations
    x = _nan_rows(np.random.default_rng(300 + act), 4, 1024)
    x[2, 700] = np.inf
    x[3, 40] = -np.inf
    got = quantize_activations(to_dev(x, dev), act).cpu().numpy()
    assert np.array_equal(got, oracle.quantize_act(act, x))


@pytest.mark.parametrize("t", ALL)
def test_forward_nan_activations(oracle, lbq, dev, t):
    rng = np.random.default_rng(310 + t)
    n, k = 300, 4096
    w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3)
    for m in (1, 4, 32, 512):
        x = _nan_rows(rng, m, k)
        y = gpu_qmatmul(t, w_raw, n, k, x, dev)
        rows = sorted({r for r in (0, 1, m // 2, m - 1) if r < m})
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert np.all(np.isfinite(ref))
        assert_rows_close(y[rows], ref, tight_bound(t, m))


def _poison(raw, t, n, nbpr, rng):
    """Set NaN / +-Inf f16 scales in a few blocks of distinct rows; returns the
    weight rows hit and, of those, the rows holding a NaN scale."""
    blocks = raw.reshape(n * nbpr, BYTES[t])
    specials = [0x7e00, 0x7c00, 0xfc00]  # NaN, +Inf, -Inf
    rows = rng.choice(n, 9, replace=False)
    nan_rows = []
    for i, r in enumerate(rows):
        b = int(r) * nbpr + int(rng.integers(0, nbpr))
        off = HDR[t][i % len(HDR[t])]
        v = specials[i % 3]
        blocks[b, off] = v & 0xff
        blocks[b, off + 1] = v >> 8
        if v == 0x7e00:
            nan_rows.append(int(r))
    return sorted(int(r) for r in rows), sorted(nan_rows)


@pytest.mark.parametrize("t", ALL)
def test_dequant_nonfinite_scales(oracle, lbq, dev, t):
    from lightbulb_amd.quantized import dequantize_tensor
    rng = np.random.default_rng(320 + t)
    nb = 64
    raw = bp.random_blocks(rng, t, nb, d_scale=0.5)
    _poison(raw, t, nb, 1, rng)
    bs = oracle.block_size(t)
    ref = oracle.dequantize(t, raw)
    got = dequantize_tensor(to_dev(raw, dev), t, nb * bs).cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.isnan(ref).any() and np.isinf(ref).any()


@pytest.mark.parametrize("t", ALL)
def test_forward_nonfinite_scales(oracle, lbq, dev, t):
    rng = np.random.default_rng(330 + t)
    n, k = 200, 1024
    bs = oracle.block_size(t)
    w_raw = bp.random_blocks(rng, t, n * k // bs, d_scale=1e-3)
    bad, nan_rows = _poison(w_raw, t, n, k // bs, rng)
    good = np.setdiff1d(np.arange(n), bad)
    for m in (1, 4, 32, 300):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = gpu_qmatmul(t, w_raw, n, k, x, dev)
        rows = sorted({r for r in (0, m // 2, m - 1) if r < m})
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert not np.isfinite(ref[:, bad]).any() and np.isfinite(ref[:, good]).all()
        # non-finite exactly where the reference is; a NaN scale gives NaN under any
        # summation order, while an Inf scale gives Inf or NaN depending on how the
        # block's partial sums are grouped (the reference keeps 8 lane sums), so
        # NaN-ness is compared on the NaN-scale rows only
        assert np.array_equal(np.isfinite(y[rows]), np.isfinite(ref)), m
        assert np.isnan(y[rows][:, nan_rows]).all() and np.isnan(ref[:, nan_rows]).all(), m
        assert_rows_close(y[rows][:, good], ref[:, good], tight_bound(t, m))


@pytest.mark.parametrize("t", ALL)
@pytest.mark.parametrize("d_scale", [1e-6, 1e-7])
def test_tiny_scales_mfma(oracle, lbq, dev, t, d_scale):
    # |d| ~ 1e-6 .. 1e-7: dequantised values far below the fp16 normal range
    # (6.1e-5); the per-row operand exponent keeps them at full precision
    rng = np.random.default_rng(340 + t)
    n, k = 260, 2048
    w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=d_scale)
    for m in (1, 32, 512):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = gpu_qmatmul(t, w_raw, n, k, x, dev)
        rows = sorted({r for r in (0, 1, m // 2, m - 1) if r < m})
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert np.abs(ref).max() > 0
        assert_rows_close(y[rows], ref, tight_bound(t, m))


def test_mixed_row_scales_mfma(oracle, lbq, dev):
    # rows whose scales differ by 2^24, up to values past the fp16 range
    # (2^8 * 63 * 15 > 65504): each row's operands are scaled on their own
    rng = np.random.default_rng(350)
    n, k, t = 128, 1024, Q4_K
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1.0).reshape(n, 4, 144)
    for r in range(n):
        scale = 2.0 ** (-16 + (r % 5) * 6)  # 2^-16 .. 2^8
        d = (rng.standard_normal(4) * scale).astype(np.float16)
        w_raw[r, :, 0:2] = d.view(np.uint8).reshape(4, 2)
        w_raw[r, :, 2:4] = (d * 0.5).astype(np.float16).view(np.uint8).reshape(4, 2)
    w_raw = w_raw.reshape(-1)
    x = rng.standard_normal((64, k)).astype(np.float32)
    y = gpu_qmatmul(t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    # per output column (one weight row): relative error against that column's own scale
    err = np.abs(y - ref).max(axis=0) / np.maximum(np.abs(ref).max(axis=0), 1e-300)
    assert err.max() < 1e-2, err.max()
    assert_rows_close(y, ref, tight_bound(t, 64))
