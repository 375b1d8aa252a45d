"""Batch decode on the matrix cores (k_gemv_mx: Q4_K / Q5_K at m = 5..64 with
n >= 1024 -- m = 33..64 as two 32-row halves -- and m = 2..8 at k > 8192; Q6_K on
the same shapes at k > 8192 only; Q8_0 at m = 9..16 from 1024 rows; and through
LBQ_GEMV_MX_ALL wherever the kernel can run) against the oracle.

The kernel forms the reference's integer sub-block sums exactly (i8 MFMA) and
the mins term exactly (f16 MFMA of integers below 2^24), so it is held to the
decode bound (f32 summation order only).  Shapes cover uneven splits of a row's
blocks over the four waves (5 blocks), waves with no block (2 blocks), the
largest k (64 blocks), a row count that is not a multiple of 32, NaN activations
and NaN / Inf weight scales.  The same calls with the kernel switched off
(LBQ_GEMV_MX_OFF, the multi-row or general decode kernel) must differ in some
bits, which shows the matrix-core kernel is the one that ran.
"""
import numpy as np
import pytest

import blockpack as bp
from test_gpu_nonfinite import _nan_rows, _poison
from test_gpu_parity import Q4_K, Q5_K, Q6_K, Q8_0, assert_rows_close, gpu_qmatmul
from test_gpu_q8_0_dense import forward_with_env

pytestmark = pytest.mark.gpu


def mx_env(t, k):
    """Plan overrides that put a call on the kernel: Q6_K takes it only at k > 8192
    by default, LBQ_GEMV_MX_ALL everywhere it can run."""
    return {"LBQ_GEMV_MX_ALL": "1"} if t == Q6_K and k <= 8192 else {}


def mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev):
    env = mx_env(t, k)
    return forward_with_env(monkeypatch, env, t, w_raw, n, k, x, dev) if env else gpu_qmatmul(t, w_raw, n, k, x, dev)

# (8224 rows: 257 workgroups, the four-wave kernel; fewer rows: one workgroup per CU at
# most, the eight-wave kernel)
SHAPES = [(4096, 4096), (2050, 2048), (4100, 1280), (4096, 512), (64, 14336), (96, 16384), (8224, 1024)]


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [5, 8])
def test_mx_matches_oracle(oracle, lbq, dev, t, n, k, m, monkeypatch):
    rng = np.random.default_rng(n * 7 + k + 31 * m + t)
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    print(f"mx t={t} n={n} k={k} m={m}", flush=True)
    y = gpu_qmatmul(t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    again = gpu_qmatmul(t, w_raw, n, k, x, dev)
    assert np.array_equal(again.view(np.uint32), y.view(np.uint32))  # deterministic
    off = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_OFF": "1"}, t, w_raw, n, k, x, dev)
    assert_rows_close(off, ref, 1e-4)
    assert not np.array_equal(off.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("n,k", [(4096, 4096), (2050, 2048), (64, 14336), (96, 16384)])
@pytest.mark.parametrize("m", [2, 5, 8])
def test_mx_q6k_small_m_forced(oracle, lbq, dev, n, k, m, monkeypatch):
    # Q6_K at m <= 8 and k <= 8192 stays on the decode kernels; LBQ_GEMV_MX_ALL runs
    # the kernel's 8-row form there (uneven and empty waves), k > 8192 takes it anyway
    rng = np.random.default_rng(n + k + 53 * m)
    w_raw = bp.random_blocks(rng, Q6_K, n * k // 256, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    print(f"mx q6k forced n={n} k={k} m={m}", flush=True)
    y = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_ALL": "1"}, Q6_K, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(Q6_K, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    # (k > 8192 and m > 2: the kernel is Q6_K's default there too)
    same = np.array_equal(gpu_qmatmul(Q6_K, w_raw, n, k, x, dev).view(np.uint32), y.view(np.uint32))
    assert same == (k > 8192 and m > 2)


@pytest.mark.parametrize("m", [16, 32])
def test_mx_q6k_extreme_codes(oracle, lbq, dev, m, monkeypatch):
    # Q6_K blocks at the ends of every integer range: scales -128 / 127, 6-bit codes
    # 0 / 63 (values -32 / 31), activations of one magnitude (codes +-127, sums
    # +-2032 per group): the int32 block sums and the offset term stay exact
    rng = np.random.default_rng(970 + m)
    n, k = 1024, 4096
    blocks = np.zeros((n * k // 256, 210), dtype=np.uint8)
    blocks[:, :192] = rng.choice(np.array([0x00, 0xff], dtype=np.uint8), size=(blocks.shape[0], 192))
    blocks[:, 192:208] = rng.choice(np.array([0x80, 0x7f], dtype=np.uint8), size=(blocks.shape[0], 16))
    blocks[:, 208:210] = (rng.standard_normal(blocks.shape[0]) * 1e-3).astype(np.float16).view(np.uint8).reshape(-1, 2)
    w_raw = blocks.reshape(-1)
    x = (np.where(rng.random((m, k)) < 0.5, -100.0, 100.0)).astype(np.float32)
    y = forward_with_env(monkeypatch, mx_env(Q6_K, k), Q6_K, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(Q6_K, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)


# m = 9..32 runs on the kernel from 1024 rows: 32-128 tiles (two workgroups each),
# 129-130 tiles (one, eight waves), 257 (one, four waves); k from 2 to 64 blocks
WIDE_SHAPES = [(4096, 4096), (1056, 4096), (4100, 1280), (4096, 512), (8224, 1024), (4096, 14336), (4160, 16384)]


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("n,k", WIDE_SHAPES)
@pytest.mark.parametrize("m", [9, 16, 17, 32])
def test_mx_wide_matches_oracle(oracle, lbq, dev, t, n, k, m, monkeypatch):
    # m = 9..16 and 17..32: the kernel's 16- and 32-row forms (every C row of the
    # 32 x 32 tile in use at m = 32)
    rng = np.random.default_rng(n * 5 + k + 37 * m + t)
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    print(f"mx wide t={t} n={n} k={k} m={m}", flush=True)
    y = mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    again = mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev)
    assert np.array_equal(again.view(np.uint32), y.view(np.uint32))  # deterministic
    # switched off: the fp16 GEMM (its own bound), which must differ in some bits
    off = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_WIDE_OFF": "1"}, t, w_raw, n, k, x, dev)
    assert_rows_close(off, ref, 2e-3)
    assert not np.array_equal(off.view(np.uint32), y.view(np.uint32))


# m = 33..64 (from 1024 rows, where the m <= 32 launch has at most one workgroup per
# CU): two 32-row halves per tile (workgroups b and b + 8 of each 16), with and
# without the two-way split (up to 128 tiles), a last tile of 4 rows, k from 5 to
# 56 blocks
HALF_SHAPES = [(4096, 4096), (1056, 4096), (4100, 1280), (8192, 1024), (4096, 14336)]


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("n,k", HALF_SHAPES)
@pytest.mark.parametrize("m", [33, 47, 64])
def test_mx_halves_match_oracle(oracle, lbq, dev, t, n, k, m, monkeypatch):
    rng = np.random.default_rng(n * 3 + k + 41 * m + t)
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    print(f"mx halves t={t} n={n} k={k} m={m}", flush=True)
    y = mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    again = mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev)
    assert np.array_equal(again.view(np.uint32), y.view(np.uint32))  # deterministic
    # switched off: the fp16 GEMM (its own bound), which must differ in some bits
    off = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_HALVES_OFF": "1"}, t, w_raw, n, k, x, dev)
    assert_rows_close(off, ref, 2e-3)
    assert not np.array_equal(off.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m,n,k", [(40, 4096, 1024), (64, 2080, 2048), (64, 8192, 1024)])
def test_mx_halves_are_two_launches(lbq, dev, t, m, n, k, monkeypatch):
    # each half is the 32-row launch over its rows: with the wave count pinned (the
    # plan picks it from the grid, which the halves double), rows 0..31 carry the
    # bits of forward(x[:32]) and rows 32.. those of forward(x[32:]), with the
    # two-way split (4096 and 2080 rows) and without (8192)
    rng = np.random.default_rng(960 + t + m + n)
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    print(f"mx halves bits t={t} m={m} n={n} k={k}", flush=True)
    env = {"LBQ_GEMV_MX_WAVES": "4", **mx_env(t, k)}
    if t == Q6_K:
        env["LBQ_GEMV_MX_ALL"] = "1"  # (Q6_K at m <= 8 runs the decode kernels otherwise)
    y = forward_with_env(monkeypatch, env, t, w_raw, n, k, x, dev)
    lo = forward_with_env(monkeypatch, env, t, w_raw, n, k, np.ascontiguousarray(x[:32]), dev)
    hi = forward_with_env(monkeypatch, env, t, w_raw, n, k, np.ascontiguousarray(x[32:]), dev)
    assert np.array_equal(y[:32].view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(y[32:].view(np.uint32), hi.view(np.uint32))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m,k,n", [(6, 4096, 4096), (7, 4096, 4096), (2, 14336, 160), (3, 14336, 33), (4, 9216, 160),
                                   (2, 8448, 1), (5, 8448, 70), (12, 512, 4097), (31, 768, 4127), (25, 8448, 4100)])
def test_mx_row_counts(oracle, lbq, dev, t, m, k, n, monkeypatch):
    # k = 8448: 33 blocks, the smallest k the kernel takes at m <= 4; n = 1 and 33:
    # a workgroup of one row, a last workgroup of one row
    rng = np.random.default_rng(900 + 10 * m + t + k + n)
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m,n,k", [(8, 96, 14336), (32, 4096, 4096)])
def test_mx_nan_activations(oracle, lbq, dev, t, m, n, k, monkeypatch):
    rng = np.random.default_rng(910 + t + m)
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    x = _nan_rows(rng, m, k)
    y = mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert np.all(np.isfinite(ref))
    assert_rows_close(y, ref, 1e-4)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m,n,k", [(8, 200, 14336), (32, 4128, 4096)])
def test_mx_nonfinite_scales(oracle, lbq, dev, t, m, n, k, monkeypatch):
    rng = np.random.default_rng(920 + t + m)
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    bad, nan_rows = _poison(w_raw, t, n, k // 256, rng)
    good = np.setdiff1d(np.arange(n), bad)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = mx_qmatmul(monkeypatch, t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert not np.isfinite(ref[:, bad]).any() and np.isfinite(ref[:, good]).all()
    assert np.array_equal(np.isfinite(y), np.isfinite(ref))
    assert np.isnan(y[:, nan_rows]).all() and np.isnan(ref[:, nan_rows]).all()
    assert_rows_close(y[:, good], ref[:, good], 1e-4)


SPLIT_CASES = [(8, 4096, 4096), (16, 4096, 14336), (32, 4096, 2048), (6, 2080, 8192), (64, 4096, 4096), (45, 2080, 4096)]
# (Q6_K: the kernel's own shapes, k > 8192)
SPLIT_CASES_Q6 = [(6, 4096, 9216), (16, 4096, 14336), (32, 2048, 9216), (64, 4096, 9216), (45, 2080, 9216)]


@pytest.mark.parametrize("t,m,n,k", [(t, *c) for t in (Q4_K, Q5_K) for c in SPLIT_CASES] +
                         [(Q6_K, *c) for c in SPLIT_CASES_Q6])
def test_mx_split_halves_same_bits(oracle, lbq, dev, t, m, n, k):
    # Up to 4096 rows a tile is split over two workgroups.  forward() zeroes y in the
    # quantisation launch and the halves are added into it atomically; the
    # pre-quantised handle (no quantisation launch) adds them through the workspace
    # and a tile counter.  Two addends: both give the same bits, as does a grouped
    # call (one quantisation zeroing both outputs) for each of its weights.
    import torch
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor, qmatmul_group
    from test_gpu_parity import to_dev
    rng = np.random.default_rng(930 + t + m + n + k)
    raws = [bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3) for _ in range(2)]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r in raws]
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    xd = to_dev(x, dev)
    print(f"mx split t={t} m={m} n={n} k={k}", flush=True)
    y = qms[0].forward(xd)
    y2 = qms[0].forward_quantized(QActivation.for_weight(qms[0], m).quantize(xd))
    yg = qmatmul_group(qms, xd)
    y1b = qms[1].forward(xd)
    torch.cuda.synchronize()
    ref = oracle.qmatmul(t, raws[0], n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y.cpu().numpy(), ref, 1e-4)
    bits = lambda a: a.cpu().numpy().view(np.uint32)
    assert np.array_equal(bits(y), bits(y2))
    assert np.array_equal(bits(y), bits(yg[0]))
    assert np.array_equal(bits(y1b), bits(yg[1]))


@pytest.mark.parametrize("t,m,k", [(Q4_K, 8, 4096), (Q5_K, 8, 4096), (Q6_K, 8, 9216)])
def test_mx_split_halves_subnormal_and_host_output(oracle, lbq, dev, t, m, k):
    # Two-way split tiles at m = 8: with tiny weight scales (f16 d ~1e-7) and a tiny
    # x (~1e-36, Q8_K scales ~1e-38) the halves are subnormal f32.  forward() adds them with f32 atomics into y (plain device
    # memory); the pre-quantised handle, and forward() into host-pinned memory
    # (which takes no atomics), add them through the workspace.  Halves in the
    # normal range give the same bits either way; subnormal ones may differ only by
    # the subnormal part (an atomic add may flush it), never by more than 2^-126.
    import ctypes
    import torch
    from lightbulb_amd import _lib
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    from test_gpu_parity import to_dev
    rng = np.random.default_rng(960 + t)
    n = 2048
    L = _lib.lib()
    bits = lambda a: np.asarray(a).view(np.uint32)
    for scale, d_scale in ((1.0, 1e-3), (1e-36, 1e-7)):
        raw = bp.random_blocks(rng, t, n * k // 256, d_scale=d_scale)
        qm = QMatMul.from_qtensor(QTensor(to_dev(raw, dev), t, (n, k)))
        x = (rng.standard_normal((m, k)) * scale).astype(np.float32)
        xd = to_dev(x, dev)
        print(f"mx split subnormal t={t} scale={scale}", flush=True)
        y = qm.forward(xd)
        y2 = qm.forward_quantized(QActivation.for_weight(qm, m).quantize(xd))
        yh = torch.empty(m, n, dtype=torch.float32, pin_memory=True)
        _lib.check(L.lbq_qmatmul_f32(qm._ctx, qm._handle, xd.data_ptr(), m, yh.data_ptr(),
                                     ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
        torch.cuda.synchronize()
        a, b, h = y.cpu().numpy(), y2.cpu().numpy(), yh.numpy()
        assert np.array_equal(bits(b), bits(h))  # the same protocol, device or host output
        normal = np.abs(b) >= np.float32(2.0 ** -126)
        assert np.array_equal(bits(a)[normal], bits(b)[normal])
        assert np.all(np.abs(a.astype(np.float64) - b) <= 2.0 ** -126)
        if scale == 1.0:
            ref = oracle.qmatmul(t, raw, n, k, x, nthreads=8).astype(np.float64)
            assert_rows_close(a, ref, 1e-4)
        else:
            assert (~normal).sum() > 0  # the case exercises subnormal halves


def test_overlapping_x_and_y_refused(lbq, dev):
    # QMatMul::forward returns a new tensor; an output that overlaps the input is refused
    import torch
    from lightbulb_amd import _lib
    from lightbulb_amd.quantized import QMatMul, QTensor
    from test_gpu_parity import to_dev
    rng = np.random.default_rng(970)
    n = k = 256
    qm = QMatMul.from_qtensor(QTensor(to_dev(bp.random_blocks(rng, Q4_K, n * k // 256, d_scale=1e-3), dev), Q4_K, (n, k)))
    buf = torch.zeros(4 * k, dtype=torch.float32, device=dev)
    L = _lib.lib()
    assert L.lbq_qmatmul_f32(qm._ctx, qm._handle, buf.data_ptr(), 2, buf[k:].data_ptr(), None) == -1
    assert b"overlap" in L.lbq_last_error()
    assert L.lbq_qmatmul_f32(qm._ctx, qm._handle, buf.data_ptr(), 1, buf[k:].data_ptr(), None) == 0
    torch.cuda.synchronize()


def test_wrapped_weight_refresh(oracle, lbq, dev):
    # a handle wrapped over zero-filled device memory, the blocks written afterwards:
    # lbq_weight_refresh recomputes the MFMA GEMM's per-row exponents, after which
    # m > 8 forwards are correct (m <= 8 never used them)
    import ctypes
    import torch
    from lightbulb_amd import _lib
    from lightbulb_amd.quantized import context
    from test_gpu_parity import to_dev
    rng = np.random.default_rng(980)
    n, k = 512, 4096
    raw = bp.random_blocks(rng, Q6_K, n * k // 256, d_scale=1e-3)
    L = _lib.lib()
    ctx = context(dev)
    buf = torch.zeros(raw.size, dtype=torch.uint8, device=dev)
    h = ctypes.c_void_p()
    _lib.check(L.lbq_weight_wrap_device(ctx, Q6_K, n, k, buf.data_ptr(), raw.size, ctypes.byref(h)))
    buf.copy_(to_dev(raw, dev))
    _lib.check(L.lbq_weight_refresh(h, ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
    for m in (1, 64):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = torch.empty(m, n, dtype=torch.float32, device=dev)
        _lib.check(L.lbq_qmatmul_f32(ctx, h, to_dev(x, dev).data_ptr(), m, y.data_ptr(),
                                     ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)))
        torch.cuda.synchronize()
        ref = oracle.qmatmul(Q6_K, raw, n, k, x, nthreads=8).astype(np.float64)
        assert_rows_close(y.cpu().numpy(), ref, 1e-4 if m == 1 else 1.5e-3)
    assert L.lbq_weight_refresh(None, None) == -1
    _lib.check(L.lbq_weight_destroy(h))


def _gate_up_env(monkeypatch, env, t, g_raw, u_raw, n, k, x, dev):
    """lbq_gate_up_silu_f32 through a context created with the given plan overrides."""
    import ctypes
    import torch
    from lightbulb_amd import _lib
    from test_gpu_parity import to_dev
    L = _lib.lib()
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    ctx = ctypes.c_void_p()
    try:
        _lib.check(L.lbq_init(dev.index or 0, ctypes.byref(ctx)))
    finally:
        for key in env:
            monkeypatch.delenv(key)
    hs, keep = [], []
    try:
        for raw in (g_raw, u_raw):
            wd = to_dev(raw, dev)
            keep.append(wd)
            h = ctypes.c_void_p()
            _lib.check(L.lbq_weight_wrap_device(ctx, t, n, k, wd.data_ptr(), wd.numel(), ctypes.byref(h)))
            hs.append(h)
        xd = to_dev(x, dev)
        out = torch.empty(x.shape[0], n, device=dev)
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(L.lbq_gate_up_silu_f32(ctx, hs[0], hs[1], xd.data_ptr(), x.shape[0], out.data_ptr(), st))
        torch.cuda.synchronize()
        return out.cpu().numpy()
    finally:
        for h in hs:
            L.lbq_weight_destroy(h)
        L.lbq_ctx_destroy(ctx)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m,n,k", [(2, 8224, 9216), (5, 8224, 2048), (16, 8240, 1024), (32, 8256, 4096)])
def test_mx_gate_up_pair(oracle, lbq, dev, t, m, n, k, monkeypatch):
    # above 8192 rows a gate/up pair at m = 2..32 is one launch (16 gate and 16 up
    # rows per tile, silu(gate) * up in the epilogue): the bits of the two separate
    # launches and the product launch (LBQ_GEMV_MX_PAIR_OFF), and the oracle's value
    rng = np.random.default_rng(940 + t + m + n + k)
    g_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    u_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    print(f"mx pair t={t} m={m} n={n} k={k}", flush=True)
    y = _gate_up_env(monkeypatch, mx_env(t, k), t, g_raw, u_raw, n, k, x, dev)
    off = _gate_up_env(monkeypatch, {"LBQ_GEMV_MX_PAIR_OFF": "1", **mx_env(t, k)}, t, g_raw, u_raw, n, k, x, dev)
    assert np.array_equal(y.view(np.uint32), off.view(np.uint32))
    gr = oracle.qmatmul(t, g_raw, n, k, x, nthreads=8).astype(np.float64)
    ur = oracle.qmatmul(t, u_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, gr / (1.0 + np.exp(-gr)) * ur, 1e-4)


GROUP_CASES = [(6, (4096, 1024, 2080), 4096), (16, (4096, 1024, 2080), 2048), (32, (1024, 4096), 4096),
               (8, (14336, 14336), 4096), (40, (4096, 1024, 2080), 4096), (64, (1024, 4096), 2048)]


GROUP_CASES_Q6 = [(6, (4096, 1024, 2080), 9216), (16, (4096, 1024, 2080), 9216), (32, (1024, 4096), 9216),
                  (40, (4096, 1024, 2080), 9216), (64, (1024, 4096), 9216)]


@pytest.mark.parametrize("t,m,ns,k", [(t, *c) for t in (Q4_K, Q5_K) for c in GROUP_CASES] +
                         [(Q6_K, *c) for c in GROUP_CASES_Q6])
def test_mx_group_one_launch(oracle, lbq, dev, t, m, ns, k):
    # a grouped call whose weights all run on the kernel is one launch (each weight's
    # workgroups as its own launch would run them): the bits of the separate calls
    import torch
    from lightbulb_amd.quantized import QMatMul, QTensor, qmatmul_group
    from test_gpu_parity import to_dev
    rng = np.random.default_rng(950 + t + m + k + len(ns))
    raws = [bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3) for n in ns]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, ns)]
    x = rng.standard_normal((m, k)).astype(np.float32)
    xd = to_dev(x, dev)
    print(f"mx group t={t} m={m} ns={ns} k={k}", flush=True)
    ys = qmatmul_group(qms, xd)
    sep = [q.forward(xd) for q in qms]
    torch.cuda.synchronize()
    for a, b in zip(ys, sep):
        assert np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))
    i = int(np.argmin(ns))
    ref = oracle.qmatmul(t, raws[i], ns[i], k, x, nthreads=8).astype(np.float64)
    assert_rows_close(ys[i].cpu().numpy(), ref, 1e-4)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m", [2, 6, 16, 32, 48])
def test_mx_rmsnorm_in_quantisation(oracle, lbq, dev, t, m):
    # at m > 1 the call-site entry points run candle's RmsNorm inside the Q8_K
    # quantisation launch when every weight reads pre-quantised activations (the
    # normalised x never reaches memory): grouped weights at k = 2304 (9 blocks, one
    # partial pass), 4096 and 14336 (56 blocks, four passes) and a gate/up pair above
    # 8192 rows, against the oracle on the numpy-normalised x
    import torch
    from lightbulb_amd.quantized import QMatMul, QTensor, rmsnorm_gate_up_silu, rmsnorm_qmatmul_group
    from test_gpu_parity import _rms_norm_ref, to_dev
    rng = np.random.default_rng(990 + t + m)
    for k, ns in ((2304, (1024, 1040)), (4096, (2048, 1024, 1056)), (14336, (1024,))):
        raws = [bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3) for n in ns]
        qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, ns)]
        w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
        x = (3.0 * rng.standard_normal((m, k)) + 0.5).astype(np.float32)
        x[rng.random(x.shape) < 0.01] *= 20
        xn = _rms_norm_ref(x, w, 1e-5)
        print(f"mx rmsnorm group t={t} m={m} k={k} ns={ns}", flush=True)
        ys = rmsnorm_qmatmul_group(qms, to_dev(x, dev), to_dev(w, dev), 1e-5)
        torch.cuda.synchronize()
        for y, r, n in zip(ys, raws, ns):
            assert_rows_close(y.cpu().numpy(), oracle.qmatmul(t, r, n, k, xn, nthreads=8).astype(np.float64), 2e-3)
    k, n = 4096, 8256
    g_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    u_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    qg = QMatMul.from_qtensor(QTensor(to_dev(g_raw, dev), t, (n, k)))
    qu = QMatMul.from_qtensor(QTensor(to_dev(u_raw, dev), t, (n, k)))
    w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    x = (3.0 * rng.standard_normal((m, k)) + 0.5).astype(np.float32)
    xn = _rms_norm_ref(x, w, 1e-5)
    print(f"mx rmsnorm pair t={t} m={m} n={n}", flush=True)
    out = rmsnorm_gate_up_silu(qg, qu, to_dev(x, dev), to_dev(w, dev), 1e-5)
    torch.cuda.synchronize()
    gr = oracle.qmatmul(t, g_raw, n, k, xn, nthreads=8).astype(np.float64)
    ur = oracle.qmatmul(t, u_raw, n, k, xn, nthreads=8).astype(np.float64)
    assert_rows_close(out.cpu().numpy(), gr / (1.0 + np.exp(-gr)) * ur, 2e-3)


# Q8_0 (m = 5..32 from 1024 rows, m = 33..64 as row halves at k <= 8192; k % 256 ==
# 0): eight 34-byte blocks per step, one v_mfma_i32_32x32x32_i8 per block,
# (sum * d_w) * d_x in f32 -- the decode bound
Q80_SHAPES = [(4096, 4096), (1056, 4096), (4100, 1280), (8224, 1024), (4096, 14336), (1024, 16384)]


@pytest.mark.parametrize("n,k,m", [(n, k, m) for (n, k) in Q80_SHAPES for m in (9, 12, 16, 17, 32, 40, 64)
                                   if m <= 32 or (k <= 8192 and n <= 8192)])
def test_mx_q8_0_matches_oracle(oracle, lbq, dev, n, k, m, monkeypatch):
    rng = np.random.default_rng(n * 11 + k + 43 * m)
    w_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    print(f"mx q8_0 n={n} k={k} m={m}", flush=True)
    y = gpu_qmatmul(Q8_0, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(Q8_0, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    again = gpu_qmatmul(Q8_0, w_raw, n, k, x, dev)
    assert np.array_equal(again.view(np.uint32), y.view(np.uint32))  # deterministic
    off = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_WIDE_OFF": "1"}, Q8_0, w_raw, n, k, x, dev)
    assert_rows_close(off, ref, 2e-3)
    assert not np.array_equal(off.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("m", [40, 64])
def test_mx_q8_0_halves_are_two_launches(lbq, dev, m, monkeypatch):
    # each 32-row half is the m <= 32 launch over its rows (the wave count pinned)
    rng = np.random.default_rng(1040 + m)
    n, k = 4096, 2048
    w_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    env = {"LBQ_GEMV_MX_WAVES": "4", "LBQ_GEMV_MX_ALL": "1"}
    y = forward_with_env(monkeypatch, env, Q8_0, w_raw, n, k, x, dev)
    lo = forward_with_env(monkeypatch, env, Q8_0, w_raw, n, k, np.ascontiguousarray(x[:32]), dev)
    hi = forward_with_env(monkeypatch, env, Q8_0, w_raw, n, k, np.ascontiguousarray(x[32:]), dev)
    assert np.array_equal(y[:32].view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(y[32:].view(np.uint32), hi.view(np.uint32))


@pytest.mark.parametrize("n,k", [(4096, 4096), (2050, 2048), (64, 14336), (96, 16384)])
@pytest.mark.parametrize("m", [2, 5, 8])
def test_mx_q8_0_small_m_forced(oracle, lbq, dev, n, k, m, monkeypatch):
    # Q8_0 at m <= 4 or below 1024 rows stays on the decode kernels;
    # LBQ_GEMV_MX_ALL runs the 8-row form there
    rng = np.random.default_rng(n + k + 59 * m)
    w_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    print(f"mx q8_0 forced n={n} k={k} m={m}", flush=True)
    y = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_ALL": "1"}, Q8_0, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(Q8_0, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    same = np.array_equal(gpu_qmatmul(Q8_0, w_raw, n, k, x, dev).view(np.uint32), y.view(np.uint32))
    assert same == (m >= 5 and n >= 1024)  # (the kernel is Q8_0's default there)


@pytest.mark.parametrize("m", [9, 16, 32])
def test_mx_q8_0_extremes_and_nonfinite(oracle, lbq, dev, m):
    # codes at -128 / 127 against activations of one magnitude (codes +-127): the
    # int32 block sums stay exact; then NaN / +-Inf block scales in a few rows
    rng = np.random.default_rng(1010 + m)
    n, k = 1024, 4096
    blocks = np.zeros((n * k // 32, 34), dtype=np.uint8)
    blocks[:, 2:] = rng.choice(np.array([0x80, 0x7f], dtype=np.uint8), size=(blocks.shape[0], 32))
    blocks[:, :2] = (rng.standard_normal(blocks.shape[0]) * 1e-3).astype(np.float16).view(np.uint8).reshape(-1, 2)
    w_raw = blocks.reshape(-1)
    x = (np.where(rng.random((m, k)) < 0.5, -100.0, 100.0)).astype(np.float32)
    y = gpu_qmatmul(Q8_0, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(Q8_0, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    w2 = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3)
    bad, nan_rows = _poison(w2, Q8_0, n, k // 32, rng)
    good = np.setdiff1d(np.arange(n), bad)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = gpu_qmatmul(Q8_0, w2, n, k, x, dev)
    ref = oracle.qmatmul(Q8_0, w2, n, k, x, nthreads=8).astype(np.float64)
    assert np.array_equal(np.isfinite(y), np.isfinite(ref))
    assert np.isnan(y[:, nan_rows]).all()
    assert_rows_close(y[:, good], ref[:, good], 1e-4)
    xn = _nan_rows(rng, m, k)
    y = gpu_qmatmul(Q8_0, w_raw, n, k, xn, dev)
    ref = oracle.qmatmul(Q8_0, w_raw, n, k, xn, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)


@pytest.mark.parametrize("m,n,k", [(16, 4096, 4096), (12, 2080, 2048), (9, 1024, 14336), (32, 2048, 4096),
                                   (64, 4096, 2048)])
def test_mx_q8_0_split_and_group_bits(oracle, lbq, dev, m, n, k):
    # two-way split tiles: forward() (y zeroed by the Q8_0 quantisation launch, halves
    # added atomically), the pre-quantised handle (partials and a tile counter) and a
    # grouped call (one quantisation, one launch) give the same bits
    import torch
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor, qmatmul_group
    from test_gpu_parity import to_dev
    rng = np.random.default_rng(1020 + m + n + k)
    raws = [bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3) for _ in range(2)]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), Q8_0, (n, k))) for r in raws]
    x = rng.standard_normal((m, k)).astype(np.float32)
    xd = to_dev(x, dev)
    y = qms[0].forward(xd)
    y2 = qms[0].forward_quantized(QActivation.for_weight(qms[0], m).quantize(xd))
    yg = qmatmul_group(qms, xd)
    y1b = qms[1].forward(xd)
    torch.cuda.synchronize()
    ref = oracle.qmatmul(Q8_0, raws[0], n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y.cpu().numpy(), ref, 1e-4)
    bits = lambda a: a.cpu().numpy().view(np.uint32)
    assert np.array_equal(bits(y), bits(y2))
    assert np.array_equal(bits(y), bits(yg[0]))
    assert np.array_equal(bits(y1b), bits(yg[1]))


@pytest.mark.parametrize("m", [9, 16, 32])
def test_mx_q8_0_gate_up_pair(oracle, lbq, dev, m, monkeypatch):
    # a Q8_0 gate/up pair above 8192 rows in one launch: the bits of the separate
    # launches and the product launch, and the oracle's value
    rng = np.random.default_rng(1030 + m)
    n, k = 8240, 1024
    g_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3)
    u_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = _gate_up_env(monkeypatch, {}, Q8_0, g_raw, u_raw, n, k, x, dev)
    off = _gate_up_env(monkeypatch, {"LBQ_GEMV_MX_PAIR_OFF": "1"}, Q8_0, g_raw, u_raw, n, k, x, dev)
    assert np.array_equal(y.view(np.uint32), off.view(np.uint32))
    gr = oracle.qmatmul(Q8_0, g_raw, n, k, x, nthreads=8).astype(np.float64)
    ur = oracle.qmatmul(Q8_0, u_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, gr / (1.0 + np.exp(-gr)) * ur, 1e-4)


# The legacy 32-value types (m = 5..16 from 1024 rows, k % 256 == 0): eight blocks per
# step, q - 8 / q - 16 formed bytewise (Q4_0 / Q5_0), + m * s (Q4_1 / Q5_1 against
# Q8_1 activations) -- the decode bound; byte sizes 18 / 20 / 22 / 24
LEG = [2, 3, 6, 7]
LEG_BYTES = {2: 18, 3: 20, 6: 22, 7: 24}


@pytest.mark.parametrize("t", LEG)
@pytest.mark.parametrize("n,k", [(4096, 4096), (1056, 4096), (4100, 1280), (4096, 14336), (1024, 16384)])
@pytest.mark.parametrize("m", [5, 9, 16])
def test_mx_legacy_matches_oracle(oracle, lbq, dev, t, n, k, m, monkeypatch):
    rng = np.random.default_rng(n * 13 + k + 47 * m + t)
    w_raw = bp.random_blocks(rng, t, n * k // 32, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    print(f"mx legacy t={t} n={n} k={k} m={m}", flush=True)
    y = gpu_qmatmul(t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    again = gpu_qmatmul(t, w_raw, n, k, x, dev)
    assert np.array_equal(again.view(np.uint32), y.view(np.uint32))  # deterministic
    off = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_OFF": "1"}, t, w_raw, n, k, x, dev)
    assert_rows_close(off, ref, 2e-3)
    assert not np.array_equal(off.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("t", LEG)
@pytest.mark.parametrize("n,k,m", [(4096, 4096, 2), (2050, 2048, 8), (64, 14336, 4), (96, 16384, 8)])
def test_mx_legacy_forced_and_extremes(oracle, lbq, dev, t, n, k, m, monkeypatch):
    # LBQ_GEMV_MX_ALL runs the kernel at m <= 4 and below 1024 rows; then blocks at the
    # ends of every field (codes 0 / 15 or 31, every fifth bit set or clear, d and m of
    # both signs) against activations of one magnitude
    rng = np.random.default_rng(1050 + t + m + n)
    w_raw = bp.random_blocks(rng, t, n * k // 32, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_ALL": "1"}, t, w_raw, n, k, x, dev)
    ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
    assert_rows_close(y, ref, 1e-4)
    blocks = w_raw.reshape(-1, LEG_BYTES[t]).copy()
    hdr = 4 if t in (3, 7) else 2
    body = rng.choice(np.array([0x00, 0xff], dtype=np.uint8), size=(blocks.shape[0], LEG_BYTES[t] - hdr))
    blocks[:, hdr:] = body
    w2 = blocks.reshape(-1)
    x2 = (np.where(rng.random((m, k)) < 0.5, -100.0, 100.0)).astype(np.float32)
    y2 = forward_with_env(monkeypatch, {"LBQ_GEMV_MX_ALL": "1"}, t, w2, n, k, x2, dev)
    ref2 = oracle.qmatmul(t, w2, n, k, x2, nthreads=8).astype(np.float64)
    assert_rows_close(y2, ref2, 1e-4)


@pytest.mark.parametrize("t", LEG)
def test_mx_legacy_nonfinite_and_bits(oracle, lbq, dev, t):
    # NaN / Inf block scales in a few rows; then forward(), the pre-quantised handle and
    # a grouped call give the same bits (two-way split tiles at 4096 rows)
    import torch
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor, qmatmul_group
    from test_gpu_parity import to_dev
    rng = np.random.default_rng(1060 + t)
    n, k, m = 4096, 2048, 12
    w_raw = bp.random_blocks(rng, t, n * k // 32, d_scale=1e-3)
    w_bad = w_raw.copy()
    bad, nan_rows = _poison(w_bad, t, n, k // 32, rng)
    good = np.setdiff1d(np.arange(n), bad)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = gpu_qmatmul(t, w_bad, n, k, x, dev)
    ref = oracle.qmatmul(t, w_bad, n, k, x, nthreads=8).astype(np.float64)
    assert np.array_equal(np.isfinite(y), np.isfinite(ref))
    assert np.isnan(y[:, nan_rows]).all()
    assert_rows_close(y[:, good], ref[:, good], 1e-4)
    raws = [w_raw, bp.random_blocks(rng, t, n * k // 32, d_scale=1e-3)]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r in raws]
    xd = to_dev(x, dev)
    y0 = qms[0].forward(xd)
    y0q = qms[0].forward_quantized(QActivation.for_weight(qms[0], m).quantize(xd))
    yg = qmatmul_group(qms, xd)
    y1 = qms[1].forward(xd)
    torch.cuda.synchronize()
    bits = lambda a: a.cpu().numpy().view(np.uint32)
    assert np.array_equal(bits(y0), bits(y0q))
    assert np.array_equal(bits(y0), bits(yg[0]))
    assert np.array_equal(bits(y1), bits(yg[1]))
