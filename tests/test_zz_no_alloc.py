"""lbq_qmatmul_f32_noalloc against lbq_qmatmul_f32, through the C ABI.

The allocation-free entry point runs the same kernels as lbq_qmatmul_f32 with
its activation scratch and GEMM workspace in a fixed per-device array, so its
outputs must equal lbq_qmatmul_f32's bit for bit, on every dispatch path (fused
decode GEMV, pre-quantised multi-row GEMV, 32-value types over row chunks, the
MFMA GEMM with and without split-k, unaligned x, dense weights), and stay within
the oracle's bar.  Calls come in pairs on the same weight, the second with a
smaller input, so a second call reading what the first left in the shared array
would show.  A call needing more than the array holds is refused before any
launch."""
import ctypes

import numpy as np
import pytest
import torch

import blockpack as bp
from test_gpu_parity import Q4_K, Q5_K, Q6_K, Q8_0, assert_rows_close, tight_bound, to_dev

pytestmark = pytest.mark.gpu
F16, Q4_0, Q4_1 = 1, 2, 3


def _weight(L, ctx, t, n, k, rng, dev):
    bs = 1 if t == F16 else (32 if t in (Q8_0, Q4_0, Q4_1) else 256)
    if t == F16:
        raw = (rng.standard_normal(n * k) * 0.05).astype(np.float16).view(np.uint8)
    else:
        raw = bp.random_blocks(rng, t, n * k // bs, d_scale=1e-3)
    wd = to_dev(raw, dev)
    h = ctypes.c_void_p()
    assert L.lbq_weight_wrap_device(ctx, t, n, k, wd.data_ptr(), wd.numel(), ctypes.byref(h)) == 0
    return h, wd, raw


def _both(L, ctx, h, x, n, dev):
    m, k = x.shape
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    y1 = torch.full((m, n), np.nan, device=dev)
    y2 = torch.full((m, n), np.nan, device=dev)
    assert L.lbq_qmatmul_f32(ctx, h, x.data_ptr(), m, y1.data_ptr(), st) == 0
    assert L.lbq_qmatmul_f32_noalloc(ctx, h, x.data_ptr(), m, y2.data_ptr(), st) == 0, L.lbq_last_error()
    torch.cuda.synchronize()
    return y1.cpu().numpy(), y2.cpu().numpy()


@pytest.mark.parametrize("t,n,k,ms", [
    (Q4_K, 1000, 4096, (1, 1)),        # fused decode GEMV (no scratch)
    (Q4_K, 1000, 4096, (8, 4)),        # pre-quantised multi-row GEMV
    (Q6_K, 700, 4096, (300, 40)),      # tall / k-sliced MFMA tiles
    (Q4_K, 4096, 14336, (512, 16)),    # split-k partials, then the integer matrix-core decode (two-way split, atomic adds)
    (Q5_K, 14336, 4096, (200, 32)),    # wide tiles, then the integer matrix-core decode
    (Q6_K, 8192, 4096, (16, 13)),      # slices added in the kernel twice (tile counters left zero)
    (Q4_K, 4096, 4096, (8, 6)),        # integer matrix-core decode, two workgroups per tile adding into y
    (Q5_K, 4096, 4096, (32, 12)),      # the same at 32 and 16 rows
    (Q8_0, 512, 4096, (64, 12)),       # Q8_0 on MFMA
    (Q4_0, 300, 1184, (20, 9)),        # activation scratch + GEMV row chunks (k % 256 != 0)
    (Q4_1, 300, 1024, (20, 9)),        # MFMA with the offset k-step operands in the workspace
    (F16, 300, 1024, (20, 3)),         # dense
])
def test_noalloc_matches_qmatmul(oracle, lbq, dev, t, n, k, ms):
    from lightbulb_amd.quantized import context
    L = lbq
    ctx = context(dev)
    rng = np.random.default_rng(600 + t + n + k)
    h, wd, raw = _weight(L, ctx, t, n, k, rng, dev)
    try:
        for m in ms:  # the second call is the smaller one
            x = rng.standard_normal((m, k)).astype(np.float32)
            y1, y2 = _both(L, ctx, h, to_dev(x, dev), n, dev)
            assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), (t, m)
            rows = sorted({0, m // 2, m - 1})
            if t == F16:
                ref = x[rows].astype(np.float64) @ raw.view(np.float16).reshape(n, k).astype(np.float64).T
                assert_rows_close(y2[rows], ref, 1e-5)
            else:
                ref = oracle.qmatmul(t, raw, n, k, x[rows], nthreads=8).astype(np.float64)
                assert_rows_close(y2[rows], ref, tight_bound(t, m) if k % 256 == 0 else 1e-4)
    finally:
        L.lbq_weight_destroy(h)


def test_noalloc_split_tiles_through_workspace(oracle, lbq, dev):
    # An output in host-pinned memory takes no atomic adds: the two workgroups of a
    # split 32-row tile store partials in the fixed array and the one that completes
    # the tile's counter (at the array's end) adds them.  Same bits as
    # lbq_qmatmul_f32 into device memory (atomic adds); two calls, the second smaller.
    from lightbulb_amd.quantized import context
    L = lbq
    ctx = context(dev)
    rng = np.random.default_rng(640)
    n, k = 4096, 4096
    h, wd, raw = _weight(L, ctx, Q4_K, n, k, rng, dev)
    try:
        for m in (8, 6):
            x = to_dev(rng.standard_normal((m, k)).astype(np.float32), dev)
            st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
            y1 = torch.full((m, n), np.nan, device=dev)
            y2 = torch.full((m, n), np.nan, dtype=torch.float32, pin_memory=True)
            assert L.lbq_qmatmul_f32(ctx, h, x.data_ptr(), m, y1.data_ptr(), st) == 0
            assert L.lbq_qmatmul_f32_noalloc(ctx, h, x.data_ptr(), m, y2.data_ptr(), st) == 0, L.lbq_last_error()
            torch.cuda.synchronize()
            a, b = y1.cpu().numpy(), y2.numpy()
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), m
            ref = oracle.qmatmul(Q4_K, raw, n, k, x.cpu().numpy()[[0, m - 1]], nthreads=8).astype(np.float64)
            assert_rows_close(b[[0, m - 1]], ref, 1e-4)
    finally:
        L.lbq_weight_destroy(h)


def test_noalloc_unaligned_x(oracle, lbq, dev):
    # x only 4-byte aligned: quantised into the scratch first, then the GEMM
    # workspace after it in the same array
    from lightbulb_amd.quantized import context
    L = lbq
    ctx = context(dev)
    rng = np.random.default_rng(650)
    n, k = 500, 2048
    h, wd, raw = _weight(L, ctx, Q4_K, n, k, rng, dev)
    try:
        for m in (40, 20):
            base = to_dev(rng.standard_normal(m * k + 1).astype(np.float32), dev)
            x = base[1:].reshape(m, k)
            y1, y2 = _both(L, ctx, h, x, n, dev)
            assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), m
    finally:
        L.lbq_weight_destroy(h)


def test_noalloc_limit(lbq, dev):
    # 4096 x 14336 operands in fp16 are 117 MB, beyond the 64 MiB array: refused
    from lightbulb_amd.quantized import context
    L = lbq
    ctx = context(dev)
    rng = np.random.default_rng(660)
    n, k, m = 64, 14336, 4096
    h, wd, raw = _weight(L, ctx, Q4_K, n, k, rng, dev)
    try:
        x = torch.zeros(m, k, device=dev)
        y = torch.full((m, n), 7.0, device=dev)
        assert L.lbq_qmatmul_f32_noalloc(ctx, h, x.data_ptr(), m, y.data_ptr(), None) == -6
        assert b"scratch" in L.lbq_last_error()
        torch.cuda.synchronize()
        assert bool((y == 7.0).all())  # nothing launched
        assert L.lbq_qmatmul_f32_noalloc(ctx, h, x.data_ptr(), 0, y.data_ptr(), None) == 0
        assert L.lbq_qmatmul_f32_noalloc(ctx, None, x.data_ptr(), 1, y.data_ptr(), None) == -1
    finally:
        L.lbq_weight_destroy(h)
