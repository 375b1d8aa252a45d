"""Q8_0 on the MFMA path and dense F32 / F16 weights, on the GPU.

* Q8_0 at m > 8 (k % 256 == 0) runs the batched MFMA kernels on fp16 operands
  of the reference's Q8_0 activation values and the d*q weight values; checked
  against the oracle (the reference's integer Q8_0 x Q8_0 path) at the MFMA
  guard on every kernel the plan reaches (k-sliced, 64-row, wide and tall
  tiles), at configs[0]'s 4096 x 4096 for M = 16 / 64 / 512, and the operands
  built from f32 x and from pre-quantised codes agree to the bit.
* Dense weights are candle's dense QMatMul variant (QMatMul::from_qtensor
  dequantises F32 / F16 / BF16 and forward is an f32 matmul): checked against a
  float64 x . W^T at the 2e-3 bar (and a 1e-5 guard: the device computes in
  f32 too), through forward, the grouped and gate/up entry points, a GGUF
  file holding F16, F32 and BF16 output.weight tensors, and the embedding gather.
  BF16 values are widened exactly (the 16 bits are the f32's upper half), so
  dequantisation and the embedding gather are bit-exact against numpy.
* Launch-plan overrides (read from the environment when a context is created)
  route shapes to every k-slice length and tile kind; results stay within the
  guard.
"""
import ctypes

import numpy as np
import pytest
import torch

import blockpack as bp
from test_gpu_parity import Q4_K, Q5_K, Q6_K, Q8_0, assert_rows_close, gpu_qmatmul, tight_bound, to_dev

pytestmark = pytest.mark.gpu
F32, F16, BF16 = 0, 1, 30


def _bf16_bits(w: np.ndarray) -> np.ndarray:
    """f32 -> bfloat16 bits (round to nearest even), as uint16."""
    u = np.ascontiguousarray(w, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- Q8_0 on MFMA
@pytest.mark.parametrize("m,n,k", [(9, 300, 256), (32, 1000, 256 * 5), (48, 130, 4096), (64, 257, 256 * 3),
                                   (100, 300, 256 * 2), (130, 77, 256 * 12), (300, 390, 256 * 3),
                                   (520, 200, 256 * 4)])
def test_q8_0_mfma_shapes(oracle, lbq, dev, m, n, k):
    rng = np.random.default_rng(400 + m + n)
    w_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = gpu_qmatmul(Q8_0, w_raw, n, k, x, dev)
    rows = sorted({0, 1, m // 3, m // 2, m - 2, m - 1})
    ref = oracle.qmatmul(Q8_0, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
    assert_rows_close(y[rows], ref, tight_bound(Q4_K, m))


@pytest.mark.parametrize("m", [16, 64, 512])
def test_q8_0_mfma_config0_shape(oracle, lbq, dev, m):
    # configs[0]'s Q8_0 4096 x 4096 weight (N(0, 0.02), quantised on the device)
    from test_gpu_configs import quantised
    qm, raw = quantised(Q8_0, 4096, 4096, dev, 0x1B0)
    rng = np.random.default_rng(410 + m)
    x = rng.standard_normal((m, 4096)).astype(np.float32)
    y = qm.forward(to_dev(x, dev)).cpu().numpy()
    rows = sorted({0, 5, m // 2, m - 1})
    ref = oracle.qmatmul(Q8_0, raw, 4096, 4096, x[rows], nthreads=oracle.nproc()).astype(np.float64)
    assert_rows_close(y[rows], ref, tight_bound(Q4_K, m))


def test_q8_0_mfma_operands_from_codes(oracle, lbq, dev):
    # forward (operands quantised from f32 x in the pre-pass) and forward_quantized
    # (operands from Q8_0 codes quantised by the standalone kernel) give the same bits
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    rng = np.random.default_rng(420)
    n, k = 333, 256 * 6
    qm = QMatMul.from_qtensor(QTensor(to_dev(bp.random_blocks(rng, Q8_0, n * k // 32), dev), Q8_0, (n, k)))
    for m in (12, 40, 200, 300):
        xd = to_dev(rng.standard_normal((m, k)).astype(np.float32), dev)
        y1 = qm.forward(xd)
        y2 = qm.forward_quantized(QActivation.for_weight(qm, m).quantize(xd))
        torch.cuda.synchronize()
        assert np.array_equal(y1.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32)), m


def test_q8_0_batched_k_not_multiple_of_256(oracle, lbq, dev):
    # k % 256 != 0: the Q8_0 batched call stays on the integer GEMV (row chunks)
    rng = np.random.default_rng(430)
    n, k = 129, 32 * 37
    w_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-2)
    x = rng.standard_normal((20, k)).astype(np.float32)
    assert_rows_close(gpu_qmatmul(Q8_0, w_raw, n, k, x, dev),
                      oracle.qmatmul(Q8_0, w_raw, n, k, x, nthreads=8).astype(np.float64), 1e-4)


def test_q8_0_grouped_batched(oracle, lbq, dev):
    # a grouped call at m > 8 shares one Q8_0 operand pre-pass between weights of different n
    from lightbulb_amd.quantized import QMatMul, QTensor, qmatmul_group
    rng = np.random.default_rng(440)
    k = 1024
    raws = [bp.random_blocks(rng, Q8_0, n * k // 32) for n in (256, 64, 64)]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), Q8_0, (r.size // 34 * 32 // k, k))) for r in raws]
    x = to_dev(rng.standard_normal((24, k)).astype(np.float32), dev)
    ys = qmatmul_group(qms, x)
    for y, qm in zip(ys, qms):
        assert np.array_equal(y.cpu().numpy().view(np.uint32), qm.forward(x).cpu().numpy().view(np.uint32))


# ---------------------------------------------------------------- dense F32 / F16
def _dense(t, n, k, rng, dev):
    from lightbulb_amd.quantized import QMatMul, QTensor
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float16 if t == F16 else np.float32)
    if t == BF16:
        b = _bf16_bits(w)
        qm = QMatMul.from_qtensor(QTensor(to_dev(b.view(np.uint8).reshape(-1), dev), t, (n, k)))
        return qm, _bf16_to_f32(b).astype(np.float64)
    qm = QMatMul.from_qtensor(QTensor(to_dev(w.view(np.uint8).reshape(-1), dev), t, (n, k)))
    return qm, w.astype(np.float64)


def _assert_dense(y, ref):
    assert_rows_close(y, ref, 1e-5)


@pytest.mark.parametrize("t", [F32, F16, BF16])
@pytest.mark.parametrize("m", [1, 3, 8, 9, 40, 130])
def test_dense_forward(lbq, dev, t, m):
    rng = np.random.default_rng(450 + m + t)
    # k = 14336 / 16392: x staged in LDS at m = 1 (57 KB) and not (64 KB + 32 B), the
    # latter also a row of five 4096-column units with a partial last one
    for n, k in ((1, 8), (77, 520), (300, 4096), (129, 1000), (64, 14336), (40, 16392)):
        qm, w = _dense(t, n, k, rng, dev)
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = qm.forward(to_dev(x, dev)).cpu().numpy()
        _assert_dense(y, x.astype(np.float64) @ w.T)


def test_dense_unaligned_x_and_entry_points(lbq, dev):
    # x views only 4-byte aligned; grouped / gate-up / norm-fused entry points on dense weights
    from lightbulb_amd.quantized import gate_up_silu, qmatmul_group, rmsnorm_gate_up_silu
    rng = np.random.default_rng(460)
    k = 512
    (qa, wa), (qb, wb) = _dense(F16, 96, k, rng, dev), _dense(F16, 96, k, rng, dev)
    for m in (1, 5, 20):
        base = to_dev(rng.standard_normal(m * k + 1).astype(np.float32), dev)
        x = base[1:].reshape(m, k)
        xh = x.cpu().numpy().astype(np.float64)
        _assert_dense(qa.forward(x).cpu().numpy(), xh @ wa.T)
        ya, yb = qmatmul_group([qa, qb], x)
        _assert_dense(ya.cpu().numpy(), xh @ wa.T)
        _assert_dense(yb.cpu().numpy(), xh @ wb.T)
        g, u = xh @ wa.T, xh @ wb.T
        _assert_dense(gate_up_silu(qa, qb, x).cpu().numpy(), g / (1.0 + np.exp(-g)) * u)
        nw = to_dev((1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32), dev)
        xn = x.cpu().numpy()
        rms = np.sqrt((xn.astype(np.float32) ** 2).sum(-1, keepdims=True) / k + 1e-5)
        xn = (xn / rms * nw.cpu().numpy()).astype(np.float64)
        g, u = xn @ wa.T, xn @ wb.T
        assert_rows_close(rmsnorm_gate_up_silu(qa, qb, x, nw, 1e-5).cpu().numpy(), g / (1.0 + np.exp(-g)) * u, 1e-4)


def test_dense_gguf_output_weight(lbq, dev, tmp_path):
    # a GGUF holding F16, F32 and BF16 output.weight tensors (and F16 / BF16
    # embedding tables): loaded both ways and forwarded as the reference's dense
    # QMatMul; extract_tensor_bytes' mirror refuses BF16 as the reference does
    import gguf_writer as gw
    from lightbulb_amd import _lib
    from lightbulb_amd.gguf import Content
    from lightbulb_amd.quantized import QEmbedding, QMatMul, context
    rng = np.random.default_rng(470)
    n, k = 1000, 256
    w16 = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    w32 = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    b16 = _bf16_bits(rng.standard_normal((n, k)) * 0.05)
    wbf = _bf16_to_f32(b16)
    blob, _, _ = gw.build([("general.architecture", gw.STR, "llama")],
                          [("output.weight", [k, n], F16, w16.tobytes()), ("output32.weight", [k, n], F32, w32.tobytes()),
                           ("token_embd.weight", [k, n], F16, w16.tobytes()), ("outputbf.weight", [k, n], BF16, b16.tobytes()),
                           ("token_embd_bf.weight", [k, n], BF16, b16.tobytes())])
    path = tmp_path / "dense.gguf"
    path.write_bytes(blob)
    L = _lib.lib()
    x = rng.standard_normal((4, k)).astype(np.float32)
    with Content.read(path) as c:
        for name, w in (("output.weight", w16), ("output32.weight", w32), ("outputbf.weight", wbf)):
            qm = QMatMul.from_qtensor(c.tensor(name, dev))
            y = qm.forward(to_dev(x, dev)).cpu().numpy()
            _assert_dense(y, x.astype(np.float64) @ w.astype(np.float64).T)
            h = ctypes.c_void_p()
            ctx = context(dev)
            _lib.check(L.lbq_weight_from_gguf(ctx, c._h, name.encode(), ctypes.byref(h)))
            y2 = torch.empty(4, n, device=dev)
            _lib.check(L.lbq_qmatmul_f32(ctx, h.value, to_dev(x, dev).data_ptr(), 4, y2.data_ptr(), None))
            torch.cuda.synchronize()
            assert np.array_equal(y.view(np.uint32), y2.cpu().numpy().view(np.uint32))
            L.lbq_weight_destroy(h.value)
        emb = QEmbedding(c.tensor("token_embd.weight", dev))
        ids = np.array([0, 999, 5, 5], dtype=np.int64)
        got = emb.forward(torch.from_numpy(ids).to(dev)).cpu().numpy()
        assert np.array_equal(got, w16.astype(np.float32)[ids])
        emb = QEmbedding(c.tensor("token_embd_bf.weight", dev))
        got = emb.forward(torch.from_numpy(ids).to(dev)).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), wbf[ids].view(np.uint32))
        # extract_tensor_bytes (lbq_gguf_tensor_bytes) keeps the reference's table: no BF16
        p, nb = ctypes.c_void_p(), ctypes.c_uint64()
        assert L.lbq_gguf_tensor_bytes(c._h, b"outputbf.weight", ctypes.byref(p), ctypes.byref(nb)) == -2
        assert b"Unknown quantization type: 30" in L.lbq_last_error()


def test_bf16_dequantize_bit_exact(lbq, dev):
    # QTensor::dequantize of a BF16 tensor: the exact widening, every bit pattern class
    from lightbulb_amd.quantized import GgmlDType, dequantize_tensor
    rng = np.random.default_rng(475)
    b = rng.integers(0, 1 << 16, size=4096, dtype=np.uint32).astype(np.uint16)
    b[:6] = [0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC1, 0x0001]  # +-0, +-inf, a NaN, a subnormal
    got = dequantize_tensor(to_dev(b.view(np.uint8), dev), GgmlDType.BF16, 4095).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), _bf16_to_f32(b)[:4095].view(np.uint32))


def test_dense_errors(lbq, dev):
    from lightbulb_amd.quantized import QActivation, context
    ctx = context(dev)
    h = ctypes.c_void_p()
    buf = torch.zeros(4096, dtype=torch.uint8, device=dev)
    assert lbq.lbq_weight_wrap_device(ctx, F16, 4, 12, buf.data_ptr(), 96, ctypes.byref(h)) == -3  # k % 8
    assert lbq.lbq_weight_wrap_device(ctx, F16, 4, 16, buf.data_ptr(), 100, ctypes.byref(h)) == -3  # bytes
    assert lbq.lbq_weight_wrap_device(ctx, 4, 4, 16, buf.data_ptr(), 128, ctypes.byref(h)) == -2   # no such type
    assert lbq.lbq_weight_wrap_device(ctx, F16, 4, 16, buf.data_ptr(), 128, ctypes.byref(h)) == 0
    act = QActivation(Q8_0, 1, 32, dev)
    y = torch.empty(1, 4, device=dev)
    assert lbq.lbq_qmatmul_act_f32(ctx, h, act._handle, y.data_ptr(), None) == -2
    assert b"dense" in lbq.lbq_last_error()
    assert lbq.lbq_weight_destroy(h) == 0


# ---------------------------------------------------------------- plan overrides
def forward_with_env(monkeypatch, env, t, w_raw, n, k, x, dev):
    """QMatMul::forward through a context created with the given plan overrides."""
    from lightbulb_amd import _lib
    L = _lib.lib()
    for key, val in env.items():
        monkeypatch.setenv(key, val)
    ctx = ctypes.c_void_p()
    try:
        _lib.check(L.lbq_init(dev.index or 0, ctypes.byref(ctx)))
    finally:
        for key in env:
            monkeypatch.delenv(key)
    try:
        wd = to_dev(w_raw, dev)
        h = ctypes.c_void_p()
        _lib.check(L.lbq_weight_wrap_device(ctx, t, n, k, wd.data_ptr(), wd.numel(), ctypes.byref(h)))
        xd = to_dev(x.astype(np.float32), dev)
        y = torch.empty(x.shape[0], n, device=dev)
        st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(L.lbq_qmatmul_f32(ctx, h, xd.data_ptr(), x.shape[0], y.data_ptr(), st))
        torch.cuda.synchronize()
        L.lbq_weight_destroy(h)
        return y.cpu().numpy()
    finally:
        L.lbq_ctx_destroy(ctx)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_gemm_routing_overrides(oracle, lbq, dev, t, monkeypatch):
    # the kernels a shape reaches only through the plan overrides stay correct:
    # 32-row tiles at m <= 32, k-sliced two-row tiles for Q4_K / Q5_K, every
    # k-slice length, wide tiles where tall ones are chosen and the reverse,
    # explicit split counts, no tall tiles
    rng = np.random.default_rng(97 + t)
    n, k = 300, 256 * 6
    w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3)
    cases = [({"LBQ_GEMM_NO_KS": "1"}, 20), ({"LBQ_GEMM_KS64": "1"}, 50), ({"LBQ_GEMM_KS": "1"}, 24),
             ({"LBQ_GEMM_KS": "2"}, 32), ({"LBQ_GEMM_KS": "3"}, 32), ({"LBQ_GEMM_KS": "4"}, 17),
             ({"LBQ_GEMM_BIG": "tall"}, 300), ({"LBQ_GEMM_BIG": "wide"}, 600), ({"LBQ_GEMM_SPLITS": "3"}, 70),
             ({"LBQ_GEMM_NO_TALL": "1"}, 260)]
    for env, m in cases:
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = forward_with_env(monkeypatch, env, t, w_raw, n, k, x, dev)
        rows = np.r_[0:2, m // 2, m - 2:m]
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert_rows_close(y[rows], ref, tight_bound(Q4_K, m))


@pytest.mark.parametrize("t", [Q5_K, Q6_K])
def test_ksliced_long_slices_large_n(oracle, lbq, dev, t):
    # slices of 3 and 4 blocks chosen by the plan itself (many 128-column tiles):
    # k = 14336 and 4096 at m = 32 with n large enough that the grid fills the chip
    rng = np.random.default_rng(480 + t)
    for n, k in ((4096, 4096), (2048, 14336)):
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
        x = rng.standard_normal((32, k)).astype(np.float32)
        y = gpu_qmatmul(t, w_raw, n, k, x, dev)
        rows = [0, 13, 31]
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert_rows_close(y[rows], ref, tight_bound(t, 32))


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0])
def test_ksliced_slice_sum_in_kernel(oracle, lbq, dev, t, monkeypatch):
    # k-sliced shapes with at least 64 column tiles add their slices in the kernel
    # (the last workgroup of a tile, found through a per-tile counter); the bits
    # equal those of the separate slice-sum launch, call after call (the counters
    # are left zero), with a ragged last tile, and through the grouped entry point
    from lightbulb_amd.quantized import QMatMul, QTensor, qmatmul_group
    rng = np.random.default_rng(620 + t)
    for (m, n, k) in ((16, 8192, 4096), (32, 8196, 2048), (13, 8192, 256 * 6)):
        w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3)
        x = rng.standard_normal((m, k)).astype(np.float32)
        y_sep = forward_with_env(monkeypatch, {"LBQ_GEMM_SPLIT_LAUNCH": "1"}, t, w_raw, n, k, x, dev)
        qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
        xd = to_dev(x, dev)
        for _ in range(3):
            y = qm.forward(xd).cpu().numpy()
            assert np.array_equal(y.view(np.uint32), y_sep.view(np.uint32)), (m, n, k)
        ys = qmatmul_group([qm, qm], xd)
        for yg in ys:
            assert np.array_equal(yg.cpu().numpy().view(np.uint32), y_sep.view(np.uint32)), (m, n, k)
        rows = [0, m // 2, m - 1]
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert_rows_close(y[rows], ref, tight_bound(t, m))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
def test_ksliced_quantise_in_kernel(oracle, lbq, dev, t, monkeypatch):
    # k-sliced launches of at most 32 column tiles quantise f32 x themselves (no
    # pre-pass launch): every slice shape (1, 2, 4 blocks; 16 and 32 quantised
    # rows; two row tiles), ragged m and n, a short last slice; checked against
    # the oracle and against the pre-pass operands (the same Q8_K values; the
    # operand exponent is per slice instead of per group of four blocks, which
    # moves no bit unless an operand is an f16 subnormal)
    from lightbulb_amd.quantized import QMatMul, QTensor, qmatmul_group
    rng = np.random.default_rng(640 + t)
    cases = [(16, 4096, 4096, {}), (13, 1000, 256 * 6, {}), (32, 1024, 4096, {}), (9, 300, 256 * 5, {}),
             (12, 4096, 256 * 34, {}),  # 4-block slices, a short last one
             (16, 4096, 4096, {"LBQ_GEMM_KS": "1"}), (20, 700, 256 * 7, {"LBQ_GEMM_KS": "2"})]
    if t != Q4_K:
        cases.append((48, 500, 4096, {"LBQ_GEMM_KS": "1"}))  # two row tiles, 64 quantised rows
    for (m, n, k, env) in cases:
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = forward_with_env(monkeypatch, env, t, w_raw, n, k, x, dev)
        y_pre = forward_with_env(monkeypatch, {**env, "LBQ_GEMM_PREPASS": "1"}, t, w_raw, n, k, x, dev)
        np.testing.assert_allclose(y, y_pre, rtol=1e-6, atol=1e-6 * float(np.abs(y_pre).max()))
        rows = sorted({0, m // 2, m - 1})
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert_rows_close(y[rows], ref, tight_bound(t, m))
    # a group whose weights take both paths (4096 rows in the kernel, 14336 after
    # the pre-pass) equals separate calls bit for bit
    k, m = 4096, 16
    raws = [bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3) for n in (4096, 14336)]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, (4096, 14336))]
    xd = to_dev(rng.standard_normal((m, k)).astype(np.float32), dev)
    ys = qmatmul_group(qms, xd)
    for q, yg in zip(qms, ys):
        assert np.array_equal(yg.cpu().numpy().view(np.uint32), q.forward(xd).cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("t", [Q4_K, Q6_K])
def test_unaligned_output_on_every_small_m_path(oracle, lbq, dev, t):
    # y only 4-byte aligned (the ABI's requirement) on the k-sliced paths that write
    # y from the kernel: slices added in the kernel (14336 columns), quantisation in
    # the kernel (4096), the separate slice sum, and the multi-row decode (m = 3)
    rng = np.random.default_rng(680 + t)
    from lightbulb_amd import _lib
    L = _lib.lib()
    for (m, n, k) in ((16, 14336, 4096), (16, 4096, 4096), (32, 1024, 4096), (3, 4096, 4096)):
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
        x = rng.standard_normal((m, k)).astype(np.float32)
        y_ref = gpu_qmatmul(t, w_raw, n, k, x, dev)
        ctx = ctypes.c_void_p()
        _lib.check(L.lbq_init(dev.index or 0, ctypes.byref(ctx)))
        try:
            wd = to_dev(w_raw, dev)
            h = ctypes.c_void_p()
            _lib.check(L.lbq_weight_wrap_device(ctx, t, n, k, wd.data_ptr(), wd.numel(), ctypes.byref(h)))
            xd = to_dev(x, dev)
            base = torch.full((m * n + 1,), float("nan"), device=dev)
            st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
            _lib.check(L.lbq_qmatmul_f32(ctx, h, xd.data_ptr(), m, base.data_ptr() + 4, st))
            torch.cuda.synchronize()
            L.lbq_weight_destroy(h)
            y = base[1:].reshape(m, n).cpu().numpy()
            assert np.isnan(base[0].item())
            assert np.array_equal(y.view(np.uint32), y_ref.view(np.uint32)), (m, n, k)
        finally:
            L.lbq_ctx_destroy(ctx)


def test_tuning_read_once_per_context(oracle, lbq, dev, monkeypatch):
    # an override set after a context exists does not change that context's plan
    from lightbulb_amd.quantized import QMatMul, QTensor
    rng = np.random.default_rng(490)
    n, k = 300, 1024
    w_raw = bp.random_blocks(rng, Q4_K, n * k // 256, d_scale=1e-3)
    qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), Q4_K, (n, k)))
    x = to_dev(rng.standard_normal((20, k)).astype(np.float32), dev)
    y0 = qm.forward(x).cpu().numpy()
    monkeypatch.setenv("LBQ_GEMM_NO_KS", "1")  # would change the summation order
    y1 = qm.forward(x).cpu().numpy()
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
@pytest.mark.parametrize("k", [1024, 2048])
def test_eight_wave_workgroups_6144_rows(oracle, lbq, dev, t, k):
    # m = 1 over 6144 rows at k <= 8192 takes eight-wave workgroups: a single
    # weight, a q|k|v group and the norm-fused group
    from lightbulb_amd.quantized import QMatMul, QTensor, qmatmul_group, rmsnorm_qmatmul_group
    rng = np.random.default_rng(500 + t + k)
    raws = [bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3) for n in (6144, 4096, 1024, 1024)]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (r.size // (144 if t == Q4_K else 176) * 256 // k, k)))
           for r in raws]
    x = rng.standard_normal((1, k)).astype(np.float32)
    xd = to_dev(x, dev)
    y = qms[0].forward(xd).cpu().numpy()
    assert_rows_close(y, oracle.qmatmul(t, raws[0], 6144, k, x, nthreads=8).astype(np.float64))
    ys = qmatmul_group(qms[1:], xd)
    for yy, r, n in zip(ys, raws[1:], (4096, 1024, 1024)):
        assert_rows_close(yy.cpu().numpy(), oracle.qmatmul(t, r, n, k, x, nthreads=8).astype(np.float64))
    w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    rms = np.sqrt((x.astype(np.float32) ** 2).sum(-1, keepdims=True, dtype=np.float32) / np.float32(k) + np.float32(1e-5))
    xn = (x / rms.astype(np.float32) * w).astype(np.float32)
    ys = rmsnorm_qmatmul_group(qms[1:], xd, to_dev(w, dev), 1e-5)
    for yy, r, n in zip(ys, raws[1:], (4096, 1024, 1024)):
        assert_rows_close(yy.cpu().numpy(), oracle.qmatmul(t, r, n, k, xn, nthreads=8).astype(np.float64), 2e-3)


@pytest.mark.parametrize("t,m,n,k", [(Q4_K, 512, 14336, 1024), (Q4_K, 256, 14336, 2048), (Q5_K, 200, 7168, 1024),
                                     (Q6_K, 130, 448, 2048), (Q8_0, 160, 672, 512)])
def test_wide_tiles_seven_waves(oracle, lbq, dev, t, m, n, k, monkeypatch):
    # where n is a multiple of 224 and seven-wave (128 x 224) wide tiles take fewer
    # rounds of the chip, the wide kernel runs with seven waves: the same columns
    # in the same k order per wave, so the bits of the eight-wave tiles
    # (LBQ_GEMM_WIDE7=0), and forced seven-wave tiles (=1) on shapes the plan
    # leaves at eight; rows against the oracle
    rng = np.random.default_rng(1400 + t + m + n)
    w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3)
    x = rng.standard_normal((m, k)).astype(np.float32)
    print(f"wide7 t={t} m={m} n={n} k={k}", flush=True)
    y = forward_with_env(monkeypatch, {}, t, w_raw, n, k, x, dev)
    y8 = forward_with_env(monkeypatch, {"LBQ_GEMM_WIDE7": "0"}, t, w_raw, n, k, x, dev)
    y7 = forward_with_env(monkeypatch, {"LBQ_GEMM_WIDE7": "1"}, t, w_raw, n, k, x, dev)
    assert np.array_equal(y.view(np.uint32), y8.view(np.uint32))
    assert np.array_equal(y7.view(np.uint32), y8.view(np.uint32))
    rows = np.r_[0:2, m // 2, m - 2:m]
    ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
    assert_rows_close(y[rows], ref, tight_bound(Q4_K, m))
