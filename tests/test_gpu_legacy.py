"""GPU parity for the remaining GGUF block types -- the 32-value legacy weights
(Q4_0, Q4_1, Q5_0, Q5_1) with their Q8_0 / Q8_1 activations, and Q2_K / Q3_K
with Q8_K activations -- through the C ABI, against the CPU oracle.

Bars as for the other types: dequantisation, activation and weight
quantisation bit-exact; QMatMul::forward per-row relative L2 <= 2e-3 and max
abs <= 1e-2 * ||row||_inf.  At m <= 8 (and at any m when k % 256 != 0) these
types run the integer-dot GEMV, whose error is f32 summation order only (1e-4
guard); above m = 8 at k % 256 == 0 they run the MFMA GEMM on fp16 operands
(1.5e-3 guard), every kernel of its plan (k-sliced, 32/64/128-row, wide and
tall tiles) checked on spread rows.
"""
import numpy as np
import pytest
import torch

import blockpack as bp

from test_gpu_parity import _special_rows, assert_rows_close, gpu_qmatmul, gpu_quant_weights, tight_bound, to_dev

pytestmark = pytest.mark.gpu

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1, Q2_K, Q3_K = 2, 3, 6, 7, 8, 9, 10, 11
LEGACY = [Q4_0, Q4_1, Q5_0, Q5_1]


@pytest.mark.parametrize("t", LEGACY)
def test_legacy_dequant_bit_exact(oracle, lbq, dev, t):
    from lightbulb_amd.quantized import dequantize_tensor
    rng = np.random.default_rng(300 + t)
    nb = 1001  # odd: 18- and 22-byte blocks alternate between 4-aligned and 2 mod 4
    raw = bp.random_blocks(rng, t, nb, d_scale=0.5)
    got = dequantize_tensor(to_dev(raw, dev), t, nb * 32).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.dequantize(t, raw).view(np.uint32))


def test_q8_1_quantize_and_dequant_bit_exact(oracle, lbq, dev):
    from lightbulb_amd.quantized import dequantize_tensor, quantize_activations
    rng = np.random.default_rng(310)
    k = 4096
    x = rng.standard_normal((9, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    x = np.concatenate([x, _special_rows(k)])
    got = quantize_activations(to_dev(x, dev), Q8_1).cpu().numpy()
    ref = oracle.quantize_act(Q8_1, x)
    assert np.array_equal(got, ref)
    deq = dequantize_tensor(to_dev(ref.reshape(-1), dev), Q8_1, x.size).cpu().numpy()
    assert np.array_equal(deq, oracle.dequantize(Q8_1, ref.reshape(-1)))


@pytest.mark.parametrize("t", LEGACY)
def test_legacy_quantize_weights_bit_exact(oracle, lbq, dev, t):
    rng = np.random.default_rng(320 + t)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0             # all-zero block
    w[1, :32] = 1e-3            # constant block
    w[2, :32] = -w[2, :32]
    w[3, 5], w[3, 9] = 0.5, -0.5  # tie in |x|: the first one sets the sign of d
    got = gpu_quant_weights(t, w, dev)
    assert np.array_equal(got, oracle.quantize_weights(t, w))


SHAPES = [(48, 32), (100, 256), (257, 32 * 37), (1024, 1024)]


@pytest.mark.parametrize("t", LEGACY)
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9, 17])
def test_legacy_qmatmul(oracle, lbq, dev, t, m):
    rng = np.random.default_rng(1000 * t + m + 7)
    for n, k in SHAPES:
        w_raw = bp.random_blocks(rng, t, n * k // 32, d_scale=1e-2)
        x = rng.standard_normal((m, k)).astype(np.float32)
        ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
        assert_rows_close(gpu_qmatmul(t, w_raw, n, k, x, dev), ref, tight_bound(t, m))


@pytest.mark.parametrize("t", LEGACY)
def test_legacy_llama_rows_and_quantised_weights(oracle, lbq, dev, t):
    # k = 4096 / 14336 with weights from the quantiser (real code statistics),
    # x with outliers; the pre-quantised activation handle gives the same bits
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor, vec_dot_type
    rng = np.random.default_rng(340 + t)
    for n, k in ((300, 4096), (77, 14336)):
        w_raw = oracle.quantize_weights(t, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
        for m in (1, 4, 12):
            x = rng.standard_normal((m, k)).astype(np.float32)
            x[rng.random(x.shape) < 0.01] *= 20
            xd = to_dev(x, dev)
            y = qm.forward(xd)
            act = QActivation.for_weight(qm, m)
            assert act.act_type == vec_dot_type(t)
            y2 = qm.forward_quantized(act.quantize(xd))
            torch.cuda.synchronize()
            ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
            assert_rows_close(y.cpu().numpy(), ref, tight_bound(t, m))
            assert np.array_equal(y.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("t", [Q4_0, Q5_1])
def test_legacy_call_site_entry_points(oracle, lbq, dev, t):
    # grouped projections and the gate/up product take the shared-quantisation
    # path for these types; outputs equal the single calls bit for bit
    from lightbulb_amd.quantized import QMatMul, QTensor, gate_up_silu, qmatmul_group
    rng = np.random.default_rng(350 + t)
    k, ns = 1024, (300, 64, 64)
    raws = [bp.random_blocks(rng, t, n * k // 32, d_scale=1e-2) for n in ns]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, ns)]
    for m in (1, 3, 20):
        x = rng.standard_normal((m, k)).astype(np.float32)
        xd = to_dev(x, dev)
        ys = qmatmul_group(qms, xd)
        singles = [q.forward(xd) for q in qms]
        g = gate_up_silu(qms[1], qms[2], xd)
        torch.cuda.synchronize()
        for y, y1 in zip(ys, singles):
            assert np.array_equal(y.cpu().numpy().view(np.uint32), y1.cpu().numpy().view(np.uint32))
        gr = oracle.qmatmul(t, raws[1], 64, k, x, nthreads=4).astype(np.float64)
        ur = oracle.qmatmul(t, raws[2], 64, k, x, nthreads=4).astype(np.float64)
        assert_rows_close(g.cpu().numpy(), gr / (1.0 + np.exp(-gr)) * ur, tight_bound(t, m))


def test_legacy_activation_type_mismatch(oracle, lbq, dev):
    from lightbulb_amd import _lib
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    rng = np.random.default_rng(360)
    qm = QMatMul.from_qtensor(QTensor(to_dev(bp.random_blocks(rng, Q4_1, 8 * 2), dev), Q4_1, (8, 64)))
    act = QActivation(Q8_0, 1, 64, dev).quantize(to_dev(rng.standard_normal((1, 64)).astype(np.float32), dev))
    with pytest.raises(_lib.LbqError, match="needs activation type 9"):
        qm.forward_quantized(act)


# ---------------------------------------------------------------- Q2_K / Q3_K
@pytest.mark.parametrize("t", [Q2_K, Q3_K])
def test_k23_dequant_bit_exact(oracle, lbq, dev, t):
    from lightbulb_amd.quantized import dequantize_tensor
    rng = np.random.default_rng(370 + t)
    nb = 333  # odd: 110-byte Q3_K blocks alternate between 4-aligned and 2 mod 4
    raw = bp.random_blocks(rng, t, nb, d_scale=0.5)
    got = dequantize_tensor(to_dev(raw, dev), t, nb * 256).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), oracle.dequantize(t, raw).view(np.uint32))


K23_SHAPES = [(48, 256), (100, 512), (257, 256 * 5), (1024, 1024)]


@pytest.mark.parametrize("t", [Q2_K, Q3_K])
@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9, 17])
def test_k23_qmatmul(oracle, lbq, dev, t, m):
    rng = np.random.default_rng(1000 * t + m + 9)
    for n, k in K23_SHAPES:
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-2)
        x = rng.standard_normal((m, k)).astype(np.float32)
        ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
        assert_rows_close(gpu_qmatmul(t, w_raw, n, k, x, dev), ref, tight_bound(t, m))


@pytest.mark.parametrize("t", [Q2_K, Q3_K])
def test_k23_llama_rows(oracle, lbq, dev, t):
    # Llama-3 row lengths, x with outliers, ragged n; the activation handle gives
    # the same bits as forward()
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    rng = np.random.default_rng(380 + t)
    for n, k in ((300, 4096), (77, 14336)):
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
        qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
        for m in (1, 4, 12):
            x = rng.standard_normal((m, k)).astype(np.float32)
            x[rng.random(x.shape) < 0.01] *= 20
            xd = to_dev(x, dev)
            y = qm.forward(xd)
            y2 = qm.forward_quantized(QActivation.for_weight(qm, m).quantize(xd))
            torch.cuda.synchronize()
            assert_rows_close(y.cpu().numpy(), oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64),
                              tight_bound(t, m))
            assert np.array_equal(y.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))


def test_k23_has_no_weight_quantiser(lbq, dev):
    from lightbulb_amd.quantized import quantize_tensor
    with pytest.raises(ValueError, match="Quantization for Q2K not yet implemented"):
        quantize_tensor(torch.zeros(256, device=dev), Q2_K)


# ---------------------------------------------------------------- MFMA plans
def _rows_of(w_raw, t, n, k, rows, oracle):
    """The weight rows `rows` as their own (len(rows) x k) tensor of blocks."""
    per = k // oracle.block_size(t) * BLOCK_BYTES[t]
    return w_raw.reshape(n, per)[rows].reshape(-1)


BLOCK_BYTES = {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q2_K: 84, Q3_K: 110}


@pytest.mark.parametrize("t", LEGACY + [Q2_K, Q3_K])
def test_mfma_plans(oracle, lbq, dev, t):
    # every batched kernel: k-sliced (m <= 32, or 64 for the heavy types, with
    # 1..4-block slices), 32/64/128-row tiles (m up to 127), wide 128 x 256 tiles
    # and tall 256 x 128 tiles; split-k on few column tiles; ragged n and m
    from lightbulb_amd.quantized import QMatMul, QTensor
    rng = np.random.default_rng(400 + t)
    bs = oracle.block_size(t)
    for n, k in ((1000, 4096), (131, 1024)):
        w_raw = bp.random_blocks(rng, t, n * k // bs, d_scale=1e-2)
        qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
        cols = np.unique(np.r_[0, 1, n // 3, n // 2 + 1, n - 2, n - 1, rng.integers(0, n, 10)])
        w_sub = _rows_of(w_raw, t, n, k, cols, oracle)
        for m in (9, 16, 33, 48, 64, 100, 128, 255, 300, 512):
            x = rng.standard_normal((m, k)).astype(np.float32)
            x[rng.random(x.shape) < 0.01] *= 20
            y = qm.forward(to_dev(x, dev))
            torch.cuda.synchronize()
            rows = sorted({r for r in (0, 1, m // 2, m - 2, m - 1) if 0 <= r < m})
            ref = oracle.qmatmul(t, w_sub, len(cols), k, x[rows], nthreads=8).astype(np.float64)
            assert_rows_close(y.cpu().numpy()[rows][:, cols], ref, tight_bound(t, m))


@pytest.mark.parametrize("t", LEGACY + [Q2_K, Q3_K])
def test_mfma_quantised_activations_and_groups(oracle, lbq, dev, t):
    # forward_quantized (pre-quantised Q8_0 / Q8_1 / Q8_K handle) and the grouped
    # entry point at m > 8 give the bits of forward(); k = 14336 takes the
    # separate quantiser (no fused pre-pass above 64 blocks of 256)
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor, qmatmul_group
    rng = np.random.default_rng(420 + t)
    bs = oracle.block_size(t)
    for k in (4096, 18432):
        ns = (96, 40)
        raws = [bp.random_blocks(rng, t, n * k // bs, d_scale=1e-2) for n in ns]
        qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, ns)]
        for m in (12, 40, 130):
            x = rng.standard_normal((m, k)).astype(np.float32)
            xd = to_dev(x, dev)
            y = qms[0].forward(xd)
            y2 = qms[0].forward_quantized(QActivation.for_weight(qms[0], m).quantize(xd))
            ys = qmatmul_group(qms, xd)
            y1 = qms[1].forward(xd)
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
            assert np.array_equal(y.cpu().numpy().view(np.uint32), ys[0].cpu().numpy().view(np.uint32))
            assert np.array_equal(y1.cpu().numpy().view(np.uint32), ys[1].cpu().numpy().view(np.uint32))
            rows = [0, m // 2, m - 1]
            ref = oracle.qmatmul(t, raws[0], ns[0], k, x[rows], nthreads=8).astype(np.float64)
            assert_rows_close(y.cpu().numpy()[rows], ref, tight_bound(t, m))
