"""GPU parity: liblbq (through its C ABI) against the CPU oracle on the same inputs.

Bars:
* dequantisation, activation quantisation, weight quantisation: bit-exact;
* QMatMul::forward: per output row, relative L2 error <= 2e-3 and max abs error
  <= 1e-2 * ||row||_inf against the oracle's CPU QMatMul (the tolerance the
  path is specified with).  The GPU reproduces the reference's Q8_K / Q8_0
  activation quantisation.  The decode path (m <= 8) also forms the integer
  sub-block sums, so its error is f32 summation order only (~1e-6) and a 1e-4
  guard checks that; the MFMA path (m > 8: k-quants, and Q8_0 at k % 256 == 0)
  rounds each dequantised weight to fp16 once (~3e-4 on a row), guarded at 1.5e-3.
"""
import ctypes

import numpy as np
import pytest
import torch

import blockpack as bp

pytestmark = pytest.mark.gpu

Q8_0, Q4_K, Q5_K, Q6_K, Q8_K = 8, 12, 13, 14, 15
TOL_REL_L2 = 2e-3
TOL_MAX_ABS = 1e-2


def tight_bound(t: int, m: int) -> float:
    # decode (m <= 8): the reference's integer arithmetic; above, the MFMA path
    # (Q4_K/Q5_K/Q6_K, and Q8_0 when k % 256 == 0) rounds operands to fp16
    return 1e-4 if m <= 8 else 1.5e-3


def assert_rows_close(y: np.ndarray, ref: np.ndarray, tight: float = 1e-4):
    y = y.reshape(ref.shape)
    assert np.all(np.isfinite(y))
    for r in range(ref.shape[0]):
        diff = y[r].astype(np.float64) - ref[r]
        nrm = np.linalg.norm(ref[r])
        rel = np.linalg.norm(diff) / nrm if nrm > 0 else np.linalg.norm(diff)
        assert rel <= TOL_REL_L2, f"row {r}: rel L2 {rel:.3e}"
        assert np.abs(diff).max() <= TOL_MAX_ABS * np.abs(ref[r]).max() + 1e-30, f"row {r}: max abs"
        assert rel <= tight, f"row {r}: rel L2 {rel:.3e} above the expected summation-order level"


def to_dev(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def gpu_quant_weights(t: int, w: np.ndarray, dev) -> np.ndarray:
    from lightbulb_amd.quantized import quantize_tensor
    out = quantize_tensor(to_dev(w.astype(np.float32).reshape(-1), dev), t, _exact=True)
    return out.cpu().numpy()


def gpu_qmatmul(t: int, w_raw: np.ndarray, n: int, k: int, x: np.ndarray, dev) -> np.ndarray:
    from lightbulb_amd.quantized import QMatMul, QTensor
    qt = QTensor(to_dev(w_raw, dev), t, (n, k))
    y = QMatMul.from_qtensor(qt).forward(to_dev(x.astype(np.float32), dev))
    torch.cuda.synchronize()
    return y.cpu().numpy()


# ---------------------------------------------------------------- dequantisation
@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q5_K, Q6_K])
def test_dequant_bit_exact_random_blocks(oracle, lbq, dev, t):
    rng = np.random.default_rng(10 + t)
    nb = 1001
    raw = bp.random_blocks(rng, t, nb, d_scale=0.5)
    bs = oracle.block_size(t)
    ref = oracle.dequantize(t, raw)
    from lightbulb_amd.quantized import dequantize_tensor
    got = dequantize_tensor(to_dev(raw, dev), t, nb * bs).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_q8k_and_truncation(oracle, lbq, dev):
    rng = np.random.default_rng(20)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    q8k = oracle.quantize_act(Q8_K, x).reshape(-1)
    from lightbulb_amd.quantized import dequantize_tensor
    got = dequantize_tensor(to_dev(q8k, dev), Q8_K, 3 * 512).cpu().numpy()
    assert np.array_equal(got, oracle.dequantize(Q8_K, q8k))
    # reference semantics: blocks rounded up, output truncated to elem_count (mod.rs:165-187)
    raw = bp.random_blocks(rng, Q4_K, 2)
    got = dequantize_tensor(to_dev(raw, dev), Q4_K, 300).cpu().numpy()
    assert got.shape == (300,) and np.array_equal(got, oracle.dequantize(Q4_K, raw)[:300])
    with pytest.raises(ValueError, match="Insufficient data for Q4K: got 200 bytes, need 288 bytes"):
        dequantize_tensor(to_dev(raw[:200], dev), Q4_K, 512)


@pytest.mark.parametrize("t", [Q4_K, Q6_K, Q8_0, 2, 7, 11])
def test_embedding_rows_bit_exact(oracle, lbq, dev, t):
    # QEmbedding gathers dequantised rows without the dense table: equal to the
    # oracle's dequantised rows (repeats, first/last row, odd row starts), NaN
    # rows for ids outside [0, n)
    from lightbulb_amd.quantized import QEmbedding, QTensor
    rng = np.random.default_rng(160 + t)
    n, k = 333, 512 if t != 7 else 160
    raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=0.5)
    dense = oracle.dequantize(t, raw).reshape(n, k)
    emb = QEmbedding(QTensor(to_dev(raw, dev), t, (n, k)))
    ids = np.array([[0, 5, 5, 332], [17, 1, 200, 0]], dtype=np.int64)
    got = emb.forward(torch.from_numpy(ids).to(dev)).cpu().numpy()
    assert got.shape == (2, 4, k)
    assert np.array_equal(got.view(np.uint32), dense[ids].view(np.uint32))
    bad = emb.forward(torch.tensor([3, -1, 333, 4], device=dev)).cpu().numpy()
    assert np.isnan(bad[1]).all() and np.isnan(bad[2]).all()
    assert np.array_equal(bad[[0, 3]], dense[[3, 4]])
    assert emb.forward(torch.zeros(0, dtype=torch.int32, device=dev)).shape == (0, k)


def test_dense_f32_f16_dequantize(lbq, dev):
    # norm weights are stored as F32 (a copy) or F16 (an exact widening)
    from lightbulb_amd.quantized import dequantize_tensor
    rng = np.random.default_rng(170)
    h = rng.standard_normal(4099).astype(np.float16)
    h[:4] = [np.inf, -np.inf, 0.0, -0.0]
    got = dequantize_tensor(to_dev(h.view(np.uint8), dev), 1, h.size).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), h.astype(np.float32).view(np.uint32))
    f = rng.standard_normal(1001).astype(np.float32)
    got = dequantize_tensor(to_dev(f.view(np.uint8), dev), 0, f.size).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), f.view(np.uint32))


# ---------------------------------------------------------------- activation quantisation
def _special_rows(k: int) -> np.ndarray:
    rows = np.zeros((7, k), dtype=np.float32)
    rows[1, 17] = -3.0                       # single non-zero
    rows[2, 3], rows[2, 7] = -2.0, 2.0       # tie with opposite signs, saturation at +128
    rows[3, 0] = -128.0                      # iscale = 1: half-away-from-zero rounding
    rows[3, 1:6] = [2.5, -2.5, 3.5, 0.5, -0.5]
    rows[4, :] = np.linspace(-1, 1, k, dtype=np.float32)
    rows[5, :] = 1e-30                       # tiny magnitudes
    near_half = np.array([0.49999997, -0.49999997, 1.4999999, -1.4999999, 2.5000002, -2.4999998,
                          126.5, -127.5, 127.49999, -127.50001, 0.5000001, 63.5], dtype=np.float32)
    for b in range(0, k, 256):               # iscale = 1 in every block: rounding at and next to halves
        rows[6, b] = -128.0
        rows[6, b + 1:b + 1 + len(near_half)] = near_half
    return rows


def _tie_rows(k: int) -> np.ndarray:
    """Rows whose block maximum is decided by order, sign, NaN kind or size:
    |max| held by both signs (first occurrence wins, within one 16-value lane and
    across lanes), signalling NaNs (passed over like quiet ones), subnormal and
    largest finite maxima, signed zeros.  k >= 768."""
    f = np.float32
    snan, nsnan, snan2 = (np.array([v], np.uint32).view(np.float32)[0] for v in (0x7F800001, 0xFF800001, 0x7FA00000))
    rows = np.zeros((6, k), dtype=np.float32)
    rows[0, 17], rows[0, 40] = -5.0, 5.0            # across lanes: -5 first
    rows[0, 256 + 3], rows[0, 256 + 200] = 6.0, -6.0
    rows[0, 512 + 1], rows[0, 512 + 2] = 0.25, -0.25
    rows[1, 0], rows[1, 9] = 7.0, -7.0              # within one lane: +7 first
    rows[1, 256 + 20], rows[1, 256 + 30] = -7.0, 7.0
    rows[1, 256 + 33], rows[1, 256 + 34] = 3.0, -3.0  # a lane tie below the block maximum
    rows[1, 512 + 100:512 + 116] = np.where(np.arange(16) % 2 == 0, f(-2.5), f(2.5))
    rows[2, 5], rows[2, 100] = f(1e-40), f(-3e-41)  # subnormal maxima: iscale overflows
    rows[2, 256 + 44], rows[2, 256 + 45] = f(-2e-39), f(1e-45)
    rows[2, 512 + 7] = f(1.4e-45)
    rows[3, :] = np.random.default_rng(5).standard_normal(k).astype(np.float32)
    rows[3, 0], rows[3, 7] = snan, snan             # signalling NaNs among normal values
    rows[3, 256 + 5], rows[3, 256 + 6] = nsnan, np.nan
    rows[3, 512:768] = snan2                        # a block of signalling NaNs only
    rows[4, 0:256] = -0.0                           # signed zeros (and a NaN) only
    rows[4, 256:512:2] = -0.0
    rows[4, 300] = np.nan
    rows[4, 512 + 9] = -0.0
    rows[5, 3], rows[5, 600] = f(-3.4028235e38), f(3.4028235e38)
    rows[5, 4] = f(1e30)
    return rows


@pytest.mark.parametrize("act", [Q8_K, Q8_0])
def test_quantize_act_bit_exact(oracle, lbq, dev, act):
    rng = np.random.default_rng(30 + act)
    k = 4096
    x = rng.standard_normal((9, k)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20      # outliers, as in the LM-head config
    x = np.concatenate([x, _special_rows(k), _tie_rows(k)])
    from lightbulb_amd.quantized import quantize_activations
    got = quantize_activations(to_dev(x, dev), act).cpu().numpy()
    ref = oracle.quantize_act(act, x)
    assert np.array_equal(got, ref)


def test_quantize_act_unaligned_input(oracle, lbq, dev):
    # an f32 view that is only 4-byte aligned takes the scalar-load variant
    rng = np.random.default_rng(33)
    base = torch.from_numpy(rng.standard_normal(2 * 256 + 1).astype(np.float32)).to(dev)
    view = base[1:]
    from lightbulb_amd.quantized import quantize_activations
    got = quantize_activations(view.reshape(2, 256), Q8_K).cpu().numpy()
    assert np.array_equal(got, oracle.quantize_act(Q8_K, view.cpu().numpy().reshape(2, 256)))


# ---------------------------------------------------------------- weight quantisation
@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q5_K, Q6_K])
def test_quantize_weights_bit_exact(oracle, lbq, dev, t):
    rng = np.random.default_rng(40 + t)
    w = (rng.standard_normal((64, 1024)) * 0.02).astype(np.float32)
    w[0, :256] = 0.0            # all-zero block
    w[1, :256] = 1e-3           # constant block
    got = gpu_quant_weights(t, w, dev)
    ref = oracle.quantize_weights(t, w)
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------- QMatMul::forward
SMALL = [(48, 256), (100, 512), (257, 768), (1024, 1024)]


@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 6, 7, 8, 9, 17])
def test_qmatmul_small(oracle, lbq, dev, t, m):
    # m = 3, 5, 6, 7 run the 4- and 8-row decode kernels with unstored padding rows
    rng = np.random.default_rng(1000 * t + m)
    for n, k in SMALL:
        bs = oracle.block_size(t)
        w_raw = bp.random_blocks(rng, t, n * k // bs, d_scale=1e-3)
        x = rng.standard_normal((m, k)).astype(np.float32)
        ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
        assert_rows_close(gpu_qmatmul(t, w_raw, n, k, x, dev), ref, tight_bound(t, m))


def test_qmatmul_q8_0_odd_block_count(oracle, lbq, dev):
    rng = np.random.default_rng(51)
    n, k = 129, 32 * 37  # 37 blocks per row: rows start 2 bytes into a dword
    w_raw = bp.random_blocks(rng, Q8_0, n * k // 32, d_scale=1e-2)
    for m in (1, 4, 12):
        x = rng.standard_normal((m, k)).astype(np.float32)
        assert_rows_close(gpu_qmatmul(Q8_0, w_raw, n, k, x, dev),
                          oracle.qmatmul(Q8_0, w_raw, n, k, x, nthreads=8).astype(np.float64))


def test_qmatmul_odd_superblock_count(oracle, lbq, dev):
    rng = np.random.default_rng(52)
    for t in (Q4_K, Q5_K, Q6_K):
        n, k = 77, 256 * 5
        w_raw = bp.random_blocks(rng, t, n * k // 256)
        x = rng.standard_normal((3, k)).astype(np.float32)
        assert_rows_close(gpu_qmatmul(t, w_raw, n, k, x, dev),
                          oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64), tight_bound(t, 3))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
def test_qmatmul_mfma_ragged(oracle, lbq, dev, t):
    # m and n not multiples of the 128 x 128 tile; k with an odd block count
    rng = np.random.default_rng(60 + t)
    n, k = 200, 256 * 3
    w_raw = bp.random_blocks(rng, t, n * k // 256)
    for m in (9, 130, 300):
        x = rng.standard_normal((m, k)).astype(np.float32)
        assert_rows_close(gpu_qmatmul(t, w_raw, n, k, x, dev),
                          oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64), tight_bound(t, m))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("k", [4096, 14336])
def test_decode_row_partition(oracle, lbq, dev, t, k):
    # m = 1 at the Llama-3 row lengths: every row split across waves (1 .. 8 rows
    # per wave), ragged row counts, fused quantisation and pre-quantised x
    # (Q8_0 at k = 14336: 448 blocks, more block scales than threads)
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    rng = np.random.default_rng(70 + t + k)
    # 8400 / 16400 rows: eight-wave workgroups, at most 7 / 9 groups per wave (the
    # static schedule with clamped duplicates / the dynamic loop past 8)
    for n in (1, 3, 257, 1000, 5000, 8400) + ((16400,) if k == 4096 else ()):
        w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3)
        x = rng.standard_normal((1, k)).astype(np.float32)
        ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
        qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
        xd = to_dev(x, dev)
        y1 = qm.forward(xd)
        y2 = qm.forward_quantized(QActivation.for_weight(qm, 1).quantize(xd))
        torch.cuda.synchronize()
        assert_rows_close(y1.cpu().numpy(), ref)
        assert_rows_close(y2.cpu().numpy(), ref)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
@pytest.mark.parametrize("k", [4096, 14336])
def test_fused_quantisation_is_bit_exact(oracle, lbq, dev, t, k):
    # At m = 1 the GEMV quantises x in its own prologue (k = 14336: four passes
    # of 16 Q8_K blocks).  The same kernel fed x quantised by the standalone
    # (bit-exact) kernel runs the same integer arithmetic, so the two outputs
    # must agree to the bit.
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    # 300 rows: four-wave workgroups (16 lanes per Q8_K block); 8400 rows at
    # k = 4096: eight-wave workgroups quantising with 32 lanes per block
    rng = np.random.default_rng(90 + t)
    xs = np.concatenate([_special_rows(k), _tie_rows(k), rng.standard_normal((4, k)).astype(np.float32)])
    xs[-1, rng.random(k) < 0.01] *= 20
    for n in (300, 8400):
        w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3)
        qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
        for row in xs:
            xd = to_dev(row[None, :], dev)
            y_fused = qm.forward(xd)
            y_act = qm.forward_quantized(QActivation.for_weight(qm, 1).quantize(xd))
            torch.cuda.synchronize()
            assert np.array_equal(y_fused.cpu().numpy().view(np.uint32), y_act.cpu().numpy().view(np.uint32)), n


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
@pytest.mark.parametrize("k", [4096, 8192])
def test_multi_row_fused_quantisation_is_bit_exact(oracle, lbq, dev, t, k):
    # At m = 2..4 (k = 4096; m = 2 at k = 8192) forward() quantises the rows in the
    # multi-row GEMV's prologue; fed the standalone kernel's codes the same kernel
    # must give the same bits (2- and 4-row launches, a padded one, special and tie
    # rows); m = 5 and 8 take the standalone quantiser and must agree as well
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    rng = np.random.default_rng(150 + t + k)
    n = 300
    w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
    qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
    pool = np.concatenate([_special_rows(k), _tie_rows(k), rng.standard_normal((4, k)).astype(np.float32)])
    pool[-1, rng.random(k) < 0.01] *= 20
    for m in (2, 3, 5, 8):
        x = pool[rng.choice(len(pool), m, replace=False)]
        xd = to_dev(x, dev)
        y_fused = qm.forward(xd)
        y_act = qm.forward_quantized(QActivation.for_weight(qm, m).quantize(xd))
        torch.cuda.synchronize()
        assert np.array_equal(y_fused.cpu().numpy().view(np.uint32), y_act.cpu().numpy().view(np.uint32)), m
    rows = [0, m - 1]
    ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
    ok = np.isfinite(ref).all(axis=1)
    if ok.any():
        assert_rows_close(y_fused.cpu().numpy()[rows][ok], ref[ok])


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
def test_batched_prepass_quantisation_is_bit_exact(oracle, lbq, dev, t):
    # At m > 8 forward() quantises x inside the GEMM's operand pre-pass; fed the
    # standalone kernel's codes instead, the same GEMM must give the same bits
    # (both tile kernels, one and four quantisation passes, special rows)
    from lightbulb_amd.quantized import QActivation, QMatMul, QTensor
    rng = np.random.default_rng(130 + t)
    for m, n, k in ((20, 200, 4096), (300, 130, 4096), (40, 96, 14336)):
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
        qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), t, (n, k)))
        x = rng.standard_normal((m, k)).astype(np.float32)
        x[:7] = _special_rows(k)
        x[7:13] = _tie_rows(k)
        x[-1, rng.random(k) < 0.01] *= 20
        xd = to_dev(x, dev)
        y_fused = qm.forward(xd)
        y_act = qm.forward_quantized(QActivation.for_weight(qm, m).quantize(xd))
        torch.cuda.synchronize()
        assert np.array_equal(y_fused.cpu().numpy().view(np.uint32), y_act.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_qmatmul_group_matches_separate_calls(oracle, lbq, dev, t):
    # q|k|v- and gate|up-like groups in one call: every output bit-identical to
    # its own forward (m = 1 streams all weights in one launch; m > 1 shares the
    # quantised x), checked against the oracle too; x offset by one float takes
    # the unfused m = 1 path
    from lightbulb_amd.quantized import QMatMul, QTensor, qmatmul_group
    rng = np.random.default_rng(110 + t)
    for k, ns in ((4096, (512, 128, 128)), (1024, (300, 77)), (14336, (64, 33, 96, 5))):
        raws = [bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3) for n in ns]
        qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, ns)]
        for m in (1, 3, 20, 48):
            x = rng.standard_normal((m, k)).astype(np.float32)
            for shift in ((0, 1) if m == 1 else (0,)):
                buf = to_dev(np.concatenate([np.zeros(shift, np.float32), x.ravel()]), dev)
                xd = buf[shift:].view(m, k)
                ys = qmatmul_group(qms, xd)
                singles = [q.forward(xd) for q in qms]
                torch.cuda.synchronize()
                for y, y1 in zip(ys, singles):
                    assert np.array_equal(y.cpu().numpy().view(np.uint32), y1.cpu().numpy().view(np.uint32))
            if m == 1:
                for y, r, n in zip(ys, raws, ns):
                    assert_rows_close(y.cpu().numpy(), oracle.qmatmul(t, r, n, k, x, nthreads=8).astype(np.float64))
            if m == 48:  # the shared pre-pass's operand layout matches every member's GEMM
                for y, r, n in zip(ys, raws, ns):
                    assert_rows_close(y.cpu().numpy()[::7], oracle.qmatmul(t, r, n, k, x[::7], nthreads=8).astype(np.float64),
                                      tight_bound(t, m))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_gate_up_silu(oracle, lbq, dev, t):
    # silu(x.Wg^T) * (x.Wu^T): one launch at m = 1 (the product in the GEMV
    # epilogue), the grouped path plus an elementwise launch otherwise; against
    # the oracle's two products combined in float64, and through Mlp.forward
    from lightbulb_amd.quantized import Mlp, QMatMul, QTensor, QuantizableLinear, gate_up_silu
    rng = np.random.default_rng(140 + t)
    bs = oracle.block_size(t)
    for k, n in ((4096, 300), (14336, 77), (1024, 513)):
        g_raw = bp.random_blocks(rng, t, n * k // bs, d_scale=1e-3)
        u_raw = bp.random_blocks(rng, t, n * k // bs, d_scale=1e-3)
        qg = QMatMul.from_qtensor(QTensor(to_dev(g_raw, dev), t, (n, k)))
        qu = QMatMul.from_qtensor(QTensor(to_dev(u_raw, dev), t, (n, k)))
        for m in (1, 3, 20, 48):
            x = rng.standard_normal((m, k)).astype(np.float32)
            for shift in ((0, 1) if m == 1 else (0,)):
                buf = to_dev(np.concatenate([np.zeros(shift, np.float32), x.ravel()]), dev)
                y = gate_up_silu(qg, qu, buf[shift:].view(m, k))
                torch.cuda.synchronize()
                gr = oracle.qmatmul(t, g_raw, n, k, x, nthreads=8).astype(np.float64)
                ur = oracle.qmatmul(t, u_raw, n, k, x, nthreads=8).astype(np.float64)
                ref = gr / (1.0 + np.exp(-gr)) * ur
                assert_rows_close(y.cpu().numpy(), ref, tight_bound(t, m))
    # the MLP forward end to end (down_proj on the fused gate/up output)
    k, n = 512, 256
    raws = [bp.random_blocks(rng, t, n * k // bs, d_scale=1e-3) for _ in range(2)]
    d_raw = bp.random_blocks(rng, t, k * n // bs, d_scale=1e-3)
    lin = lambda raw, shape: QuantizableLinear.from_qmatmul(QMatMul.from_qtensor(QTensor(to_dev(raw, dev), t, shape)))
    mlp = Mlp(lin(raws[0], (n, k)), lin(raws[1], (n, k)), lin(d_raw, (k, n)))
    x = rng.standard_normal((2, 1, k)).astype(np.float32)
    y = mlp.forward(to_dev(x, dev))
    assert tuple(y.shape) == (2, 1, k)
    xf = x.reshape(2, k)
    gr = oracle.qmatmul(t, raws[0], n, k, xf, nthreads=4).astype(np.float64)
    ur = oracle.qmatmul(t, raws[1], n, k, xf, nthreads=4).astype(np.float64)
    h = (gr / (1.0 + np.exp(-gr)) * ur).astype(np.float32)
    ref = oracle.qmatmul(t, d_raw, k, n, h, nthreads=4).astype(np.float64)
    assert_rows_close(y.cpu().numpy().reshape(2, k), ref, 2e-3)


def test_gguf_to_qmatmul(oracle, lbq, dev, tmp_path):
    # GGUF file -> device through pinned staging, both ways (Content.tensor and
    # lbq_weight_from_gguf), then QMatMul::forward against the oracle on the
    # same bytes; the two loads give the same bits
    import gguf_writer as gw
    from lightbulb_amd import _lib
    from lightbulb_amd.gguf import Content
    from lightbulb_amd.quantized import QMatMul, context
    rng = np.random.default_rng(150)
    w = {t: (bp.random_blocks(rng, t, n * k // oracle.block_size(t)), n, k)
         for t, n, k in ((Q4_K, 300, 512), (Q6_K, 64, 1024), (Q8_0, 33, 256), (2, 41, 96), (7, 17, 160), (10, 23, 512), (11, 19, 512))}
    tensors = [("token_norm", [512], 0, rng.standard_normal(512).astype(np.float32).tobytes())]
    tensors += [(f"blk.0.w{t}", [k, n], t, raw.tobytes()) for t, (raw, n, k) in w.items()]
    blob, _, _ = gw.build([("general.architecture", gw.STR, "llama"), ("general.alignment", gw.U32, 64)], tensors,
                          alignment=64)
    path = tmp_path / "w.gguf"
    path.write_bytes(blob)
    L = _lib.lib()
    with Content.read(path) as c:
        for t, (raw, n, k) in w.items():
            qt = c.tensor(f"blk.0.w{t}", dev)
            assert qt.shape() == (n, k) and int(qt.dtype()) == t
            assert np.array_equal(qt.data.cpu().numpy(), raw)
            x = rng.standard_normal((3, k)).astype(np.float32)
            y = QMatMul.from_qtensor(qt).forward(to_dev(x, dev))
            ref = oracle.qmatmul(t, raw, n, k, x, nthreads=4).astype(np.float64)
            assert_rows_close(y.cpu().numpy(), ref)
            h = ctypes.c_void_p()
            ctx = context(dev)
            _lib.check(L.lbq_weight_from_gguf(ctx, c._h, f"blk.0.w{t}".encode(), ctypes.byref(h)))
            y2 = torch.empty(3, n, device=dev)
            _lib.check(L.lbq_qmatmul_f32(ctx, h.value, to_dev(x, dev).data_ptr(), 3, y2.data_ptr(), None))
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
            L.lbq_weight_destroy(h.value)
        # a 1-D tensor is not a weight
        h = ctypes.c_void_p()
        assert L.lbq_weight_from_gguf(context(dev), c._h, b"token_norm", ctypes.byref(h)) == -3
        with pytest.raises(ValueError, match="2"):
            c.tensor("token_norm", dev)


def _rms_norm_ref(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    # candle RmsNorm in f32: x / sqrt(sum(x^2) / k + eps) * w
    x32 = x.astype(np.float32)
    ss = (x32 * x32).sum(axis=-1, dtype=np.float32, keepdims=True)
    rms = np.sqrt(ss / np.float32(x.shape[-1]) + np.float32(eps)).astype(np.float32)
    return (x32 / rms * w.astype(np.float32)).astype(np.float32)


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_rmsnorm_fused_projections(oracle, lbq, dev, t):
    # the input norm in the GEMV prologue (m = 1, k-quants, k <= 8192) or in its
    # own launch (otherwise), then grouped projections / the gate-up product;
    # against the oracle on the numpy-normalised x
    from lightbulb_amd.quantized import (QMatMul, QTensor, qmatmul_group, rms_norm, rmsnorm_gate_up_silu,
                                         rmsnorm_qmatmul_group)
    rng = np.random.default_rng(160 + t)
    bs = oracle.block_size(t)
    for k, ns in ((4096, (256, 64, 64)), (1024, (96, 33)), (14336, (40, 24))):
        raws = [bp.random_blocks(rng, t, n * k // bs, d_scale=1e-3) for n in ns]
        qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, ns)]
        w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
        wd = to_dev(w, dev)
        for m in (1, 3):
            x = (3.0 * rng.standard_normal((m, k)) + 0.5).astype(np.float32)
            xd = to_dev(x, dev)
            xn = _rms_norm_ref(x, w, 1e-5)
            got_norm = rms_norm(xd, wd, 1e-5).cpu().numpy()
            assert np.allclose(got_norm, xn, rtol=2e-6, atol=1e-6)
            ys = rmsnorm_qmatmul_group(qms, xd, wd, 1e-5)
            torch.cuda.synchronize()
            for y, r, n in zip(ys, raws, ns):
                assert_rows_close(y.cpu().numpy(), oracle.qmatmul(t, r, n, k, xn, nthreads=8).astype(np.float64), 2e-3)
            if ns[0] == ns[1]:
                continue
            # gate/up product over the first two weights cut to a common n
            n2 = min(ns[0], ns[1])
            cut = [r[: n2 * (r.size // n)] for r, n in zip(raws[:2], ns[:2])]  # the first n2 rows
            gq = [QMatMul.from_qtensor(QTensor(to_dev(c, dev), t, (n2, k))) for c in cut]
            out = rmsnorm_gate_up_silu(gq[0], gq[1], xd, wd, 1e-5)
            torch.cuda.synchronize()
            gr = oracle.qmatmul(t, cut[0], n2, k, xn, nthreads=8).astype(np.float64)
            ur = oracle.qmatmul(t, cut[1], n2, k, xn, nthreads=8).astype(np.float64)
            assert_rows_close(out.cpu().numpy(), gr / (1.0 + np.exp(-gr)) * ur, 2e-3)


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
def test_eight_wave_fused_launches(oracle, lbq, dev, t):
    # fused m = 1 launches on eight-wave workgroups: grouped q|k|v at Llama-3
    # sizes (6144 rows), gate/up pairs past 8192 rows and both with the RMS norm
    # in the prologue; grouped outputs bit-identical to the separate (four-wave)
    # calls, all against the oracle
    from lightbulb_amd.quantized import (QMatMul, QTensor, gate_up_silu, qmatmul_group, rmsnorm_gate_up_silu,
                                         rmsnorm_qmatmul_group)
    rng = np.random.default_rng(180 + t)
    k, ns = 4096, (4096, 1024, 1024)
    raws = [bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3) for n in ns]
    qms = [QMatMul.from_qtensor(QTensor(to_dev(r, dev), t, (n, k))) for r, n in zip(raws, ns)]
    x = rng.standard_normal((1, k)).astype(np.float32)
    xd = to_dev(x, dev)
    ys = qmatmul_group(qms, xd)
    singles = [q.forward(xd) for q in qms]
    torch.cuda.synchronize()
    for y, y1, r, n in zip(ys, singles, raws, ns):
        assert np.array_equal(y.cpu().numpy().view(np.uint32), y1.cpu().numpy().view(np.uint32))
        assert_rows_close(y.cpu().numpy(), oracle.qmatmul(t, r, n, k, x, nthreads=8).astype(np.float64))
    w = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32)
    wd = to_dev(w, dev)
    xn = _rms_norm_ref(x, w, 1e-5)
    ys = rmsnorm_qmatmul_group(qms, xd, wd, 1e-5)
    torch.cuda.synchronize()
    for y, r, n in zip(ys, raws, ns):
        assert_rows_close(y.cpu().numpy(), oracle.qmatmul(t, r, n, k, xn, nthreads=8).astype(np.float64), 2e-3)
    n2 = 4200  # 8400 interleaved rows
    g_raw = bp.random_blocks(rng, t, n2 * k // 256, d_scale=1e-3)
    u_raw = bp.random_blocks(rng, t, n2 * k // 256, d_scale=1e-3)
    qg = QMatMul.from_qtensor(QTensor(to_dev(g_raw, dev), t, (n2, k)))
    qu = QMatMul.from_qtensor(QTensor(to_dev(u_raw, dev), t, (n2, k)))
    for fn, xin, xr, tol in ((lambda: gate_up_silu(qg, qu, xd), x, x, 1e-4),
                             (lambda: rmsnorm_gate_up_silu(qg, qu, xd, wd, 1e-5), x, xn, 2e-3)):
        out = fn()
        torch.cuda.synchronize()
        gr = oracle.qmatmul(t, g_raw, n2, k, xr, nthreads=8).astype(np.float64)
        ur = oracle.qmatmul(t, u_raw, n2, k, xr, nthreads=8).astype(np.float64)
        assert_rows_close(out.cpu().numpy(), gr / (1.0 + np.exp(-gr)) * ur, tol)


def test_qmatmul_group_errors(oracle, lbq, dev):
    from lightbulb_amd import _lib
    from lightbulb_amd.quantized import QMatMul, QTensor, qmatmul_group
    rng = np.random.default_rng(120)
    a = QMatMul.from_qtensor(QTensor(to_dev(bp.random_blocks(rng, Q4_K, 8 * 2), dev), Q4_K, (8, 512)))
    b = QMatMul.from_qtensor(QTensor(to_dev(bp.random_blocks(rng, Q4_K, 8 * 1), dev), Q4_K, (8, 256)))
    c = QMatMul.from_qtensor(QTensor(to_dev(bp.random_blocks(rng, Q5_K, 8 * 2), dev), Q5_K, (8, 512)))
    x = torch.zeros(1, 512, device=dev)
    with pytest.raises(ValueError, match="share"):
        qmatmul_group([a, b], x)
    with pytest.raises(ValueError, match="between 1 and 4"):
        qmatmul_group([a] * 5, x)
    assert [tuple(y.shape) for y in qmatmul_group([a], torch.zeros(0, 512, device=dev))] == [(0, 8)]
    # the C ABI checks the same things itself
    L = _lib.lib()
    y = torch.empty(1, 8, device=dev)
    for ws, cnt, want in (([a, c], 2, -3), ([a, b], 2, -3), ([a], 0, -6), ([a] * 4 + [a], 5, -6)):
        hs = (ctypes.c_void_p * len(ws))(*[q._handle for q in ws])
        outs = (ctypes.c_void_p * len(ws))(*([y.data_ptr()] * len(ws)))
        assert L.lbq_qmatmul_group_f32(a._ctx, hs, cnt, x.data_ptr(), 1, outs, None) == want
    hs = (ctypes.c_void_p * 2)(a._handle, None)
    outs = (ctypes.c_void_p * 2)(y.data_ptr(), y.data_ptr())
    assert L.lbq_qmatmul_group_f32(a._ctx, hs, 2, x.data_ptr(), 1, outs, None) == -1
    # gate/up pairs must match in type and shape
    from lightbulb_amd.quantized import gate_up_silu
    with pytest.raises(ValueError, match="share"):
        gate_up_silu(a, c, x)
    assert L.lbq_gate_up_silu_f32(a._ctx, a._handle, c._handle, x.data_ptr(), 1, y.data_ptr(), None) == -3
    assert L.lbq_gate_up_silu_f32(a._ctx, a._handle, None, x.data_ptr(), 1, y.data_ptr(), None) == -1


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_batch_decode_row_chunks(oracle, lbq, dev, t):
    # m = 2..8 at k = 4096 takes the multi-row decode kernel: activation rows in
    # chunks of at most 4 or 8 (m = 5 and 7 leave a ragged last chunk), ragged n
    rng = np.random.default_rng(90 + t)
    k = 4096
    for n in (1, 257, 1000):
        w_raw = bp.random_blocks(rng, t, n * k // oracle.block_size(t), d_scale=1e-3)
        for m in (2, 5, 7, 8):
            x = rng.standard_normal((m, k)).astype(np.float32)
            ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
            assert_rows_close(gpu_qmatmul(t, w_raw, n, k, x, dev), ref, tight_bound(t, m))


@pytest.mark.parametrize("t", [Q4_K, Q5_K])
@pytest.mark.parametrize("k", [4096, 14336])
def test_ksliced_tiles_split_k(oracle, lbq, dev, t, k):
    # 9 <= m <= 32 takes the k-sliced tiles (32 rows x 128 columns, k split over
    # workgroups): ragged m and n, both Llama-3 row lengths
    rng = np.random.default_rng(95 + t + k)
    for n in (40, 1000):
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
        for m in (9, 23, 32):
            x = rng.standard_normal((m, k)).astype(np.float32)
            ref = oracle.qmatmul(t, w_raw, n, k, x, nthreads=8).astype(np.float64)
            assert_rows_close(gpu_qmatmul(t, w_raw, n, k, x, dev), ref, tight_bound(t, m))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
def test_qmatmul_wide_tiles(oracle, lbq, dev, t):
    # 128 <= m < 256 (and Q4_K up to 512) takes the 128 x 256 eight-wave tiles:
    # ragged m and n, odd block counts, split-k over 12 one-block slices
    rng = np.random.default_rng(85 + t)
    for (m, n, k) in ((128, 256, 256), (200, 77, 256 * 3), (255, 300, 256 * 12), (400, 290, 256 * 2)):
        w_raw = bp.random_blocks(rng, t, n * k // 256)
        x = rng.standard_normal((m, k)).astype(np.float32)
        rows = np.r_[0:4, m // 2:m // 2 + 4, m - 4:m]
        y = gpu_qmatmul(t, w_raw, n, k, x, dev)
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert_rows_close(y[rows], ref, tight_bound(t, m))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
def test_split_k_shapes_deterministic(oracle, lbq, dev, t):
    # shapes that split k (k-sliced m <= 32, 32-row tiles, wide, tall): partial
    # sums are added in slice order, so repeated calls give the same bits
    rng = np.random.default_rng(88 + t)
    for (m, n, k) in ((16, 300, 256 * 16), (32, 1000, 256 * 56), (48, 300, 256 * 8), (130, 300, 256 * 12),
                      (300, 100, 256 * 16)):
        w_raw = bp.random_blocks(rng, t, n * k // 256, d_scale=1e-3)
        x = rng.standard_normal((m, k)).astype(np.float32)
        y1 = gpu_qmatmul(t, w_raw, n, k, x, dev)
        y2 = gpu_qmatmul(t, w_raw, n, k, x, dev)
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32)), (m, n, k)
        rows = np.r_[0:2, m - 2:m]
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert_rows_close(y1[rows], ref, tight_bound(t, m))


@pytest.mark.parametrize("t", [Q4_K, Q5_K, Q6_K])
def test_qmatmul_tall_tiles(oracle, lbq, dev, t):
    # Q5_K / Q6_K at m >= 256 and Q4_K above 512 take the 256 x 128 tiles: ragged
    # m and n, odd and even block counts (Q4_K at m = 256, 300: the wide tiles)
    rng = np.random.default_rng(80 + t)
    for (m, n, k) in ((256, 128, 256), (300, 200, 256 * 3), (520, 390, 256 * 4), (640, 130, 256 * 5)):
        w_raw = bp.random_blocks(rng, t, n * k // 256)
        x = rng.standard_normal((m, k)).astype(np.float32)
        rows = np.r_[0:4, m // 2:m // 2 + 4, m - 4:m]
        y = gpu_qmatmul(t, w_raw, n, k, x, dev)
        ref = oracle.qmatmul(t, w_raw, n, k, x[rows], nthreads=8).astype(np.float64)
        assert_rows_close(y[rows], ref, tight_bound(t, m))


def test_qmatmul_shapes_and_errors(oracle, lbq, dev):
    from lightbulb_amd.quantized import QMatMul, QTensor, QuantizableLinear
    rng = np.random.default_rng(53)
    n, k = 64, 512
    w_raw = bp.random_blocks(rng, Q4_K, n * k // 256)
    qm = QMatMul.from_qtensor(QTensor(to_dev(w_raw, dev), Q4_K, (n, k)))
    lin = QuantizableLinear.from_qmatmul(qm)
    assert lin.is_quantized()
    x = rng.standard_normal((4, 1, k)).astype(np.float32)  # decode [B, 1, K]
    y = lin.forward(to_dev(x, dev))
    assert tuple(y.shape) == (4, 1, n)
    ref = oracle.qmatmul(Q4_K, w_raw, n, k, x.reshape(4, k), nthreads=4)
    assert_rows_close(y.cpu().numpy().reshape(4, n), ref.astype(np.float64))
    with pytest.raises(ValueError, match="incompatible"):
        qm.forward(torch.zeros(2, k + 256, device=dev))
    with pytest.raises(ValueError, match="only one dimension"):
        qm.forward(torch.zeros(k, device=dev))
    with pytest.raises(ValueError, match="must be f32"):
        qm.forward(torch.zeros(2, k, device=dev, dtype=torch.float16))
    with pytest.raises(ValueError, match="not contiguous"):
        qm.forward(torch.zeros(k, 2, device=dev).t())
    assert qm.forward(torch.zeros(0, k, device=dev)).shape == (0, n)


def test_c_abi_error_paths(lbq, dev):
    from lightbulb_amd import _lib
    from lightbulb_amd.quantized import context
    ctx = context(dev)
    h = ctypes.c_void_p()
    buf = torch.zeros(144 * 4, dtype=torch.uint8, device=dev)
    assert lbq.lbq_weight_wrap_device(ctx, 5, 4, 256, buf.data_ptr(), 2 * 4 * 256, ctypes.byref(h)) == -2  # no type 5
    assert lbq.lbq_weight_wrap_device(ctx, Q4_K, 4, 255, buf.data_ptr(), buf.numel(), ctypes.byref(h)) == -3
    assert lbq.lbq_weight_wrap_device(ctx, Q4_K, 4, 256, buf.data_ptr(), buf.numel() - 1, ctypes.byref(h)) == -3
    assert lbq.lbq_weight_wrap_device(ctx, Q4_K, 4, 256, buf.data_ptr() + 4, 144 * 4, ctypes.byref(h)) == -1
    assert b"16-byte" in lbq.lbq_last_error()
    assert lbq.lbq_weight_wrap_device(ctx, Q4_K, 4, 256, buf.data_ptr(), buf.numel(), ctypes.byref(h)) == 0
    assert lbq.lbq_qmatmul_f32(ctx, h, None, 1, None, None) == -1
    assert lbq.lbq_qmatmul_f32(ctx, h, None, -1, None, None) == -1
    assert lbq.lbq_qmatmul_f32(ctx, h, None, 0, None, None) == 0
    assert lbq.lbq_weight_destroy(h) == 0
    with pytest.raises(_lib.LbqError):
        _lib.check(lbq.lbq_init(1 << 20, ctypes.byref(ctypes.c_void_p())))
