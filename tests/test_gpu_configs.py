"""BASELINE.json configs at their full shapes, on the GPU, against the oracle.

Rows of y are independent (each is one activation row against all weight rows),
so at the large batched sizes the oracle checks a sample of rows spread over the
batch; every row is checked for finiteness, and the decode configs are checked
whole.  Weights are N(0, 0.02) quantised on the device (the device quantiser is
bit-exact with the oracle's, tests/test_gpu_parity.py)."""
import numpy as np
import pytest
import torch

from test_gpu_parity import Q4_K, Q5_K, Q6_K, Q8_0, assert_rows_close, tight_bound

pytestmark = pytest.mark.gpu


def quantised(t, n, k, dev, seed):
    from lightbulb_amd.quantized import QMatMul, QTensor
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    w = torch.randn(n, k, generator=g, device=dev) * 0.02
    qt = QTensor.quantize(w, t)
    del w
    return QMatMul.from_qtensor(qt), qt.data.cpu().numpy()


def check(oracle, qm, raw, t, n, k, x, rows=None):
    y = qm.forward(torch.from_numpy(x).to(qm.qtensor().data.device))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert np.all(np.isfinite(y))
    rows = np.arange(x.shape[0]) if rows is None else np.asarray(rows)
    ref = oracle.qmatmul(t, raw, n, k, x[rows], nthreads=oracle.nproc()).astype(np.float64)
    assert_rows_close(y[rows], ref, tight_bound(t, x.shape[0]))


def test_config1_q8_0_gemv(oracle, lbq, dev):
    qm, raw = quantised(Q8_0, 4096, 4096, dev, 0x1B0)
    x = np.random.default_rng(1).standard_normal((1, 4096)).astype(np.float32)
    check(oracle, qm, raw, Q8_0, 4096, 4096, x)


@pytest.mark.parametrize("n,k", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_config2_q4k_decode(oracle, lbq, dev, n, k):
    qm, raw = quantised(Q4_K, n, k, dev, 0x1B1 + n + k)
    x = np.random.default_rng(2).standard_normal((1, k)).astype(np.float32)
    check(oracle, qm, raw, Q4_K, n, k, x)


@pytest.mark.parametrize("b", [1, 4, 8])
def test_config3_q6k_head_and_q5k(oracle, lbq, dev, b):
    rng = np.random.default_rng(3 + b)
    x = rng.standard_normal((b, 4096)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20  # ~1% outliers
    qm, raw = quantised(Q6_K, 128256, 4096, dev, 0x1B2)
    check(oracle, qm, raw, Q6_K, 128256, 4096, x)
    del qm, raw
    qm, raw = quantised(Q5_K, 14336, 4096, dev, 0x1B3)
    check(oracle, qm, raw, Q5_K, 14336, 4096, x)


@pytest.mark.parametrize("b", [2, 3])
def test_config3_q6k_head_few_rows(oracle, lbq, dev, b):
    # the head's long per-wave stream takes the deeper weight ring at m = 1..4
    rng = np.random.default_rng(30 + b)
    x = rng.standard_normal((b, 4096)).astype(np.float32)
    x[rng.random(x.shape) < 0.01] *= 20
    qm, raw = quantised(Q6_K, 128256, 4096, dev, 0x1B2)
    check(oracle, qm, raw, Q6_K, 128256, 4096, x)


@pytest.mark.parametrize("m", [16, 64, 512, 2048])
def test_config4_q4k_prefill(oracle, lbq, dev, m):
    rng = np.random.default_rng(4 + m)
    rows = sorted(set([0, 1, m // 3, m // 2, m - 1]))
    for (n, k) in [(14336, 4096), (4096, 14336)]:
        qm, raw = quantised(Q4_K, n, k, dev, 0x1B4 + n)
        x = rng.standard_normal((m, k)).astype(np.float32)
        check(oracle, qm, raw, Q4_K, n, k, x, rows)
