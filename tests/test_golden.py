"""Frozen restatement vectors (tests/golden/restatement_vectors.npz, written by
tests/golden/make_fixtures.py): the oracle must still reproduce them exactly, and the GPU
library must match them to the parity bar.  They are restatement outputs, not reference
outputs (the reference's tests hold no vectors for this path)."""
import sys
from pathlib import Path

import numpy as np
import pytest

GOLD = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLD))
import make_fixtures as mf  # noqa: E402

TYPES = ((8, "q8_0"), (12, "q4_k"), (13, "q5_k"), (14, "q6_k"))


@pytest.fixture(scope="module")
def vec():
    return dict(np.load(GOLD / "restatement_vectors.npz"))


def weights(t):
    n, k = mf.N, mf.K
    return (mf.normal(0x1B0 + t, n * k) * 0.02).reshape(n, k)


def test_generator_is_stable(vec):
    x = mf.normal(0x1B0 + 100, mf.M * mf.K).reshape(mf.M, mf.K)
    pick = ((mf.splitmix64(0x1B0 + 101, mf.M * mf.K) % np.uint64(100)) == 0).reshape(mf.M, mf.K)
    x[pick] *= 20.0
    assert np.array_equal(x, vec["x"])


@pytest.mark.parametrize("t,name", TYPES)
def test_oracle_reproduces_vectors(oracle, vec, t, name):
    n, k, m = (int(v) for v in vec["shape"])
    blocks = vec[f"{name}_blocks"]
    assert np.array_equal(oracle.quantize_weights(t, weights(t)), blocks)
    assert np.array_equal(oracle.dequantize(t, blocks).view(np.uint32), vec[f"{name}_dequant"].view(np.uint32))
    assert np.array_equal(oracle.qmatmul(t, blocks, n, k, vec["x"], nthreads=4), vec[f"{name}_y"])


def test_oracle_reproduces_activation_vectors(oracle, vec):
    assert np.array_equal(oracle.quantize_act(15, vec["x"]), vec["x_q8_k"])
    assert np.array_equal(oracle.quantize_act(8, vec["x"]), vec["x_q8_0"])


@pytest.mark.gpu
@pytest.mark.parametrize("t,name", TYPES)
def test_gpu_matches_vectors(lbq, dev, vec, t, name):
    import torch
    from lightbulb_amd.quantized import QMatMul, QTensor, dequantize_tensor, quantize_tensor
    from test_gpu_parity import assert_rows_close
    n, k, m = (int(v) for v in vec["shape"])
    blocks = vec[f"{name}_blocks"]
    w = torch.from_numpy(weights(t)).to(dev)
    assert np.array_equal(quantize_tensor(w.reshape(-1), t, _exact=True).cpu().numpy(), blocks)
    d = torch.from_numpy(blocks).to(dev)
    got = dequantize_tensor(d, t, n * k).cpu().numpy()
    assert np.array_equal(got.view(np.uint32), vec[f"{name}_dequant"].view(np.uint32))
    qm = QMatMul.from_qtensor(QTensor(d, t, (n, k)))
    for rows in (1, m):  # decode GEMV (m = 1) and the general path
        y = qm.forward(torch.from_numpy(vec["x"][:rows]).to(dev))
        torch.cuda.synchronize()
        assert_rows_close(y.cpu().numpy(), vec[f"{name}_y"][:rows].astype(np.float64))


@pytest.mark.gpu
def test_gpu_matches_activation_vectors(lbq, dev, vec):
    import torch
    from lightbulb_amd.quantized import quantize_activations
    x = torch.from_numpy(vec["x"]).to(dev)
    assert np.array_equal(quantize_activations(x, 15).cpu().numpy(), vec["x_q8_k"])
    assert np.array_equal(quantize_activations(x, 8).cpu().numpy(), vec["x_q8_0"])
