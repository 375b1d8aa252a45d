"""BASELINE configs[4] at batch 32 (and its shapes at batch 1), on the GPU, against the oracle.

The stack's B = 32 step runs every distinct (type, shape) of the Llama-3-8B
Q4_K_M mix at m = 32, where the k-sliced MFMA kernel's slice length depends on
the number of 128-column tiles, so on n.  Each shape is checked here at its full
size on rows spread over the batch (the oracle's per-row cost is the full
weight), and the call-site entry points the stack's fused step uses (grouped
q|k, gate|up with the SiLU product) are checked at B = 32 as well.  Weights are
N(0, 0.02) quantised on the device (bit-exact with the oracle's quantiser);
x ~ N(0, 1).  Shapes as /root/reference/src/model/custom_attention.rs:265-267
(q/k/v), mlp_wrapper.rs:190-195 (gate/up/down) and custom_transformer.rs:603-625
(the head) run them."""
import numpy as np
import pytest
import torch

from test_gpu_configs import quantised
from test_gpu_parity import Q4_K, Q5_K, Q6_K, assert_rows_close, tight_bound

pytestmark = pytest.mark.gpu

B = 32
ROWS = [0, 7, 15, 16, 31]  # both 16-row halves of the MFMA tile, first and last


def _check(oracle, qm, raw, t, n, k, x):
    y = qm.forward(torch.from_numpy(x).to(qm.qtensor().data.device))
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert np.all(np.isfinite(y))
    ref = oracle.qmatmul(t, raw, n, k, x[ROWS], nthreads=oracle.nproc()).astype(np.float64)
    assert_rows_close(y[ROWS], ref, tight_bound(t, B))
    return y


@pytest.mark.parametrize("t,n,k", [(Q4_K, 4096, 4096), (Q4_K, 1024, 4096), (Q6_K, 1024, 4096),
                                   (Q4_K, 14336, 4096), (Q5_K, 14336, 4096), (Q6_K, 4096, 14336),
                                   (Q4_K, 4096, 14336), (Q6_K, 128256, 4096)])
def test_stack_shape_b32(oracle, lbq, dev, t, n, k):
    qm, raw = quantised(t, n, k, dev, 0x1B5 + n + k + t)
    x = np.random.default_rng(5 + n + t).standard_normal((B, k)).astype(np.float32)
    _check(oracle, qm, raw, t, n, k, x)


@pytest.mark.parametrize("t,n,k", [(Q6_K, 1024, 4096), (Q6_K, 4096, 14336), (Q4_K, 1024, 4096),
                                   (Q4_K, 4096, 4096), (Q4_K, 14336, 4096), (Q4_K, 4096, 14336)])
def test_stack_shape_b1(oracle, lbq, dev, t, n, k):
    # the same stack shapes at batch 1 (the decode launch plan depends on n through
    # the groups per wave), every row against the oracle at the decode bound
    qm, raw = quantised(t, n, k, dev, 0x1B9 + n + k + t)
    x = np.random.default_rng(9 + n + t).standard_normal((1, k)).astype(np.float32)
    y = qm.forward(torch.from_numpy(x).to(qm.qtensor().data.device))
    torch.cuda.synchronize()
    ref = oracle.qmatmul(t, raw, n, k, x, nthreads=oracle.nproc()).astype(np.float64)
    assert_rows_close(y.cpu().numpy(), ref, tight_bound(t, 1))


def test_stack_call_sites_b32(oracle, lbq, dev):
    # the B = 32 fused step: q|k grouped (one operand pre-pass), gate|up through
    # gate_up_silu, down on its output -- against separate calls (bit-identical)
    # and the oracle
    from lightbulb_amd.quantized import gate_up_silu, qmatmul_group
    rng = np.random.default_rng(0x32)
    q, q_raw = quantised(Q4_K, 4096, 4096, dev, 0x1C0)
    kp, k_raw = quantised(Q4_K, 1024, 4096, dev, 0x1C1)
    gate, g_raw = quantised(Q4_K, 14336, 4096, dev, 0x1C2)
    up, u_raw = quantised(Q4_K, 14336, 4096, dev, 0x1C3)
    down, d_raw = quantised(Q6_K, 4096, 14336, dev, 0x1C4)
    x = rng.standard_normal((B, 4096)).astype(np.float32)
    xd = torch.from_numpy(x).to(dev)
    yq, yk = qmatmul_group([q, kp], xd)
    h = gate_up_silu(gate, up, xd)
    yd = down.forward(h)
    torch.cuda.synchronize()
    for got, qm in ((yq, q), (yk, kp)):
        assert np.array_equal(got.cpu().numpy().view(np.uint32), qm.forward(xd).cpu().numpy().view(np.uint32))
    n8 = oracle.nproc()
    for got, raw, n in ((yq, q_raw, 4096), (yk, k_raw, 1024)):
        ref = oracle.qmatmul(Q4_K, raw, n, 4096, x[ROWS], nthreads=n8).astype(np.float64)
        assert_rows_close(got.cpu().numpy()[ROWS], ref, tight_bound(Q4_K, B))
    gr = oracle.qmatmul(Q4_K, g_raw, 14336, 4096, x[ROWS], nthreads=n8).astype(np.float64)
    ur = oracle.qmatmul(Q4_K, u_raw, 14336, 4096, x[ROWS], nthreads=n8).astype(np.float64)
    assert_rows_close(h.cpu().numpy()[ROWS], gr / (1.0 + np.exp(-gr)) * ur, tight_bound(Q4_K, B))
    hh = h.cpu().numpy()
    ref = oracle.qmatmul(Q6_K, d_raw, 4096, 14336, hh[ROWS], nthreads=n8).astype(np.float64)
    assert_rows_close(yd.cpu().numpy()[ROWS], ref, tight_bound(Q6_K, B))
