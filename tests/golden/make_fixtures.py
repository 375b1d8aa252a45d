"""Write tests/golden/restatement_vectors.npz: frozen input/output vectors of the CPU
restatement (oracle/) for the quantized-linear path.

These are RESTATEMENT OUTPUTS, NOT REFERENCE OUTPUTS: the reference's arithmetic lives in
candle-core 0.10.2 / ggml-quants 0.1.0 (Rust, not vendored, no toolchain here) and its own
tests hold no vectors for QMatMul.  Freezing the restatement's outputs pins it against
regressions, and the GPU library is checked against the same vectors.

Inputs are drawn from a splitmix64-seeded generator written here (no numpy RNG, so the
vectors do not depend on numpy's generator versions).  Run from the repo root:
    python tests/golden/make_fixtures.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
import oracle  # noqa: E402

OUT = Path(__file__).resolve().parent / "restatement_vectors.npz"
N, K, M = 16, 512, 3


def splitmix64(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint64)
    s = seed & 0xFFFFFFFFFFFFFFFF
    for i in range(count):
        s = (s + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        out[i] = z ^ (z >> 31)
    return out


def normal(seed: int, count: int) -> np.ndarray:
    """Box-Muller over splitmix64 uniforms, float64 -> float32."""
    u = (splitmix64(seed, 2 * count) >> np.uint64(11)).astype(np.float64) * (1.0 / (1 << 53))
    u1, u2 = np.maximum(u[0::2], 1e-300), u[1::2]
    return (np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)).astype(np.float32)


def main() -> None:
    oracle.build()
    vec = {"shape": np.array([N, K, M], dtype=np.int64)}
    x = normal(0x1B0 + 100, M * K).reshape(M, K)
    pick = (splitmix64(0x1B0 + 101, M * K) % np.uint64(100)) == 0  # ~1% outliers, x20
    x[pick.reshape(M, K)] *= 20.0
    vec["x"] = x
    for t, name in ((oracle.Q8_0, "q8_0"), (oracle.Q4_K, "q4_k"), (oracle.Q5_K, "q5_k"), (oracle.Q6_K, "q6_k")):
        w = (normal(0x1B0 + t, N * K) * 0.02).reshape(N, K)
        blocks = oracle.quantize_weights(t, w)
        vec[f"{name}_blocks"] = blocks
        vec[f"{name}_dequant"] = oracle.dequantize(t, blocks)
        vec[f"{name}_y"] = oracle.qmatmul(t, blocks, N, K, x, nthreads=1)
    vec["x_q8_k"] = oracle.quantize_act(oracle.Q8_K, x)
    vec["x_q8_0"] = oracle.quantize_act(oracle.Q8_0, x)
    np.savez_compressed(OUT, **vec)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
