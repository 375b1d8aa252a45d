"""CPU oracle for the quantized-linear path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline).  The product (``lightbulb_amd``) never imports it.

It wraps ``oracle/_build/liblbq_oracle.so``, a C restatement of the reference's
CPU path (candle-core 0.10.2 quantized CPU kernels behind ``QMatMul::forward``,
reached through /root/reference/src/model/quantizable_linear.rs:63-69); see
``lbq_oracle.c`` for the function-by-function restatement.

How each function is pinned (tests/test_oracle.py), given that the reference
itself (Rust) cannot be built or run here and holds no golden vectors for
this path:

* type table          -- asserted against the GgmlDType table
                         (/root/reference/src/quantization/mod.rs:99-126) and the
                         reference's own test_dtype_properties (:114-120).
* f16 <-> f32          -- exhaustive over all 65536 half patterns against numpy's
                         IEEE float16, and RNE narrowing on random f32.
* dequantize           -- known-answer blocks assembled by an independent Python
                         bit-packer from chosen (d, dmin, sc, m, q) per value, for
                         every scale-unpack branch, nibble, qh bit plane and
                         Q6_K quarter, the Q2_K/Q3_K 2-bit planes, hmask bits and
                         6-bit scale layout (packed the way ggml's quantisers
                         write them), and every code of the 32-value types; plus
                         the reference's own Q8_0 round-trip bound (|err| < 0.01
                         on i/256 ramps, mod.rs:99-112).
* Q8_K / Q8_0 / Q8_1   -- closed-form special cases (single non-zero -> -128,
  act quant              negative max, all-zero, ties, saturation), the bsums
                         invariant, |x - d*q| <= |d|/2 on random rows, and Q8_1's
                         s = f16(f16(sum q) * d) recomputed from its codes.
* vec_dot / qmatmul    -- float64 brute force over the dequantised weights and
                         dequantised activations (the exact value the integer
                         path computes) on tiny shapes, to ~1e-6 relative.
* weight quantisers    -- "parity unpinned": only validity of the produced
                         blocks and a reconstruction-error bound are checked; the
                         kernels consume the same bytes as the oracle, so the
                         quantiser's exact choices never affect kernel parity.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_BUILD = HERE / "_build"

Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, Q8_1 = 2, 3, 6, 7, 8, 9
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K, Q8_K = 10, 11, 12, 13, 14, 15
BLOCK_SIZE = {Q4_0: 32, Q4_1: 32, Q5_0: 32, Q5_1: 32, Q8_0: 32, Q8_1: 32,
              Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256, Q8_K: 256}
TYPE_SIZE = {Q4_0: 18, Q4_1: 20, Q5_0: 22, Q5_1: 24, Q8_0: 34, Q8_1: 36,
             Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 292}
# the activation type each weight type's vec_dot takes (candle GgmlType::VecDotType)
VEC_DOT_TYPE = {Q4_0: Q8_0, Q5_0: Q8_0, Q8_0: Q8_0, Q4_1: Q8_1, Q5_1: Q8_1,
                Q2_K: Q8_K, Q3_K: Q8_K, Q4_K: Q8_K, Q5_K: Q8_K, Q6_K: Q8_K}

_libs: dict[str, ctypes.CDLL] = {}


def build() -> None:
    """Compile the oracle with its Makefile (outputs only under oracle/_build)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def _load(native: bool | str = False) -> ctypes.CDLL:
    """The scalar build, the -march=native build made here (native=True), or the
    build for the host running this process (native="host", made by `make host`)."""
    name = ("liblbq_oracle_host.so" if native == "host" else "liblbq_oracle_native.so" if native
            else "liblbq_oracle.so")
    if name in _libs:
        return _libs[name]
    path = _BUILD / name
    if native == "host":
        subprocess.run(["make", "-s", "-C", str(HERE), "host"], check=True)
    elif not path.exists():
        build()
    lib = ctypes.CDLL(str(path))
    c = ctypes
    lib.oracle_f16_to_f32.argtypes = [c.c_uint16]
    lib.oracle_f16_to_f32.restype = c.c_float
    lib.oracle_f32_to_f16.argtypes = [c.c_float]
    lib.oracle_f32_to_f16.restype = c.c_uint16
    lib.oracle_dequantize.argtypes = [c.c_uint32, c.c_void_p, c.c_int64, c.c_void_p]
    lib.oracle_quantize_act.argtypes = [c.c_uint32, c.c_void_p, c.c_int64, c.c_int64, c.c_void_p]
    lib.oracle_vec_dot.argtypes = [c.c_uint32, c.c_int64, c.c_void_p, c.c_void_p, c.c_void_p]
    lib.oracle_qmatmul.argtypes = [c.c_uint32, c.c_void_p, c.c_int64, c.c_int64, c.c_void_p, c.c_int64,
                                   c.c_void_p, c.c_int]
    lib.oracle_quantize_weights.argtypes = [c.c_uint32, c.c_void_p, c.c_int64, c.c_void_p]
    lib.oracle_unpack_scales_k4.argtypes = [c.c_void_p, c.c_void_p, c.c_void_p]
    for f in ("oracle_dequantize", "oracle_quantize_act", "oracle_vec_dot", "oracle_qmatmul",
              "oracle_quantize_weights", "oracle_block_size", "oracle_type_size"):
        getattr(lib, f).restype = c.c_int
    _libs[name] = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def block_size(t: int) -> int:
    return _load().oracle_block_size(t)


def type_size(t: int) -> int:
    return _load().oracle_type_size(t)


def f16_to_f32(bits: int) -> float:
    return _load().oracle_f16_to_f32(bits)


def f32_to_f16(x: float) -> int:
    return _load().oracle_f32_to_f16(x)


def dequantize(t: int, blocks: np.ndarray) -> np.ndarray:
    """Raw GGUF bytes (uint8) -> f32 values."""
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    ts, bs = TYPE_SIZE[t], BLOCK_SIZE[t]
    assert blocks.size % ts == 0
    nb = blocks.size // ts
    out = np.empty(nb * bs, dtype=np.float32)
    assert _load().oracle_dequantize(t, _ptr(blocks), nb, _ptr(out)) == 0
    return out


def quantize_act(t: int, x: np.ndarray) -> np.ndarray:
    """x f32 [m, k] -> GGUF blocks of Q8_K (t=15), Q8_0 (t=8) or Q8_1 (t=9) as uint8 [m, k/QK*TS]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.ndim == 1:
        x = x[None]
    m, k = x.shape
    out = np.zeros((m, k // BLOCK_SIZE[t] * TYPE_SIZE[t]), dtype=np.uint8)
    assert _load().oracle_quantize_act(t, _ptr(x), m, k, _ptr(out)) == 0
    return out


def vec_dot(t: int, k: int, wrow: np.ndarray, xrow: np.ndarray) -> float:
    r = np.zeros(1, dtype=np.float32)
    wrow = np.ascontiguousarray(wrow, dtype=np.uint8)
    xrow = np.ascontiguousarray(xrow, dtype=np.uint8)
    assert _load().oracle_vec_dot(t, k, _ptr(wrow), _ptr(xrow), _ptr(r)) == 0
    return float(r[0])


def qmatmul(t: int, w_blocks: np.ndarray, n: int, k: int, x: np.ndarray, nthreads: int = 1,
            native: bool | str = False) -> np.ndarray:
    """candle's CPU QMatMul::forward restated: y[m, n] = x[m, k] . W^T."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, k)
    w_blocks = np.ascontiguousarray(w_blocks, dtype=np.uint8)
    m = x.shape[0]
    y = np.zeros((m, n), dtype=np.float32)
    assert _load(native).oracle_qmatmul(t, _ptr(w_blocks), n, k, _ptr(x), m, _ptr(y), nthreads) == 0
    return y


def quantize_weights(t: int, w: np.ndarray) -> np.ndarray:
    """f32 weights (row-major, rows along k) -> GGUF blocks (uint8)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n = w.size // BLOCK_SIZE[t]
    out = np.zeros(n * TYPE_SIZE[t], dtype=np.uint8)
    assert _load().oracle_quantize_weights(t, _ptr(w), w.size, _ptr(out)) == 0
    return out


def unpack_scales_k4(scales12: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    s = np.ascontiguousarray(scales12, dtype=np.uint8)
    sc = np.zeros(8, dtype=np.uint8)
    mn = np.zeros(8, dtype=np.uint8)
    _load().oracle_unpack_scales_k4(_ptr(s), _ptr(sc), _ptr(mn))
    return sc, mn


def nproc() -> int:
    return len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
