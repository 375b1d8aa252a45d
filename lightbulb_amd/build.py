"""Build liblbq.so (the HIP library behind include/lbq.h) for gfx950.

Run as ``python -m lightbulb_amd.build`` or through ``__graft_entry__.build()``.
Every translation unit is compiled by hipcc for gfx950 only and linked into
``lightbulb_amd/liblbq.so``.  No torch, no JIT cache: the library sits in-tree
so it travels with the repository to the GPU box.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "liblbq.so"
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for all device code: the compiler is
# free to emit them from plain float code, and some forms have produced wrong
# results on this hardware pool without raising an error.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
]
# Sources whose float arithmetic must be rounded op by op (bit-exact restatements).
NO_CONTRACT = {"lbq_wquant.hip"}
# Matrix-core results consumed by VALU right away: keep them in VGPRs (no AGPR
# copies, fewer registers, so two waves per SIMD).
EXTRA_FLAGS = {"lbq_gemv_mx.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}

SOURCES = ["lbq_act.hip", "lbq_gemv.hip", "lbq_gemv_q4k.hip", "lbq_gemv_q5k.hip", "lbq_gemv_q6k.hip",
           "lbq_gemv_q8_0.hip", "lbq_gemv_legacy.hip", "lbq_gemv_k23.hip", "lbq_gemv_mx.hip", "lbq_gemm.hip", "lbq_gemm_q4k.hip", "lbq_gemm_q5k.hip",
           "lbq_gemm_q6k.hip", "lbq_gemm_q8_0.hip", "lbq_gemm_q4_0.hip", "lbq_gemm_q5_0.hip",
           "lbq_gemm_k23.hip", "lbq_dense.hip", "lbq_wquant.hip",
           "lbq_api.cpp", "lbq_gguf.cpp"]


def _hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _compile(src: str) -> Path:
    hipcc = _hipcc()
    out = OBJ / (src + ".o")
    cmd = [hipcc, *HIP_FLAGS]
    if src in NO_CONTRACT:
        cmd.append("-ffp-contract=off")
    cmd += EXTRA_FLAGS.get(src, [])
    if src.endswith(".cpp"):
        cmd += ["-x", "hip"]
    cmd += ["-c", str(CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return out


# measurement-only kernels for bench.py (a read-only stream), kept out of liblbq.so
PROBE_SOURCES = ["lbq_probe.hip"]
PROBE_LIB = PKG / "liblbq_probe.so"


def _link(objs, lib: Path) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = True) -> Path:
    OBJ.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES) + len(PROBE_SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES + PROBE_SOURCES))
    _link(objs[len(SOURCES):], PROBE_LIB)
    objs = objs[:len(SOURCES)]
    _link(objs, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
