"""ctypes binding of liblbq.so (the C ABI declared in include/lbq.h).

The library is the product: there is no fallback.  If ``liblbq.so`` has not
been built, or cannot be loaded, every entry point raises instead of quietly
computing something else.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liblbq.so"

LBQ_OK = 0
STATUS_NAMES = {
    -1: "LBQ_ERR_INVALID_ARG",
    -2: "LBQ_ERR_UNSUPPORTED_TYPE",
    -3: "LBQ_ERR_SHAPE",
    -4: "LBQ_ERR_OOM",
    -5: "LBQ_ERR_HIP",
    -6: "LBQ_ERR_LIMIT",
    -7: "LBQ_ERR_FORMAT",
    -8: "LBQ_ERR_NOT_FOUND",
    -9: "LBQ_ERR_IO",
}

# name -> (restype, argtypes); must list every function include/lbq.h declares
_c = ctypes
_VP, _I64, _U32, _SZ = _c.c_void_p, _c.c_int64, _c.c_uint32, _c.c_size_t
SIGNATURES = {
    "lbq_last_error": (_c.c_char_p, []),
    "lbq_type_block_size": (_c.c_int, [_U32]),
    "lbq_type_size": (_c.c_int, [_U32]),
    "lbq_type_block_bytes": (_c.c_int, [_U32]),
    "lbq_init": (_c.c_int, [_c.c_int, _c.POINTER(_VP)]),
    "lbq_ctx_destroy": (_c.c_int, [_VP]),
    "lbq_weight_create": (_c.c_int, [_VP, _U32, _I64, _I64, _VP, _SZ, _c.POINTER(_VP)]),
    "lbq_weight_wrap_device": (_c.c_int, [_VP, _U32, _I64, _I64, _VP, _SZ, _c.POINTER(_VP)]),
    "lbq_weight_destroy": (_c.c_int, [_VP]),
    "lbq_weight_info": (_c.c_int, [_VP, _c.POINTER(_U32), _c.POINTER(_I64), _c.POINTER(_I64)]),
    "lbq_weight_refresh": (_c.c_int, [_VP, _VP]),
    "lbq_qmatmul_f32": (_c.c_int, [_VP, _VP, _VP, _I64, _VP, _VP]),
    "lbq_qmatmul_f32_noalloc": (_c.c_int, [_VP, _VP, _VP, _I64, _VP, _VP]),
    "lbq_qmatmul_group_f32": (_c.c_int, [_VP, _c.POINTER(_VP), _c.c_int, _VP, _I64, _c.POINTER(_VP), _VP]),
    "lbq_gate_up_silu_f32": (_c.c_int, [_VP, _VP, _VP, _VP, _I64, _VP, _VP]),
    "lbq_rmsnorm_f32": (_c.c_int, [_VP, _VP, _c.c_float, _I64, _I64, _VP, _VP]),
    "lbq_rmsnorm_qmatmul_group_f32": (_c.c_int, [_VP, _c.POINTER(_VP), _c.c_int, _VP, _VP, _c.c_float, _I64,
                                                 _c.POINTER(_VP), _VP]),
    "lbq_rmsnorm_gate_up_silu_f32": (_c.c_int, [_VP, _VP, _VP, _VP, _VP, _c.c_float, _I64, _VP, _VP]),
    "lbq_act_create": (_c.c_int, [_VP, _U32, _I64, _I64, _c.POINTER(_VP)]),
    "lbq_act_quantize": (_c.c_int, [_VP, _VP, _VP]),
    "lbq_act_destroy": (_c.c_int, [_VP]),
    "lbq_qmatmul_act_f32": (_c.c_int, [_VP, _VP, _VP, _VP, _VP]),
    "lbq_dequantize_f32": (_c.c_int, [_VP, _VP, _VP, _VP]),
    "lbq_dequantize_blocks_f32": (_c.c_int, [_U32, _VP, _I64, _VP, _VP]),
    "lbq_embedding_f32": (_c.c_int, [_VP, _VP, _VP, _I64, _VP, _VP]),
    "lbq_quantize_act": (_c.c_int, [_U32, _VP, _I64, _I64, _VP, _VP]),
    "lbq_quantize_weights_f32": (_c.c_int, [_U32, _VP, _I64, _VP, _VP]),
    "lbq_gguf_open": (_c.c_int, [_c.c_char_p, _c.POINTER(_VP)]),
    "lbq_gguf_close": (_c.c_int, [_VP]),
    "lbq_gguf_header": (_c.c_int, [_VP, _c.POINTER(_U32), _c.POINTER(_I64), _c.POINTER(_I64), _c.POINTER(_c.c_uint64),
                                   _c.POINTER(_c.c_uint64), _c.POINTER(_c.c_uint64)]),
    "lbq_gguf_tensor_info": (_c.c_int, [_VP, _I64, _c.POINTER(_c.c_char_p), _c.POINTER(_U32), _c.POINTER(_U32),
                                        _c.POINTER(_c.c_uint64), _c.POINTER(_c.c_uint64)]),
    "lbq_gguf_find_tensor": (_c.c_int, [_VP, _c.c_char_p, _c.POINTER(_I64)]),
    "lbq_gguf_tensor_bytes": (_c.c_int, [_VP, _c.c_char_p, _c.POINTER(_VP), _c.POINTER(_SZ)]),
    "lbq_gguf_meta_key": (_c.c_int, [_VP, _I64, _c.POINTER(_c.c_char_p), _c.POINTER(_U32)]),
    "lbq_gguf_meta_int": (_c.c_int, [_VP, _c.c_char_p, _c.POINTER(_I64)]),
    "lbq_gguf_meta_float": (_c.c_int, [_VP, _c.c_char_p, _c.POINTER(_c.c_double)]),
    "lbq_gguf_meta_string": (_c.c_int, [_VP, _c.c_char_p, _c.POINTER(_VP), _c.POINTER(_SZ)]),
    "lbq_gguf_meta_array": (_c.c_int, [_VP, _c.c_char_p, _c.POINTER(_U32), _c.POINTER(_c.c_uint64)]),
    "lbq_gguf_copy_tensor": (_c.c_int, [_VP, _c.c_char_p, _VP, _SZ]),
    "lbq_weight_from_gguf": (_c.c_int, [_VP, _VP, _c.c_char_p, _c.POINTER(_VP)]),
}


class LbqError(RuntimeError):
    """A non-zero status from liblbq, with the library's own message."""

    def __init__(self, status: int, message: str):
        self.status = status
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")


_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first "
                "(python -m lightbulb_amd.build, or __graft_entry__.build())")
        # torch-ROCm bundles its own libamdhip64.so.7 / libhsa-runtime64.so.1.  If
        # liblbq.so were loaded first, the system runtime would be mapped and torch
        # would then map a second copy, and one of the two finds no device.  Loading
        # torch first makes liblbq bind (by soname) to the one runtime in the process.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != LBQ_OK:
        msg = lib().lbq_last_error()
        raise LbqError(status, msg.decode() if msg else "")
