"""GGUF container access and the direct GGUF -> device weight path.

Mirrors the reference's Lightning loader (src/gguf/mod.rs ``Content``,
src/gguf/parser.rs ``parse_gguf``, src/quantization/gguf_ops.rs
``extract_tensor_bytes``) over the C ABI in liblbq (``lbq_gguf_*``): the file is
mapped read-only, parsed with every read bounds-checked, and a tensor's bytes
go to the device through pinned staging.
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple

import numpy as np
import torch

from . import _lib
from .quantized import GgmlDType, QTensor


class TensorInfo(NamedTuple):
    """``TensorInfo`` (src/gguf/parser.rs:103-109); dimensions list ne0 (= k) first."""
    name: str
    dimensions: tuple
    tensor_type: int
    offset: int


class Content:
    """``Content::read`` + accessors (src/gguf/mod.rs:62-252)."""

    def __init__(self, handle: int, path: str):
        self._h = handle
        self.path = path
        L = _lib.lib()
        ver, nt, nm = ctypes.c_uint32(), ctypes.c_int64(), ctypes.c_int64()
        al, off, size = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _lib.check(L.lbq_gguf_header(handle, ctypes.byref(ver), ctypes.byref(nt), ctypes.byref(nm), ctypes.byref(al),
                                     ctypes.byref(off), ctypes.byref(size)))
        self.version, self.tensor_count, self.metadata_count = ver.value, nt.value, nm.value
        self.alignment, self.tensor_data_offset, self.file_size = al.value, off.value, size.value

    @classmethod
    def read(cls, path) -> "Content":
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().lbq_gguf_open(str(path).encode(), ctypes.byref(h)))
        return cls(h.value, str(path))

    def tensor_infos(self) -> list[TensorInfo]:
        L = _lib.lib()
        out = []
        for i in range(self.tensor_count):
            name, t, nd, off = ctypes.c_char_p(), ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
            dims = (ctypes.c_uint64 * 8)()
            _lib.check(L.lbq_gguf_tensor_info(self._h, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd), dims,
                                              ctypes.byref(off)))
            out.append(TensorInfo(name.value.decode(), tuple(dims[d] for d in range(nd.value)), t.value, off.value))
        return out

    def metadata_keys(self) -> list[tuple[str, int]]:
        L = _lib.lib()
        out = []
        for i in range(self.metadata_count):
            key, t = ctypes.c_char_p(), ctypes.c_uint32()
            _lib.check(L.lbq_gguf_meta_key(self._h, i, ctypes.byref(key), ctypes.byref(t)))
            out.append((key.value.decode(), t.value))
        return out

    def meta_int(self, key: str) -> int:
        v = ctypes.c_int64()
        _lib.check(_lib.lib().lbq_gguf_meta_int(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_float(self, key: str) -> float:
        v = ctypes.c_double()
        _lib.check(_lib.lib().lbq_gguf_meta_float(self._h, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_str(self, key: str) -> str:
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        _lib.check(_lib.lib().lbq_gguf_meta_string(self._h, key.encode(), ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value).decode() if n.value else ""

    def meta_array(self, key: str) -> tuple[int, int]:
        t, n = ctypes.c_uint32(), ctypes.c_uint64()
        _lib.check(_lib.lib().lbq_gguf_meta_array(self._h, key.encode(), ctypes.byref(t), ctypes.byref(n)))
        return t.value, n.value

    def get_tensor_data(self, name: str) -> np.ndarray:
        """The tensor's bytes (``extract_tensor_bytes``): a read-only uint8 view of
        the mapping, valid while this Content is open."""
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        _lib.check(_lib.lib().lbq_gguf_tensor_bytes(self._h, name.encode(), ctypes.byref(p), ctypes.byref(n)))
        if not n.value:
            return np.zeros(0, dtype=np.uint8)
        arr = np.ctypeslib.as_array((ctypes.c_uint8 * n.value).from_address(p.value))
        arr.flags.writeable = False
        return arr

    def tensor(self, name: str, device="cuda") -> QTensor:
        """A 2-D quantized weight on the device (``Content::tensor``): shape (n, k)
        from dims (k, n), bytes copied through pinned staging."""
        info = next((t for t in self.tensor_infos() if t.name == name), None)
        if info is None:
            raise ValueError(f"Tensor '{name}' not found in GGUF file")
        if len(info.dimensions) != 2:
            raise ValueError(f"tensor {name} has {len(info.dimensions)} dimensions, a weight has 2")
        dt = GgmlDType(info.tensor_type)
        numel = int(np.prod(info.dimensions, dtype=np.uint64))
        nbytes = -(-numel // dt.block_size()) * dt.block_bytes()  # the blocks lbq_gguf_copy_tensor copies
        data = torch.empty(nbytes, dtype=torch.uint8, device=device)
        if nbytes:
            _lib.check(_lib.lib().lbq_gguf_copy_tensor(self._h, name.encode(), data.data_ptr(), nbytes))
        k, n = info.dimensions
        return QTensor(data, dt, (n, k))

    def close(self):
        h = getattr(self, "_h", None)
        if h:
            _lib.lib().lbq_gguf_close(h)
            self._h = None

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
