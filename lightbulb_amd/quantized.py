"""Host-side mirror of the reference's quantized-linear surface, over liblbq.

The reference (Rust) serves every GGUF projection through these types:

* ``GgmlDType``          -- /root/reference/src/quantization/mod.rs:58-147
* ``QTensor`` / ``QMatMul`` (candle-core 0.10.2, external) -- built at
  src/model/custom_attention.rs:195-206, mlp_wrapper.rs:127-135 and
  custom_transformer.rs:360-363; ``forward`` called at custom_attention.rs:265-267,
  :671, mlp_wrapper.rs:190-195 and custom_transformer.rs:625
* ``QuantizableLinear``  -- src/model/quantizable_linear.rs:36-70
* ``dequantize_tensor`` / ``quantize_tensor`` -- src/quantization/mod.rs:158-327

Same names, same argument meaning, same failure cases (raised as exceptions
where Rust returns ``Err``).  The arithmetic runs in liblbq's HIP kernels on the
GPU; torch only provides device memory and the current stream.  There is no
CPU fallback: without the built library or a GPU these raise.
"""
from __future__ import annotations

import ctypes
import threading
from enum import IntEnum

import numpy as np
import torch

from . import _lib


class GgmlDType(IntEnum):
    """GGML quantisation type ids (GGUF ``ggml_type``).

    The reference's table (src/quantization/mod.rs:60-77) plus ``BF16 = 30``:
    candle-core's GgmlDType carries it, so a BF16 tensor reaches
    ``QMatMul::from_qtensor`` through candle's GGUF reader
    (custom_transformer.rs:358-363) and is served as the dense variant.
    ``from_u32`` keeps the reference's own table (it returns None for 30).
    """

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q8_1 = 9
    Q2K = 10
    Q3K = 11
    Q4K = 12
    Q5K = 13
    Q6K = 14
    Q8K = 15
    BF16 = 30

    @classmethod
    def from_u32(cls, value: int) -> "GgmlDType | None":
        """The reference's ``GgmlDType::from_u32`` (mod.rs:80-97): ids of its table only."""
        if value == cls.BF16:
            return None
        try:
            return cls(value)
        except ValueError:
            return None

    def is_dense(self) -> bool:
        """F32 / F16 / BF16: candle's dense QMatMul variant (an f32 matmul)."""
        return self in (GgmlDType.F32, GgmlDType.F16, GgmlDType.BF16)

    def block_size(self) -> int:
        if self.is_dense():
            return 1
        if self in (GgmlDType.Q4_0, GgmlDType.Q4_1, GgmlDType.Q5_0, GgmlDType.Q5_1, GgmlDType.Q8_0, GgmlDType.Q8_1):
            return 32
        return 256

    def type_size(self) -> int:
        return {
            GgmlDType.F32: 4, GgmlDType.F16: 2, GgmlDType.Q4_0: 18, GgmlDType.Q4_1: 20, GgmlDType.Q5_0: 22,
            GgmlDType.Q5_1: 24, GgmlDType.Q8_0: 34, GgmlDType.Q8_1: 36, GgmlDType.Q2K: 82, GgmlDType.Q3K: 110,
            GgmlDType.Q4K: 144, GgmlDType.Q5K: 176, GgmlDType.Q6K: 210, GgmlDType.Q8K: 292, GgmlDType.BF16: 2,
        }[self]

    def block_bytes(self) -> int:
        """Bytes of one block as the kernels (and candle) lay it out.  Equal to
        ``type_size`` except for Q2_K: the reference's table gives 82, the block
        (scales[16], qs[64], d, dmin) is 84."""
        return 84 if self == GgmlDType.Q2K else self.type_size()

    def type_name(self) -> str:
        """Human-readable name as the reference prints it (``GgmlDType::name``)."""
        return {
            GgmlDType.Q2K: "Q2_K", GgmlDType.Q3K: "Q3_K", GgmlDType.Q4K: "Q4_K", GgmlDType.Q5K: "Q5_K",
            GgmlDType.Q6K: "Q6_K", GgmlDType.Q8K: "Q8_K",
        }.get(self, self.name)


#: weight types the GPU path serves; the others are rejected with LBQ_ERR_UNSUPPORTED_TYPE.
#: F32 / F16 / BF16 are candle's dense QMatMul variant (an f32 matmul, no activation quantisation).
SERVED = (GgmlDType.F32, GgmlDType.F16, GgmlDType.BF16, GgmlDType.Q4_0, GgmlDType.Q4_1, GgmlDType.Q5_0, GgmlDType.Q5_1,
          GgmlDType.Q8_0, GgmlDType.Q2K, GgmlDType.Q3K, GgmlDType.Q4K, GgmlDType.Q5K, GgmlDType.Q6K)

#: weight types quantize_tensor can produce (no Q2_K / Q3_K quantiser; dense types are not quantised)
QUANTIZABLE = tuple(t for t in SERVED if t not in (GgmlDType.Q2K, GgmlDType.Q3K) and not t.is_dense())

#: activation-only block types (the vec-dot partners)
ACT_TYPES = (GgmlDType.Q8_0, GgmlDType.Q8_1, GgmlDType.Q8K)


def vec_dot_type(dtype: GgmlDType) -> GgmlDType:
    """The activation block type QMatMul::forward quantises x to for a weight type
    (candle GgmlType::VecDotType): Q8_K for k-quants, Q8_1 for Q4_1/Q5_1, else Q8_0."""
    dtype = GgmlDType(dtype)
    if dtype in (GgmlDType.Q2K, GgmlDType.Q3K, GgmlDType.Q4K, GgmlDType.Q5K, GgmlDType.Q6K):
        return GgmlDType.Q8K
    if dtype in (GgmlDType.Q4_1, GgmlDType.Q5_1):
        return GgmlDType.Q8_1
    return GgmlDType.Q8_0


# ---------------------------------------------------------------------------
# contexts: one liblbq context per device, created on first use
# ---------------------------------------------------------------------------
_ctx_lock = threading.Lock()
_ctxs: dict[int, int] = {}


def _device_index(device) -> int:
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"the quantized path runs on the GPU; got device {dev}")
    return dev.index if dev.index is not None else torch.cuda.current_device()


def context(device="cuda") -> int:
    idx = _device_index(device)
    with _ctx_lock:
        if idx not in _ctxs:
            out = ctypes.c_void_p()
            _lib.check(_lib.lib().lbq_init(idx, ctypes.byref(out)))
            _ctxs[idx] = out.value
        return _ctxs[idx]


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(torch.device(device)).cuda_stream)


# ---------------------------------------------------------------------------
# QTensor: GGUF blocks resident in HBM, in their on-disk layout
# ---------------------------------------------------------------------------
class QTensor:
    """Quantised tensor of shape (n, k): n rows of k/block_size GGUF blocks.

    ``data`` is a flat uint8 device tensor holding the blocks unchanged.  The
    shape is candle's (n, k) order; a GGUF tensor-info lists it as ne0 = k,
    ne1 = n (/root/reference/src/gguf/parser.rs:180-199).
    """

    def __init__(self, data: torch.Tensor, dtype: GgmlDType, shape: tuple[int, int]):
        dtype = GgmlDType(dtype)
        n, k = (int(s) for s in shape)
        if data.dtype != torch.uint8 or data.dim() != 1 or not data.is_contiguous():
            raise ValueError("QTensor data must be a contiguous 1-D uint8 tensor")
        if k % dtype.block_size():
            raise ValueError(f"{dtype.type_name()}: k = {k} is not a multiple of {dtype.block_size()}")
        need = n * (k // dtype.block_size()) * dtype.block_bytes()
        if data.numel() != need:
            raise ValueError(f"{dtype.type_name()}: {data.numel()} bytes for shape ({n}, {k}), expected {need}")
        self.data = data
        self._dtype = dtype
        self._shape = (n, k)

    @classmethod
    def from_bytes(cls, raw, dtype: GgmlDType, shape: tuple[int, int], device="cuda") -> "QTensor":
        """Upload raw GGUF block bytes (bytes / numpy uint8) to the device unchanged."""
        host = torch.from_numpy(np.frombuffer(bytes(raw), dtype=np.uint8).copy()) if not isinstance(
            raw, np.ndarray) else torch.from_numpy(np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1))
        return cls(host.to(device), dtype, shape)

    @classmethod
    def quantize(cls, w: torch.Tensor, dtype: GgmlDType) -> "QTensor":
        """Quantise an f32 [n, k] device tensor to ``dtype`` blocks on the device."""
        if w.dim() != 2:
            raise ValueError("QTensor.quantize expects a 2-D (n, k) tensor")
        n, k = w.shape
        blocks = quantize_tensor(w.reshape(-1), dtype, _exact=True)
        return cls(blocks, dtype, (n, k))

    def dtype(self) -> GgmlDType:
        return self._dtype

    def shape(self) -> tuple[int, int]:
        return self._shape

    def storage_size_in_bytes(self) -> int:
        return self.data.numel()

    def dequantize(self) -> torch.Tensor:
        """f32 [n, k], bit-exact with the reference's dequantisation."""
        n, k = self._shape
        return dequantize_tensor(self.data, self._dtype, n * k).reshape(n, k)

    def __repr__(self) -> str:
        return f"QTensor({self._dtype.type_name()}, shape={self._shape}, device={self.data.device})"


# ---------------------------------------------------------------------------
# QMatMul
# ---------------------------------------------------------------------------
class QMatMul:
    """``QMatMul::from_qtensor`` + ``Module::forward`` over liblbq."""

    def __init__(self, qtensor: QTensor, _handle: int, _ctx: int):
        self._qt = qtensor
        self._handle = _handle
        self._ctx = _ctx

    @classmethod
    def from_qtensor(cls, qtensor: QTensor) -> "QMatMul":
        dt = qtensor.dtype()
        if dt not in SERVED:
            raise ValueError(f"quantized matmul for {dt.type_name()} is not served by the GPU path")
        n, k = qtensor.shape()
        ctx = context(qtensor.data.device)
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().lbq_weight_wrap_device(ctx, int(dt), n, k, qtensor.data.data_ptr(),
                                                     qtensor.data.numel(), ctypes.byref(h)))
        return cls(qtensor, h.value, ctx)

    def qtensor(self) -> QTensor:
        return self._qt

    def forward(self, xs: torch.Tensor) -> torch.Tensor:
        n, k = self._qt.shape()
        if xs.dtype != torch.float32:
            raise ValueError(f"the lhs for quantized matmul must be f32, got {xs.dtype}")
        if xs.dim() < 2:
            raise ValueError(f"input tensor has only one dimension {tuple(xs.shape)}")
        if xs.shape[-1] != k:
            raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with {(n, k)}")
        if not xs.is_contiguous():
            raise ValueError(f"input tensor is not contiguous {tuple(xs.shape)}")
        if xs.device != self._qt.data.device:
            raise ValueError(f"input on {xs.device}, weights on {self._qt.data.device}")
        m = xs.numel() // k
        y = torch.empty(*xs.shape[:-1], n, dtype=torch.float32, device=xs.device)
        if m:
            _lib.check(_lib.lib().lbq_qmatmul_f32(self._ctx, self._handle, xs.data_ptr(), m, y.data_ptr(),
                                                  _stream(xs.device)))
        return y

    __call__ = forward

    def forward_quantized(self, act: "QActivation", out: torch.Tensor | None = None) -> torch.Tensor:
        """The dot half of ``forward`` on an activation quantised once by ``QActivation``."""
        n, k = self._qt.shape()
        if act.k != k:
            raise ValueError(f"activation k = {act.k} incompatible with {(n, k)}")
        if out is None:
            out = torch.empty(act.m, n, dtype=torch.float32, device=self._qt.data.device)
        elif out.dtype != torch.float32 or not out.is_contiguous() or out.numel() != act.m * n:
            raise ValueError("out must be a contiguous f32 tensor of m*n values")
        _lib.check(_lib.lib().lbq_qmatmul_act_f32(self._ctx, self._handle, act._handle, out.data_ptr(),
                                                  _stream(out.device)))
        return out

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h:
            try:
                _lib.lib().lbq_weight_destroy(h)
            except Exception:
                pass
            self._handle = None

    def __repr__(self) -> str:
        return f"QMatMul({self._qt!r})"


GROUP_MAX = 4  # LBQ_GROUP_MAX


def qmatmul_group(qmatmuls, xs: torch.Tensor) -> list[torch.Tensor]:
    """``[q.forward(xs) for q in qmatmuls]`` in one call: the runs of
    ``QMatMul::forward`` on one input at the q/k/v projections
    (src/model/custom_attention.rs:265-267) and gate/up (src/model/mlp_wrapper.rs:190,193).
    x is quantised once and, at m = 1, all weights stream in one launch; the
    outputs are bit-identical to separate ``forward`` calls.  The weights must
    share the ggml type and k."""
    qmatmuls = list(qmatmuls)
    if not 1 <= len(qmatmuls) <= GROUP_MAX:
        raise ValueError(f"between 1 and {GROUP_MAX} weights per group, got {len(qmatmuls)}")
    q0 = qmatmuls[0]
    n0, k = q0.qtensor().shape()
    for q in qmatmuls[1:]:
        if q.qtensor().dtype() != q0.qtensor().dtype() or q.qtensor().shape()[1] != k:
            raise ValueError("grouped weights must share the ggml type and k")
    if xs.dtype != torch.float32:
        raise ValueError(f"the lhs for quantized matmul must be f32, got {xs.dtype}")
    if xs.dim() < 2:
        raise ValueError(f"input tensor has only one dimension {tuple(xs.shape)}")
    if xs.shape[-1] != k:
        raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with {(n0, k)}")
    if not xs.is_contiguous():
        raise ValueError(f"input tensor is not contiguous {tuple(xs.shape)}")
    m = xs.numel() // k
    ys = [torch.empty(*xs.shape[:-1], q.qtensor().shape()[0], dtype=torch.float32, device=xs.device)
          for q in qmatmuls]
    if m:
        cnt = len(qmatmuls)
        hs = (ctypes.c_void_p * cnt)(*[q._handle for q in qmatmuls])
        outs = (ctypes.c_void_p * cnt)(*[y.data_ptr() for y in ys])
        _lib.check(_lib.lib().lbq_qmatmul_group_f32(q0._ctx, hs, cnt, xs.data_ptr(), m, outs, _stream(xs.device)))
    return ys


def gate_up_silu(gate: "QMatMul", up: "QMatMul", xs: torch.Tensor) -> torch.Tensor:
    """``silu(gate.forward(xs)) * up.forward(xs)`` -- the gate/up half of the
    reference's MLP forward (src/model/mlp_wrapper.rs:190-194) -- in one call
    (one launch at m = 1).  gate and up share the ggml type, n and k."""
    (n, k), (nu, ku) = gate.qtensor().shape(), up.qtensor().shape()
    if gate.qtensor().dtype() != up.qtensor().dtype() or (n, k) != (nu, ku):
        raise ValueError("gate and up must share the ggml type and shape")
    if xs.dtype != torch.float32:
        raise ValueError(f"the lhs for quantized matmul must be f32, got {xs.dtype}")
    if xs.dim() < 2:
        raise ValueError(f"input tensor has only one dimension {tuple(xs.shape)}")
    if xs.shape[-1] != k:
        raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with {(n, k)}")
    if not xs.is_contiguous():
        raise ValueError(f"input tensor is not contiguous {tuple(xs.shape)}")
    m = xs.numel() // k
    out = torch.empty(*xs.shape[:-1], n, dtype=torch.float32, device=xs.device)
    if m:
        _lib.check(_lib.lib().lbq_gate_up_silu_f32(gate._ctx, gate._handle, up._handle, xs.data_ptr(), m,
                                                   out.data_ptr(), _stream(xs.device)))
    return out


def _check_norm(xs: torch.Tensor, weight: torch.Tensor, k: int):
    if weight.dtype != torch.float32 or not weight.is_contiguous() or weight.numel() != k:
        raise ValueError(f"the norm weight must be a contiguous f32 tensor of {k} values")
    if weight.device != xs.device:
        raise ValueError(f"norm weight on {weight.device}, input on {xs.device}")


def rms_norm(xs: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """candle's ``RmsNorm`` in f32: ``x / sqrt(mean(x^2) + eps) * weight`` over the last dim."""
    if xs.dtype != torch.float32 or not xs.is_contiguous():
        raise ValueError("rms_norm takes a contiguous f32 tensor")
    k = xs.shape[-1]
    _check_norm(xs, weight, k)
    y = torch.empty_like(xs)
    m = xs.numel() // k
    if m:
        _lib.check(_lib.lib().lbq_rmsnorm_f32(xs.data_ptr(), weight.data_ptr(), float(eps), m, k, y.data_ptr(),
                                              _stream(xs.device)))
    return y


def rmsnorm_qmatmul_group(qmatmuls, xs: torch.Tensor, weight: torch.Tensor, eps: float) -> list[torch.Tensor]:
    """``qmatmul_group(qmatmuls, rms_norm(xs, weight, eps))`` -- the input norm
    and the q/k/v projections that read it in one call (one launch at m = 1)."""
    qmatmuls = list(qmatmuls)
    if not 1 <= len(qmatmuls) <= GROUP_MAX:
        raise ValueError(f"between 1 and {GROUP_MAX} weights per group, got {len(qmatmuls)}")
    k = qmatmuls[0].qtensor().shape()[1]
    if xs.dtype != torch.float32 or not xs.is_contiguous() or xs.shape[-1] != k:
        raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with k = {k}")
    _check_norm(xs, weight, k)
    m = xs.numel() // k
    ys = [torch.empty(*xs.shape[:-1], q.qtensor().shape()[0], dtype=torch.float32, device=xs.device) for q in qmatmuls]
    if m:
        cnt = len(qmatmuls)
        hs = (ctypes.c_void_p * cnt)(*[q._handle for q in qmatmuls])
        outs = (ctypes.c_void_p * cnt)(*[y.data_ptr() for y in ys])
        _lib.check(_lib.lib().lbq_rmsnorm_qmatmul_group_f32(qmatmuls[0]._ctx, hs, cnt, xs.data_ptr(), weight.data_ptr(),
                                                            float(eps), m, outs, _stream(xs.device)))
    return ys


def rmsnorm_gate_up_silu(gate: "QMatMul", up: "QMatMul", xs: torch.Tensor, weight: torch.Tensor,
                         eps: float) -> torch.Tensor:
    """``gate_up_silu(gate, up, rms_norm(xs, weight, eps))`` in one call."""
    n, k = gate.qtensor().shape()
    if gate.qtensor().dtype() != up.qtensor().dtype() or up.qtensor().shape() != (n, k):
        raise ValueError("gate and up must share the ggml type and shape")
    if xs.dtype != torch.float32 or not xs.is_contiguous() or xs.shape[-1] != k:
        raise ValueError(f"input tensor {tuple(xs.shape)} incompatible with k = {k}")
    _check_norm(xs, weight, k)
    m = xs.numel() // k
    out = torch.empty(*xs.shape[:-1], n, dtype=torch.float32, device=xs.device)
    if m:
        _lib.check(_lib.lib().lbq_rmsnorm_gate_up_silu_f32(gate._ctx, gate._handle, up._handle, xs.data_ptr(),
                                                           weight.data_ptr(), float(eps), m, out.data_ptr(),
                                                           _stream(xs.device)))
    return out


class Mlp:
    """``Mlp`` (src/model/mlp_wrapper.rs): ``down_proj(silu(gate_proj(x)) * up_proj(x))``
    over ``QuantizableLinear`` projections; quantized gate/up pairs take the fused
    ``gate_up_silu`` path."""

    def __init__(self, gate_proj: "QuantizableLinear", up_proj: "QuantizableLinear", down_proj: "QuantizableLinear"):
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj

    def forward(self, xs: torch.Tensor) -> torch.Tensor:
        g, u = self.gate_proj, self.up_proj
        if (g.is_quantized() and u.is_quantized() and g.inner.qtensor().dtype() == u.inner.qtensor().dtype()
                and g.inner.qtensor().shape() == u.inner.qtensor().shape()):
            h = gate_up_silu(g.inner, u.inner, xs)
        else:
            h = torch.nn.functional.silu(g.forward(xs)) * u.forward(xs)
        return self.down_proj.forward(h)

    __call__ = forward


class QActivation:
    """x [m, k] quantised once to the weights' vec-dot type (``vec_dot_type``),
    reusable by every QMatMul that reads the same x -- q/k/v and gate/up."""

    def __init__(self, act_type: GgmlDType, m: int, k: int, device="cuda"):
        self.act_type = GgmlDType(act_type)
        self.m, self.k = int(m), int(k)
        self.device = torch.device(device)
        h = ctypes.c_void_p()
        _lib.check(_lib.lib().lbq_act_create(context(self.device), int(self.act_type), self.m, self.k,
                                             ctypes.byref(h)))
        self._handle = h.value

    @classmethod
    def for_weight(cls, qmatmul: "QMatMul", m: int) -> "QActivation":
        t = vec_dot_type(qmatmul.qtensor().dtype())
        return cls(t, m, qmatmul.qtensor().shape()[1], qmatmul.qtensor().data.device)

    def quantize(self, x: torch.Tensor) -> "QActivation":
        if x.dtype != torch.float32 or not x.is_contiguous() or x.numel() != self.m * self.k:
            raise ValueError(f"x must be a contiguous f32 tensor of {self.m}x{self.k} values")
        _lib.check(_lib.lib().lbq_act_quantize(self._handle, x.data_ptr(), _stream(x.device)))
        return self

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h:
            try:
                _lib.lib().lbq_act_destroy(h)
            except Exception:
                pass
            self._handle = None


# ---------------------------------------------------------------------------
# token embedding straight from the quantized table
# ---------------------------------------------------------------------------
class QEmbedding:
    """``Embedding::new(qtensor.dequantize(), hidden)`` then ``forward(ids)``
    (/root/reference/src/model/custom_transformer.rs:321-323) without the dense
    table: each call dequantises only the rows it gathers, bit-identical to
    index_select on the dequantised weight.  Ids outside [0, n) give NaN rows."""

    def __init__(self, qtensor: QTensor):
        self._qmatmul = QMatMul.from_qtensor(qtensor)
        self.num_embeddings, self.hidden_size = qtensor.shape()

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        dev = self._qmatmul.qtensor().data.device
        flat = ids.reshape(-1).to(device=dev, dtype=torch.int32).contiguous()
        out = torch.empty(flat.numel(), self.hidden_size, dtype=torch.float32, device=dev)
        _lib.check(_lib.lib().lbq_embedding_f32(context(dev), self._qmatmul._handle, flat.data_ptr(), flat.numel(),
                                                out.data_ptr(), _stream(dev)))
        return out.reshape(*ids.shape, self.hidden_size)

    __call__ = forward


# ---------------------------------------------------------------------------
# QuantizableLinear (src/model/quantizable_linear.rs)
# ---------------------------------------------------------------------------
class QuantizableLinear:
    """Either ``Regular`` (dense f32 weight [n, k], optional bias) or ``Quantized(QMatMul)``."""

    def __init__(self, kind: str, inner):
        self.kind = kind
        self.inner = inner

    @classmethod
    def from_linear(cls, weight: torch.Tensor, bias: torch.Tensor | None = None) -> "QuantizableLinear":
        return cls("Regular", (weight, bias))

    @classmethod
    def from_qmatmul(cls, qmatmul: QMatMul) -> "QuantizableLinear":
        return cls("Quantized", qmatmul)

    def is_quantized(self) -> bool:
        return self.kind == "Quantized"

    def forward(self, xs: torch.Tensor) -> torch.Tensor:
        if self.kind == "Quantized":
            return self.inner.forward(xs)
        w, b = self.inner
        y = xs.matmul(w.t())
        return y + b if b is not None else y

    __call__ = forward


# ---------------------------------------------------------------------------
# dequantize_tensor / quantize_tensor (src/quantization/mod.rs:158-327)
# ---------------------------------------------------------------------------
def dequantize_tensor(data: torch.Tensor, dtype: GgmlDType, elem_count: int) -> torch.Tensor:
    """Raw device blocks -> f32 [elem_count]; blocks beyond elem_count are cut off.
    Errors name the type as the reference's ``{:?}`` does (the variant: ``Q4K``)."""
    dtype = GgmlDType(dtype)
    if dtype not in SERVED and dtype not in ACT_TYPES:
        raise ValueError(f"Dequantization for {dtype.name} not yet implemented")
    bs, ts = dtype.block_size(), dtype.block_bytes()
    num_blocks = (elem_count + bs - 1) // bs
    expected = num_blocks * ts
    if data.numel() < expected:
        raise ValueError(f"Insufficient data for {dtype.name}: got {data.numel()} bytes, "
                         f"need {expected} bytes")
    out = torch.empty(num_blocks * bs, dtype=torch.float32, device=data.device)
    if num_blocks:
        _lib.check(_lib.lib().lbq_dequantize_blocks_f32(int(dtype), data.data_ptr(), num_blocks * bs,
                                                        out.data_ptr(), _stream(data.device)))
    return out[:elem_count]


def quantize_tensor(data: torch.Tensor, dtype: GgmlDType, _exact: bool = False) -> torch.Tensor:
    """f32 device values -> GGUF blocks (uint8); the last block is zero-padded."""
    dtype = GgmlDType(dtype)
    if dtype not in QUANTIZABLE:
        raise ValueError(f"Quantization for {dtype.name} not yet implemented")
    if data.dtype != torch.float32:
        raise ValueError("quantize_tensor expects f32 values")
    flat = data.reshape(-1)
    bs = dtype.block_size()
    num_blocks = (flat.numel() + bs - 1) // bs
    if num_blocks * bs != flat.numel():
        if _exact:
            raise ValueError(f"{flat.numel()} values are not a whole number of {bs}-value blocks")
        padded = torch.zeros(num_blocks * bs, dtype=torch.float32, device=flat.device)
        padded[:flat.numel()] = flat
        flat = padded
    flat = flat.contiguous()
    out = torch.empty(num_blocks * dtype.block_bytes(), dtype=torch.uint8, device=flat.device)
    if num_blocks:
        _lib.check(_lib.lib().lbq_quantize_weights_f32(int(dtype), flat.data_ptr(), flat.numel(), out.data_ptr(),
                                                       _stream(flat.device)))
    return out


def quantize_activations(x: torch.Tensor, act_type: GgmlDType) -> torch.Tensor:
    """The activation step of QMatMul::forward on its own: x f32 [m, k] -> Q8_K / Q8_0 / Q8_1 blocks (uint8)."""
    act_type = GgmlDType(act_type)
    if act_type not in ACT_TYPES:
        raise ValueError("activations quantise to Q8_K, Q8_0 or Q8_1")
    x = x.contiguous()
    k = x.shape[-1]
    m = x.numel() // k
    out = torch.empty(m, k // act_type.block_size() * act_type.type_size(), dtype=torch.uint8, device=x.device)
    if m:
        _lib.check(_lib.lib().lbq_quantize_act(int(act_type), x.data_ptr(), m, k, out.data_ptr(), _stream(x.device)))
    return out
