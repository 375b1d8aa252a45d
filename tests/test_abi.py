"""The C ABI library loads, exports every symbol include/lbq.h declares, and rejects
bad arguments before touching a device (these run without a GPU)."""
import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def declared_functions() -> list[str]:
    text = (ROOT / "include" / "lbq.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lbq_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound(lbq):
    from lightbulb_amd import _lib
    names = declared_functions()
    assert len(names) >= 14
    for name in names:
        assert hasattr(lbq, name), name
    assert sorted(_lib.SIGNATURES) == names


def test_type_table_matches_reference(lbq):
    # GgmlDType::block_size / type_size, /root/reference/src/quantization/mod.rs:99-126
    # (Q2_K: the table's 82); lbq_type_block_bytes is the block in memory (Q2_K: 84)
    for t, bs, ts in [(0, 1, 4), (1, 1, 2), (2, 32, 18), (3, 32, 20), (6, 32, 22), (7, 32, 24), (8, 32, 34), (9, 32, 36),
                      (10, 256, 82), (11, 256, 110), (12, 256, 144), (13, 256, 176), (14, 256, 210), (15, 256, 292)]:
        assert lbq.lbq_type_block_size(t) == bs and lbq.lbq_type_size(t) == ts
        assert lbq.lbq_type_block_bytes(t) == (84 if t == 10 else ts)
    for t in (4, 5, 16, 29, 31, 999):
        assert lbq.lbq_type_block_size(t) == 0 and lbq.lbq_type_size(t) == 0 and lbq.lbq_type_block_bytes(t) == 0


def test_bf16_is_served(lbq):
    # candle's GgmlDType::BF16 (GGUF id 30), which QMatMul::from_qtensor serves as
    # its dense variant: one 2-byte value per block; the weight path accepts it
    # (lbq_dequantize_blocks_f32 checks the type before the size: an unknown id
    # gives -2, a served one with a bad size -3)
    from lightbulb_amd.quantized import SERVED, GgmlDType
    assert lbq.lbq_type_block_size(30) == 1 and lbq.lbq_type_size(30) == 2 and lbq.lbq_type_block_bytes(30) == 2
    assert GgmlDType.BF16 == 30 and GgmlDType.BF16 in SERVED and GgmlDType.BF16.is_dense()
    assert GgmlDType.from_u32(30) is None  # the reference's own from_u32 does not know it
    dummy = ctypes.c_void_p(256)
    assert lbq.lbq_dequantize_blocks_f32(29, dummy, -1, dummy, None) == -2
    assert lbq.lbq_dequantize_blocks_f32(30, dummy, -1, dummy, None) == -3


def test_argument_errors_without_device(lbq):
    # unsupported types, bad shapes and null pointers are refused before any HIP call
    dummy = ctypes.c_void_p(256)
    assert lbq.lbq_quantize_act(12, dummy, 1, 256, dummy, None) == -2
    assert lbq.lbq_quantize_act(15, dummy, 1, 255, dummy, None) == -3
    assert lbq.lbq_quantize_act(15, None, 1, 256, dummy, None) == -1
    assert lbq.lbq_dequantize_blocks_f32(4, dummy, 256, dummy, None) == -2
    assert lbq.lbq_embedding_f32(None, None, dummy, 1, dummy, None) == -1
    assert lbq.lbq_dequantize_blocks_f32(11, dummy, 300, dummy, None) == -3
    assert lbq.lbq_quantize_weights_f32(10, dummy, 256, dummy, None) == -2  # no Q2_K quantiser
    assert lbq.lbq_dequantize_blocks_f32(2, dummy, 48, dummy, None) == -3
    assert lbq.lbq_quantize_act(9, dummy, 1, 48, dummy, None) == -3
    assert lbq.lbq_quantize_weights_f32(9, dummy, 32, dummy, None) == -2
    assert lbq.lbq_dequantize_blocks_f32(12, dummy, 100, dummy, None) == -3
    assert lbq.lbq_quantize_weights_f32(15, dummy, 256, dummy, None) == -2
    assert lbq.lbq_quantize_weights_f32(14, dummy, 300, dummy, None) == -3
    assert lbq.lbq_qmatmul_f32(None, None, None, 1, None, None) == -1
    assert lbq.lbq_weight_create(None, 12, 1, 256, None, 144, ctypes.byref(ctypes.c_void_p())) == -1
    msg = lbq.lbq_last_error()
    assert msg and b"null" in msg
    assert lbq.lbq_init(0, None) == -1
    assert lbq.lbq_weight_destroy(None) == 0 and lbq.lbq_ctx_destroy(None) == 0


def test_product_does_not_import_oracle():
    # the product path must never route through the test oracle
    for p in (ROOT / "lightbulb_amd").rglob("*"):
        if p.suffix in (".py", ".cpp", ".hip", ".hpp", ".h"):
            src = p.read_text()
            assert "import oracle" not in src and "from oracle" not in src and "lbq_oracle" not in src, p


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from lightbulb_amd import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    monkeypatch.setattr(_lib, "_lib", None)
    try:
        _lib.lib()
    except RuntimeError as e:
        assert "missing" in str(e)
    else:
        raise AssertionError("no error without the library")
