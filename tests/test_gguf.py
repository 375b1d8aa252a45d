"""GGUF container parsing through the C ABI (host only: no device needed).

The expected values come from an independent writer (tests/gguf_writer.py) and
from the reference's own parser tests (src/gguf/parser.rs:352-386: the alignment
rule, little-endian u32/u64, u64-length strings) and error messages
(parser.rs:140-157, 293-309)."""
import ctypes
import struct

import numpy as np
import pytest

import gguf_writer as gw

pytestmark = pytest.mark.filterwarnings("ignore")


@pytest.fixture(scope="module")
def L():
    from lightbulb_amd import _lib
    return _lib.lib()


def open_raw(L, path):
    h = ctypes.c_void_p()
    rc = L.lbq_gguf_open(str(path).encode(), ctypes.byref(h))
    return rc, h.value, L.lbq_last_error().decode()


def write(tmp_path, blob, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    return p


KVS = [("general.architecture", gw.STR, "llama"), ("u8", gw.U8, 200), ("i8", gw.I8, -5), ("u16", gw.U16, 65000),
       ("i16", gw.I16, -30000), ("u32", gw.U32, 4000000000), ("i32", gw.I32, -2000000000), ("f32", gw.F32, 0.25),
       ("flag", gw.BOOL, 1), ("u64", gw.U64, 2 ** 40 + 3), ("i64", gw.I64, -(2 ** 40)), ("f64", gw.F64, -1.5),
       ("tokens", gw.ARR, (gw.STR, ["<s>", "</s>", "hi"])), ("ids", gw.ARR, (gw.U32, [1, 2, 3, 4])),
       ("empty", gw.STR, "")]


def test_header_metadata_tensors(tmp_path):
    from lightbulb_amd.gguf import Content
    rng = np.random.default_rng(1)
    norm = rng.standard_normal(64).astype(np.float32).tobytes()
    q4 = rng.integers(0, 256, 8 * 2 * 144, dtype=np.uint8).tobytes()       # 8 rows x 512 (2 blocks)
    q8 = rng.integers(0, 256, 3 * 34, dtype=np.uint8).tobytes()            # 70 values -> 3 blocks (ceil)
    blob, data_off, offs = gw.build(KVS, [("norm", [64], 0, norm), ("blk.0.w", [512, 8], 12, q4),
                                          ("odd", [70], 8, q8)])
    with Content.read(write(tmp_path, blob)) as c:
        assert (c.version, c.tensor_count, c.metadata_count, c.alignment) == (3, 3, len(KVS), 32)
        assert c.tensor_data_offset == data_off and data_off % 32 == 0 and c.file_size == len(blob)
        assert [k for k, _ in c.metadata_keys()] == [k for k, _, _ in KVS]
        assert [t for _, t in c.metadata_keys()] == [t for _, t, _ in KVS]
        for key, t, v in KVS:
            if t in (gw.U8, gw.I8, gw.U16, gw.I16, gw.U32, gw.I32, gw.BOOL, gw.U64, gw.I64):
                assert c.meta_int(key) == v
            elif t in (gw.F32, gw.F64):
                assert c.meta_float(key) == v
            elif t == gw.STR:
                assert c.meta_str(key) == v
        assert c.meta_array("tokens") == (gw.STR, 3) and c.meta_array("ids") == (gw.U32, 4)
        infos = c.tensor_infos()
        assert [(t.name, t.dimensions, t.tensor_type, t.offset) for t in infos] == \
            [("norm", (64,), 0, offs[0]), ("blk.0.w", (512, 8), 12, offs[1]), ("odd", (70,), 8, offs[2])]
        assert all(o % 32 == 0 for o in offs)
        assert c.get_tensor_data("norm").tobytes() == norm
        assert c.get_tensor_data("blk.0.w").tobytes() == q4
        assert c.get_tensor_data("odd").tobytes() == q8   # ceil(70/32) * 34 bytes
        with pytest.raises(RuntimeError, match="Tensor not found: nope"):
            c.get_tensor_data("nope")
        with pytest.raises(RuntimeError, match="not a string"):
            c.meta_str("u32")
        with pytest.raises(RuntimeError, match="metadata key not found"):
            c.meta_int("missing")


def test_q2k_extent_follows_the_reference_table(tmp_path):
    # extract_tensor_bytes sizes a Q2_K tensor with GgmlDType::type_size = 82
    # (quantization/mod.rs:118); the block itself is 84 bytes, which is what
    # lbq_gguf_copy_tensor and the weight upload take
    from lightbulb_amd.gguf import Content
    from lightbulb_amd.quantized import GgmlDType
    rng = np.random.default_rng(3)
    q2 = rng.integers(0, 256, 4 * 84, dtype=np.uint8).tobytes()  # 2 rows x 512
    blob, _, _ = gw.build(KVS, [("w2", [512, 2], 10, q2)])
    with Content.read(write(tmp_path, blob)) as c:
        assert c.get_tensor_data("w2").tobytes() == q2[:4 * 82]
    assert GgmlDType.Q2K.type_size() == 82 and GgmlDType.Q2K.block_bytes() == 84


def test_alignment_rule(tmp_path):
    # parser.rs:374-380: align(0)=0, align(1)=32, align(31)=32, align(32)=32,
    # align(33)=64 -- here as header ends at 64 + r for r in 0, 1, 31, 32, 33
    from lightbulb_amd.gguf import Content
    base = 24 + (8 + 1) + 4 + 8  # header + a 1-char key + its type + an empty string value
    for r, want in ((0, 64), (1, 96), (31, 96), (32, 96), (33, 128)):
        pad = 64 + r - base
        blob = gw.build([("k" * (1 + pad), gw.STR, "")], [])[0]
        hdr_end = base + pad
        assert hdr_end == 64 + r
        with Content.read(write(tmp_path, blob[:hdr_end])) as c:
            assert c.tensor_data_offset == want
    # general.alignment (UInt32) overrides; another type is ignored (default 32)
    blob, off, offs = gw.build([("general.alignment", gw.U32, 256)], [("a", [3], 0, b"x" * 12), ("b", [5], 0, b"y" * 20)],
                               alignment=256)
    with Content.read(write(tmp_path, blob)) as c:
        assert c.alignment == 256 and c.tensor_data_offset == off and off % 256 == 0
        assert [t.offset for t in c.tensor_infos()] == [0, 256]
        assert c.get_tensor_data("b").tobytes() == b"y" * 20
    blob = gw.build([("general.alignment", gw.U64, 256)], [])[0]
    with Content.read(write(tmp_path, blob)) as c:
        assert c.alignment == 32


def test_little_endian_primitives(tmp_path):
    # parser.rs:357-368 and 371-379: bytes 12 34 56 78 read as u32 0x78563412,
    # 01..08 as u64 0x0807060504030201; a u64 length 5 then "hello"
    from lightbulb_amd.gguf import Content
    blob = b"GGUF" + struct.pack("<IQQ", 3, 0, 3)
    blob += gw.s("a") + struct.pack("<I", gw.U32) + bytes([0x12, 0x34, 0x56, 0x78])
    blob += gw.s("b") + struct.pack("<I", gw.U64) + bytes(range(1, 9))
    blob += gw.s("c") + struct.pack("<I", gw.STR) + bytes([5, 0, 0, 0, 0, 0, 0, 0]) + b"hello"
    with Content.read(write(tmp_path, blob)) as c:
        assert c.meta_int("a") == 0x78563412
        assert c.meta_int("b") == 0x0807060504030201
        assert c.meta_str("c") == "hello"


def test_errors(L, tmp_path):
    good, _, _ = gw.build(KVS[:3], [("w", [256, 2], 12, bytes(288))])
    cases = [
        (b"GGUJ" + good[4:], -7, "Invalid GGUF magic number: 0x4A554747 (expected 0x46554747)"),
        (good[:4] + struct.pack("<I", 2) + good[8:], -7, "Unsupported GGUF version: 2 (expected 3)"),
        (b"", -7, "Unexpected EOF"),
        (gw.build([("flag", gw.BOOL, 2)], [])[0], -7, "Invalid bool value: 2 (must be 0 or 1)"),
        (gw.build([("arr", gw.ARR, (gw.BOOL, [0, 1, 3]))], [])[0], -7, "Invalid bool value: 3"),
        (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw.s("x") + struct.pack("<I", 13) + bytes(8), -7,
         "Invalid metadata value type: 13"),
        (b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + gw.s("x") + struct.pack("<IIQ", gw.ARR, 14, 0), -7,
         "Invalid metadata value type: 14"),
        (gw.build([("general.alignment", gw.U32, 0)], [])[0], -7, "general.alignment is 0"),
    ]
    for blob, status, msg in cases:
        rc, h, err = open_raw(L, write(tmp_path, blob))
        assert rc == status and msg in err, (rc, err)
        assert not h
    rc, _, err = open_raw(L, tmp_path / "does-not-exist.gguf")
    assert rc == -9 and "Failed to open GGUF file" in err
    # every truncation of a valid file is an error (never a fault), the full file parses
    p, n = ctypes.c_void_p(), ctypes.c_size_t()
    for cut in range(len(good)):
        rc, h, err = open_raw(L, write(tmp_path, good[:cut], "cut.gguf"))
        if rc == 0:  # the tensor infos are complete: the data is what is missing
            assert L.lbq_gguf_tensor_bytes(h, b"w", ctypes.byref(p), ctypes.byref(n)) == -7
            assert "extends beyond file" in L.lbq_last_error().decode()
            L.lbq_gguf_close(h)
        else:
            assert rc == -7 and "Unexpected EOF" in err
    rc, h, _ = open_raw(L, write(tmp_path, good))
    assert rc == 0
    assert L.lbq_gguf_tensor_bytes(h, b"w", ctypes.byref(p), ctypes.byref(n)) == 0 and n.value == 288
    L.lbq_gguf_close(h)
    # a tensor past the end of the file, an unknown ggml type
    blob, _, _ = gw.build([], [("w", [256, 4], 12, bytes(288))])
    rc, h, _ = open_raw(L, write(tmp_path, blob))
    assert rc == 0
    assert L.lbq_gguf_tensor_bytes(h, b"w", ctypes.byref(p), ctypes.byref(n)) == -7
    assert "extends beyond file" in L.lbq_last_error().decode()
    L.lbq_gguf_close(h)
    blob, _, _ = gw.build([], [("w", [32], 4, bytes(64))])
    rc, h, _ = open_raw(L, write(tmp_path, blob))
    assert L.lbq_gguf_tensor_bytes(h, b"w", ctypes.byref(p), ctypes.byref(n)) == -2
    assert "Unknown quantization type: 4" in L.lbq_last_error().decode()
    L.lbq_gguf_close(h)


def test_byte_flips_never_fault(L, tmp_path):
    # random single-byte corruptions of a valid file: parse or fail cleanly
    good, _, _ = gw.build(KVS, [("w", [256, 2], 12, bytes(288)), ("n", [7], 0, bytes(28))])
    rng = np.random.default_rng(7)
    path = tmp_path / "flip.gguf"
    for _ in range(300):
        b = bytearray(good)
        b[int(rng.integers(0, len(b)))] = int(rng.integers(0, 256))
        path.write_bytes(bytes(b))
        rc, h, _ = open_raw(L, path)
        if rc == 0:
            p, n = ctypes.c_void_p(), ctypes.c_size_t()
            for nm in (b"w", b"n"):
                L.lbq_gguf_tensor_bytes(h, nm, ctypes.byref(p), ctypes.byref(n))
            L.lbq_gguf_close(h)
        else:
            assert rc in (-7, -1)
