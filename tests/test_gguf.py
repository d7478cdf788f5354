"""GGUF reader (mx_gguf_*, host code): parsing, metadata, tensor table, error
paths.  No GPU needed.  The reader is pinned by a file assembled byte by byte
from the public GGUF layout (independent of maxuna_amd.gguf.write_gguf), then
the writer is checked against the reader for every value type."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from maxuna_amd import gguf as G
from maxuna_amd._lib import MaxunaError


def _s(b: bytes) -> bytes:
    return struct.pack("<Q", len(b)) + b


def test_hand_assembled_file(tmp_path):
    # magic | version 3 | 2 tensors | 2 kv
    raw = b"GGUF" + struct.pack("<IQQ", 3, 2, 2)
    raw += _s(b"laguna.expert_count") + struct.pack("<I", 4) + struct.pack("<I", 64)
    raw += _s(b"general.name") + struct.pack("<I", 8) + _s(b"tiny")
    # tensor "a": F32 [3 x 8] (ne = 8, 3), offset 0; tensor "b": Q8_0 [2 x 32], offset 96
    raw += _s(b"a") + struct.pack("<I", 2) + struct.pack("<QQ", 8, 3) + struct.pack("<IQ", 0, 0)
    raw += _s(b"b") + struct.pack("<I", 2) + struct.pack("<QQ", 32, 2) + struct.pack("<IQ", 8, 96)
    data_start = (len(raw) + 31) // 32 * 32
    raw += b"\0" * (data_start - len(raw))
    a = np.arange(24, dtype=np.float32)
    raw += a.tobytes()                      # 96 bytes at offset 0
    qb = bytes(range(68))                   # 2 Q8_0 blocks of 34 bytes at offset 96
    raw += qb
    p = tmp_path / "hand.gguf"
    p.write_bytes(raw)
    with G.GgufFile(p) as gf:
        assert gf.version == 3 and gf.alignment == 32
        assert gf.get_int("laguna.expert_count") == 64
        assert gf.get_str("general.name") == "tiny"
        ta, tb = gf.tensor("a"), gf.tensor("b")
        assert (ta.ggml_type, ta.shape, ta.offset, ta.nbytes) == (0, (3, 8), data_start, 96)
        assert (tb.ggml_type, tb.shape, tb.offset, tb.nbytes) == (8, (2, 32), data_start + 96, 68)
        assert np.array_equal(gf.read_host("a").view(np.float32), a)
        assert gf.read_host("b").tobytes() == qb


def test_writer_roundtrip_all_value_types(tmp_path):
    meta = {
        "u8": (G.GGUF_U8, 200), "i8": (G.GGUF_I8, -100), "u16": (G.GGUF_U16, 60000), "i16": (G.GGUF_I16, -30000),
        "u32": (G.GGUF_U32, 4_000_000_000), "i32": (G.GGUF_I32, -2_000_000_000), "f32": (G.GGUF_F32, 2.5),
        "bool_t": (G.GGUF_BOOL, True), "bool_f": (G.GGUF_BOOL, False), "str": (G.GGUF_STRING, "héllo"),
        "u64": (G.GGUF_U64, 2**62), "i64": (G.GGUF_I64, -(2**62)), "f64": (G.GGUF_F64, 1e-300),
        "arr_i32": (G.GGUF_ARRAY, (G.GGUF_I32, [1, -2, 3])),
        "arr_str": (G.GGUF_ARRAY, (G.GGUF_STRING, ["a", "bc", ""])),
        "arr_arr": (G.GGUF_ARRAY, (G.GGUF_ARRAY, [(G.GGUF_U8, [1, 2]), (G.GGUF_U8, [])])),
    }
    rng = np.random.default_rng(0)
    q4 = rng.integers(0, 256, 3 * 4 * 144, dtype=np.uint8)
    f16 = rng.standard_normal((5, 7)).astype(np.float16)
    tensors = [("stack", 12, (3, 4, 256), q4.tobytes()), ("h", 1, (5, 7), f16.tobytes()),
               ("one", 0, (1,), np.float32([7.0]).tobytes())]
    for align, version in ((32, 3), (64, 3), (32, 2)):
        p = tmp_path / f"w{align}_{version}.gguf"
        G.write_gguf(p, meta, tensors, version=version, alignment=align)
        with G.GgufFile(p) as gf:
            assert gf.version == version and gf.alignment == align
            for k in ("u8", "i8", "u16", "i16", "u32", "i32", "u64", "i64"):
                assert gf.get_int(k) == meta[k][1], k
            assert gf.get_float("f32") == 2.5 and gf.get_float("f64") == 1e-300
            assert gf.get_float("u32") == 4e9  # integers read as numbers too
            assert gf.get_bool("bool_t") is True and gf.get_bool("bool_f") is False
            assert gf.get_str("str") == "héllo"
            assert gf.array_info("arr_i32") == (G.GGUF_I32, 3)
            assert gf.array_info("arr_str") == (G.GGUF_STRING, 3)
            assert gf.array_info("arr_arr") == (G.GGUF_ARRAY, 2)
            assert gf.get_int("missing", 5) == 5 and not gf.has("missing")
            for name, gt, shape, raw in tensors:
                t = gf.tensor(name)
                assert (t.ggml_type, t.shape, t.nbytes) == (gt, shape, len(raw))
                assert t.offset % align == 0
                assert gf.read_host(name).tobytes() == raw
            with pytest.raises(MaxunaError) as e:
                gf.get_int("str")
            assert e.value.code == 3
            with pytest.raises(MaxunaError) as e:
                gf.get_int("nope")
            assert e.value.code == 13


def test_malformed_files_fail_cleanly(tmp_path):
    p = tmp_path / "good.gguf"
    G.write_gguf(p, {"k": (G.GGUF_STRING, "v" * 40), "a": (G.GGUF_ARRAY, (G.GGUF_U32, list(range(9))))},
                 [("t", 12, (2, 256), bytes(288)), ("u", 0, (4,), bytes(16))])
    good = p.read_bytes()

    def expect(raw, code, name):
        q = tmp_path / name
        q.write_bytes(raw)
        with pytest.raises(MaxunaError) as e:
            G.GgufFile(q)
        assert e.value.code == code, (name, e.value)

    expect(b"GGUX" + good[4:], 12, "magic.gguf")
    expect(good[:4] + struct.pack("<I", 1) + good[8:], 12, "v1.gguf")
    # every truncation point is rejected (no read past the end); the file ends in
    # alignment padding, so the last cuts go into the last tensor's data
    with G.GgufFile(p) as gf:
        end_u = gf.tensor("u").offset + gf.tensor("u").nbytes
        end_t = gf.tensor("t").offset + gf.tensor("t").nbytes
    for cut in list(range(0, 120, 7)) + [end_u - 1, end_t - 1]:
        expect(good[:cut], 12, f"cut{cut}.gguf")
    # tensor offset not aligned: patch the last tensor's offset (its u64 sits just
    # before the padding that ends the tensor table)
    hdr_end = good.index(b"u") + 1 + 4 + 8 + 4  # name 'u', n_dims, ne[0], type
    bad = bytearray(good)
    bad[hdr_end:hdr_end + 8] = struct.pack("<Q", 300 + 3)
    expect(bytes(bad), 12, "misaligned.gguf")
    # duplicate names
    q = tmp_path / "dup.gguf"
    G.write_gguf(q, {}, [("t", 0, (4,), bytes(16)), ("t", 0, (4,), bytes(16))])
    with pytest.raises(MaxunaError) as e:
        G.GgufFile(q)
    assert e.value.code == 12
    with pytest.raises(MaxunaError) as e:
        G.GgufFile(tmp_path / "absent.gguf")
    assert e.value.code == 11


def test_element_count_overflow_rejected(tmp_path):
    """Four dimensions of 2^40 each multiply past any 128-bit product: the
    reader rejects the tensor as soon as its running element count passes 2^62
    instead of wrapping to a small size."""
    raw = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    raw += _s(b"huge") + struct.pack("<I", 4) + struct.pack("<QQQQ", 2**40, 2**40, 2**40, 2**40)
    raw += struct.pack("<IQ", 0, 0)
    raw += b"\0" * ((len(raw) + 31) // 32 * 32 - len(raw)) + b"\0" * 64
    p = tmp_path / "huge.gguf"
    p.write_bytes(raw)
    with pytest.raises(MaxunaError, match="more than 2\\^62 elements"):
        G.GgufFile(p)
