"""GGUF reader (host code of the library; no GPU): the reference's own GGUF
tests (src/gguf/tests.rs) and the directory checks of gguf.rs:156-237."""
import struct

import numpy as np
import pytest

import gguf_writer as G


@pytest.fixture()
def oco():
    import oco_amd
    oco_amd.load_library()
    return oco_amd


def write(tmp_path, data: bytes, name="f.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return str(p)


def test_metadata_scan_checks_truncation_and_skips_unused_arrays(oco, tmp_path):
    """gguf/tests.rs:41-69."""
    data = G.build(metadata=[("unused", G.ARRAY, (G.STRING, ["one", "two"])), ("count", G.U64, 23)])
    path = write(tmp_path, data)
    with oco.Gguf(path, ["count"]) as g:
        assert g.has("count") and not g.has("unused")
        assert g.optional_unsigned("count") == 23
    with oco.Gguf(path, ["unused", "count"]) as g:
        assert g.strings("unused") == ["one", "two"]
        with pytest.raises(oco.OcoError):
            g.unsigned_integers("unused")
        with pytest.raises(oco.OcoError):
            g.strings("count")
    for cut in range(len(data)):
        path = write(tmp_path, data[:cut], f"cut{cut}.gguf")
        with pytest.raises(oco.OcoError):
            oco.Gguf(path, ["count"])


def _raw(tmp_path, meta_bytes: bytes, entries: int = 1):
    return write(tmp_path, G.header(0, entries) + meta_bytes)


def test_metadata_work_and_nesting_are_bounded(oco, tmp_path):
    """gguf/tests.rs:71-102, through whole files."""
    key = G.string("k")
    # array of u8 with a count past the file
    with pytest.raises(oco.OcoError, match="excessive or truncated"):
        oco.Gguf(_raw(tmp_path, key + struct.pack("<IIQ", G.ARRAY, G.U8, 2 ** 64 - 1)))
    # arrays nested five deep
    nest = struct.pack("<I", G.ARRAY) + b"".join(struct.pack("<IQ", G.ARRAY, 1) for _ in range(4))
    nest += struct.pack("<IQ", G.U8, 1) + b"\0"
    with pytest.raises(oco.OcoError, match="too deep"):
        oco.Gguf(_raw(tmp_path, key + nest))
    # unknown metadata type, bad boolean read, duplicate keys
    with pytest.raises(oco.OcoError, match="unknown metadata type"):
        oco.Gguf(_raw(tmp_path, key + struct.pack("<I", 13)))
    dup = G.build(metadata=[("a", G.U8, 1), ("a", G.U8, 2)])
    with pytest.raises(oco.OcoError, match="duplicate"):
        oco.Gguf(write(tmp_path, dup))
    bad_bool = key + struct.pack("<IB", G.BOOL, 2)
    with oco.Gguf(_raw(tmp_path, bad_bool), ["k"]) as g:
        with pytest.raises(oco.OcoError, match="boolean"):
            g.boolean("k")


def test_header_checks(oco, tmp_path):
    with pytest.raises(oco.OcoError, match="not a GGUF"):
        oco.Gguf(write(tmp_path, b"GGML" + bytes(20)))
    with pytest.raises(oco.OcoError, match="version 3"):
        oco.Gguf(write(tmp_path, b"GGUF" + struct.pack("<IQQ", 2, 0, 0)))


def test_typed_metadata(oco, tmp_path):
    meta = [("u8", G.U8, 7), ("i8", G.I8, -3), ("u16", G.U16, 500), ("i32", G.I32, -9), ("f32", G.F32, 1.5),
            ("b", G.BOOL, 1), ("s", G.STRING, "qwen3"), ("u64", G.U64, 2 ** 40), ("f64", G.F64, -2.25),
            ("ids", G.ARRAY, (G.I32, [1, 2, 3])), ("neg", G.ARRAY, (G.I32, [1, -2])),
            ("names", G.ARRAY, (G.STRING, ["a", "bc", ""])), ("nan", G.F32, float("nan"))]
    with oco.Gguf(write(tmp_path, G.build(metadata=meta)), [k for k, _, _ in meta]) as g:
        assert g.number("u8") == 7 and g.number("i8") == -3 and g.number("f32") == 1.5 and g.number("f64") == -2.25
        assert g.optional_unsigned("u64") == 2 ** 40 and g.optional_unsigned("missing") is None
        assert g.boolean("b") and g.text("s") == "qwen3"
        assert g.unsigned_integers("ids") == [1, 2, 3] and g.strings("names") == ["a", "bc", ""]
        for bad, fn in (("i8", g.optional_unsigned), ("s", g.number), ("u16", g.boolean), ("neg", g.unsigned_integers),
                        ("nan", g.number), ("ids", g.text)):
            with pytest.raises(oco.OcoError):
                fn(bad)


def test_selected_tensors_require_aligned_complete_payloads(oco, tmp_path):
    """gguf/tests.rs:104-135."""
    data = G.build(tensors=[("weight", [4], 0, bytes(16))])
    path = write(tmp_path, data)
    with oco.Gguf(path) as g:
        e = g.directory()["weight"]
        assert g.select(e).bytes == 16
        e.offset += 1
        with pytest.raises(oco.OcoError, match="unaligned tensor data"):
            g.select(e)
    path = write(tmp_path, data[:-1], "short.gguf")
    with oco.Gguf(path) as g:
        with pytest.raises(oco.OcoError, match="truncated or overlapping"):
            g.select(g.directory()["weight"])


def test_directory_checks(oco, tmp_path):
    ok = G.build(metadata=[("general.alignment", G.U32, 64)],
                 tensors=[("a", [32, 2], 8, bytes(68)), ("b", [64], 39, bytes(34)), ("c", [256, 3], 14, bytes(630))],
                 alignment=64)
    with oco.Gguf(write(tmp_path, ok), ["general.alignment"]) as g:
        d = g.directory()
        assert sorted(d) == ["a", "b", "c"]
        start = d["a"].offset
        assert start % 64 == 0 and d["b"].offset == start + 128 and d["c"].offset == start + 192
        t = g.select(d["c"])
        assert (t.format, t.rank, list(t.shape)[:2], t.bytes) == (14, 2, [256, 3], 630)
        assert d["a"].extent == 128 and d["c"].extent == 630
        assert g.select(d["b"]).bytes == 34
    # tensor offset not a multiple of the alignment
    bad = bytearray(G.build(tensors=[("a", [4], 0, bytes(16)), ("b", [4], 0, bytes(16))]))
    i = bad.find(G.string("b")) + len(G.string("b")) + 4 + 8 + 4
    struct.pack_into("<Q", bad, i, 40)
    with oco.Gguf(write(tmp_path, bytes(bad))) as g:
        with pytest.raises(oco.OcoError, match="unaligned tensor"):
            g.directory()
    # two tensors at one offset; a zero dimension; a block-misaligned row; an unknown type
    same = bytearray(G.build(tensors=[("a", [4], 0, bytes(16)), ("b", [4], 0, bytes(16))]))
    struct.pack_into("<Q", same, i, 0)
    with oco.Gguf(write(tmp_path, bytes(same))) as g:
        with pytest.raises(oco.OcoError, match="overlapping"):
            g.directory()
    with oco.Gguf(write(tmp_path, G.build(tensors=[("z", [0], 0, b"")]))) as g:
        with pytest.raises(oco.OcoError, match="zero tensor dimension"):
            g.directory()
    with oco.Gguf(write(tmp_path, G.build(tensors=[("q", [48], 8, bytes(64))]))) as g:
        with pytest.raises(oco.OcoError, match="block alignment"):
            g.select(g.directory()["q"])
    with oco.Gguf(write(tmp_path, G.build(tensors=[("u", [32], 6, bytes(32))]))) as g:
        with pytest.raises(oco.OcoError, match="unsupported GGUF tensor type"):
            g.select(g.directory()["u"])
    with oco.Gguf(write(tmp_path, G.build(metadata=[("general.alignment", G.U32, 48)]),
                       "al.gguf"), ["general.alignment"]) as g:
        with pytest.raises(oco.OcoError, match="alignment"):
            g.directory()


def test_data_view_matches_payload(oco, tmp_path):
    rng = np.random.default_rng(0)
    payload = rng.integers(0, 256, 210 * 8, dtype=np.uint8).tobytes()
    with oco.Gguf(write(tmp_path, G.build(tensors=[("w", [256, 8], 14, payload)]))) as g:
        t = g.select(g.directory()["w"])
        assert g.data(t).tobytes() == payload
