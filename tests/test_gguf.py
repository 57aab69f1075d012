"""GGUF ingestion on the CPU: the POSIX file layer (include/kq_file.h) and
the GGUF v3 parser (include/kq_gguf.h) of libkq_hip.so.

Golden cases: the synthetic fixture and the 20 malformed files of the
reference's tests/gguf_test.c (fixture at :130-238, view checks at :339-364,
accessor checks at :374-461, failure cases at :475-620), each with the status
the reference expects. The parser oracle (oracle/kq_gguf_oracle.py) is
checked against the same cases, then used on seeded mutations of the fixture
to compare every status and every parsed field with the library's.
"""
from __future__ import annotations

import ctypes as C
import random
import struct

import pytest

import kq_gguf_oracle as ORC
import kq_hip as K
import kq_synth as S

T_F32, T_Q5_1, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_IQ4_NL, T_BF16 = 0, 7, 8, 12, 13, 14, 20, 30
FIX_TYPES = [T_F32, T_BF16, T_Q5_1, T_Q8_0, T_Q4_K, T_Q5_K, T_IQ4_NL]
FIX_DIMS = [4, 4, 32, 32, 256, 256, 32]
FIX_PACKED = [16, 8, 24, 34, 144, 176, 18]
U64MAX = (1 << 64) - 1


class Fixture:
    """The reference test's fixture (tests/gguf_test.c:130-238), with the
    byte offsets its failure cases patch."""

    def __init__(self):
        b = bytearray()
        u32 = lambda v: b.extend(struct.pack("<I", v))
        u64 = lambda v: b.extend(struct.pack("<Q", v))

        def string(s: bytes):
            u64(len(s))
            b.extend(s)

        b.extend(b"GGUF")
        u32(3)
        u64(7)
        u64(4)
        self.first_key_length = len(b)
        string(b"general.architecture")
        u32(8)
        string(b"testarch")
        string(b"general.alignment")
        u32(4)
        self.alignment_value = len(b)
        u32(32)
        self.array_key = [len(b) + 8]
        string(b"test.array0")
        u32(9)
        self.array_element_type = len(b)
        u32(5)
        self.array_length = len(b)
        u64(3)
        for v in (1, 2, 3):
            u32(v)
        self.array_key.append(len(b) + 8)
        string(b"test.array1")
        u32(9)
        u32(8)
        u64(2)
        string(b"one")
        string(b"two")
        rel, self.rel = 0, []
        self.name, self.rank, self.dim, self.type, self.offset = [], [], [], [], []
        for i in range(7):
            self.rel.append(rel)
            rel = (rel + FIX_PACKED[i] + 31) // 32 * 32
            u64(2)
            self.name.append(len(b))
            b.extend(b"t%d" % i)
            self.rank.append(len(b))
            u32(1)
            self.dim.append(len(b))
            u64(FIX_DIMS[i])
            self.type.append(len(b))
            u32(FIX_TYPES[i])
            self.offset.append(len(b))
            u64(self.rel[i])
        self.directory_end = len(b)
        b.extend(bytes(-len(b) % 32))
        self.data_section = len(b)
        b.extend(b"\xa5" * (self.rel[6] + FIX_PACKED[6]))
        self.bytes = bytes(b)

    def patched(self, at: int, fmt: str, value) -> bytes:
        b = bytearray(self.bytes)
        struct.pack_into(fmt, b, at, value)
        return bytes(b)


FX = Fixture()


def _failure_cases():
    f = FX
    b0 = bytearray(f.bytes)
    b0[0] = ord("B")
    key = bytearray(f.bytes)
    key[f.first_key_length + 8] = 0xC0
    dup_meta = bytearray(f.bytes)
    dup_meta[f.array_key[1]:f.array_key[1] + 11] = f.bytes[f.array_key[0]:f.array_key[0] + 11]
    dup_tensor = bytearray(f.bytes)
    dup_tensor[f.name[1]:f.name[1] + 2] = b"t0"
    return [
        ("bad magic", bytes(b0), "BAD_MAGIC"),
        ("bad version", f.patched(4, "<I", 2), "UNSUPPORTED_VERSION"),
        ("truncated fixed header", f.bytes[:20], "TRUNCATED"),
        ("absurd string length", f.patched(f.first_key_length, "<Q", (128 << 20) + 1),
         "LIMIT_EXCEEDED"),
        ("invalid UTF-8 string", bytes(key), "MALFORMED_METADATA"),
        ("nested metadata array", f.patched(f.array_element_type, "<I", 9),
         "UNSUPPORTED_METADATA"),
        ("absurd metadata array", f.patched(f.array_length, "<Q", 2000001), "LIMIT_EXCEEDED"),
        ("directory allocation overflow", f.patched(8, "<Q", U64MAX), "ARITHMETIC_OVERFLOW"),
        ("tensor count defensive limit", f.patched(8, "<Q", 8193), "LIMIT_EXCEEDED"),
        ("zero tensor rank", f.patched(f.rank[0], "<I", 0), "MALFORMED_TENSOR"),
        ("excessive tensor rank", f.patched(f.rank[0], "<I", 9), "MALFORMED_TENSOR"),
        ("zero tensor dimension", f.patched(f.dim[0], "<Q", 0), "MALFORMED_TENSOR"),
        ("packed tensor byte overflow", f.patched(f.dim[0], "<Q", U64MAX), "ARITHMETIC_OVERFLOW"),
        ("unsupported tensor type", f.patched(f.type[0], "<I", 1), "UNSUPPORTED_TENSOR_TYPE"),
        ("duplicate metadata name", bytes(dup_meta), "DUPLICATE_METADATA"),
        ("duplicate tensor name", bytes(dup_tensor), "DUPLICATE_TENSOR"),
        ("invalid GGUF alignment", f.patched(f.alignment_value, "<I", 3), "INVALID_ALIGNMENT"),
        ("unaligned tensor offset", f.patched(f.offset[1], "<Q", 1), "INVALID_ALIGNMENT"),
        ("missing zero data-section origin", f.patched(f.offset[0], "<Q", 32),
         "INCONSISTENT_DATA_SECTION"),
        ("tensor span past EOF", f.bytes[:-1], "SPAN_OUT_OF_RANGE"),
        ("invalid quantized block geometry", f.patched(f.dim[3], "<Q", 31), "MALFORMED_TENSOR"),
    ]


FAILURES = _failure_cases()


def lib_status(path) -> str:
    """Status name of kq_file_open_readonly + kq_gguf_open on path."""
    try:
        K.Gguf(path).close()
        return "OK"
    except K.KqError as e:
        return e.name


def lib_parse(path) -> dict:
    """Every field the library reports, in the oracle's shape."""
    with K.Gguf(path) as g:
        info = g.info()
        info["architecture"] = info["architecture"].encode()
        meta = []
        for i in range(info["metadata_count"]):
            m = g.metadata_at(i).contents
            meta.append({"key": m.key.bytes(), "type": m.value_type,
                         "etype": m.array_element_type, "alen": m.array_length,
                         "scalar": m.scalar_value,
                         "string": m.string_value.bytes() if m.value_type == ORC.STRING else None,
                         "array": m.array_data.bytes() if m.value_type == ORC.ARRAY else None})
        tensors = []
        for i in range(info["tensor_count"]):
            t = g.tensor_at(i).contents
            tensors.append({"name": t.name.bytes(), "rank": t.rank,
                            "dims": list(t.dimensions[:t.rank]), "type": t.type_id,
                            "elements": t.element_count, "rel": t.relative_offset,
                            "packed": t.packed_bytes, "data_offset": t.data_offset})
        info["metadata"], info["tensors"] = meta, tensors
        return info


def write(tmp_path, data: bytes, name="f.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return p


# ------------------------------------------------------------ the oracle


def test_oracle_valid_fixture():
    r = ORC.parse(FX.bytes)
    assert r["packed_bytes"] == 420 and r["tensor_count"] == 7 and r["metadata_count"] == 4
    assert r["directory_end"] == FX.directory_end == r["bytes_parsed"]
    assert r["data_section"] == FX.data_section
    assert r["overhead_bytes"] == len(FX.bytes) - 420
    assert [t["packed"] for t in r["tensors"]] == FIX_PACKED


@pytest.mark.parametrize("name,data,expected", FAILURES, ids=[c[0] for c in FAILURES])
def test_oracle_failure_cases(name, data, expected):
    assert ORC.status(data) == expected


UTF8_CASES = [b"", b"a", b"\x7f", b"\xc0\x80", b"\xc1\xbf", b"\xc2\x80", b"\xdf\xbf",
              b"\xe0\x9f\xbf", b"\xe0\xa0\x80", b"\xed\x9f\xbf", b"\xed\xa0\x80",
              b"\xef\xbf\xbf", b"\xee\x80", b"\xf0\x8f\xbf\xbf", b"\xf0\x90\x80\x80",
              b"\xf4\x8f\xbf\xbf", b"\xf4\x90\x80\x80", b"\xf5\x80\x80\x80", b"\xf8\x88\x80\x80\x80",
              b"\xff", b"\x80", b"\xbf", b"\xc2", b"\xe1\x80", b"\xf1\x80\x80", b"\xc2\x41",
              b"\xe1\x41\x80", b"\xf1\x80\x41\x80", "日本語".encode(), "\U0001f600".encode(),
              b"ok\xe2\x82\xac", b"\xe2\x82\xacok\xc3"]


@pytest.mark.parametrize("s", UTF8_CASES, ids=[s.hex() or "empty" for s in UTF8_CASES])
def test_oracle_utf8_matches_strict_decoder(s):
    try:
        s.decode("utf-8", errors="strict")
        ok = True
    except UnicodeDecodeError:
        ok = False
    assert ORC.utf8_valid(s) == ok


# ------------------------------------------------------------ file layer


def test_file_views(tmp_path):
    p = write(tmp_path, FX.bytes)
    with K.File(p) as f:
        assert f.size == len(FX.bytes)
        off, n, data = f.view(3, 13)
        assert (off, n, data) == (3, 13, FX.bytes[3:16])
        off, n, data = f.view(4095, len(FX.bytes) - 4095) if len(FX.bytes) > 4096 else f.view(
            1, len(FX.bytes) - 1)
        assert data == FX.bytes[off:off + n]
        for args, status in [((0, 0), "INVALID_ARGUMENT"), ((U64MAX, 2), "ARITHMETIC_OVERFLOW"),
                             ((len(FX.bytes), 1), "SPAN_OUT_OF_RANGE")]:
            with pytest.raises(K.KqError) as e:
                f.view(*args)
            assert e.value.name == status


def test_file_views_across_pages(tmp_path):
    data = bytes(random.Random(7).getrandbits(8) for _ in range(3 * 4096 + 123))
    p = write(tmp_path, data)
    with K.File(p) as f:
        for off, n in [(0, len(data)), (4095, 2), (4096, 4096), (8191, 4096 + 124), (12000, 411)]:
            o, m, got = f.view(off, n)
            assert (o, m) == (off, n) and got == data[off:off + n]


def test_file_open_errors(tmp_path):
    with pytest.raises(K.KqError) as e:
        K.File(tmp_path / "missing.gguf")
    assert e.value.name == "FILE_OPEN_FAILED"
    with pytest.raises(K.KqError) as e:
        K.File(tmp_path)
    assert e.value.name == "FILE_SIZE_FAILED"


def test_file_wide_path(tmp_path):
    p = write(tmp_path, FX.bytes, "tést-日本.gguf")
    with K.File(p, wide=True) as f:
        assert f.size == len(FX.bytes)
    with K.Gguf(p, wide=True) as g:
        assert g.info()["tensor_count"] == 7


# ------------------------------------------------------------ parser


def test_valid_fixture(tmp_path):
    p = write(tmp_path, FX.bytes)
    with K.Gguf(p) as g:
        info = g.info()
        assert info["version"] == 3
        assert info["metadata_count"] == 4 and info["tensor_count"] == 7
        assert info["alignment"] == 32
        assert info["directory_end"] == FX.directory_end
        assert info["data_section"] == FX.data_section
        assert info["packed_bytes"] == 420
        assert info["overhead_bytes"] == len(FX.bytes) - 420
        assert info["bytes_parsed"] == FX.directory_end < info["data_section"]
        assert info["payload_bytes_accessed"] == 0
        assert info["architecture"] == "testarch"
        assert g.metadata_at(4) is None and g.tensor_at(7) is None
        assert g.tensor("missing") is None and g.metadata("missing") is None
        assert g.scalar(g.metadata("general.alignment"), "u32") == 32
        assert g.scalar(g.metadata("general.alignment"), "i32") is None
        a0 = g.metadata("test.array0")
        assert [g.array_item(a0, "i32", i) for i in range(4)] == [1, 2, 3, None]
        assert g.array_item(a0, "u64", 0) is None
        a1 = g.metadata("test.array1")
        assert [g.array_item(a1, "string", i) for i in range(3)] == [b"one", b"two", None]
        t3 = g.tensor("t3")
        assert t3 is not None and t3.contents.type_id == T_Q8_0
        for i in range(7):
            t = g.tensor_at(i).contents
            assert t.name.bytes() == b"t%d" % i and t.rank == 1
            assert t.dimensions[0] == FIX_DIMS[i] and t.type_id == FIX_TYPES[i]
            assert t.packed_bytes == FIX_PACKED[i] and t.element_count == FIX_DIMS[i]
            assert t.relative_offset == FX.rel[i]
            assert t.data_offset == FX.data_section + FX.rel[i] >= info["data_section"]
            assert K.gguf_type_info(t.type_id)[1:] == (t.block_elements, t.bytes_per_block)


@pytest.mark.parametrize("name,data,expected", FAILURES, ids=[c[0] for c in FAILURES])
def test_failure_cases(tmp_path, name, data, expected):
    assert lib_status(write(tmp_path, data)) == expected


def test_type_table():
    assert K.gguf_type_info(T_Q4_K) == ("Q4_K", 256, 144)
    assert K.gguf_type_info(T_Q6_K) == ("Q6_K", 256, 210)
    for t, (be, bpb) in ORC.TYPES.items():
        assert K.gguf_type_info(t)[1:] == (be, bpb) == K.GEOMETRY[t]
    for t in (1, 2, 3, 6, 9, 10, 11, 15, 16, 19, 21, 29, 31, 1000):
        assert K.gguf_type_info(t) is None


def meta_file(metadata, tensors=None, alignment=32):
    tensors = tensors or [("w", T_Q8_0, [32, 2], bytes(68))]
    return S.gguf_bytes(tensors, metadata, alignment)


ARCH = ("general.architecture", S.GGUF_STRING, "qwen3moe")


def test_metadata_value_types(tmp_path):
    md = [ARCH, ("u16", S.GGUF_UINT16, 65535), ("i32", S.GGUF_INT32, -7),
          ("f32", S.GGUF_FLOAT32, 1.5), ("b0", S.GGUF_BOOL, 0), ("b1", S.GGUF_BOOL, 1),
          ("u64s", S.GGUF_ARRAY, (S.GGUF_UINT64, [0, 1 << 40, U64MAX])),
          ("empty", S.GGUF_ARRAY, (S.GGUF_STRING, [])),
          ("general.alignment", S.GGUF_UINT32, 64)]
    data = meta_file(md, alignment=64)
    p = write(tmp_path, data)
    with K.Gguf(p) as g:
        assert g.scalar(g.metadata("u16"), "u16") == 65535
        assert g.scalar(g.metadata("i32"), "i32") == -7
        m = g.metadata("f32").contents
        assert m.value_type == S.GGUF_FLOAT32
        assert struct.unpack("<f", struct.pack("<I", m.scalar_value))[0] == 1.5
        assert g.metadata("b1").contents.scalar_value == 1
        u = g.metadata("u64s")
        assert [g.array_item(u, "u64", i) for i in range(4)] == [0, 1 << 40, U64MAX, None]
        assert g.array_item(g.metadata("empty"), "string", 0) is None
        assert g.info()["alignment"] == 64
    assert lib_parse(p) == ORC.parse(data)


@pytest.mark.parametrize("md,expected", [
    ([ARCH, ("b", S.GGUF_BOOL, 2)], "MALFORMED_METADATA"),
    ([ARCH, ("u64", S.GGUF_UINT64, 1)], "UNSUPPORTED_METADATA"),
    ([ARCH, ("i8", 1, 0)], "UNSUPPORTED_METADATA"),
    ([ARCH, ("f64s", S.GGUF_ARRAY, (12, []))], "UNSUPPORTED_METADATA"),
    ([ARCH, ("f32s", S.GGUF_ARRAY, (S.GGUF_FLOAT32, [1.0]))], "UNSUPPORTED_METADATA"),
    ([("general.architecture", S.GGUF_UINT32, 1)], "MALFORMED_METADATA"),
    ([("x", S.GGUF_STRING, "y")], "MALFORMED_METADATA"),
    ([ARCH, ("general.alignment", S.GGUF_UINT16, 32)], "MALFORMED_METADATA"),
    ([ARCH, ("general.alignment", S.GGUF_UINT32, 0)], "INVALID_ALIGNMENT"),
    ([ARCH, ("general.alignment", S.GGUF_UINT32, 8192)], "INVALID_ALIGNMENT"),
    ([ARCH, ("general.alignment", S.GGUF_UINT32, 48)], "INVALID_ALIGNMENT"),
    ([ARCH, ARCH], "DUPLICATE_METADATA"),
], ids=["bool2", "u64-scalar", "int8", "f64-array", "f32-array", "arch-u32", "no-arch",
        "align-u16", "align-0", "align-8192", "align-48", "dup-arch"])
def test_metadata_errors(tmp_path, md, expected):
    data = meta_file(md)
    assert ORC.status(data) == expected
    assert lib_status(write(tmp_path, data)) == expected


def _patch(data: bytes, at: int, fmt: str, value) -> bytes:
    b = bytearray(data)
    struct.pack_into(fmt, b, at, value)
    return bytes(b)


def test_directory_errors(tmp_path):
    w = ("w", T_Q8_0, [32, 2], bytes(68))
    b = S.gguf_bytes([w, ("v", T_Q8_0, [32], bytes(34))], [ARCH])
    # tensor "v": 8-byte name length, name, rank, one dimension, type, offset
    v_offset = b.index(struct.pack("<Q", 1) + b"v") + 8 + 1 + 4 + 8 + 4
    cases = [
        (_patch(b, v_offset, "<Q", 32), "INCONSISTENT_DATA_SECTION"),  # overlaps "w"
        (_patch(b, 8, "<Q", 0), "MALFORMED_METADATA"),   # no tensors
        (_patch(b, 16, "<Q", 0), "MALFORMED_METADATA"),  # no metadata
        (_patch(b, 16, "<Q", 1025), "LIMIT_EXCEEDED"),
    ]
    # file cut inside the directory / inside the data
    cases.append((bytes(b[:40]), "TRUNCATED"))
    cases.append((bytes(b[:len(b) - 40]), "SPAN_OUT_OF_RANGE"))
    # Q6_K is read (an addition to the reference's table); F16 is not
    cases.append((S.gguf_bytes([("q", T_Q6_K, [256, 3], bytes(630))], [ARCH]), "OK"))
    cases.append((S.gguf_bytes([("h", 1, [4], bytes(8))], [ARCH]), "UNSUPPORTED_TENSOR_TYPE"))
    # rank 8 with a dimension product overflowing uint64
    big = S.gguf_bytes([("r", T_F32, [1 << 16] * 4 + [2] * 4, bytes(4))], [ARCH])
    cases.append((big, "ARITHMETIC_OVERFLOW"))
    for i, (data, expected) in enumerate(cases):
        assert ORC.status(data) == expected, i
        assert lib_status(write(tmp_path, data, f"c{i}.gguf")) == expected, i


def test_multi_dimensional_stack(tmp_path):
    """A routed expert stack as GGUF stores it: dims [cols, rows, experts]."""
    cols, rows, experts = 512, 8, 6
    gate = bytes(random.Random(1).getrandbits(8) for _ in range(experts * rows * cols // 256 * 144))
    data = S.gguf_bytes([("blk.0.ffn_gate_exps.weight", T_Q4_K, [cols, rows, experts], gate),
                         ("blk.0.ffn_gate_inp.weight", T_F32, [cols, experts],
                          bytes(4 * cols * experts))],
                        [ARCH, ("general.alignment", S.GGUF_UINT32, 256)], alignment=256)
    p = write(tmp_path, data)
    with K.Gguf(p) as g:
        t = g.tensor("blk.0.ffn_gate_exps.weight")
        assert t.contents.packed_bytes == len(gate) and t.contents.rank == 3
        member = rows * cols // 256 * 144
        for e in range(experts):
            assert K.gguf_expert_member(t, e) == (e * member, member)
        with pytest.raises(K.KqError) as e:
            K.gguf_expert_member(t, experts)
        assert e.value.name == "SPAN_OUT_OF_RANGE"
        r = g.tensor("blk.0.ffn_gate_inp.weight")
        assert K.gguf_expert_member(r, 5) == (5 * 4 * cols, 4 * cols)
        with K.Gguf(write(tmp_path, FX.bytes, "fx.gguf")) as fx:
            with pytest.raises(K.KqError) as e:
                K.gguf_expert_member(fx.tensor("t0"), 0)
            assert e.value.name == "INVALID_QUANTIZED_GEOMETRY"
    assert lib_parse(p) == ORC.parse(data)


def _mutations(rng: random.Random, base: bytes, fx: Fixture):
    fields = ([(fx.first_key_length, "<Q"), (fx.alignment_value, "<I"),
               (fx.array_element_type, "<I"), (fx.array_length, "<Q"), (8, "<Q"), (16, "<Q"),
               (4, "<I")] + [(a, "<I") for a in fx.rank] + [(a, "<Q") for a in fx.dim]
              + [(a, "<I") for a in fx.type] + [(a, "<Q") for a in fx.offset])
    interesting = [0, 1, 2, 3, 4, 5, 7, 8, 9, 10, 12, 13, 14, 20, 30, 31, 32, 33, 64, 256,
                   4096, 8192, 1024, 1025, 8193, 2000001, (128 << 20) + 1, 0xFFFFFFFF, U64MAX,
                   1 << 63, 1 << 32]
    kind = rng.randrange(4)
    b = bytearray(base)
    if kind == 0:
        for _ in range(rng.randint(1, 3)):
            b[rng.randrange(fx.directory_end)] = rng.randrange(256)
    elif kind == 1:
        at, fmt = rng.choice(fields)
        v = rng.choice(interesting)
        v &= 0xFFFFFFFF if fmt == "<I" else U64MAX
        struct.pack_into(fmt, b, at, v)
    elif kind == 2:
        b = b[:rng.randrange(len(b))]
    else:
        at, fmt = rng.choice(fields)
        struct.pack_into(fmt, b, at, rng.getrandbits(32 if fmt == "<I" else 64) %
                         rng.choice([2, 16, 1024, 1 << 32]))
    return bytes(b)


def test_mutations_match_oracle(tmp_path):
    """1,500 seeded mutations of the fixture: flipped directory bytes,
    boundary values in every field, truncations. The library and the oracle
    agree on the status and, when it parses, on every field."""
    rng = random.Random(0x6A1F)
    seen = {}
    p = tmp_path / "m.gguf"
    for i in range(1500):
        data = _mutations(rng, FX.bytes, FX)
        p.write_bytes(data)
        try:
            want = ORC.parse(data)
        except ORC.Fail as f:
            want = f.status
        got = lib_status(p)
        if isinstance(want, dict):
            assert got == "OK", (i, got)
            assert lib_parse(p) == want, i
            seen["OK"] = seen.get("OK", 0) + 1
        else:
            assert got == want, (i, data.hex())
            seen[want] = seen.get(want, 0) + 1
    # the mutations reach most of the statuses the parser can return
    assert len(seen) >= 12, seen


def test_view_limit_exceeded(tmp_path):
    """A directory longer than the 512 MiB view of a longer file is
    LIMIT_EXCEEDED (not TRUNCATED). Sparse file: the strings are zero bytes,
    which are valid UTF-8."""
    p = tmp_path / "big.gguf"
    with open(p, "wb") as f:
        f.write(b"GGUF" + struct.pack("<IQQ", 3, 1, 5))
        at = 24
        for n in [110 << 20, 111 << 20, 112 << 20, 113 << 20, 114 << 20]:
            f.seek(at)
            f.write(struct.pack("<Q", n))   # key length (zero-byte key)
            f.seek(at + 8 + n)
            f.write(struct.pack("<IQ", 8, 0))  # STRING value of length 0
            at += 8 + n + 12
        f.truncate(600 << 20)
    assert lib_status(p) == "LIMIT_EXCEEDED"
    # the same file cut to 500 MiB reads to its end: TRUNCATED
    with open(p, "r+b") as f:
        f.truncate(500 << 20)
    assert lib_status(p) == "TRUNCATED"


def test_tensor_descriptor_pointers(tmp_path):
    """Descriptors stay valid while the GGUF is open; kq_string_view_equal
    compares names byte for byte."""
    p = write(tmp_path, FX.bytes)
    L = K.lib()
    with K.Gguf(p) as g:
        a, b = g.tensor("t1"), g.tensor_at(1)
        assert C.addressof(a.contents) == C.addressof(b.contents)
        na, n0 = a.contents.name, g.tensor_at(0).contents.name
        assert L.kq_string_view_equal(C.byref(na), C.byref(na)) == 1
        assert L.kq_string_view_equal(C.byref(na), C.byref(n0)) == 0
        assert L.kq_string_view_equal_cstr(C.byref(na), b"t1") == 1
        assert L.kq_string_view_equal_cstr(C.byref(na), b"t") == 0
