"""GGUF v3 directory parser restated in plain Python.

TEST INFRASTRUCTURE ONLY: the checker that tests/ run the library's GGUF
parser against. Nothing in the product package imports this module.

It restates src/kq_gguf.c step by step, in the reference's order, so that
the status of any malformed file is the one the reference returns:
  - reader: bounds and the LIMIT_EXCEEDED / TRUNCATED split, :115-150;
  - UTF-8 byte-range rule, :207-255 (written as the reference's table of
    lead-byte ranges, not as a decoder);
  - strings :256-285; scalar values :349-393; arrays :395-469;
  - metadata :471-551; tensors :553-668; spans :688-796; open :798-967;
  - the string-array walk of kq_gguf_metadata_array_string_at, :1200-1237.
The type table is the reference's (:57-65) plus Q6_K (type 14), which the
library accepts as an addition.

Pinned by: the valid fixture and all 20 failure cases of tests/gguf_test.c
(run against this module in tests/test_gguf.py), and Python's strict UTF-8
decoder on boundary sequences.
"""
from __future__ import annotations

import struct

VIEW_LIMIT = 512 << 20
STRING_LIMIT = 128 << 20
ARRAY_LIMIT = 2_000_000
METADATA_LIMIT = 1024
TENSOR_LIMIT = 8192
DEFAULT_ALIGNMENT = 32
ALIGNMENT_LIMIT = 4096
U64 = (1 << 64) - 1
# SIZE_MAX / sizeof(descriptor) on LP64: kq_gguf_metadata is 72 bytes,
# kq_gguf_tensor 144.
META_ALLOC_LIMIT = U64 // 72
TENSOR_ALLOC_LIMIT = U64 // 144

TYPES = {0: (1, 4), 7: (32, 24), 8: (32, 34), 12: (256, 144), 13: (256, 176),
         14: (256, 210), 20: (32, 18), 30: (1, 2)}

UINT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64 = 2, 4, 5, 6, 7, 8, 9, 10


class Fail(Exception):
    def __init__(self, status: str):
        super().__init__(status)
        self.status = status


def utf8_valid(b: bytes) -> bool:
    i, n = 0, len(b)
    cont = lambda x: (x & 0xC0) == 0x80
    while i < n:
        f = b[i]
        if f <= 0x7F:
            i += 1
        elif 0xC2 <= f <= 0xDF:
            if n - i < 2 or not cont(b[i + 1]):
                return False
            i += 2
        elif 0xE0 <= f <= 0xEF:
            if n - i < 3:
                return False
            s = b[i + 1]
            if not cont(b[i + 2]):
                return False
            if f == 0xE0 and not 0xA0 <= s <= 0xBF:
                return False
            if f == 0xED and not 0x80 <= s <= 0x9F:
                return False
            if f not in (0xE0, 0xED) and not cont(s):
                return False
            i += 3
        elif 0xF0 <= f <= 0xF4:
            if n - i < 4:
                return False
            s = b[i + 1]
            if not cont(b[i + 2]) or not cont(b[i + 3]):
                return False
            if f == 0xF0 and not 0x90 <= s <= 0xBF:
                return False
            if f == 0xF4 and not 0x80 <= s <= 0x8F:
                return False
            if f not in (0xF0, 0xF4) and not cont(s):
                return False
            i += 4
        else:
            return False
    return True


class _Reader:
    def __init__(self, data: bytes, file_size: int):
        self.data, self.file_size = data, file_size
        self.at = self.furthest = 0

    def take(self, n: int) -> bytes:
        end = self.at + n
        if end > U64:
            raise Fail("ARITHMETIC_OVERFLOW")
        if end > len(self.data):
            raise Fail("LIMIT_EXCEEDED" if len(self.data) < self.file_size else "TRUNCATED")
        out = self.data[self.at:end]
        self.at = end
        self.furthest = max(self.furthest, end)
        return out

    def u(self, n: int) -> int:
        return int.from_bytes(self.take(n), "little")

    def string(self) -> bytes:
        n = self.u(8)
        if n > STRING_LIMIT:
            raise Fail("LIMIT_EXCEEDED")
        s = self.take(n)
        if not utf8_valid(s):
            raise Fail("MALFORMED_METADATA")
        return s


def _scalar(r: _Reader, vtype: int) -> int:
    if vtype == UINT16:
        return r.u(2)
    if vtype in (UINT32, INT32, FLOAT32):
        return r.u(4)
    if vtype == BOOL:
        v = r.u(1)
        if v > 1:
            raise Fail("MALFORMED_METADATA")
        return v
    raise Fail("UNSUPPORTED_METADATA")


def _array(r: _Reader) -> tuple[int, int, bytes]:
    etype = r.u(4)
    n = r.u(8)
    if n > ARRAY_LIMIT:
        raise Fail("LIMIT_EXCEEDED")
    if etype == INT32:
        return etype, n, r.take(n * 4)
    if etype == UINT64:
        return etype, n, r.take(n * 8)
    if etype == STRING:
        start = r.at
        for _ in range(n):
            r.string()
        return etype, n, r.data[start:r.at]
    raise Fail("UNSUPPORTED_METADATA")


def parse(image: bytes, file_size: int | None = None, view_limit: int = VIEW_LIMIT) -> dict:
    """Parse a GGUF image (the whole file). Raises Fail(status name)."""
    size = len(image) if file_size is None else file_size
    if size < 24:
        raise Fail("TRUNCATED")
    r = _Reader(image[:min(size, view_limit)], size)
    if r.u(4) != 0x46554747:
        raise Fail("BAD_MAGIC")
    version = r.u(4)
    if version != 3:
        raise Fail("UNSUPPORTED_VERSION")
    tcount, mcount = r.u(8), r.u(8)
    if tcount == 0 or mcount == 0:
        raise Fail("MALFORMED_METADATA")
    if mcount > META_ALLOC_LIMIT or tcount > TENSOR_ALLOC_LIMIT:
        raise Fail("ARITHMETIC_OVERFLOW")
    if mcount > METADATA_LIMIT or tcount > TENSOR_LIMIT:
        raise Fail("LIMIT_EXCEEDED")

    meta, keys, arch, alignment = [], set(), None, DEFAULT_ALIGNMENT
    for _ in range(mcount):
        key = r.string()
        if key in keys:
            raise Fail("DUPLICATE_METADATA")
        keys.add(key)
        vtype = r.u(4)
        entry = {"key": key, "type": vtype, "etype": 0, "alen": 0, "scalar": 0,
                 "string": None, "array": None}
        if vtype == STRING:
            entry["string"] = r.string()
        elif vtype == ARRAY:
            entry["etype"], entry["alen"], entry["array"] = _array(r)
        else:
            entry["scalar"] = _scalar(r, vtype)
        if key == b"general.architecture":
            if vtype != STRING:
                raise Fail("MALFORMED_METADATA")
            arch = entry["string"]
        elif key == b"general.alignment":
            if vtype != UINT32:
                raise Fail("MALFORMED_METADATA")
            alignment = entry["scalar"]
        meta.append(entry)
    if arch is None:
        raise Fail("MALFORMED_METADATA")
    if alignment == 0 or alignment > ALIGNMENT_LIMIT or alignment & (alignment - 1):
        raise Fail("INVALID_ALIGNMENT")

    tensors, names = [], set()
    for _ in range(tcount):
        name = r.string()
        if name in names:
            raise Fail("DUPLICATE_TENSOR")
        names.add(name)
        rank = r.u(4)
        if rank == 0 or rank > 8:
            raise Fail("MALFORMED_TENSOR")
        dims, count = [], 1
        for _ in range(rank):
            d = r.u(8)
            if d == 0:
                raise Fail("MALFORMED_TENSOR")
            count *= d
            if count > U64:
                raise Fail("ARITHMETIC_OVERFLOW")
            dims.append(d)
        type_id = r.u(4)
        if type_id not in TYPES:
            raise Fail("UNSUPPORTED_TENSOR_TYPE")
        rel = r.u(8)
        if rel % alignment:
            raise Fail("INVALID_ALIGNMENT")
        be, bpb = TYPES[type_id]
        if dims[0] % be:
            raise Fail("MALFORMED_TENSOR")
        packed = count // be * bpb
        if packed > U64:
            raise Fail("ARITHMETIC_OVERFLOW")
        tensors.append({"name": name, "rank": rank, "dims": dims, "type": type_id,
                        "elements": count, "rel": rel, "packed": packed})

    dir_end = r.at
    if dir_end + alignment - 1 > U64:
        raise Fail("ARITHMETIC_OVERFLOW")
    data = (dir_end + alignment - 1) & ~(alignment - 1)
    if data > size:
        raise Fail("INCONSISTENT_DATA_SECTION")

    order = sorted(range(tcount), key=lambda i: (tensors[i]["rel"], i))
    if tensors[order[0]]["rel"] != 0:
        raise Fail("INCONSISTENT_DATA_SECTION")
    total = 0
    for pos, i in enumerate(order):
        t = tensors[i]
        rel_end = t["rel"] + t["packed"]
        t["data_offset"] = data + t["rel"]
        abs_end = t["data_offset"] + t["packed"]
        if rel_end > U64 or t["data_offset"] > U64 or abs_end > U64:
            raise Fail("ARITHMETIC_OVERFLOW")
        if abs_end > size:
            raise Fail("SPAN_OUT_OF_RANGE")
        if pos + 1 < tcount and rel_end > tensors[order[pos + 1]]["rel"]:
            raise Fail("INCONSISTENT_DATA_SECTION")
        total += t["packed"]
        if total > U64:
            raise Fail("ARITHMETIC_OVERFLOW")
    if total > size:
        raise Fail("INCONSISTENT_DATA_SECTION")
    return {"version": version, "metadata_count": mcount, "tensor_count": tcount,
            "alignment": alignment, "directory_end": dir_end, "data_section": data,
            "packed_bytes": total, "overhead_bytes": size - total, "bytes_parsed": r.furthest,
            "payload_bytes_accessed": 0, "architecture": arch, "metadata": meta,
            "tensors": tensors}


def status(image: bytes, **kw) -> str:
    try:
        parse(image, **kw)
        return "OK"
    except Fail as f:
        return f.status


def array_string_at(array: bytes, count: int, index: int):
    """kq_gguf_metadata_array_string_at over an array's encoded bytes."""
    if index >= count:
        return None
    at = 0
    for k in range(index + 1):
        if len(array) - at < 8:
            return None
        (n,) = struct.unpack_from("<Q", array, at)
        at += 8
        if n > len(array) - at:
            return None
        if k == index:
            return array[at:at + n]
        at += n
    return None
