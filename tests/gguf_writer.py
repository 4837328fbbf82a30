"""Writes GGUF files for the reader tests, from the GGUF specification (the
container the reference's test fixtures build byte by byte,
tests/test_utils.h:16-97): little-endian header {magic "GGUF", version u32,
tensor_count u64, metadata_kv_count u64}, key/value pairs {string key, u32
type, value}, tensor infos {string name, u32 n_dims, u64 dims[n_dims], u32
ggml type, u64 offset}, zero padding to the alignment, then the data section.
Strings are u64 length + bytes; arrays are u32 element type + u64 count +
elements.  Independent of the C++ reader under test."""
from __future__ import annotations

import struct

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
        BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def _string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


class GGUFWriter:
    def __init__(self, version: int = 3, alignment: int | None = None):
        self.version = version
        self.alignment = alignment
        self.kvs: list[tuple[str, int, object]] = []
        self.tensors: list[tuple[str, list[int], int, bytes]] = []
        if alignment is not None:
            self.kvs.append(("general.alignment", UINT32, alignment))

    def add_kv(self, key: str, vtype: int, value) -> "GGUFWriter":
        self.kvs.append((key, vtype, value))
        return self

    def add_tensor(self, name: str, dims: list[int], ggml_type: int, data: bytes) -> "GGUFWriter":
        self.tensors.append((name, list(dims), ggml_type, bytes(data)))
        return self

    def build(self, tensor_count: int | None = None, kv_count: int | None = None, magic: bytes = b"GGUF",
              trailing: bytes = b"") -> bytes:
        align = self.alignment or 32
        out = bytearray(magic + struct.pack("<IQQ", self.version,
                                            len(self.tensors) if tensor_count is None else tensor_count,
                                            len(self.kvs) if kv_count is None else kv_count))
        for key, vtype, value in self.kvs:
            out += _string(key) + struct.pack("<I", vtype) + _value(vtype, value)
        offsets, off = [], 0
        for _, _, _, data in self.tensors:
            offsets.append(off)
            off = (off + len(data) + align - 1) // align * align
        for (name, dims, t, _), o in zip(self.tensors, offsets):
            out += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", t, o)
        out += b"\0" * ((-len(out)) % align)
        self.data_offset = len(out)
        for (_, _, _, data), o in zip(self.tensors, offsets):
            out += b"\0" * (self.data_offset + o - len(out)) + data
        return bytes(out) + trailing

    def write(self, path, **kw) -> bytes:
        b = self.build(**kw)
        with open(path, "wb") as fh:
            fh.write(b)
        return b
