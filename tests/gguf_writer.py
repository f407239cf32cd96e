"""A minimal GGUF v2/v3 writer for the tests (the role of the reference's
tests/gguf_writer.hpp): typed metadata, tensor infos and aligned data.

Layout: "GGUF" | u32 version | u64 n_tensors | u64 n_kv | kv pairs |
tensor infos | padding to the alignment | tensor data (each tensor at its
offset from the data start, offsets aligned).
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}

# ggml tensor type ids
T_F32, T_F16, T_Q4_0, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_BF16 = 0, 1, 2, 8, 12, 13, 14, 30


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        return struct.pack("<IQ", etype, len(items)) + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


class GgufWriter:
    def __init__(self, alignment: int = 32):
        self.alignment = alignment
        self.kv = []
        self.tensors = []

    def add(self, key: str, vtype: int, value):
        self.kv.append((key, vtype, value))
        return self

    def add_tensor(self, name: str, dims, ttype: int, data: bytes):
        self.tensors.append((name, list(dims), ttype, bytes(data)))
        return self

    def to_bytes(self, version: int = 3, magic: bytes = b"GGUF") -> bytes:
        out = bytearray(magic)
        out += struct.pack("<IQQ", version, len(self.tensors), len(self.kv))
        for key, vtype, value in self.kv:
            out += _str(key) + struct.pack("<I", vtype) + _value(vtype, value)
        offsets, off = [], 0
        for _, _, _, data in self.tensors:
            offsets.append(off)
            off += len(data)
            off = (off + self.alignment - 1) // self.alignment * self.alignment
        for (name, dims, ttype, _), o in zip(self.tensors, offsets):
            out += _str(name) + struct.pack("<I", len(dims))
            out += b"".join(struct.pack("<Q", d) for d in dims)
            out += struct.pack("<IQ", ttype, o)
        pad = (-len(out)) % self.alignment
        out += b"\0" * pad
        data_start = len(out)
        for (_, _, _, data), o in zip(self.tensors, offsets):
            out += b"\0" * (data_start + o - len(out))
            out += data
        return bytes(out)

    def write(self, path: str, **kw) -> str:
        with open(path, "wb") as f:
            f.write(self.to_bytes(**kw))
        return path
