"""Byte builder for GGUF v3 test files: header, metadata entries, tensor infos, padding to the
alignment, tensor data (the file layout src/gguf.zig:263-330 parses)."""
import struct


class GgufBuilder:
    def __init__(self):
        self.b = bytearray()

    def u8(self, v):
        self.b += struct.pack("<B", v)
        return self

    def u32(self, v):
        self.b += struct.pack("<I", v)
        return self

    def u64(self, v):
        self.b += struct.pack("<Q", v)
        return self

    def str(self, s):
        s = s.encode() if isinstance(s, str) else s
        self.u64(len(s))
        self.b += s
        return self

    def header(self, n_tensors, n_kv, version=3, magic=b"GGUF"):
        self.b += magic
        return self.u32(version).u64(n_tensors).u64(n_kv)

    def kv_u32(self, key, v):
        return self.str(key).u32(4).u32(v)

    def kv_str(self, key, v):
        return self.str(key).u32(8).str(v)

    def tensor(self, name, dims, type_id, offset):
        self.str(name).u32(len(dims))
        for d in dims:
            self.u64(d)
        return self.u32(type_id).u64(offset)

    def pad(self, alignment=32):
        while len(self.b) % alignment:
            self.b += b"\0"
        return self

    def bytes(self):
        return bytes(self.b)
