"""Minimal GGUF reader (TEST INFRASTRUCTURE): header, key/values and tensor
directory of a GGUF v2/v3 file, and each tensor's bytes.

It reads what the reference converter writes (hy3_convert.c:712-742 header and
key/values, :894-901 tensor infos, data aligned to general.alignment, 32 by
default) so that fixtures can be taken from the converter's own output.
"""
import struct

import numpy as np

_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q",
           11: "<q", 12: "<d"}
# ggml type -> (block elements, block bytes); type 8 is hy3's 36-byte Q8_0
TYPE_SIZE = {0: (1, 4), 1: (1, 2), 8: (32, 36), 12: (256, 144)}


class Reader:
    def __init__(self, path):
        with open(path, "rb") as f:
            self.buf = f.read()
        self.pos = 0
        assert self._take(4) == b"GGUF", "not a GGUF file"
        self.version = self._u32()
        n_tensors, n_kv = self._u64(), self._u64()
        self.kv = {}
        for _ in range(n_kv):
            k = self._str()
            self.kv[k] = self._value(self._u32())
        self.tensors = {}
        for _ in range(n_tensors):
            name = self._str()
            nd = self._u32()
            dims = [self._u64() for _ in range(nd)]
            ty = self._u32()
            off = self._u64()
            self.tensors[name] = (dims, ty, off)
        align = int(self.kv.get("general.alignment", 32))
        self.data_start = (self.pos + align - 1) // align * align

    def _take(self, n):
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def _u32(self):
        return struct.unpack("<I", self._take(4))[0]

    def _u64(self):
        return struct.unpack("<Q", self._take(8))[0]

    def _str(self):
        return self._take(self._u64()).decode()

    def _value(self, ty):
        if ty == 8:
            return self._str()
        if ty == 9:
            et, n = self._u32(), self._u64()
            return [self._value(et) for _ in range(n)]
        fmt = _SCALAR[ty]
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def tensor_bytes(self, name):
        dims, ty, off = self.tensors[name]
        elems = int(np.prod(dims))
        be, bb = TYPE_SIZE[ty]
        n = elems // be * bb
        start = self.data_start + off
        return np.frombuffer(self.buf[start:start + n], np.uint8).copy(), dims, ty
