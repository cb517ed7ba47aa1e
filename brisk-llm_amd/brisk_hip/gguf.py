"""GGUF v3 reading and writing (host side).

The reader follows the format as the reference parses it (src/gguf.cpp:263-343):
little-endian header ``GGUF``, version 2 or 3, tensor and key/value counts,
typed metadata, tensor infos with dims innermost-first (src/gguf.h:52-56), then
the data section aligned to ``general.alignment`` (default 32,
src/gguf.cpp:15-16, :318-321).  Tensor bytes are exposed as numpy views into a
read-only memory map, so loading a model does not copy it.

The writer emits the same layout; it is what builds the seeded random-weight
model files the parity tests and the benchmark run on.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = 0x46554747
DEFAULT_ALIGNMENT = 32

# Metadata value types (src/gguf.h:16-19).
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
           U64: "<Q", I64: "<q", F64: "<d"}

# Tensor types (ggml numbering, src/gguf.h:22-27) and their (elements, bytes) per block
# (src/gguf.cpp:135-161).
T_F32, T_F16, T_Q4_0, T_Q8_0, T_Q4_K, T_Q6_K, T_TQ2_0, T_BF16 = 0, 1, 2, 8, 12, 14, 35, 30
T_Q4_1, T_Q5_0, T_Q5_K = 3, 6, 13
BLOCK = {T_F32: (1, 4), T_F16: (1, 2), T_BF16: (1, 2), T_Q4_0: (32, 18), T_Q4_1: (32, 20), T_Q5_0: (32, 22),
         T_Q8_0: (32, 34), T_Q4_K: (256, 144), T_Q5_K: (256, 176), T_Q6_K: (256, 210), T_TQ2_0: (256, 66)}
TYPE_NAMES = {T_F32: "F32", T_F16: "F16", T_BF16: "BF16", T_Q4_0: "Q4_0", T_Q4_1: "Q4_1", T_Q5_0: "Q5_0",
              T_Q8_0: "Q8_0", T_Q4_K: "Q4_K", T_Q5_K: "Q5_K", T_Q6_K: "Q6_K", T_TQ2_0: "TQ2_0"}


class GgufError(RuntimeError):
    pass


@dataclass
class Tensor:
    name: str
    dims: tuple          # ggml order: innermost first
    type: int
    offset: int          # relative to the data section
    data: np.ndarray = field(repr=False, default=None)  # uint8 view of the tensor's bytes

    @property
    def rows(self) -> int:
        n = 1
        for d in self.dims[1:]:
            n *= d
        return n

    @property
    def cols(self) -> int:
        return self.dims[0]

    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


class GgufFile:
    """A parsed GGUF file; ``metadata`` maps key -> python value, ``tensors`` name -> Tensor."""

    def __init__(self, path: str):
        self.path = path
        self._map = np.memmap(path, dtype=np.uint8, mode="r")
        buf = memoryview(self._map)
        pos = 0

        def take(n):
            nonlocal pos
            if n > len(buf) - pos:
                raise GgufError("gguf: unexpected end of file")
            out = buf[pos:pos + n]
            pos += n
            return out

        def read(fmt):
            return struct.unpack(fmt, take(struct.calcsize(fmt)))[0]

        def read_string():
            n = read("<Q")
            return bytes(take(n)).decode("utf-8", errors="replace")

        def read_value(t):
            if t in _SCALAR:
                v = read(_SCALAR[t])
                return bool(v) if t == BOOL else v
            if t == STRING:
                return read_string()
            if t == ARRAY:
                et = read("<I")
                count = read("<Q")
                if et == ARRAY:
                    raise GgufError("gguf: nested arrays are not supported")
                if et == STRING:
                    return [read_string() for _ in range(count)]
                fmt = _SCALAR[et]
                size = struct.calcsize(fmt)
                raw = bytes(take(count * size))
                return list(np.frombuffer(raw, dtype=np.dtype(fmt)))
            raise GgufError(f"gguf: unknown metadata type {t}")

        if read("<I") != GGUF_MAGIC:
            raise GgufError("gguf: bad magic, not a GGUF file")
        self.version = read("<I")
        if self.version not in (2, 3):
            raise GgufError(f"gguf: unsupported version {self.version}")
        n_tensors = read("<Q")
        n_kv = read("<Q")
        self.metadata = {}
        for _ in range(n_kv):
            key = read_string()
            t = read("<I")
            if key in self.metadata:
                raise GgufError(f"gguf: duplicate metadata key '{key}'")
            self.metadata[key] = read_value(t)
        self.tensors = {}
        order = []
        for _ in range(n_tensors):
            name = read_string()
            nd = read("<I")
            if nd > 4:
                raise GgufError(f"gguf: tensor '{name}' has too many dimensions")
            dims = tuple(read("<Q") for _ in range(nd))
            ttype = read("<I")
            off = read("<Q")
            if name in self.tensors:
                raise GgufError(f"gguf: duplicate tensor name '{name}'")
            self.tensors[name] = Tensor(name, dims, ttype, off)
            order.append(name)
        align = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        pos += (align - pos % align) % align
        self.data_offset = pos
        for name in order:
            t = self.tensors[name]
            if t.type not in BLOCK:
                continue
            be, bb = BLOCK[t.type]
            n = t.n_elements()
            if n % be:
                raise GgufError(f"gguf: tensor '{name}' size is not a whole number of blocks")
            size = n // be * bb
            start = self.data_offset + t.offset
            if start + size > len(self._map):
                raise GgufError(f"gguf: tensor '{name}' data lies outside the file")
            t.data = self._map[start:start + size]

    def get(self, key, default=None):
        return self.metadata.get(key, default)

    def tensor(self, name):
        return self.tensors.get(name)


class GgufWriter:
    """Streams a GGUF v3 file: metadata and tensor infos first, then aligned tensor data."""

    def __init__(self, alignment: int = DEFAULT_ALIGNMENT):
        self.alignment = alignment
        self.kv = []       # (key, type, value)
        self.infos = []    # (name, dims, type, nbytes, producer)

    def add(self, key, vtype, value):
        self.kv.append((key, vtype, value))

    def add_tensor(self, name, dims, ttype, producer):
        """``producer()`` returns the tensor's bytes (uint8 array) when the data is written."""
        be, bb = BLOCK[ttype]
        n = 1
        for d in dims:
            n *= d
        assert n % be == 0, name
        self.infos.append((name, tuple(dims), ttype, n // be * bb, producer))

    @staticmethod
    def _string(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def _value(self, vtype, value) -> bytes:
        if vtype in _SCALAR:
            return struct.pack(_SCALAR[vtype], value)
        if vtype == STRING:
            return self._string(value)
        if vtype == ARRAY:
            et, items = value
            out = struct.pack("<IQ", et, len(items))
            if et == STRING:
                return out + b"".join(self._string(s) for s in items)
            return out + np.asarray(items, dtype=np.dtype(_SCALAR[et])).tobytes()
        raise GgufError(f"unknown metadata type {vtype}")

    def write(self, path: str):
        kvs = [(k, t, v) for k, t, v in self.kv]
        if self.alignment != DEFAULT_ALIGNMENT:
            kvs.append(("general.alignment", U32, self.alignment))
        head = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, 3, len(self.infos), len(kvs)))
        for k, t, v in kvs:
            head += self._string(k) + struct.pack("<I", t) + self._value(t, v)
        offset = 0
        offsets = []
        for name, dims, ttype, nbytes, _ in self.infos:
            offsets.append(offset)
            head += self._string(name) + struct.pack("<I", len(dims))
            head += b"".join(struct.pack("<Q", d) for d in dims)
            head += struct.pack("<IQ", ttype, offset)
            offset += nbytes
            offset += (self.alignment - offset % self.alignment) % self.alignment
        head += b"\0" * ((self.alignment - len(head) % self.alignment) % self.alignment)
        with open(path, "wb") as f:
            f.write(head)
            pos = 0
            for (name, dims, ttype, nbytes, producer), off in zip(self.infos, offsets):
                assert pos == off
                data = np.ascontiguousarray(producer(), dtype=np.uint8).reshape(-1)
                if data.size != nbytes:
                    raise GgufError(f"tensor '{name}': producer gave {data.size} bytes, expected {nbytes}")
                f.write(data.tobytes())
                pos += nbytes
                pad = (self.alignment - pos % self.alignment) % self.alignment
                f.write(b"\0" * pad)
                pos += pad
