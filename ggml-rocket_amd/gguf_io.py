"""GGUF v3 files: a streaming writer and a memory-mapped reader.

The container format ggml models ship in, as ggml's published GGUF specification lays it out
(the `gguf` Python package is not available here, so this is our own code for the format):
little-endian; header = magic "GGUF", u32 version 3, u64 tensor count, u64 metadata count; then
the metadata pairs (string key, u32 value type, value), then one info record per tensor (string
name, u32 n_dims, u64 ne[n_dims] innermost first, u32 ggml type, u64 offset into the data
section), then padding to `general.alignment` (32 unless the metadata says otherwise), then the
data section, each tensor at its offset, every offset a multiple of the alignment. A string is
a u64 byte length and the UTF-8 bytes; an array is a u32 element type, a u64 count and the
elements.

Used to write the random-init Llama-3-8B GGUF of the end-to-end prefill configuration
(`llama3_gguf.py`) and to read one back for the GGUF-driven plugin path (`bench.py --host-path
--gguf`) and the tests.
"""
import mmap
import os
import struct

import numpy as np

MAGIC = b"GGUF"
VERSION = 3
DEFAULT_ALIGNMENT = 32

# metadata value types
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}

# ggml block facts of the types the writer emits: (values per block, bytes per block)
TYPE_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176),
              14: (256, 210), 30: (1, 2)}


class GGUFError(ValueError):
    pass


def tensor_nbytes(ggml_type: int, ne) -> int:
    if ggml_type not in TYPE_BLOCK:
        raise GGUFError(f"no block size known for ggml type {ggml_type}")
    blk, size = TYPE_BLOCK[ggml_type]
    if ne[0] % blk:
        raise GGUFError(f"ne0 = {ne[0]} is not a whole number of {blk}-value blocks")
    n = 1
    for d in ne:
        n *= int(d)
    return n // blk * size


def _pack_string(s) -> bytes:
    b = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _pack_value(vtype: int, value) -> bytes:
    if vtype == STRING:
        return _pack_string(value)
    if vtype == ARRAY:
        etype, items = value
        if etype == STRING:
            return struct.pack("<IQ", STRING, len(items)) + b"".join(_pack_string(x) for x in items)
        if etype == ARRAY:
            raise GGUFError("arrays of arrays are not written")
        arr = np.asarray(items, dtype=np.dtype(_SCALAR[etype]))
        return struct.pack("<IQ", etype, len(arr)) + arr.tobytes()
    return struct.pack(_SCALAR[vtype], value)


def _infer_type(value):
    if isinstance(value, bool):
        return BOOL, value
    if isinstance(value, int):
        return (UINT32 if 0 <= value < 2**32 else INT64), value
    if isinstance(value, float):
        return FLOAT32, value
    if isinstance(value, str):
        return STRING, value
    raise GGUFError(f"give the type of {value!r} explicitly as (type, value)")


class Writer:
    """Streams a GGUF file: declare every tensor first (name, type, ne), then write their data
    in the declared order (the header goes out with the first data)."""

    def __init__(self, path: str, alignment: int = DEFAULT_ALIGNMENT):
        self.path = path
        self.alignment = alignment
        self.kv = []          # (key, type, value)
        self.tensors = []     # (name, type, ne, nbytes, offset)
        self._data_off = 0
        self._f = None
        self._next = 0
        if alignment != DEFAULT_ALIGNMENT:
            self.add("general.alignment", alignment, UINT32)

    def add(self, key: str, value, vtype: int = None):
        """A metadata pair; `vtype` defaults to u32 / i64 / f32 / str / bool by the value.
        An array: add(key, (element type, items), ARRAY)."""
        if vtype is None:
            vtype, value = _infer_type(value)
        self.kv.append((key, vtype, value))

    def add_tensor(self, name: str, ggml_type: int, ne):
        if self._f is not None:
            raise GGUFError("tensors must be declared before the header is written")
        nb = tensor_nbytes(ggml_type, ne)
        off = self._data_off
        self.tensors.append((name, ggml_type, [int(x) for x in ne], nb, off))
        self._data_off = (off + nb + self.alignment - 1) // self.alignment * self.alignment

    def _header(self) -> bytes:
        out = [MAGIC, struct.pack("<IQQ", VERSION, len(self.tensors), len(self.kv))]
        for key, vtype, v in self.kv:
            out.append(_pack_string(key) + struct.pack("<I", vtype) + _pack_value(vtype, v))
        for name, t, ne, _, off in self.tensors:
            out.append(_pack_string(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) +
                       struct.pack("<IQ", t, off))
        h = b"".join(out)
        pad = (-len(h)) % self.alignment
        return h + b"\0" * pad

    def write_data(self, data):
        """Data of the next declared tensor: bytes, or a numpy array of exactly its size."""
        if self._f is None:
            self._f = open(self.path, "wb")
            self._f.write(self._header())
            self._base = self._f.tell()
        if self._next >= len(self.tensors):
            raise GGUFError("more data than declared tensors")
        name, _, _, nb, off = self.tensors[self._next]
        buf = memoryview(np.ascontiguousarray(data).view(np.uint8).reshape(-1)) if isinstance(data, np.ndarray) \
            else memoryview(data)
        if buf.nbytes != nb:
            raise GGUFError(f"{name}: {buf.nbytes} bytes given, {nb} declared")
        pos = self._f.tell() - self._base
        if pos != off:
            self._f.write(b"\0" * (off - pos))
        self._f.write(buf)
        self._next += 1

    def close(self):
        if self._f is None:
            self._f = open(self.path, "wb")
            self._f.write(self._header())
        if self._next != len(self.tensors):
            self._f.close()
            raise GGUFError(f"{len(self.tensors) - self._next} declared tensors have no data")
        self._f.close()
        self._f = None


class Reader:
    """A GGUF file mapped read-only: `kv` (key -> value), `tensors` (name -> (type, ne, offset
    in the file, nbytes)), and `data(name)`, a uint8 view of the tensor's bytes in the map."""

    def __init__(self, path: str):
        self.path = path
        self._fh = open(path, "rb")
        size = os.fstat(self._fh.fileno()).st_size
        if size < 24:
            raise GGUFError("file too short for a GGUF header")
        self._mm = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        self._p = 0
        if self._take(4) != MAGIC:
            raise GGUFError("not a GGUF file (bad magic)")
        version, n_tensors, n_kv = struct.unpack("<IQQ", self._take(20))
        if version != VERSION:
            raise GGUFError(f"GGUF version {version}, only {VERSION} is read")
        self.kv = {}
        for _ in range(n_kv):
            key = self._string()
            (vtype,) = struct.unpack("<I", self._take(4))
            self.kv[key] = self._value(vtype)
        infos = []
        for _ in range(n_tensors):
            name = self._string()
            (nd,) = struct.unpack("<I", self._take(4))
            ne = list(struct.unpack(f"<{nd}Q", self._take(8 * nd)))
            t, off = struct.unpack("<IQ", self._take(12))
            infos.append((name, t, ne, off))
        align = int(self.kv.get("general.alignment", DEFAULT_ALIGNMENT))
        base = (self._p + align - 1) // align * align
        self.data_offset = base
        self.tensors = {}
        for name, t, ne, off in infos:
            if off % align:
                raise GGUFError(f"{name}: offset {off} is not aligned to {align}")
            nb = tensor_nbytes(t, ne) if t in TYPE_BLOCK else None
            if nb is not None and base + off + nb > size:
                raise GGUFError(f"{name}: data runs past the end of the file")
            self.tensors[name] = (t, ne, base + off, nb)

    def _take(self, n):
        b = self._mm[self._p:self._p + n]
        if len(b) != n:
            raise GGUFError("truncated GGUF header")
        self._p += n
        return b

    def _string(self):
        (n,) = struct.unpack("<Q", self._take(8))
        return self._take(n).decode("utf-8")

    def _value(self, vtype):
        if vtype == STRING:
            return self._string()
        if vtype == ARRAY:
            etype, n = struct.unpack("<IQ", self._take(12))
            if etype == STRING:
                return [self._string() for _ in range(n)]
            dt = np.dtype(_SCALAR[etype])
            return np.frombuffer(self._take(n * dt.itemsize), dtype=dt).copy()
        if vtype not in _SCALAR:
            raise GGUFError(f"unknown metadata value type {vtype}")
        fmt = _SCALAR[vtype]
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def data(self, name: str) -> np.ndarray:
        t, ne, off, nb = self.tensors[name]
        if nb is None:
            raise GGUFError(f"{name}: type {t} has no block size known here")
        return np.frombuffer(self._mm, dtype=np.uint8, count=nb, offset=off)

    def close(self):
        self._mm.close()
        self._fh.close()
