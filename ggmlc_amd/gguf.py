"""GGUF v3 reader and writer — the on-disk format ggmlc compiles models to.

Layout (little endian), as ggml's `gguf.cpp` reads it and ggmlc's writer
(`python/ggmlc/serialization/gguf.py:225-362`) emits it:

    "GGUF"  u32 version (3)  u64 n_tensors  u64 n_kv
    n_kv x  { string key, u32 value_type, value }
    n_tensors x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset }
    zero padding to `general.alignment` (default 32)
    tensor data; each tensor starts at data_start + offset, offsets aligned

A string is u64 length + UTF-8 bytes; an array value is u32 element type + u64
count + elements. ggmlc stores its execution graph as the JSON string
`ggmlc.graph_spec` (see :mod:`ggmlc_amd.graph_spec`) and the graph's parameters
as tensors named like the graph's tensors.

The reader maps the file (numpy memmap) and hands out tensor bytes without
copying; it runs on the host and never touches a device.
"""

from __future__ import annotations

import io
import mmap
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any, BinaryIO

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32

# value types (gguf.h)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)

_SCALAR = {
    UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i",
    FLOAT32: "<f", BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d",
}
_NUMPY = {
    UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16, UINT32: np.uint32,
    INT32: np.int32, FLOAT32: np.float32, BOOL: np.bool_, UINT64: np.uint64, INT64: np.int64,
    FLOAT64: np.float64,
}

# ggml tensor types this path reads and writes (ggml.h enum ggml_type), with
# (block elements, block bytes)
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 8: ("Q8_0", 32, 34),
    24: ("I8", 1, 1), 25: ("I16", 1, 2), 26: ("I32", 1, 4), 27: ("I64", 1, 8), 28: ("F64", 1, 8),
    30: ("BF16", 1, 2),
}


def tensor_nbytes(ggml_type: int, ne: list[int]) -> int:
    """Bytes of a contiguous tensor of this type and shape (ggml_nbytes for a
    contiguous tensor: rows of ne[0] elements in whole blocks)."""
    if ggml_type not in GGML_TYPES:
        raise ValueError(f"unsupported ggml type {ggml_type}")
    _, blk, size = GGML_TYPES[ggml_type]
    if ne and ne[0] % blk:
        raise ValueError(f"ne[0] = {ne[0]} is not a whole number of {blk}-element blocks")
    n = 1
    for d in ne[1:]:
        n *= int(d)
    return (int(ne[0]) // blk * size if ne else size) * n


@dataclass
class TensorInfo:
    name: str
    ne: list[int]       # ggml order: ne[0] is the innermost dimension
    ggml_type: int
    offset: int         # from the start of the data section
    nbytes: int


class GGUFReader:
    """Parsed GGUF v3 file (path or bytes). `metadata` maps key -> value
    (arrays become lists; strings str); `value_types` keeps each key's GGUF type;
    `tensors` maps name -> TensorInfo; `tensor_bytes(name)` is a zero-copy view."""

    def __init__(self, source: str | Path | bytes | bytearray | memoryview):
        if isinstance(source, (str, Path)):
            self.path = Path(source)
            with open(self.path, "rb") as f:
                self._buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        else:
            self.path = None
            self._buf = memoryview(bytes(source))
        self._parse()

    # -- parsing ------------------------------------------------------------------
    def _take(self, n: int) -> bytes:
        if self._pos + n > len(self._buf):
            raise ValueError("GGUF: truncated file")
        b = bytes(self._buf[self._pos:self._pos + n])
        self._pos += n
        return b

    def _u(self, fmt: str):
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def _string(self) -> str:
        return self._take(self._u("<Q")).decode("utf-8")

    def _value(self, vtype: int):
        if vtype == STRING:
            return self._string()
        if vtype == ARRAY:
            etype, count = self._u("<I"), self._u("<Q")
            if etype == STRING:
                return [self._string() for _ in range(count)]
            if etype == ARRAY:
                return [self._value(ARRAY) for _ in range(count)]
            if etype not in _SCALAR:
                raise ValueError(f"GGUF: bad array element type {etype}")
            size = struct.calcsize(_SCALAR[etype])
            arr = np.frombuffer(self._take(size * count), dtype=np.dtype(_NUMPY[etype]).newbyteorder("<"))
            return arr.tolist()
        if vtype not in _SCALAR:
            raise ValueError(f"GGUF: bad value type {vtype}")
        return self._u(_SCALAR[vtype])

    def _parse(self) -> None:
        self._pos = 0
        if self._take(4) != GGUF_MAGIC:
            raise ValueError("GGUF: magic header mismatch")
        self.version = self._u("<I")
        if self.version not in (2, 3):
            raise ValueError(f"GGUF: unsupported version {self.version}")
        n_tensors, n_kv = self._u("<Q"), self._u("<Q")
        self.metadata: dict[str, Any] = {}
        self.value_types: dict[str, tuple[int, int | None]] = {}
        for _ in range(n_kv):
            key = self._string()
            vtype = self._u("<I")
            etype = None
            if vtype == ARRAY:  # peek the element type for round trips
                etype = struct.unpack_from("<I", self._buf, self._pos)[0]
            self.metadata[key] = self._value(vtype)
            self.value_types[key] = (vtype, etype)
        self.tensors: dict[str, TensorInfo] = {}
        order = []
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._u("<I")
            ne = [self._u("<Q") for _ in range(n_dims)]
            gtype = self._u("<I")
            offset = self._u("<Q")
            info = TensorInfo(name, ne, gtype, offset, tensor_nbytes(gtype, ne) if gtype in GGML_TYPES else -1)
            if name in self.tensors:
                raise ValueError(f"GGUF: duplicate tensor name {name!r}")
            self.tensors[name] = info
            order.append(name)
        self.tensor_order = order
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise ValueError(f"GGUF: alignment {self.alignment} is not a power of two")
        self.data_start = (self._pos + self.alignment - 1) // self.alignment * self.alignment
        for t in self.tensors.values():
            if t.offset % self.alignment:
                raise ValueError(f"GGUF: tensor {t.name!r} offset {t.offset} is not aligned")
            if t.nbytes >= 0 and self.data_start + t.offset + t.nbytes > len(self._buf):
                raise ValueError(f"GGUF: tensor {t.name!r} runs past the end of the file")

    # -- access -------------------------------------------------------------------
    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 array (no copy)."""
        t = self.tensors[name]
        if t.nbytes < 0:
            raise ValueError(f"GGUF: tensor {name!r} has unsupported type {t.ggml_type}")
        start = self.data_start + t.offset
        return np.frombuffer(self._buf, dtype=np.uint8, count=t.nbytes, offset=start)

    def tensor_array(self, name: str) -> np.ndarray:
        """Plain-typed tensors (F32, F16, I32, ...) as numpy arrays in C order
        (shape = reversed ne without the leading unit dims: ne [K, N, 1, 1] is [N, K]);
        quantized tensors as uint8 rows [..., rows, row_bytes]."""
        t = self.tensors[name]
        raw = self.tensor_bytes(name)
        kind, blk, size = GGML_TYPES[t.ggml_type]
        ne = list(t.ne) or [1]
        while len(ne) > (2 if blk > 1 else 1) and ne[-1] == 1:
            ne.pop()
        shape = list(reversed(ne))
        if blk > 1:
            return raw.reshape(shape[:-1] + [t.ne[0] // blk * size])
        dt = {"F32": np.float32, "F16": np.float16, "I8": np.int8, "I16": np.int16, "I32": np.int32,
              "I64": np.int64, "F64": np.float64, "BF16": np.uint16}[kind]
        return raw.view(dt).reshape(shape)


class GGUFWriter:
    """GGUF v3 writer: typed metadata, then tensors laid out at aligned offsets in
    the order they were added (the order of ggmlc's writer)."""

    def __init__(self, alignment: int = DEFAULT_ALIGNMENT):
        if alignment <= 0 or alignment & (alignment - 1):
            raise ValueError("alignment must be a power of two")
        self.alignment = alignment
        self._kv: list[tuple[str, int, bytes]] = []
        self._tensors: list[tuple[str, list[int], int, Any]] = []

    # -- metadata -----------------------------------------------------------------
    @staticmethod
    def _enc_string(s: str) -> bytes:
        b = s.encode("utf-8")
        return struct.pack("<Q", len(b)) + b

    def add(self, key: str, value_type: int, value: Any, elem_type: int | None = None) -> None:
        if value_type == STRING:
            payload = self._enc_string(value)
        elif value_type == ARRAY:
            if elem_type is None:
                raise ValueError("array needs an element type")
            out = io.BytesIO()
            out.write(struct.pack("<IQ", elem_type, len(value)))
            for v in value:
                out.write(self._enc_string(v) if elem_type == STRING else struct.pack(_SCALAR[elem_type], v))
            payload = out.getvalue()
        else:
            payload = struct.pack(_SCALAR[value_type], value)
        self._kv.append((key, value_type, payload))

    def add_string(self, key: str, v: str) -> None:
        self.add(key, STRING, v)

    def add_uint32(self, key: str, v: int) -> None:
        self.add(key, UINT32, v)

    def add_int32(self, key: str, v: int) -> None:
        self.add(key, INT32, v)

    def add_float32(self, key: str, v: float) -> None:
        self.add(key, FLOAT32, float(v))

    def add_bool(self, key: str, v: bool) -> None:
        self.add(key, BOOL, bool(v))

    def add_string_array(self, key: str, v: list[str]) -> None:
        self.add(key, ARRAY, list(v), STRING)

    def add_float_array(self, key: str, v: list[float]) -> None:
        self.add(key, ARRAY, [float(x) for x in v], FLOAT32)

    # -- tensors ------------------------------------------------------------------
    def add_tensor(self, name: str, ne: list[int], ggml_type: int, data) -> None:
        """data: bytes-like of exactly tensor_nbytes(ggml_type, ne) bytes."""
        mv = memoryview(data).cast("B")
        want = tensor_nbytes(ggml_type, ne)
        if mv.nbytes != want:
            raise ValueError(f"tensor {name!r}: {mv.nbytes} bytes, shape/type need {want}")
        if len(name.encode("utf-8")) >= 64:
            raise ValueError(f"tensor name {name!r} is too long for ggml (< 64 bytes)")
        self._tensors.append((name, [int(d) for d in ne], int(ggml_type), mv))

    # -- output -------------------------------------------------------------------
    def _pad(self, n: int) -> int:
        return (-n) % self.alignment

    def write(self, out: BinaryIO) -> int:
        pos = 0

        def put(b: bytes | memoryview) -> None:
            nonlocal pos
            out.write(b)
            pos += len(b) if isinstance(b, bytes) else b.nbytes

        put(GGUF_MAGIC + struct.pack("<IQQ", GGUF_VERSION, len(self._tensors), len(self._kv)))
        for key, vtype, payload in self._kv:
            put(self._enc_string(key) + struct.pack("<I", vtype) + payload)
        offsets, off = [], 0
        for _, ne, gtype, mv in self._tensors:
            off += self._pad(off)
            offsets.append(off)
            off += mv.nbytes
        for (name, ne, gtype, _), o in zip(self._tensors, offsets):
            put(self._enc_string(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) +
                struct.pack("<IQ", gtype, o))
        put(b"\0" * self._pad(pos))
        data_start = pos
        for (_, _, _, mv), o in zip(self._tensors, offsets):
            put(b"\0" * (data_start + o - pos))
            put(mv)
        put(b"\0" * self._pad(pos))
        return pos

    def to_bytes(self) -> bytes:
        buf = io.BytesIO()
        self.write(buf)
        return buf.getvalue()

    def write_file(self, path: str | Path) -> Path:
        p = Path(path)
        p.parent.mkdir(parents=True, exist_ok=True)
        with open(p, "wb") as f:
            self.write(f)
        return p
