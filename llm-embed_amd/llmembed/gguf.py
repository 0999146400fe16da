"""GGUF v2/v3 reader and writer (numpy memory-mapped tensor data).

The reader follows the rules of the reference reader, internal/gguf/reader.go:
  * header: magic 0x46554747, version 2 or 3, u64 tensor and KV counts (:228-240);
  * KV values are typed; getters type-switch strictly (u32 / f32 / string, :293-342);
  * tensor info: name, u32 n_dims, u64 dims (dims[0] = inner K), u32 type, u64 offset;
  * the data section starts at the next 32-byte boundary after the tensor table, and
    `general.alignment` is ignored (:266-269);
  * ByteSize = nel / blockSize * typeSize (:196-204).
The writer produces files that reader accepts (32-byte aligned tensors).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from . import quant

MAGIC = 0x46554747
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
           T_F32: "<f", T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}
ALIGN = 32

# BlockSize / TypeSize of the reference's GGMLType (reader.go:106-194), for ByteSize.
_BS = {0: 1, 1: 1, 2: 32, 3: 32, 6: 32, 7: 32, 8: 32, 9: 32, 10: 256, 11: 256, 12: 256,
       13: 256, 14: 256, 15: 256, 24: 1, 25: 1, 26: 1, 27: 1}
_TS = {0: 4, 1: 2, 2: 18, 3: 20, 6: 22, 7: 24, 8: 34, 9: 36, 10: 84, 11: 110, 12: 144,
       13: 176, 14: 210, 15: 292, 24: 1, 25: 2, 26: 4, 27: 8}


class GGUFError(ValueError):
    pass


@dataclass
class TensorInfo:
    name: str
    dims: list
    type: int
    offset: int

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n

    @property
    def byte_size(self) -> int:
        bs, ts = _BS.get(self.type, 0), _TS.get(self.type, 0)
        if bs == 0 or ts == 0:
            return 0
        return (self.n_elements // bs) * ts


@dataclass
class GGUFFile:
    path: str
    version: int
    kv: dict = field(default_factory=dict)       # key -> (type, value)
    tensors: dict = field(default_factory=dict)  # name -> TensorInfo
    data_offset: int = 0
    _mm: np.ndarray | None = None

    def get_u32(self, key):
        t = self.kv.get(key)
        return t[1] if t is not None and t[0] == T_U32 else None

    def get_f32(self, key):
        t = self.kv.get(key)
        return t[1] if t is not None and t[0] == T_F32 else None

    def get_str(self, key):
        t = self.kv.get(key)
        return t[1] if t is not None and t[0] == T_STR else None

    def tensor_bytes(self, name: str) -> np.ndarray:
        ti = self.tensors.get(name)
        if ti is None:
            raise GGUFError(f"tensor {name!r} not found")
        if self._mm is None:
            self._mm = np.memmap(self.path, dtype=np.uint8, mode="r")
        o = self.data_offset + ti.offset
        n = ti.byte_size
        if o + n > self._mm.shape[0]:
            raise GGUFError(f"tensor {name!r} extends past end of file")
        return self._mm[o:o + n]


class _Reader:
    def __init__(self, f):
        self.f = f

    def read(self, n):
        b = self.f.read(n)
        if len(b) != n:
            raise GGUFError("unexpected end of file")
        return b

    def u32(self):
        return struct.unpack("<I", self.read(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.read(8))[0]

    def str(self):
        n = self.u64()
        return self.read(n).decode("utf-8", errors="replace")

    def value(self, t):
        if t in _SCALAR:
            fmt = _SCALAR[t]
            return struct.unpack(fmt, self.read(struct.calcsize(fmt)))[0]
        if t == T_STR:
            return self.str()
        if t == T_ARR:
            et = self.u32()
            n = self.u64()
            if et == T_STR:
                return [self.str() for _ in range(n)]
            if et in _SCALAR:
                fmt = _SCALAR[et]
                sz = struct.calcsize(fmt)
                raw = self.read(sz * n)
                return list(struct.unpack("<" + fmt[1] * n, raw))
            return [self.value(et) for _ in range(n)]
        raise GGUFError(f"unknown value type: {t}")


def read(path: str) -> GGUFFile:
    with open(path, "rb") as f:
        r = _Reader(f)
        magic = r.u32()
        if magic != MAGIC:
            raise GGUFError(f"invalid magic: 0x{magic:08x} (expected 0x{MAGIC:08x})")
        version = r.u32()
        if version < 2 or version > 3:
            raise GGUFError(f"unsupported version: {version}")
        n_t, n_kv = r.u64(), r.u64()
        g = GGUFFile(path=path, version=version)
        for _ in range(n_kv):
            key = r.str()
            t = r.u32()
            g.kv[key] = (t, r.value(t))
        for _ in range(n_t):
            name = r.str()
            nd = r.u32()
            dims = [r.u64() for _ in range(nd)]
            ty = r.u32()
            off = r.u64()
            g.tensors[name] = TensorInfo(name, dims, ty, off)
        pos = f.tell()
        g.data_offset = (pos + ALIGN - 1) & ~(ALIGN - 1)
    return g


def _pack_str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_kv(key: str, t: int, v) -> bytes:
    out = _pack_str(key) + struct.pack("<I", t)
    if t in _SCALAR:
        return out + struct.pack(_SCALAR[t], v)
    if t == T_STR:
        return out + _pack_str(v)
    if t == T_ARR:
        et, items = v
        out += struct.pack("<IQ", et, len(items))
        if et == T_STR:
            return out + b"".join(_pack_str(s) for s in items)
        return out + b"".join(struct.pack(_SCALAR[et], x) for x in items)
    raise GGUFError(f"cannot write value type {t}")


def write(path: str, kvs: list, tensors: list) -> None:
    """kvs: [(key, type, value)]; tensors: [(name, dims, ggml_type, uint8 ndarray)]."""
    head = struct.pack("<IIQQ", MAGIC, 3, len(tensors), len(kvs))
    head += b"".join(_pack_kv(k, t, v) for k, t, v in kvs)
    off = 0
    infos = []
    for name, dims, ty, data in tensors:
        nb = int(np.asarray(data).nbytes)
        ti = TensorInfo(name, list(dims), ty, off)
        if ti.byte_size != nb:
            raise GGUFError(f"{name}: {nb} bytes, ByteSize says {ti.byte_size}")
        infos.append(_pack_str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
                     + struct.pack("<IQ", ty, off))
        off += (nb + ALIGN - 1) & ~(ALIGN - 1)
    head += b"".join(infos)
    pad = ((len(head) + ALIGN - 1) & ~(ALIGN - 1)) - len(head)
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * pad)
        for name, dims, ty, data in tensors:
            b = np.ascontiguousarray(data, dtype=np.uint8).tobytes()
            f.write(b)
            p = ((len(b) + ALIGN - 1) & ~(ALIGN - 1)) - len(b)
            if p:
                f.write(b"\0" * p)


__all__ = ["read", "write", "GGUFFile", "TensorInfo", "GGUFError", "quant"]
