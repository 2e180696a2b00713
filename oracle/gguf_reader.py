"""Pure-Python GGUF v3 reader: a restatement of the reference's file parser.

TEST INFRASTRUCTURE ONLY (part of the oracle).  It is written independently of
the product's C++ reader so that each checks the other.

Follows src/file_parser/:
  gguf_header.rs:13-24        u32 magic (not validated), u32 version, u64 counts
  gguf_metadata.rs:15-25      key string, u32 value type, typed value
  gguf_metadata_value.rs:49-80 scalar types, strings, recursive arrays
  gguf_tensor_info.rs:25-65   name, u32 n_dims, u64 dims, u32 ggml type, u64 offset
  gguf_file.rs:10,44-46       data starts at the next multiple of 32 (fixed)
  binary_reader_common.rs     little-endian readers; bool must be 0 or 1
"""
from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

# GGUFType (gguf_metadata_value.rs:10-24)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           U64: "<Q", I64: "<q", F64: "<d"}

# GGMLType ids (ggml_type.rs:8-41) and their storage (ggml_type.rs:45-62)
GGML_NAMES = {0: "F32", 1: "F16", 2: "Q4_0", 3: "Q4_1", 6: "Q5_0", 7: "Q5_1", 8: "Q8_0",
              9: "Q8_1", 10: "Q2_K", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K",
              15: "Q8_K", 16: "IQ2_XXS", 17: "IQ2_XS", 18: "IQ3_XXS", 19: "IQ1_S",
              20: "IQ4_NL", 21: "IQ3_S", 22: "IQ2_S", 23: "IQ4_XS", 24: "I8", 25: "I16",
              26: "I32", 27: "I64", 28: "F64", 29: "IQ1_M", 30: "BF16", 34: "TQ1_0",
              35: "TQ2_0", 39: "MXFP4"}
BLOCK = {0: (1, 4), 30: (1, 2), 8: (32, 34), 2: (32, 18)}  # type -> (elems, bytes)
ALIGN = 32


class GGUFError(Exception):
    """Malformed or unsupported file (the reference's io::Error / Error cases)."""


@dataclass
class TensorInfo:
    name: str
    dims: tuple
    ggml_type: int
    offset: int

    @property
    def numel(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    def nbytes(self) -> int:
        """tensor_bytes_size (gguf_tensor_info.rs:52-65)."""
        if self.ggml_type not in BLOCK:
            raise GGUFError(f"UnsupportedQuantScheme({GGML_NAMES[self.ggml_type]})")
        elems, nb = BLOCK[self.ggml_type]
        if self.numel % elems:
            raise GGUFError(f"UnsupportedQuantScheme({GGML_NAMES[self.ggml_type]})")
        return self.numel // elems * nb


class _Cursor:
    def __init__(self, buf):
        self.buf = buf
        self.pos = 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise GGUFError("unexpected end of file")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(U64)
        try:
            return self.take(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GGUFError("invalid utf-8 string") from e

    def value(self, t: int):
        if t == BOOL:
            b = self.scalar(U8)
            if b not in (0, 1):
                raise GGUFError("Invalid bool data!")
            return bool(b)
        if t == STRING:
            return self.string()
        if t == ARRAY:
            at = self.scalar(U32)
            if at > F64:
                raise GGUFError("Invalid GGUF array type!")
            n = self.scalar(U64)
            return (at, [self.value(at) for _ in range(n)])
        return self.scalar(t)


class GGUFFile:
    """Header, typed metadata {key: (type, value)}, tensor infos, data offset."""

    def __init__(self, path: str):
        self.path = path
        self.mm = np.memmap(path, dtype=np.uint8, mode="r")
        c = _Cursor(self.mm)
        self.magic = c.scalar(U32)
        self.version = c.scalar(U32)
        n_tensors = c.scalar(U64)
        n_kv = c.scalar(U64)
        self.metadata = {}
        for _ in range(n_kv):
            key = c.string()
            t = c.scalar(U32)
            if t > F64:
                raise GGUFError("Invalid GGUF Type!")
            self.metadata[key] = (t, c.value(t))
        self.tensors = {}
        for _ in range(n_tensors):
            name = c.string()
            nd = c.scalar(U32)
            dims = tuple(c.scalar(U64) for _ in range(nd))
            gt = c.scalar(U32)
            if gt not in GGML_NAMES:
                raise GGUFError(f"unknown GGML type id {gt} in tensor {name!r}")
            off = c.scalar(U64)
            self.tensors[name] = TensorInfo(name, dims, gt, off)
        self.data_offset = (c.pos + ALIGN - 1) & ~(ALIGN - 1)

    def tensor_bytes(self, name: str) -> np.ndarray:
        """Zero-copy view of one tensor's bytes (NonOwningTensor::from_info,
        src/kernels/tensor.rs:152-169)."""
        info = self.tensors[name]
        start = self.data_offset + info.offset
        end = start + info.nbytes()
        if end > len(self.mm):
            raise GGUFError(f"tensor {name!r} runs past the end of the file")
        return self.mm[start:end]
