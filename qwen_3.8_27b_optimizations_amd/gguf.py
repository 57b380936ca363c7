"""Memory-mapped reader for GGUF model files (format version 2 and 3), for
bringing IQ4_XS weight tensors into HBM as the raw 136-byte super-blocks the
kernels read.

The reference reads its model with gguf-py (tools/dump_matmul_fixtures.py:
26-31, 168-170), which is not part of this build; this module follows the
published GGUF layout:

    magic "GGUF" | u32 version | u64 tensor_count | u64 kv_count
    kv:     string key | u32 value_type | value
    tensor: string name | u32 n_dims | u64 ne[n_dims] | u32 ggml_type | u64 offset
    padding to `general.alignment` (default 32), then the tensor data; each
    offset is relative to the start of the data and aligned
    string: u64 length | bytes (UTF-8, no terminator)
    array:  u32 element type | u64 count | elements

ne[0] is the length of a row (K for a weight matrix), ne[1] the number of
rows (N), as in ggml and in the reference's extraction
(tools/dump_matmul_fixtures.py:77-78).  Nothing in a file is executed:
values are decoded with struct/numpy from a read-only map.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass, field

import numpy as np

GGUF_MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<?", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
_NP = {UINT8: "<u1", INT8: "<i1", UINT16: "<u2", INT16: "<i2", UINT32: "<u4", INT32: "<i4", FLOAT32: "<f4",
       BOOL: "<u1", UINT64: "<u8", INT64: "<i8", FLOAT64: "<f8"}
# the short names llama.cpp prints for them (startup-log.txt:26-66 of the reference shows str, u32, i32, f32, arr)
TYPE_NAMES = {UINT8: "u8", INT8: "i8", UINT16: "u16", INT16: "i16", UINT32: "u32", INT32: "i32", FLOAT32: "f32",
              BOOL: "bool", STRING: "str", ARRAY: "arr", UINT64: "u64", INT64: "i64", FLOAT64: "f64"}

# ggml tensor types: id -> (name, elements per block, bytes per block)
GGML_TYPES = {
    0: ("f32", 1, 4), 1: ("f16", 1, 2), 2: ("q4_0", 32, 18), 3: ("q4_1", 32, 20), 6: ("q5_0", 32, 22),
    7: ("q5_1", 32, 24), 8: ("q8_0", 32, 34), 9: ("q8_1", 32, 36), 10: ("q2_K", 256, 84), 11: ("q3_K", 256, 110),
    12: ("q4_K", 256, 144), 13: ("q5_K", 256, 176), 14: ("q6_K", 256, 210), 15: ("q8_K", 256, 292),
    16: ("iq2_xxs", 256, 66), 17: ("iq2_xs", 256, 74), 18: ("iq3_xxs", 256, 98), 19: ("iq1_s", 256, 50),
    20: ("iq4_nl", 32, 18), 21: ("iq3_s", 256, 110), 22: ("iq2_s", 256, 82), 23: ("iq4_xs", 256, 136),
    24: ("i8", 1, 1), 25: ("i16", 1, 2), 26: ("i32", 1, 4), 27: ("i64", 1, 8), 28: ("f64", 1, 8),
    29: ("iq1_m", 256, 56), 30: ("bf16", 1, 2),
}
GGML_TYPE_IQ4_XS = 23

# general.file_type values (llama_ftype) this reader names; the reference's
# model reports 30 as "IQ4_XS - 4.25 bpw" (startup-log.txt:63,73)
FILE_TYPES = {0: "all F32", 1: "F16", 30: "IQ4_XS - 4.25 bpw"}


class GGUFError(ValueError):
    pass


@dataclass
class TensorInfo:
    name: str
    ne: tuple           # ggml order: ne[0] = row length
    ggml_type: int
    offset: int         # from the start of the data section
    nbytes: int
    data: np.ndarray = field(repr=False, default=None)  # read-only uint8 view into the map

    @property
    def type_name(self) -> str:
        return GGML_TYPES.get(self.ggml_type, (f"type{self.ggml_type}",))[0]

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.ne:
            n *= d
        return n


class _Cursor:
    def __init__(self, buf, pos: int = 0):
        self.buf, self.pos = buf, pos

    def take(self, n: int) -> memoryview:
        if n < 0 or self.pos + n > len(self.buf):
            raise GGUFError(f"truncated file: need {n} bytes at offset {self.pos}, have {len(self.buf) - self.pos}")
        v = memoryview(self.buf)[self.pos:self.pos + n]
        self.pos += n
        return v

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar(UINT64)
        try:
            return bytes(self.take(n)).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GGUFError(f"string at offset {self.pos - n} is not UTF-8") from e

    def value(self, t: int):
        if t == STRING:
            return self.string()
        if t == ARRAY:
            et = self.scalar(UINT32)
            n = self.scalar(UINT64)
            if et == STRING:
                return [self.string() for _ in range(n)]
            if et == ARRAY:
                return [self.value(ARRAY) for _ in range(n)]
            if et not in _NP:
                raise GGUFError(f"unknown array element type {et}")
            a = np.frombuffer(self.take(n * np.dtype(_NP[et]).itemsize), dtype=_NP[et]).copy()
            return a.astype(bool) if et == BOOL else a
        if t not in _SCALAR:
            raise GGUFError(f"unknown metadata value type {t}")
        return self.scalar(t)


class GGUFReader:
    """Header, metadata and tensor table of a GGUF file; tensor bytes are
    views into a read-only memory map (nothing is read until used)."""

    def __init__(self, path: str):
        self.path = path
        with open(path, "rb") as f:
            size = os.fstat(f.fileno()).st_size
            if size < 24:
                raise GGUFError(f"{path}: {size} bytes is too short for a GGUF header")
            self._map = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        c = _Cursor(self._map)
        if bytes(c.take(4)) != GGUF_MAGIC:
            raise GGUFError(f"{path}: not a GGUF file (bad magic)")
        self.version = c.scalar(UINT32)
        if self.version not in (2, 3):
            raise GGUFError(f"{path}: GGUF version {self.version} is not supported (2 and 3 are)")
        n_tensors = c.scalar(UINT64)
        n_kv = c.scalar(UINT64)
        self.metadata: dict = {}
        self.metadata_types: dict = {}
        for _ in range(n_kv):
            key = c.string()
            t = c.scalar(UINT32)
            pos = c.pos
            self.metadata[key] = c.value(t)
            if t == ARRAY:
                et = struct.unpack_from("<I", self._map, pos)[0]
                self.metadata_types[key] = (ARRAY, et)
            else:
                self.metadata_types[key] = (t, None)
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GGUFError(f"general.alignment {self.alignment} is not a power of two")
        infos = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.scalar(UINT32)
            if nd > 8:
                raise GGUFError(f"tensor {name}: {nd} dimensions")
            ne = tuple(c.scalar(UINT64) for _ in range(nd))
            t = c.scalar(UINT32)
            off = c.scalar(UINT64)
            infos.append((name, ne, t, off))
        self.data_offset = (c.pos + self.alignment - 1) // self.alignment * self.alignment
        self.tensors: list[TensorInfo] = []
        self._by_name: dict = {}
        for name, ne, t, off in infos:
            if off % self.alignment:
                raise GGUFError(f"tensor {name}: offset {off} is not {self.alignment}-aligned")
            nbytes = self._tensor_bytes(name, ne, t)
            start = self.data_offset + off
            if nbytes is not None and start + nbytes > size:
                raise GGUFError(f"tensor {name}: data [{start}, {start + nbytes}) runs past the end ({size})")
            data = None
            if nbytes is not None:
                data = np.frombuffer(self._map, dtype=np.uint8, count=nbytes, offset=start)
            ti = TensorInfo(name, ne, t, off, nbytes if nbytes is not None else -1, data)
            if name in self._by_name:
                raise GGUFError(f"duplicate tensor name {name}")
            self.tensors.append(ti)
            self._by_name[name] = ti

    @staticmethod
    def _tensor_bytes(name: str, ne: tuple, t: int):
        if t not in GGML_TYPES:
            return None  # listed, but its extent is unknown to this reader
        _, blk, bb = GGML_TYPES[t]
        n_el = 1
        for d in ne:
            n_el *= d
        if ne and ne[0] % blk:
            raise GGUFError(f"tensor {name}: row length {ne[0]} is not a multiple of the {blk}-element block")
        return n_el // blk * bb

    # -- queries ---------------------------------------------------------
    def tensor(self, name: str) -> TensorInfo:
        try:
            return self._by_name[name]
        except KeyError:
            raise KeyError(f"{self.path}: no tensor {name!r}") from None

    def type_counts(self) -> dict:
        """{type name: tensor count}, like llama.cpp's '- type iq4_xs: 440 tensors'."""
        out: dict = {}
        for t in self.tensors:
            out[t.type_name] = out.get(t.type_name, 0) + 1
        return out

    def file_type(self) -> str:
        ft = self.metadata.get("general.file_type")
        return FILE_TYPES.get(int(ft), f"unknown ({ft})") if ft is not None else "unspecified"

    def iq4xs_matrix(self, name: str):
        """(raw blocks as uint8 [N * K/256 * 136], K, N) of a 2-D IQ4_XS tensor."""
        t = self.tensor(name)
        if t.ggml_type != GGML_TYPE_IQ4_XS:
            raise GGUFError(f"tensor {name} is {t.type_name}, not iq4_xs")
        if len(t.ne) != 2:
            raise GGUFError(f"tensor {name} has {len(t.ne)} dimensions, not 2")
        K, N = int(t.ne[0]), int(t.ne[1])
        return t.data, K, N

    def close(self) -> None:
        self.tensors, self._by_name = [], {}
        try:
            self._map.close()
        except BufferError:
            pass  # tensor views handed out are still alive; the map is released with the last of them

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def to_device(blocks: np.ndarray, device=None, chunk_bytes: int = 256 << 20):
    """Copy raw tensor bytes (e.g. GGUFReader.iq4xs_matrix(...)[0]) into a new
    uint8 device tensor, streaming through one pinned host buffer."""
    import torch

    n = int(blocks.size)
    out = torch.empty(n, dtype=torch.uint8, device=device or "cuda")
    stage = torch.empty(min(n, chunk_bytes), dtype=torch.uint8, pin_memory=True)
    stage_np = stage.numpy()
    for lo in range(0, n, chunk_bytes):
        hi = min(n, lo + chunk_bytes)
        stage_np[:hi - lo] = blocks[lo:hi]
        out[lo:hi].copy_(stage[:hi - lo], non_blocking=False)
    return out
