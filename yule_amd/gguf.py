"""GGUF v3 files: a writer, and a reader over libyule_hip.so's parser.

Format (yule-core/src/gguf.rs:255-432): little-endian header
  magic u32 "GGUF" | version u32 = 3 | tensor_count u64 | kv_count u64
then kv_count pairs (string key, u32 value type, value), then tensor_count
infos (string name, u32 n_dims, n_dims x u64 dims, u32 GGUF dtype, u64
offset), then the data section at the header end rounded up to
general.alignment (default 32).  Strings are u64 length + bytes; arrays are
u32 element type + u64 length + elements.  Tensor offsets are relative to
the data section; dims are GGUF order, dims[0] the row length.

The writer places each tensor at the next multiple of the alignment, so the
files it makes satisfy the reader's bounds and overlap checks.  The reader
is the C parser (yule_hip_gguf_*): it maps the file read-only, checks it as
gguf.rs does, and hands out tensor bytes from the mapping.
"""
from __future__ import annotations

import ctypes as C
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .formats import DType

GGUF_MAGIC = 0x46554747
GGUF_VERSION = 3
DEFAULT_ALIGNMENT = 32
MAX_STRING_LEN = 1024 * 1024
MAX_TENSOR_COUNT = 100_000
MAX_KV_COUNT = 100_000
MAX_ARRAY_LEN = 10_000_000
MAX_DIMS = 8


class ValueType:
    """GGUF metadata value types (gguf.rs:19-32)."""
    U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)


_SCALAR = {ValueType.U8: "<B", ValueType.I8: "<b", ValueType.U16: "<H", ValueType.I16: "<h",
           ValueType.U32: "<I", ValueType.I32: "<i", ValueType.F32: "<f", ValueType.BOOL: "<B",
           ValueType.U64: "<Q", ValueType.I64: "<q", ValueType.F64: "<d"}


@dataclass(frozen=True)
class Value:
    """An explicitly typed metadata value; `elem` is the element type of an array."""
    type: int
    value: object
    elem: int | None = None


def _infer(v) -> Value:
    if isinstance(v, Value):
        return v
    if isinstance(v, bool):
        return Value(ValueType.BOOL, v)
    if isinstance(v, int):
        return Value(ValueType.U32 if 0 <= v < 2**32 else ValueType.I64 if v < 0 else ValueType.U64, v)
    if isinstance(v, float):
        return Value(ValueType.F32, v)
    if isinstance(v, str):
        return Value(ValueType.STRING, v)
    if isinstance(v, (list, tuple)):
        elem = _infer(v[0]).type if v else ValueType.U32
        return Value(ValueType.ARRAY, list(v), elem)
    raise TypeError(f"no GGUF type for {type(v).__name__}")


def _string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _payload(t: int, v, elem: int | None = None) -> bytes:
    if t == ValueType.STRING:
        return _string(v)
    if t == ValueType.ARRAY:
        if elem is None:
            elem = _infer(v[0]).type if v else ValueType.U32
        return struct.pack("<IQ", elem, len(v)) + b"".join(_payload(elem, x) for x in v)
    if t == ValueType.BOOL:
        return struct.pack("<B", 1 if v else 0)
    return struct.pack(_SCALAR[t], v)


def encode_kv(key: str, value) -> bytes:
    v = _infer(value)
    return _string(key) + struct.pack("<I", v.type) + _payload(v.type, v.value, v.elem)


@dataclass
class TensorEntry:
    name: str
    dtype: int
    dims: tuple            # GGUF order: (cols, rows) for a matrix
    data: bytes | np.ndarray


def write_gguf(path: Path | str, metadata: dict, tensors: list[TensorEntry]) -> int:
    """Write a GGUF v3 file; returns the data-section offset.  A
    `general.alignment` entry in `metadata` sets the alignment (its value is
    taken as u32, as the reader does)."""
    align = int(_infer(metadata["general.alignment"]).value) if "general.alignment" in metadata else DEFAULT_ALIGNMENT
    head = [struct.pack("<IIQQ", GGUF_MAGIC, GGUF_VERSION, len(tensors), len(metadata))]
    head += [encode_kv(k, v) for k, v in metadata.items()]
    blobs, off = [], 0
    for t in tensors:
        raw = np.ascontiguousarray(t.data).view(np.uint8).tobytes() if isinstance(t.data, np.ndarray) else t.data
        head.append(_string(t.name) + struct.pack("<I", len(t.dims)) + struct.pack(f"<{len(t.dims)}Q", *t.dims) +
                    struct.pack("<IQ", int(t.dtype), off))
        blobs.append((off, raw))
        off = (off + len(raw) + align - 1) // align * align
    header = b"".join(head)
    data_offset = (len(header) + align - 1) // align * align
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (data_offset - len(header)))
        pos = 0
        for o, raw in blobs:
            f.write(b"\0" * (o - pos))
            f.write(raw)
            pos = o + len(raw)
    return data_offset


class _TensorInfo(C.Structure):
    """yule_gguf_tensor"""
    _fields_ = [("name", C.c_char_p), ("dtype", C.c_uint32), ("n_dims", C.c_uint32), ("dims", C.c_uint64 * 8),
                ("offset", C.c_uint64), ("size_bytes", C.c_uint64), ("data", C.c_void_p)]


@dataclass(frozen=True)
class TensorInfo:
    """TensorInfo (yule-core/src/tensor.rs): name, GGUF dtype id, dims in
    GGUF order, offset relative to the data section, size in bytes."""
    name: str
    dtype: int
    dims: tuple
    offset: int
    size_bytes: int

    @property
    def num_elements(self) -> int:
        return int(np.prod(self.dims, dtype=np.uint64)) if self.dims else 1


class GgufFile:
    """A parsed, mapped GGUF file (GgufFile, gguf.rs:465-619).  Parse
    errors raise YuleGpuError with code YULE_ERR_PARSE (6), unreadable files
    code YULE_ERR_IO (7)."""

    def __init__(self, path: Path | str):
        from .backend import load_library
        self._lib = load_library()
        h = C.c_void_p()
        self._check(self._lib.yule_hip_gguf_open(str(path).encode(), C.byref(h)))
        self._g = h
        ver, n_t, n_kv = C.c_uint32(), C.c_uint64(), C.c_uint64()
        align, doff = C.c_uint64(), C.c_uint64()
        self._check(self._lib.yule_hip_gguf_header(h, C.byref(ver), C.byref(align), C.byref(doff), C.byref(n_t),
                                                   C.byref(n_kv)))
        self.version, self.alignment, self.data_offset = ver.value, align.value, doff.value
        self.n_kv = n_kv.value
        self.tensors = [self._info(i) for i in range(n_t.value)]

    def _check(self, rc: int) -> None:
        if rc:
            from .backend import YuleGpuError
            raise YuleGpuError(rc, self._lib.yule_hip_last_error().decode(errors="replace"))

    def _info(self, i: int) -> TensorInfo:
        t = _TensorInfo()
        self._check(self._lib.yule_hip_gguf_tensor(self._g, i, C.byref(t)))
        return TensorInfo(t.name.decode(), t.dtype, tuple(t.dims[:t.n_dims]), t.offset, t.size_bytes)

    def close(self) -> None:
        if getattr(self, "_g", None):
            self._lib.yule_hip_gguf_close(self._g)
            self._g = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def tensor_data(self, name: str) -> np.ndarray:
        """A copy of the tensor's bytes (tensor_data, gguf.rs:595-606)."""
        t = _TensorInfo()
        self._check(self._lib.yule_hip_gguf_find(self._g, name.encode(), C.byref(t)))
        return np.frombuffer(C.string_at(t.data, t.size_bytes), dtype=np.uint8).copy()

    def get_u32(self, key: str) -> int | None:
        v = C.c_uint32()
        return v.value if self._lib.yule_hip_gguf_get_u32(self._g, key.encode(), C.byref(v)) == 0 else None

    def get_f64(self, key: str) -> float | None:
        v = C.c_double()
        return v.value if self._lib.yule_hip_gguf_get_f64(self._g, key.encode(), C.byref(v)) == 0 else None

    def get_str(self, key: str) -> str | None:
        v = C.c_char_p()
        return v.value.decode() if self._lib.yule_hip_gguf_get_str(self._g, key.encode(), C.byref(v)) == 0 else None

    def get_array_len(self, key: str) -> int | None:
        v = C.c_uint64()
        return v.value if self._lib.yule_hip_gguf_get_array_len(self._g, key.encode(), C.byref(v)) == 0 else None


def model_metadata(cfg, arch: str = "llama", name: str = "synthetic") -> dict:
    """llama.* keys GgufFile::to_loaded_model reads (gguf.rs:493-599)."""
    return {
        "general.architecture": arch,
        "general.name": name,
        "general.alignment": Value(ValueType.U32, DEFAULT_ALIGNMENT),
        f"{arch}.block_count": Value(ValueType.U32, cfg.n_layers),
        f"{arch}.context_length": Value(ValueType.U32, cfg.max_seq),
        f"{arch}.embedding_length": Value(ValueType.U32, cfg.dim),
        f"{arch}.feed_forward_length": Value(ValueType.U32, cfg.ff_dim),
        f"{arch}.attention.head_count": Value(ValueType.U32, cfg.n_heads),
        f"{arch}.attention.head_count_kv": Value(ValueType.U32, cfg.n_kv_heads),
        f"{arch}.attention.layer_norm_rms_epsilon": Value(ValueType.F32, cfg.norm_eps),
        f"{arch}.rope.freq_base": Value(ValueType.F32, cfg.rope_base),
        "tokenizer.ggml.vocab_size": Value(ValueType.U32, cfg.vocab),
    }


__all__ = ["GGUF_MAGIC", "GGUF_VERSION", "ValueType", "Value", "TensorEntry", "write_gguf", "encode_kv", "GgufFile",
           "TensorInfo", "model_metadata", "DType"]
