"""GGUF container: the on-disk format boundary of the decode path.

Reader: GgufParser (crates/janus-engine/src/formats/gguf/parser.rs:21-139,
143-481): magic "GGUF", versions 2..3, little-endian counts, typed metadata
key/value pairs (arrays of scalars or strings; nested arrays rejected),
tensor infos, and tensor data at the header end rounded up to
`general.alignment` (default 32). The file is memory-mapped and tensor bytes
are returned as read-only views, never copied.

Sizes follow the reference's GGMLType table (types.rs:79-106, 150-187):
32-element blocks for Q4_0/Q4_1/Q5_0/Q5_1/Q8_0/Q8_1 and 256-element
super-blocks for the K and IQ families, with the reference's byte counts
(it gives Q4_1, Q5_1 and Q8_1 the byte sizes of Q4_0, Q5_0 and Q8_0; none of
them is accepted by the weight upload, so no tensor of the path depends on it).

Config: model_config_from_gguf_metadata (model/config.rs:377-446): the
architecture prefix (default "llama"), head_count_kv falling back to
head_count, rope.freq_base falling back to the unprefixed key and then 5e5,
vocab_size falling back to the tokenizer token list, context_length clamped to
4096, integer fields accepting any non-negative integer type and float fields
any numeric type (config.rs:304-359).

Writer: produces files of the same layout (version 3); used to build test
models and by callers that export weights.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np

GGUF_MAGIC = b"GGUF"
VERSION_MIN, VERSION_MAX = 2, 3
DEFAULT_ALIGNMENT = 32
HARD_MAX_SEQ_LEN = 4096   # config.rs:13

# metadata value types (types.rs MetadataValueType)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
_INTEGER = (UINT8, INT8, UINT16, INT16, UINT32, INT32, UINT64, INT64)

# GGML tensor types accepted by the reader (types.rs:9-75) -> (elements, bytes) per block
_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 18), 6: (32, 22), 7: (32, 22), 8: (32, 34), 9: (32, 34),
          10: (256, 82), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
          16: (1, 1), 17: (1, 2), 18: (1, 4), 19: (1, 8), 20: (1, 8),
          21: (256, 66), 22: (256, 74), 23: (256, 98), 24: (256, 50), 25: (256, 136), 26: (256, 110),
          27: (256, 82), 28: (256, 136), 29: (256, 56)}


class GgufError(Exception):
    """formats/gguf/error.rs:5-43."""


class InvalidMagic(GgufError):
    pass


class UnsupportedVersion(GgufError):
    pass


class IncompleteData(GgufError):
    pass


class InvalidTensorType(GgufError):
    pass


class ParseError(GgufError):
    pass


class ConfigError(Exception):
    """model/config.rs ConfigError: MissingGgufMetadata / InvalidConfig."""


class MissingGgufMetadata(ConfigError):
    pass


@dataclass(frozen=True)
class Value:
    """A typed metadata value (types.rs MetadataValue). Strings stay bytes;
    arrays hold Values of their element type."""
    type: int
    value: Any


@dataclass
class TensorInfo:
    name: str
    dimensions: list
    ggml_type: int
    offset: int

    def element_count(self) -> int:
        n = 1
        for d in self.dimensions:
            n *= int(d)
        return n

    def size_bytes(self) -> int:
        per, nbytes = _BLOCK[self.ggml_type]
        return (self.element_count() + per - 1) // per * nbytes

    def shape_nk(self) -> tuple[int, int]:
        """(n rows, k columns) in the [out][in] order of the weight upload;
        GGUF lists the innermost dimension first, k = 0 for 1-D tensors."""
        if len(self.dimensions) == 1:
            return int(self.dimensions[0]), 0
        if len(self.dimensions) == 2:
            return int(self.dimensions[1]), int(self.dimensions[0])
        raise ParseError(f"tensor {self.name}: {len(self.dimensions)}-D tensors are not weights of the path")


@dataclass
class GgufMetadata:
    version: int
    metadata: dict
    tensors: list
    alignment: int
    data_offset: int = 0
    extra: dict = field(default_factory=dict)


class _Reader:
    def __init__(self, buf):
        self.buf = buf
        self.pos = 0

    def take(self, n: int, what: str):
        if self.pos + n > len(self.buf):
            raise IncompleteData(f"Failed to read {what}")
        b = self.buf[self.pos:self.pos + n]
        self.pos += n
        return b

    def scalar(self, fmt: str, what: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt), what))[0]

    def bytes_(self, what: str) -> bytes:
        n = self.scalar("<Q", f"{what} length")
        return bytes(self.take(n, f"{what} data"))

    def key(self) -> str:
        b = self.bytes_("string")
        try:
            return b.decode("utf-8")
        except UnicodeDecodeError as e:
            raise ParseError(f"Invalid UTF-8 in metadata key: {e}") from None


def _value(r: _Reader, vtype: int, in_array: bool = False) -> Value:
    if vtype in _SCALAR:
        v = r.scalar(_SCALAR[vtype], "metadata value")
        return Value(vtype, (v != 0) if vtype == BOOL else v)
    if vtype == STRING:
        return Value(STRING, r.bytes_("string"))
    if vtype == ARRAY:
        if in_array:
            raise ParseError("Nested arrays not supported")
        etype = r.scalar("<I", "array element type")
        if etype not in _SCALAR and etype not in (STRING, ARRAY):
            raise ParseError(f"Invalid metadata value type {etype}")
        count = r.scalar("<Q", "array count")
        return Value(ARRAY, [_value(r, etype, True) for _ in range(count)])
    raise ParseError(f"Invalid metadata value type {vtype}")


def parse_header(buf) -> GgufMetadata:
    """parse_header (parser.rs:73-139) over a bytes-like object."""
    r = _Reader(buf)
    magic = bytes(r.take(4, "magic number"))
    if magic != GGUF_MAGIC:
        raise InvalidMagic(f"invalid GGUF magic {magic!r}")
    version = r.scalar("<I", "version")
    if not VERSION_MIN <= version <= VERSION_MAX:
        raise UnsupportedVersion(f"unsupported GGUF version {version}")
    n_tensors = r.scalar("<Q", "tensor count")
    n_kv = r.scalar("<Q", "metadata count")
    md = {}
    for _ in range(n_kv):
        k = r.key()
        md[k] = _value(r, r.scalar("<I", "metadata type"))
    a = md.get("general.alignment")
    alignment = a.value if a is not None and a.type == UINT32 else DEFAULT_ALIGNMENT
    if alignment == 0:
        raise ParseError("general.alignment must be positive")
    tensors = []
    for _ in range(n_tensors):
        name = r.key()
        nd = r.scalar("<I", "tensor dimension count")
        dims = [r.scalar("<Q", "tensor dimension") for _ in range(nd)]
        t = r.scalar("<I", "tensor type")
        off = r.scalar("<Q", "tensor offset")
        if t not in _BLOCK:
            raise InvalidTensorType(f"invalid tensor type {t}")
        tensors.append(TensorInfo(name, dims, t, off))
    data_offset = (r.pos + alignment - 1) // alignment * alignment
    return GgufMetadata(version, md, tensors, alignment, data_offset)


class GgufFile:
    """GgufParser::open: a memory-mapped GGUF file."""

    def __init__(self, path):
        self.path = Path(path)
        with open(self.path, "rb") as f:
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        self.meta = parse_header(self._mm)

    @property
    def tensors(self) -> list:
        return self.meta.tensors

    def get(self, key: str):
        v = self.meta.metadata.get(key)
        return None if v is None else v.value

    def tensor_data(self, t: TensorInfo) -> np.ndarray:
        """get_tensor_data (parser.rs:63-67) as a read-only uint8 view."""
        start = self.meta.data_offset + t.offset
        end = start + t.size_bytes()
        if end > len(self._mm):
            raise IncompleteData(f"tensor {t.name}: data runs past the end of the file")
        return np.frombuffer(self._mm, dtype=np.uint8, count=end - start, offset=start)

    def close(self) -> None:
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                pass   # views handed out are still alive: the mapping goes when they do
            self._mm = None


# ---- config (model/config.rs:304-446) ----------------------------------------

def metadata_as_u32(md: dict, key: str) -> int:
    v = md.get(key)
    if v is None:
        raise MissingGgufMetadata(key)
    if v.type not in _INTEGER or v.value < 0:
        raise ConfigError(f"GGUF metadata '{key}' is not a positive integer")
    if v.value > 0xFFFFFFFF:
        raise ConfigError(f"GGUF metadata '{key}' does not fit in u32")
    return int(v.value)


def metadata_as_f32(md: dict, key: str) -> float:
    v = md.get(key)
    if v is None:
        raise MissingGgufMetadata(key)
    if v.type not in _INTEGER and v.type not in (FLOAT32, FLOAT64):
        raise ConfigError(f"GGUF metadata '{key}' is not numeric")
    return float(np.float32(v.value))


@dataclass
class GgufConfig:
    hidden: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    max_seq_len: int
    rms_eps: float
    rope_theta: float


def config_from_metadata(md: dict, tokenizer_vocab_size: int = 0) -> GgufConfig:
    arch_v = md.get("general.architecture")
    arch = "llama"
    if arch_v is not None and arch_v.type == STRING:
        v = arch_v.value   # bytes as parsed, or str in metadata built in memory
        try:
            arch = v.decode("utf-8") if isinstance(v, (bytes, bytearray)) else str(v)
        except UnicodeDecodeError:
            pass
    hidden = metadata_as_u32(md, f"{arch}.embedding_length")
    layers = metadata_as_u32(md, f"{arch}.block_count")
    heads = metadata_as_u32(md, f"{arch}.attention.head_count")
    try:
        kv_heads = metadata_as_u32(md, f"{arch}.attention.head_count_kv")
    except MissingGgufMetadata:
        kv_heads = heads
    ffn = metadata_as_u32(md, f"{arch}.feed_forward_length")
    max_seq = min(metadata_as_u32(md, f"{arch}.context_length"), HARD_MAX_SEQ_LEN)
    eps = metadata_as_f32(md, f"{arch}.attention.layer_norm_rms_epsilon")
    try:
        theta = metadata_as_f32(md, f"{arch}.rope.freq_base")
    except MissingGgufMetadata:
        try:
            theta = metadata_as_f32(md, "rope.freq_base")
        except MissingGgufMetadata:
            theta = 500000.0
    try:
        vocab = metadata_as_u32(md, f"{arch}.vocab_size")
    except MissingGgufMetadata:
        toks = md.get("tokenizer.ggml.tokens")
        vocab = len(toks.value) if toks is not None and toks.type == ARRAY else tokenizer_vocab_size
    if heads == 0:
        raise ConfigError("attention.head_count must be positive")
    return GgufConfig(hidden, layers, heads, kv_heads, hidden // heads, ffn, vocab, max_seq, eps, theta)


# ---- writer --------------------------------------------------------------------

def _pack_value(v: Value, in_array: bool = False) -> bytes:
    if v.type in _SCALAR:
        return struct.pack(_SCALAR[v.type], int(v.value) if v.type == BOOL else v.value)
    if v.type == STRING:
        b = v.value.encode("utf-8") if isinstance(v.value, str) else bytes(v.value)
        return struct.pack("<Q", len(b)) + b
    if v.type == ARRAY and not in_array:
        items = list(v.value)
        et = items[0].type if items else UINT32
        if any(x.type != et for x in items):
            raise ParseError("array elements must share one type")
        return struct.pack("<IQ", et, len(items)) + b"".join(_pack_value(x, True) for x in items)
    raise ParseError(f"cannot write metadata value type {v.type}")


def write(path, metadata: dict, tensors: list, alignment: int = DEFAULT_ALIGNMENT, version: int = 3) -> None:
    """Write a GGUF file. metadata: key -> Value. tensors: (name, dims innermost
    first, ggml_type, bytes-like) in file order; each tensor's data is placed
    at an offset rounded up to the alignment."""
    md = dict(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        md["general.alignment"] = Value(UINT32, alignment)
    head = [GGUF_MAGIC, struct.pack("<IQQ", version, len(tensors), len(md))]
    for k, v in md.items():
        kb = k.encode("utf-8")
        head += [struct.pack("<Q", len(kb)), kb, struct.pack("<I", v.type), _pack_value(v)]
    blobs, off = [], 0
    for name, dims, gtype, data in tensors:
        raw = np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes()
        info = TensorInfo(name, list(dims), gtype, 0)
        if gtype not in _BLOCK:
            raise InvalidTensorType(f"invalid tensor type {gtype}")
        if len(raw) != info.size_bytes():
            raise ParseError(f"tensor {name}: {len(raw)} bytes, dims need {info.size_bytes()}")
        off = (off + alignment - 1) // alignment * alignment
        nb = name.encode("utf-8")
        head += [struct.pack("<Q", len(nb)), nb, struct.pack("<I", len(dims)),
                 struct.pack(f"<{len(dims)}Q", *dims), struct.pack("<IQ", gtype, off)]
        blobs.append((off, raw))
        off += len(raw)
    header = b"".join(head)
    data_offset = (len(header) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (data_offset - len(header)))
        pos = 0
        for o, raw in blobs:
            f.write(b"\0" * (o - pos))
            f.write(raw)
            pos = o + len(raw)
