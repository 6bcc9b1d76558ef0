"""GGUF checkpoints on the host side of the token loop.

`GgufFile` mirrors the managed reader (Gguf/GgufFile.cs:53-347): the file is
mapped read-only, the header's metadata and tensor table are parsed with a
bounds check on every read, a file too short for its own tensor table is
rejected up front, and tensor bytes are zero-copy views into the mapping.
Those views are what `load_gguf` hands to `jev_bind_tensor`, exactly as the
managed loader would pass `GetTensorPointer` (WeightMatrix.cs:53-65): the
library copies the bytes into HBM during the call, so the mapping can be
closed once the model is bound.

`write_gguf` writes a version-3 file with the key names the converter uses
(tools/convert_shieldstral_to_gguf.py:309-369) and the reader expects
(ModelConfig.cs:62-112, TekkenTokenizer.cs:86-110), so a synthetic checkpoint
can go through the unchanged loading path.

Errors follow the reference: InvalidDataException -> `DataError`,
NotSupportedException -> `NotSupportedError`, IOException (truncated file) ->
`OSError`, KeyNotFoundException -> `KeyError`.
"""
from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass
from typing import Iterable, Optional

import numpy as np

from . import _lib as L
from .model import MinistralModel, ModelConfig

GGUF_MAGIC = 0x46554747  # "GGUF" read as a little-endian u32
DEFAULT_ALIGNMENT = 32

# GGUF metadata value types (GgufFile.cs:11-17).
(UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY,
 UINT64, INT64, FLOAT64) = range(13)

_SCALAR = {  # value type -> (struct code, bytes)
    UINT8: ("B", 1), INT8: ("b", 1), UINT16: ("H", 2), INT16: ("h", 2), UINT32: ("I", 4), INT32: ("i", 4),
    FLOAT32: ("f", 4), UINT64: ("Q", 8), INT64: ("q", 8), FLOAT64: ("d", 8),
}
_NUMPY = {UINT8: "<u1", INT8: "<i1", UINT16: "<u2", INT16: "<i2", UINT32: "<u4", INT32: "<i4",
          FLOAT32: "<f4", UINT64: "<u8", INT64: "<i8", FLOAT64: "<f8"}

# ggml_type ids and block geometry (elements per block, bytes per block): the
# on-disk format's own table, as GgmlTypeInfo states it (GgmlType.cs:10-105).
GGML_TYPES = {
    "F32": (0, 1, 4), "F16": (1, 1, 2), "Q4_0": (2, 32, 18), "Q4_1": (3, 32, 20), "Q5_0": (6, 32, 22),
    "Q5_1": (7, 32, 24), "Q8_0": (8, 32, 34), "Q8_1": (9, 32, 36), "Q2_K": (10, 256, 84), "Q3_K": (11, 256, 110),
    "Q4_K": (12, 256, 144), "Q5_K": (13, 256, 176), "Q6_K": (14, 256, 210), "Q8_K": (15, 256, 292),
    "IQ2_XXS": (16, 256, 66), "IQ2_XS": (17, 256, 74), "IQ3_XXS": (18, 256, 98), "IQ1_S": (19, 256, 50),
    "IQ4_NL": (20, 32, 18), "IQ3_S": (21, 256, 110), "IQ2_S": (22, 256, 82), "IQ4_XS": (23, 256, 136),
    "I8": (24, 1, 1), "I16": (25, 1, 2), "I32": (26, 1, 4), "I64": (27, 1, 8), "F64": (28, 1, 8),
    "IQ1_M": (29, 256, 56), "BF16": (30, 1, 2), "TQ1_0": (34, 256, 54), "TQ2_0": (35, 256, 66),
    "MXFP4": (39, 32, 17),
}
_GEOMETRY = {tid: (bs, ts) for tid, bs, ts in GGML_TYPES.values()}
GGML_TYPE_NAME = {tid: name for name, (tid, _, _) in GGML_TYPES.items()}


class NotSupportedError(Exception):
    """NotSupportedException: a well-formed file this runtime does not handle."""


def block_geometry(ggml_type: int) -> tuple[int, int]:
    """(elements per block, bytes per block); GgmlTypeInfo.BlockSize/TypeSize (GgmlType.cs:52-97)."""
    try:
        return _GEOMETRY[int(ggml_type)]
    except KeyError:
        raise NotSupportedError(f"Unknown GGML tensor type: {ggml_type}") from None


def row_bytes(ggml_type: int, elements: int) -> int:
    """GgmlTypeInfo.RowBytes (GgmlType.cs:112-120)."""
    bs, ts = block_geometry(ggml_type)
    if elements % bs != 0:
        raise ValueError(f"{GGML_TYPE_NAME.get(ggml_type, ggml_type)} rows must be a multiple of {bs} "
                         f"elements; got {elements}.")
    return elements // bs * ts


@dataclass(frozen=True)
class GgufTensorInfo:
    """One entry of the tensor table (GgufFile.cs:19-46); shape[0] varies fastest."""
    name: str
    shape: tuple
    ggml_type: int
    offset: int  # from the start of the tensor-data section

    @property
    def element_count(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def row_elements(self) -> int:
        return self.shape[0] if self.shape else 0

    @property
    def row_count(self) -> int:
        n = 1
        for d in self.shape[1:]:
            n *= d
        return n

    @property
    def byte_count(self) -> int:
        return row_bytes(self.ggml_type, self.row_elements) * self.row_count


class GgufFile:
    """Memory-mapped GGUF reader (GgufFile.cs:53-347).  Use as a context manager or call close()."""

    def __init__(self, path: str):
        self.path = str(path)
        if not os.path.isfile(self.path):
            raise FileNotFoundError(f"GGUF not found: {self.path}")
        self.metadata: dict = {}
        self.tensors: dict[str, GgufTensorInfo] = {}
        self.version = 0
        self.data_offset = 0
        self._mm: Optional[mmap.mmap] = None
        with open(self.path, "rb") as f:
            self._length = os.fstat(f.fileno()).st_size
            if self._length > 0:
                self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        # A rejected header releases the mapping before the exception leaves:
        # there is no instance for the caller to close.
        try:
            self._parse()
        except BaseException:
            self.close()
            raise

    # ------------------------------------------------------------- parsing
    def _window(self, at: int, count: int):
        if at < 0 or count < 0 or at + count > self._length:
            raise L.DataError(L.JEV_EDATA, f"{self.path}: read of {count} bytes at {at} runs past the file.")
        return self._mm[at:at + count]

    def _unpack(self, code: str, size: int):
        v = struct.unpack("<" + code, self._window(self._cur, size))[0]
        self._cur += size
        return v

    def _string(self) -> str:
        n = self._unpack("Q", 8)
        if n > 0x7FFFFFFF:
            raise L.DataError(L.JEV_EDATA, f"{self.path}: implausible string length {n}.")
        s = bytes(self._window(self._cur, n)).decode("utf-8", errors="replace")
        self._cur += n
        return s

    def _value(self, vtype: int):
        if vtype in _SCALAR:
            return self._unpack(*_SCALAR[vtype])
        if vtype == BOOL:
            return self._unpack("B", 1) != 0
        if vtype == STRING:
            return self._string()
        if vtype == ARRAY:
            return self._array()
        raise NotSupportedError(f"{self.path}: unknown GGUF value type {vtype}.")

    def _array(self):
        elem = self._unpack("I", 4)
        n = self._unpack("Q", 8)
        if n > 0x7FFFFFFF:
            raise L.DataError(L.JEV_EDATA, f"{self.path}: implausible array length {n}.")
        if elem == STRING:
            return [self._string() for _ in range(n)]
        if elem in _NUMPY:
            size = np.dtype(_NUMPY[elem]).itemsize * n
            arr = np.frombuffer(self._window(self._cur, size), dtype=_NUMPY[elem]).copy()
            self._cur += size
            return arr
        if elem == BOOL:
            arr = np.frombuffer(self._window(self._cur, n), dtype=np.uint8) != 0
            self._cur += n
            return arr
        if elem == ARRAY:
            raise NotSupportedError(f"{self.path}: nested GGUF arrays are not supported.")
        raise NotSupportedError(f"{self.path}: unknown GGUF array element type {elem}.")

    def _parse(self) -> None:
        self._cur = 0
        magic = self._unpack("I", 4)
        if magic != GGUF_MAGIC:
            raise L.DataError(L.JEV_EDATA, f"{self.path} is not a GGUF file (magic 0x{magic:08X}).")
        self.version = self._unpack("I", 4)
        if self.version not in (2, 3):
            raise NotSupportedError(f"GGUF version {self.version} is not supported (expected 2 or 3).")
        n_tensors = self._unpack("Q", 8)
        n_kv = self._unpack("Q", 8)
        for _ in range(n_kv):
            key = self._string()
            self.metadata[key] = self._value(self._unpack("I", 4))
        for _ in range(n_tensors):
            name = self._string()
            dims = self._unpack("I", 4)
            shape = tuple(self._unpack("Q", 8) for _ in range(dims))
            ttype = self._unpack("I", 4)
            offset = self._unpack("Q", 8)
            self.tensors[name] = GgufTensorInfo(name, shape, ttype, offset)
        align = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        self.data_offset = self._cur + (align - self._cur % align) % align
        self._check_length()

    def _check_length(self) -> None:
        """ThrowIfTruncated (GgufFile.cs:166-186): a short file fails here, not inside a kernel."""
        required, last = self.data_offset, None
        for t in self.tensors.values():
            try:
                end = self.data_offset + t.offset + t.byte_count
            except (NotSupportedError, ValueError):
                continue
            if end > required:
                required, last = end, t.name
        if self._length >= required:
            return
        missing = (required - self._length) / float(1 << 30)
        raise OSError(f"{self.path} is incomplete: {self._length} bytes on disk but its {len(self.tensors)} "
                      f"tensors need {required} ({missing:.2f} GiB missing; '{last}' is the last one). "
                      "Re-download it.")

    # ------------------------------------------------------------- access
    def get_tensor(self, name: str) -> GgufTensorInfo:
        try:
            return self.tensors[name]
        except KeyError:
            raise KeyError(f"{self.path} has no tensor '{name}'.") from None

    def tensor_bytes(self, info: GgufTensorInfo) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view into the mapping (no copy)."""
        if self._mm is None:
            raise ValueError("the GGUF file is closed")
        at = self.data_offset + info.offset
        return np.frombuffer(self._mm, dtype=np.uint8, count=info.byte_count, offset=at)

    def get(self, key: str, fallback=None):
        return self.metadata.get(key, fallback)

    def get_string(self, key: str, fallback: Optional[str] = None) -> Optional[str]:
        v = self.metadata.get(key)
        return v if isinstance(v, str) else fallback

    def get_uint32(self, key: str, fallback: int = 0) -> int:
        return int(self.metadata[key]) if key in self.metadata else fallback

    def get_float32(self, key: str, fallback: float = 0.0) -> float:
        return float(np.float32(self.metadata[key])) if key in self.metadata else fallback

    def get_bool(self, key: str, fallback: bool = False) -> bool:
        return bool(self.metadata[key]) if key in self.metadata else fallback

    def get_string_array(self, key: str) -> Optional[list]:
        v = self.metadata.get(key)
        return v if isinstance(v, list) else None

    def close(self) -> None:
        mm, self._mm = self._mm, None
        if mm is not None:
            try:
                mm.close()
            except BufferError:
                # a tensor view is still alive; the mapping goes with its last reference
                pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ------------------------------------------------------------------ config

def config_from_gguf(g: GgufFile, initial_kv_capacity: int = 512) -> ModelConfig:
    """ModelConfig.FromGguf (ModelConfig.cs:62-112)."""
    arch = g.get_string("general.architecture")
    if arch is None:
        raise L.DataError(L.JEV_EDATA, f"{g.path} has no general.architecture.")
    if arch not in ("mistral3", "ministral3", "llama"):
        raise NotSupportedError(f"{g.path} is architecture '{arch}'; this runtime implements the Ministral-3 "
                                "backbone (GGUF architecture \"mistral3\").")
    a = arch + "."
    heads = g.get_uint32(a + "attention.head_count")
    hidden = g.get_uint32(a + "embedding_length")
    head_dim = g.get_uint32(a + "attention.key_length", hidden // max(1, heads))
    tokens = g.get_string_array("tokenizer.ggml.tokens")

    def f2(key1, key2, default):
        return g.get_float32(key1, g.get_float32(key2, default))

    cfg = ModelConfig(
        n_layers=g.get_uint32(a + "block_count"),
        hidden=hidden,
        n_heads=heads,
        n_kv_heads=g.get_uint32(a + "attention.head_count_kv", heads),
        head_dim=head_dim,
        ffn=g.get_uint32(a + "feed_forward_length"),
        vocab=len(tokens) if tokens is not None else g.get_uint32(a + "vocab_size"),
        rms_eps=g.get_float32(a + "attention.layer_norm_rms_epsilon", 1e-5),
        rope_freq_base=g.get_float32(a + "rope.freq_base", 10000.0),
        rope_dim=g.get_uint32(a + "rope.dimension_count", head_dim),
        rope_scale_factor=g.get_float32(a + "rope.scaling.factor", 1.0),
        rope_scaling_yarn=1 if (g.get_string(a + "rope.scaling.type", "") or "") == "yarn" else 0,
        rope_original_context=g.get_uint32(a + "rope.scaling.original_context_length", 0),
        yarn_beta_fast=f2(a + "rope.scaling.yarn_beta_fast", a + "rope.scaling.beta_fast", 32.0),
        yarn_beta_slow=f2(a + "rope.scaling.yarn_beta_slow", a + "rope.scaling.beta_slow", 1.0),
        yarn_ext_factor=g.get_float32(a + "rope.scaling.yarn_ext_factor", 1.0),
        yarn_mscale=g.get_float32(a + "rope.scaling.mscale", 0.0),
        yarn_mscale_all_dim=f2(a + "rope.scaling.yarn_log_multiplier", a + "rope.scaling.mscale_all_dim", 0.0),
        rope_attn_factor=f2(a + "rope.scaling.attn_factor", a + "rope.scaling.yarn_attn_factor", 1.0),
        attention_temperature_scale=f2(a + "attention.temperature_scale", a + "rope.scaling_beta", 0.0),
        initial_kv_capacity=initial_kv_capacity,
        architecture=arch,
    )
    if cfg.n_kv_heads == 0 or cfg.n_heads % cfg.n_kv_heads != 0:
        raise L.DataError(L.JEV_EDATA, f"{cfg.n_heads} attention heads do not divide into {cfg.n_kv_heads} KV heads.")
    return cfg


# ------------------------------------------------------------------ binding

_LAYER_TENSORS = (("attn_norm", L.SLOT_ATTN_NORM), ("attn_q", L.SLOT_Q), ("attn_k", L.SLOT_K),
                  ("attn_v", L.SLOT_V), ("attn_output", L.SLOT_O), ("ffn_norm", L.SLOT_FFN_NORM),
                  ("ffn_gate", L.SLOT_GATE), ("ffn_up", L.SLOT_UP), ("ffn_down", L.SLOT_DOWN))
_VECTOR_SLOTS = (L.SLOT_OUTPUT_NORM, L.SLOT_ATTN_NORM, L.SLOT_FFN_NORM)


def _bind(model: MinistralModel, g: GgufFile, name: str, slot: int, layer: int, required: bool = True) -> bool:
    info = g.tensors.get(name)
    if info is None:
        if required:
            raise KeyError(f"{g.path} is missing tensor '{name}'.")
        return False
    if slot in _VECTOR_SLOTS:
        # VectorParameter.From (WeightMatrix.cs:80-98): every element, one row
        rows, cols = 1, info.element_count
    else:
        # WeightMatrix.From (WeightMatrix.cs:53-65): rows = Shape[1], cols = Shape[0]
        if len(info.shape) != 2:
            raise L.DataError(L.JEV_EDATA, f"'{name}' has {len(info.shape)} dimensions; a weight matrix needs 2.")
        rows, cols = info.shape[1], info.shape[0]
    model.bind(slot, layer, info.ggml_type, rows, cols, g.tensor_bytes(info))
    return True


def bind_gguf(model: MinistralModel, g: GgufFile) -> MinistralModel:
    """The tensor binding of MinistralModel's constructor (MinistralModel.cs:74-96), then ValidateShapes."""
    _bind(model, g, "token_embd.weight", L.SLOT_TOKEN_EMBD, 0)
    _bind(model, g, "output_norm.weight", L.SLOT_OUTPUT_NORM, 0)
    # a tied head has no output.weight: the embedding table serves as the head
    _bind(model, g, "output.weight", L.SLOT_OUTPUT, 0, required=False)
    for layer in range(model.config.n_layers):
        for suffix, slot in _LAYER_TENSORS:
            _bind(model, g, f"blk.{layer}.{suffix}.weight", slot, layer)
    model.finalize()
    return model


def load_gguf(path: str, device: int = 0, initial_kv_capacity: int = 512) -> MinistralModel:
    """MinistralModel over a GGUF file: parse, bind every tensor into HBM, unmap."""
    with GgufFile(path) as g:
        model = MinistralModel(config_from_gguf(g, initial_kv_capacity), device)
        try:
            bind_gguf(model, g)
        except BaseException:
            model.close()
            raise
    model.model_path = path
    return model


# ------------------------------------------------------------------ writer

@dataclass
class WriterTensor:
    name: str
    shape: tuple  # GGUF order: shape[0] varies fastest
    ggml_type: int
    data: np.ndarray  # raw bytes


def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(vtype: int, value) -> bytes:
    if vtype in _SCALAR:
        return struct.pack("<" + _SCALAR[vtype][0], value)
    if vtype == BOOL:
        return struct.pack("<B", 1 if value else 0)
    if vtype == STRING:
        return _pack_string(value)
    if vtype == ARRAY:
        elem, items = value
        head = struct.pack("<IQ", elem, len(items))
        if elem == STRING:
            return head + b"".join(_pack_string(s) for s in items)
        if elem == BOOL:
            return head + np.asarray(items, dtype=np.uint8).tobytes()
        return head + np.asarray(items, dtype=_NUMPY[elem]).tobytes()
    raise NotSupportedError(f"cannot write GGUF value type {vtype}")


def write_gguf(path: str, metadata: Iterable[tuple], tensors: Iterable[WriterTensor],
               alignment: int = DEFAULT_ALIGNMENT) -> None:
    """A version-3 GGUF.  `metadata` holds (key, value type, value); an array value is
    (element type, items).  The file appears under `path` only once complete."""
    tensors = list(tensors)
    meta = list(metadata)
    if alignment != DEFAULT_ALIGNMENT:
        meta.append(("general.alignment", UINT32, alignment))
    head = [struct.pack("<IIQQ", GGUF_MAGIC, 3, len(tensors), len(meta))]
    for key, vtype, value in meta:
        head.append(_pack_string(key) + struct.pack("<I", vtype) + _pack_value(vtype, value))
    offset, offsets = 0, []
    for t in tensors:
        need = row_bytes(t.ggml_type, t.shape[0]) * int(np.prod(t.shape[1:], dtype=np.int64))
        if t.data.nbytes != need:
            raise ValueError(f"'{t.name}' holds {t.data.nbytes} bytes; its shape needs {need}")
        offsets.append(offset)
        offset += need + (alignment - need % alignment) % alignment
    for t, off in zip(tensors, offsets):
        head.append(_pack_string(t.name) + struct.pack("<I", len(t.shape))
                    + struct.pack("<%dQ" % len(t.shape), *t.shape) + struct.pack("<IQ", t.ggml_type, off))
    header = b"".join(head)
    partial = str(path) + ".partial"
    with open(partial, "wb") as f:
        f.write(header)
        f.write(b"\0" * ((alignment - len(header) % alignment) % alignment))
        for t in tensors:
            raw = np.ascontiguousarray(t.data).view(np.uint8).reshape(-1)
            f.write(memoryview(raw))
            f.write(b"\0" * ((alignment - raw.nbytes % alignment) % alignment))
    os.replace(partial, path)


def ministral_metadata(config: ModelConfig, file_type: int, name: str = "synthetic") -> list:
    """The converter's keys for the text model (convert_shieldstral_to_gguf.py:309-369)
    with a placeholder vocabulary of `config.vocab` tokens."""
    a = "mistral3."
    md = [
        ("general.architecture", STRING, "mistral3"),
        ("general.name", STRING, name),
        ("general.file_type", UINT32, file_type),
        (a + "context_length", UINT32, 262144),
        (a + "embedding_length", UINT32, config.hidden),
        (a + "block_count", UINT32, config.n_layers),
        (a + "feed_forward_length", UINT32, config.ffn),
        (a + "attention.head_count", UINT32, config.n_heads),
        (a + "attention.head_count_kv", UINT32, config.n_kv_heads),
        (a + "attention.key_length", UINT32, config.head_dim),
        (a + "attention.value_length", UINT32, config.head_dim),
        (a + "attention.layer_norm_rms_epsilon", FLOAT32, config.rms_eps),
        (a + "vocab_size", UINT32, config.vocab),
        (a + "rope.freq_base", FLOAT32, config.rope_freq_base),
        (a + "rope.dimension_count", UINT32, config.rope_dim),
    ]
    if config.rope_scaling_yarn:
        md += [
            (a + "rope.scaling.type", STRING, "yarn"),
            (a + "rope.scaling.factor", FLOAT32, config.rope_scale_factor),
            (a + "rope.scaling.original_context_length", UINT32, config.rope_original_context),
            (a + "rope.scaling.yarn_beta_fast", FLOAT32, config.yarn_beta_fast),
            (a + "rope.scaling.yarn_beta_slow", FLOAT32, config.yarn_beta_slow),
            (a + "rope.scaling.yarn_ext_factor", FLOAT32, config.yarn_ext_factor),
            (a + "rope.scaling.mscale", FLOAT32, config.yarn_mscale),
            (a + "rope.scaling.yarn_log_multiplier", FLOAT32, config.yarn_mscale_all_dim),
            (a + "rope.scaling.attn_factor", FLOAT32, config.rope_attn_factor),
        ]
    if config.attention_temperature_scale:
        md.append((a + "attention.temperature_scale", FLOAT32, config.attention_temperature_scale))
    md += [
        ("tokenizer.ggml.model", STRING, "gpt2"),
        ("tokenizer.ggml.pre", STRING, "tekken"),
        ("tokenizer.ggml.tokens", ARRAY, (STRING, [f"<tok{i}>" for i in range(config.vocab)])),
        ("tokenizer.ggml.token_type", ARRAY, (INT32, np.ones(config.vocab, np.int32))),
        ("tokenizer.ggml.bos_token_id", UINT32, 1),
        ("tokenizer.ggml.eos_token_id", UINT32, 2),
        ("tokenizer.ggml.add_bos_token", BOOL, True),
        ("tokenizer.ggml.add_eos_token", BOOL, False),
    ]
    return md
