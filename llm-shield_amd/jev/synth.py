"""Synthetic Ministral-shaped checkpoints for offline runs.

Stands in for the converter (tools/convert_shieldstral_to_gguf.py) when no
real weights are available: every linear weight is N(0, stddev) from a
counter-based generator keyed by (seed, tensor name), quantized with the ggml
reference quantizers into GGUF blocks; norms are 1.0 (F32).  Tensor names are
the GGUF names MinistralModel binds (MinistralModel.cs:74-96).
"""
from __future__ import annotations

import os
import zlib
from dataclasses import dataclass

import numpy as np

from . import _lib as L
from .model import MinistralModel, ModelConfig

SEED = 20261201
VERDICT_YES, VERDICT_NO = 13059, 2649


def _threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def synth_tensor(name: str, ggml_type: int, rows: int, cols: int, stddev: float = 0.02, seed: int = SEED) -> np.ndarray:
    """GGUF bytes (rows x row_bytes) of one synthetic tensor."""
    rb = L.row_bytes(ggml_type, cols)
    out = np.empty(rows * rb, np.uint8)
    stream = zlib.crc32(name.encode())
    L.check(L.lib().jev_synth_tensor(seed, stream, ggml_type, rows, cols, stddev,
                                     out.ctypes.data_as(L.c_void_p), out.nbytes, _threads()))
    return out


def quantize(values: np.ndarray, ggml_type: int) -> np.ndarray:
    """ggml reference quantizer over a flat float32 array (whole blocks)."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    out = np.empty(L.row_bytes(ggml_type, v.size), np.uint8)
    import ctypes
    L.check(L.lib().jev_quantize(ggml_type, v.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), v.size,
                                 out.ctypes.data_as(L.c_void_p), out.nbytes))
    return out


@dataclass
class Tensor:
    slot: int
    layer: int
    ggml_type: int
    rows: int
    cols: int
    data: np.ndarray


class SynthModel:
    """All tensors of a synthetic checkpoint, held as host GGUF bytes."""

    def __init__(self, config: ModelConfig, ggml_type: int = L.TYPE_Q8_0, seed: int = SEED, stddev: float = 0.02):
        self.config = config
        self.ggml_type = ggml_type
        self.tensors: dict[str, Tensor] = {}
        c = config
        ones = np.ones(c.hidden, np.float32).view(np.uint8)
        self._add("token_embd.weight", L.SLOT_TOKEN_EMBD, 0, ggml_type, c.vocab, c.hidden, seed, stddev)
        self.tensors["output_norm.weight"] = Tensor(L.SLOT_OUTPUT_NORM, 0, L.TYPE_F32, 1, c.hidden, ones)
        for l in range(c.n_layers):
            p = f"blk.{l}."
            self.tensors[p + "attn_norm.weight"] = Tensor(L.SLOT_ATTN_NORM, l, L.TYPE_F32, 1, c.hidden, ones)
            self.tensors[p + "ffn_norm.weight"] = Tensor(L.SLOT_FFN_NORM, l, L.TYPE_F32, 1, c.hidden, ones)
            for nm, slot, r, k in (("attn_q", L.SLOT_Q, c.qdim, c.hidden), ("attn_k", L.SLOT_K, c.kvdim, c.hidden),
                                   ("attn_v", L.SLOT_V, c.kvdim, c.hidden), ("attn_output", L.SLOT_O, c.hidden, c.qdim),
                                   ("ffn_gate", L.SLOT_GATE, c.ffn, c.hidden), ("ffn_up", L.SLOT_UP, c.ffn, c.hidden),
                                   ("ffn_down", L.SLOT_DOWN, c.hidden, c.ffn)):
                self._add(p + nm + ".weight", slot, l, ggml_type, r, k, seed, stddev)

    def _add(self, name, slot, layer, t, rows, cols, seed, stddev):
        self.tensors[name] = Tensor(slot, layer, t, rows, cols, synth_tensor(name, t, rows, cols, stddev, seed))

    def bind(self, model: MinistralModel) -> MinistralModel:
        for t in self.tensors.values():
            model.bind(t.slot, t.layer, t.ggml_type, t.rows, t.cols, t.data)
        model.finalize()
        return model

    def open(self, device: int = 0) -> MinistralModel:
        return self.bind(MinistralModel(self.config, device))

    def write_gguf(self, path: str) -> None:
        """The checkpoint as a GGUF file with the converter's names and keys; the
        converter records the quantization type's ggml id as general.file_type."""
        from .gguf import WriterTensor, ministral_metadata, write_gguf
        ts = []
        for name, t in self.tensors.items():
            shape = (t.cols,) if t.slot in (L.SLOT_OUTPUT_NORM, L.SLOT_ATTN_NORM, L.SLOT_FFN_NORM) else (t.cols, t.rows)
            ts.append(WriterTensor(name, shape, t.ggml_type, t.data))
        write_gguf(path, ministral_metadata(self.config, self.ggml_type), ts)


def random_tokens(n: int, vocab: int, seed: int) -> np.ndarray:
    """Uniform token ids on [0, vocab)."""
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.int64).astype(np.int32)
