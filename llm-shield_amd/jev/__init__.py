"""jev: MI355X token loop behind Jevstral's managed API (ctypes over libjev)."""
from ._lib import (MATMUL_AUTO, MATMUL_FLOAT, MATMUL_INTEGER, ArgumentError, CancelledError, DataError, JevError,
                   OUT_FULL, OUT_LAST_FULL, OUT_NONE, OUT_SELECTED, TYPE_F16, TYPE_F32, TYPE_NAMES, TYPE_Q4_0,
                   TYPE_Q5_1, TYPE_Q8_0, lib, row_bytes)
from .model import MINISTRAL_3B, DeviceSnapshot, MinistralModel, ModelConfig, TokenLayout, margins, rope_table
from .gguf import GgufFile, GgufTensorInfo, NotSupportedError, bind_gguf, config_from_gguf, load_gguf, write_gguf
from .synth import SEED, VERDICT_NO, VERDICT_YES, SynthModel, quantize, random_tokens, synth_tensor
from .weight import QuantWeight, get_matmul_strategy, quantize_activations, set_matmul_strategy
from .prefix_cache import InvalidOperationError, SystemPromptCache
from .decider import DecisionResult, TreeDecider, common_prefix, temperature_for
from .reasoning import batched_greedy, decode_batch, index_of_max, plan_batches, row_bases

__all__ = [
    "ArgumentError", "CancelledError", "DeviceSnapshot", "DataError", "GgufFile", "GgufTensorInfo", "JevError", "NotSupportedError",
    "bind_gguf", "config_from_gguf", "load_gguf", "write_gguf", "MINISTRAL_3B", "MinistralModel", "ModelConfig",
    "OUT_FULL", "OUT_LAST_FULL", "OUT_NONE", "OUT_SELECTED", "QuantWeight", "SEED", "SynthModel", "TYPE_F16", "TYPE_F32",
    "TYPE_NAMES", "TYPE_Q4_0", "TYPE_Q5_1", "TYPE_Q8_0", "TokenLayout", "VERDICT_NO", "VERDICT_YES", "lib",
    "margins", "rope_table", "quantize", "random_tokens", "row_bytes", "synth_tensor", "MATMUL_AUTO", "MATMUL_FLOAT",
    "MATMUL_INTEGER", "get_matmul_strategy", "quantize_activations", "set_matmul_strategy",
    "InvalidOperationError", "SystemPromptCache", "DecisionResult", "TreeDecider", "common_prefix", "temperature_for",
    "batched_greedy", "decode_batch", "index_of_max", "plan_batches", "row_bases",
]
