"""ctypes binding of libjev (include/jev.h).

The library is loaded from the package directory (llm-shield_amd/libjev.so),
where the build puts it.  There is no fallback: if the shared object is
missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_size_t, c_uint64, c_void_p

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libjev.so")

JEV_OK, JEV_EINVAL, JEV_EDATA, JEV_ENOMEM, JEV_EDEVICE, JEV_ECANCELED, JEV_ESTATE = range(7)
TYPE_F32, TYPE_F16, TYPE_Q4_0, TYPE_Q5_1, TYPE_Q8_0 = 0, 1, 2, 7, 8
(SLOT_TOKEN_EMBD, SLOT_OUTPUT_NORM, SLOT_OUTPUT, SLOT_ATTN_NORM, SLOT_Q, SLOT_K, SLOT_V, SLOT_O,
 SLOT_FFN_NORM, SLOT_GATE, SLOT_UP, SLOT_DOWN) = range(12)
OUT_NONE, OUT_LAST_FULL, OUT_SELECTED, OUT_FULL = range(4)
PROF_GEMM, PROF_ATTN, PROF_GEMV, PROF_DECODE_ATTN = range(4)
# MatMulStrategy (QuantMatMul.cs:10-18), same numbering
MATMUL_AUTO, MATMUL_FLOAT, MATMUL_INTEGER = range(3)

TYPE_NAMES = {"F32": TYPE_F32, "F16": TYPE_F16, "Q4_0": TYPE_Q4_0, "Q5_1": TYPE_Q5_1, "Q8_0": TYPE_Q8_0}
BLOCK = {TYPE_F32: (1, 4), TYPE_F16: (1, 2), TYPE_Q4_0: (32, 18), TYPE_Q5_1: (32, 24), TYPE_Q8_0: (32, 34)}


def row_bytes(ggml_type: int, cols: int) -> int:
    """GgmlTypeInfo.RowBytes (GgmlType.cs:112-120)."""
    bs, ts = BLOCK[ggml_type]
    return cols // bs * ts


class Config(ctypes.Structure):
    """jev_config: the ModelConfig fields (ModelConfig.cs:12-118)."""
    _fields_ = [
        ("n_layers", c_int32), ("hidden", c_int32), ("n_heads", c_int32), ("n_kv_heads", c_int32),
        ("head_dim", c_int32), ("ffn", c_int32), ("vocab", c_int32), ("rms_eps", c_float),
        ("rope_freq_base", c_float), ("rope_dim", c_int32), ("rope_scale_factor", c_float),
        ("rope_scaling_yarn", c_int32), ("rope_original_context", c_int32),
        ("yarn_beta_fast", c_float), ("yarn_beta_slow", c_float), ("yarn_ext_factor", c_float),
        ("yarn_mscale", c_float), ("yarn_mscale_all_dim", c_float), ("rope_attn_factor", c_float),
        ("attention_temperature_scale", c_float), ("initial_kv_capacity", c_int32),
    ]


class Layout(ctypes.Structure):
    """jev_layout: TokenLayout (MinistralModel.cs:703-781)."""
    _fields_ = [
        ("slot", POINTER(c_int32)), ("position", POINTER(c_int32)), ("shared_lo", POINTER(c_int32)),
        ("shared_hi", POINTER(c_int32)), ("segment", POINTER(c_int32)), ("outputs", POINTER(c_int32)),
        ("n_outputs", c_int32), ("end", c_int32),
    ]


# jev_sink: IActivationSink.Observe (MinistralModel.cs:787-790)
SINK = ctypes.CFUNCTYPE(None, c_void_p, c_char_p, POINTER(c_float), c_int32, c_int32)


class JevError(RuntimeError):
    """A non-zero status from libjev, with the library's message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class ArgumentError(JevError, ValueError):
    pass


class DataError(JevError):
    pass


class CancelledError(JevError):
    pass


_EXC = {JEV_EINVAL: ArgumentError, JEV_EDATA: DataError, JEV_ECANCELED: CancelledError}

_lib = None


def lib():
    """The loaded libjev; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libjev is not built ({LIB_PATH} is missing); run __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    I32P, F32P = POINTER(c_int32), POINTER(c_float)
    sig = {
        "jev_last_error": (c_char_p, []),
        "jev_create": (c_int, [POINTER(Config), c_int, POINTER(c_void_p)]),
        "jev_destroy": (None, [c_void_p]),
        "jev_bind_tensor": (c_int, [c_void_p, c_int, c_int, c_int, c_int64, c_int64, c_void_p, c_size_t]),
        "jev_finalize": (c_int, [c_void_p]),
        "jev_kv_length": (c_int, [c_void_p, I32P]),
        "jev_kv_capacity": (c_int, [c_void_p, I32P]),
        "jev_kv_reserve": (c_int, [c_void_p, c_int32]),
        "jev_kv_truncate": (c_int, [c_void_p, c_int32]),
        "jev_kv_reset": (c_int, [c_void_p]),
        "jev_kv_snapshot": (c_int, [c_void_p, c_int32, F32P, c_size_t]),
        "jev_kv_restore": (c_int, [c_void_p, F32P, c_size_t, c_int32]),
        "jev_kv_snapshot_device": (c_int, [c_void_p, c_int32, POINTER(c_void_p)]),
        "jev_kv_restore_device": (c_int, [c_void_p, c_void_p]),
        "jev_snapshot_length": (c_int, [c_void_p, I32P]),
        "jev_snapshot_read": (c_int, [c_void_p, F32P, c_size_t]),
        "jev_snapshot_destroy": (None, [c_void_p]),
        "jev_forward": (c_int, [c_void_p, I32P, c_int32, POINTER(Layout), c_int, I32P, c_int32, F32P, c_size_t]),
        "jev_forward_tree": (c_int, [c_void_p, I32P, c_int32, I32P, I32P, c_int32, I32P, c_int32, F32P, c_size_t]),
        "jev_capture": (c_int, [c_void_p, I32P, c_int32, SINK, c_void_p, F32P, c_size_t]),
        "jev_decode_greedy": (c_int, [c_void_p, c_int32, c_int32, I32P, c_size_t]),
        "jev_decode_rows_greedy": (c_int, [c_void_p, c_int32, c_int32, I32P, I32P, I32P, c_int32, I32P, c_size_t]),
        "jev_margins": (c_int, [F32P, c_int32, c_int32, c_int32, c_float, F32P, F32P]),
        "jev_cancel": (None, [c_void_p]),
        "jev_forward_device": (c_int, [c_void_p, c_void_p, c_int32, POINTER(Layout), c_int, I32P, c_int32, c_void_p]),
        "jev_sync": (c_int, [c_void_p]),
        "jev_stream": (c_void_p, [c_void_p]),
        "jev_profile_enable": (c_int, [c_void_p, c_int]),
        "jev_profile_read": (c_int, [c_void_p, c_int, POINTER(c_int64), POINTER(ctypes.c_double),
                                     POINTER(ctypes.c_double), POINTER(ctypes.c_double)]),
        "jev_profile_steps": (c_int, [c_void_p, F32P, c_int32, I32P]),
        "jev_weight_create": (c_int, [c_int, c_int64, c_int64, c_void_p, c_size_t, c_int, POINTER(c_void_p)]),
        "jev_weight_destroy": (None, [c_void_p]),
        "jev_matmul_device": (c_int, [c_void_p, c_void_p, c_int32, c_void_p]),
        "jev_matmul_device_noalloc": (c_int, [c_void_p, c_void_p, c_int32, c_void_p]),
        "jev_weight_sync": (c_int, [c_void_p]),
        "jev_weight_stream": (c_void_p, [c_void_p]),
        "jev_rope_table": (c_int, [POINTER(Config), F32P, c_int32, F32P]),
        "jev_dequantize": (c_int, [c_int, c_void_p, c_size_t, F32P, c_int64]),
        "jev_matmul_q": (c_int, [c_int, c_void_p, c_int64, c_int64, F32P, c_int32, F32P]),
        "jev_set_matmul_strategy": (c_int, [c_int]),
        "jev_get_matmul_strategy": (c_int, []),
        "jev_quantize_activations": (c_int, [F32P, c_int64, c_void_p, c_size_t, F32P]),
        "jev_quantize": (c_int, [c_int, F32P, c_int64, c_void_p, c_size_t]),
        "jev_synth_tensor": (c_int, [c_uint64, c_uint64, c_int, c_int64, c_int64, c_float, c_void_p, c_size_t, c_int]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(rc: int) -> None:
    if rc != JEV_OK:
        msg = lib().jev_last_error().decode(errors="replace")
        raise _EXC.get(rc, JevError)(rc, msg)


EXPORTED = [
    "jev_last_error", "jev_create", "jev_destroy", "jev_bind_tensor", "jev_finalize", "jev_kv_length",
    "jev_kv_capacity", "jev_kv_reserve", "jev_kv_truncate", "jev_kv_reset", "jev_kv_snapshot", "jev_kv_restore",
    "jev_forward", "jev_forward_tree", "jev_decode_greedy", "jev_decode_rows_greedy", "jev_margins", "jev_cancel", "jev_forward_device",
    "jev_sync", "jev_stream", "jev_profile_enable", "jev_profile_read", "jev_profile_steps", "jev_weight_create", "jev_weight_destroy",
    "jev_matmul_device", "jev_weight_sync", "jev_dequantize", "jev_matmul_q", "jev_quantize", "jev_synth_tensor",
    "jev_set_matmul_strategy", "jev_get_matmul_strategy", "jev_quantize_activations", "jev_rope_table",
    "jev_matmul_device_noalloc", "jev_capture", "jev_weight_stream", "jev_kv_snapshot_device",
    "jev_kv_restore_device", "jev_snapshot_length", "jev_snapshot_read", "jev_snapshot_destroy",
]
