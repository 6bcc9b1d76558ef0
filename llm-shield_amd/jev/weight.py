"""A single quantized weight resident in HBM: the QuantMatMul.ForwardAsync seam
(QuantMatMul.cs:66-121) over libjev's jev_weight_* entry points."""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L


class QuantWeight:
    """WeightMatrix (WeightMatrix.cs:53-65) uploaded once; rows = output features."""

    def __init__(self, ggml_type: int, rows: int, cols: int, data: np.ndarray, device: int = 0):
        self._lib = L.lib()
        raw = np.ascontiguousarray(data).view(np.uint8)
        self._h = ctypes.c_void_p()
        L.check(self._lib.jev_weight_create(ggml_type, rows, cols, raw.ctypes.data_as(ctypes.c_void_p), raw.nbytes,
                                            device, ctypes.byref(self._h)))
        self.type, self.rows, self.cols = ggml_type, rows, cols

    def close(self) -> None:
        if self._h:
            self._lib.jev_weight_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def matmul_device(self, x_ptr: int, tokens: int, y_ptr: int) -> None:
        """Enqueue y = x . W^T on the weight's stream (x, y: fp32 device pointers)."""
        L.check(self._lib.jev_matmul_device(self._h, ctypes.c_void_p(x_ptr), tokens, ctypes.c_void_p(y_ptr)))

    def matmul_device_noalloc(self, x_ptr: int, tokens: int, y_ptr: int) -> None:
        """matmul_device without allocation: the call's scratch is the library's
        static 16 MiB device array (shared by every call on the GPU)."""
        L.check(self._lib.jev_matmul_device_noalloc(self._h, ctypes.c_void_p(x_ptr), tokens, ctypes.c_void_p(y_ptr)))

    def sync(self) -> None:
        L.check(self._lib.jev_weight_sync(self._h))

    @property
    def stream(self) -> int:
        """The weight's HIP stream handle (for graph capture or event timing by the caller)."""
        return int(self._lib.jev_weight_stream(self._h) or 0)


def set_matmul_strategy(strategy: int) -> None:
    """QuantMatMul.Strategy setter (QuantMatMul.cs:41): process-wide, read by
    every QuantWeight / matmul call; AUTO and FLOAT take the float path,
    INTEGER the int8 path."""
    L.check(L.lib().jev_set_matmul_strategy(strategy))


def get_matmul_strategy() -> int:
    return int(L.lib().jev_get_matmul_strategy())


def quantize_activations(x: np.ndarray):
    """IntegerDot.QuantizeActivations on the device: (Q8_0 blocks as uint8,
    block sums d * sum(q) with the float d)."""
    xx = np.ascontiguousarray(x, np.float32).reshape(-1)
    out = np.empty(xx.size // 32 * 34, np.uint8)
    sums = np.empty(xx.size // 32, np.float32)
    F = ctypes.POINTER(ctypes.c_float)
    L.check(L.lib().jev_quantize_activations(xx.ctypes.data_as(F), xx.size, out.ctypes.data_as(ctypes.c_void_p),
                                             out.nbytes, sums.ctypes.data_as(F)))
    return out, sums
