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

    def sync(self) -> None:
        L.check(self._lib.jev_weight_sync(self._h))
