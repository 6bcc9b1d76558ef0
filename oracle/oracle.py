"""ctypes wrapper of the CPU oracle (liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, by __graft_entry__.smoke() as the checker and by bench.py's
cpu_baseline leg; the product (llm-shield_amd/) never imports it.  Mirrors the
MinistralModel API of llm-shield_amd/jev/model.py so parity tests read the
same on both sides.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OUT_NONE, OUT_LAST_FULL, OUT_SELECTED, OUT_FULL = range(4)


class OrcConfig(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32), ("hidden", c_int32), ("n_heads", c_int32), ("n_kv_heads", c_int32),
        ("head_dim", c_int32), ("ffn", c_int32), ("vocab", c_int32), ("rms_eps", c_float),
        ("rope_freq_base", c_float), ("rope_dim", c_int32), ("rope_scale_factor", c_float),
        ("rope_scaling_yarn", c_int32), ("rope_original_context", c_int32),
        ("yarn_beta_fast", c_float), ("yarn_beta_slow", c_float), ("yarn_ext_factor", c_float),
        ("yarn_mscale", c_float), ("yarn_mscale_all_dim", c_float), ("rope_attn_factor", c_float),
        ("attention_temperature_scale", c_float), ("initial_kv_capacity", c_int32),
    ]


class OrcLayout(ctypes.Structure):
    _fields_ = [
        ("slot", POINTER(c_int32)), ("position", POINTER(c_int32)), ("shared_lo", POINTER(c_int32)),
        ("shared_hi", POINTER(c_int32)), ("segment", POINTER(c_int32)), ("outputs", POINTER(c_int32)),
        ("n_outputs", c_int32), ("end", c_int32),
    ]


_lib = None

# IActivationSink.Observe (MinistralModel.cs:787-790) as a C callback
SINK = ctypes.CFUNCTYPE(None, c_void_p, ctypes.c_char_p, POINTER(c_float), c_int, c_int)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH}")
        L = ctypes.CDLL(LIB_PATH)
        F, I = POINTER(c_float), POINTER(c_int32)
        sig = {
            "orc_dequantize": (c_int, [c_int, c_void_p, F, c_int64]),
            "orc_matmul": (None, [c_int, c_void_p, c_int, c_int, F, c_int, F]),
            "orc_quantize_activations": (c_int, [F, c_int64, c_void_p, F]),
            "orc_matmul_integer": (c_int, [c_int, c_void_p, c_int, c_int, F, c_int, F]),
            "orc_rmsnorm": (None, [F, F, c_float, c_int, F]),
            "orc_softmax": (None, [F, c_int]),
            "orc_swiglu": (None, [F, F, F, c_int]),
            "orc_dot": (c_float, [F, F, c_int]),
            "orc_attend": (None, [F, F, F, c_int, c_int, c_int, c_int, c_int, c_float, F, F]),
            "orc_model_create": (c_void_p, [POINTER(OrcConfig)]),
            "orc_model_destroy": (None, [c_void_p]),
            "orc_model_bind": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p]),
            "orc_forward": (c_int, [c_void_p, I, c_int, POINTER(OrcLayout), c_int, I, c_int, F, c_size_t]),
            "orc_forward_tree": (c_int, [c_void_p, I, c_int, I, I, c_int, I, c_int, F, c_size_t]),
            "orc_forward_capture": (c_int, [c_void_p, I, c_int, SINK, c_void_p, F, c_size_t]),
            "orc_kv_length": (c_int, [c_void_p]),
            "orc_kv_truncate": (None, [c_void_p, c_int]),
            "orc_kv_reset": (None, [c_void_p]),
            "orc_kv_snapshot": (c_int, [c_void_p, c_int, F, c_size_t]),
            "orc_kv_restore": (c_int, [c_void_p, F, c_size_t, c_int]),
            "orc_kv_key": (F, [c_void_p, c_int, c_int, c_int]),
            "orc_kv_value": (F, [c_void_p, c_int, c_int, c_int]),
            "orc_rope_freqs": (c_int, [POINTER(OrcConfig), F, F]),
            "orc_rope_apply": (None, [F, c_int, c_float, F, c_int, c_int, c_int]),
            "orc_layout_tree": (c_int, [c_int, c_int, I, c_int, c_int, I, I, I, I, I]),
            "orc_layout_rows": (c_int, [c_int, I, I, I, c_int, I, I, I, I, I]),
            "orc_margins": (None, [F, c_int, c_int, c_int, c_float, F, F]),
            "orc_set_threads": (None, [c_int]),
            "orc_set_vector_bits": (None, [c_int]),
            "orc_get_vector_bits": (c_int, []),
            "orc_get_threads": (c_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def fp(a):
    return a.ctypes.data_as(POINTER(c_float))


def ip(a):
    return None if a is None else a.ctypes.data_as(POINTER(c_int32))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def i32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


def set_vector_bits(bits: int) -> None:
    """PanelGemm.VectorBits: 512, 256, or 0 for the host's widest (same bits either way)."""
    lib().orc_set_vector_bits(bits)


def vector_bits() -> int:
    return int(lib().orc_get_vector_bits())


def dequantize(ggml_type: int, raw: np.ndarray, count: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    b = np.ascontiguousarray(raw).view(np.uint8)
    if lib().orc_dequantize(ggml_type, b.ctypes.data_as(c_void_p), fp(out), count) != 0:
        raise ValueError("bad type or count")
    return out


def matmul(ggml_type: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, tokens: int) -> np.ndarray:
    """QuantMatMul.ForwardAsync with Strategy = Float."""
    xx = f32(x)
    y = np.empty(tokens * rows, np.float32)
    wb = np.ascontiguousarray(w).view(np.uint8)
    lib().orc_matmul(ggml_type, wb.ctypes.data_as(c_void_p), rows, cols, fp(xx), tokens, fp(y))
    return y.reshape(tokens, rows)


def quantize_activations(x: np.ndarray):
    """IntegerDot.QuantizeActivations: (34-byte blocks as uint8, float block sums d * sum(q))."""
    xx = f32(x).reshape(-1)
    out = np.empty(xx.size // 32 * 34, np.uint8)
    sums = np.empty(xx.size // 32, np.float32)
    if lib().orc_quantize_activations(fp(xx), xx.size, out.ctypes.data_as(c_void_p), fp(sums)) != 0:
        raise ValueError("count is not whole blocks")
    return out, sums


def matmul_integer(ggml_type: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray, tokens: int) -> np.ndarray:
    """QuantMatMul.ForwardAsync with Strategy = Integer."""
    xx = f32(x)
    y = np.empty(tokens * rows, np.float32)
    wb = np.ascontiguousarray(w).view(np.uint8)
    if lib().orc_matmul_integer(ggml_type, wb.ctypes.data_as(c_void_p), rows, cols, fp(xx), tokens, fp(y)) != 0:
        raise ValueError("unsupported type or shape")
    return y.reshape(tokens, rows)


def rmsnorm(x, w, eps=1e-5):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_rmsnorm(fp(x), fp(w), eps, x.size, fp(y))
    return y


def softmax(x):
    x = f32(x).copy()
    lib().orc_softmax(fp(x), x.size)
    return x


def swiglu(g, u):
    g, u = f32(g).copy(), f32(u).copy()
    d = np.empty_like(g)
    lib().orc_swiglu(fp(g), fp(u), fp(d), g.size)
    return d


def dot(a, b):
    a, b = f32(a), f32(b)
    return float(lib().orc_dot(fp(a), fp(b), a.size))


def attend(q, keys, values, shared_lo, shared_hi, segment, slot, scale):
    q, k, v = f32(q), f32(keys), f32(values)
    hd = q.size
    n_sh = shared_hi - shared_lo
    limit = n_sh + (slot - segment + 1)
    scores = np.empty(max(limit, 1), np.float32)
    out = np.empty(hd, np.float32)
    lib().orc_attend(fp(q), fp(k), fp(v), hd, shared_lo, shared_hi, segment, slot, scale, fp(scores), fp(out))
    return out


def config_from(cfg) -> OrcConfig:
    c = OrcConfig()
    for name, _ in OrcConfig._fields_:
        setattr(c, name, getattr(cfg, name))
    return c


def rope_freqs(cfg):
    c = config_from(cfg)
    f = np.empty(512, np.float32)
    m = np.empty(1, np.float32)
    half = lib().orc_rope_freqs(ctypes.byref(c), fp(f), fp(m))
    return f[:half].copy(), float(m[0])


def rope_apply(freqs, mscale, data, heads, head_dim, position):
    freqs = f32(freqs)
    d = f32(data).copy()
    lib().orc_rope_apply(fp(freqs), freqs.size, mscale, fp(d), heads, head_dim, position)
    return d


def layout_tree(start_pos, trunk, offsets, tokens):
    o = i32(offsets)
    arrs = [np.empty(tokens, np.int32) for _ in range(4)]
    outs = np.empty(len(o), np.int32)
    end = lib().orc_layout_tree(start_pos, trunk, ip(o), len(o), tokens, *[ip(a) for a in arrs], ip(outs))
    return (*arrs, outs, end)


def layout_rows(shared, row_base, row_length, row_tokens):
    rb, rl, rt = i32(row_base), i32(row_length), i32(row_tokens)
    n = int(rt.sum())
    arrs = [np.empty(n, np.int32) for _ in range(4)]
    outs = np.empty(len(rt), np.int32)
    end = lib().orc_layout_rows(shared, ip(rb), ip(rl), ip(rt), len(rt), *[ip(a) for a in arrs], ip(outs))
    return (*arrs, outs, end)


def margins(verdicts, n_yes, n_no, temperature=1.0):
    v = f32(verdicts)
    n = v.size // (n_yes + n_no)
    m, p = np.empty(n, np.float32), np.empty(n, np.float32)
    lib().orc_margins(fp(v), n, n_yes, n_no, temperature, fp(m), fp(p))
    return m, p


class OracleModel:
    """The oracle's MinistralModel: same method names as jev.MinistralModel."""

    def __init__(self, config):
        self.config = config
        self._c = config_from(config)
        self._h = lib().orc_model_create(ctypes.byref(self._c))
        if not self._h:
            raise ValueError("bad config")
        self._keep = []

    def close(self):
        if self._h:
            lib().orc_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def bind(self, slot, layer, ggml_type, rows, cols, data):
        b = np.ascontiguousarray(data).view(np.uint8)
        self._keep.append(b)
        if lib().orc_model_bind(self._h, slot, layer, ggml_type, rows, cols, b.ctypes.data_as(c_void_p)) != 0:
            raise ValueError("bind failed")

    def bind_synth(self, synth):
        for t in synth.tensors.values():
            self.bind(t.slot, t.layer, t.ggml_type, t.rows, t.cols, t.data)
        return self

    @property
    def cached_token_count(self):
        return lib().orc_kv_length(self._h)

    def kv_truncate(self, n):
        lib().orc_kv_truncate(self._h, n)

    def reset_kv_cache(self):
        lib().orc_kv_reset(self._h)

    def kv_snapshot(self, length):
        c = self.config
        n = 2 * c.n_layers * c.n_kv_heads * length * c.head_dim
        out = np.empty(n, np.float32)
        if lib().orc_kv_snapshot(self._h, length, fp(out), n) != 0:
            raise ValueError("snapshot")
        return out

    def kv_restore(self, snap, length):
        s = f32(snap)
        if lib().orc_kv_restore(self._h, fp(s), s.size, length) != 0:
            raise ValueError("restore")

    def kv_key(self, layer, head, slot):
        p = lib().orc_kv_key(self._h, layer, head, slot)
        return np.ctypeslib.as_array(p, shape=(self.config.head_dim,)).copy()

    def kv_value(self, layer, head, slot):
        p = lib().orc_kv_value(self._h, layer, head, slot)
        return np.ctypeslib.as_array(p, shape=(self.config.head_dim,)).copy()

    def forward_layout(self, tokens, layout, mode, rows=None):
        tok = i32(tokens)
        r = i32(rows) if rows is not None else None
        n_out = 1 if layout is None else len(layout.outputs)
        size = {OUT_NONE: 0, OUT_LAST_FULL: self.config.vocab,
                OUT_SELECTED: n_out * (0 if r is None else len(r)), OUT_FULL: n_out * self.config.vocab}[mode]
        out = np.empty(max(size, 1), np.float32)
        lay = None
        if layout is not None:
            lay = OrcLayout(ip(layout.slot), ip(layout.position), ip(layout.shared_lo), ip(layout.shared_hi),
                            ip(layout.segment), ip(layout.outputs), len(layout.outputs), layout.end)
        rc = lib().orc_forward(self._h, ip(tok), len(tok), ctypes.byref(lay) if lay is not None else None, mode,
                               ip(r), 0 if r is None else len(r), fp(out), out.size)
        if rc != 0:
            raise ValueError("oracle forward rejected its arguments")
        return out[:size]

    def forward(self, tokens):
        return self.forward_layout(tokens, None, OUT_LAST_FULL)

    def prefill(self, tokens):
        self.forward_layout(tokens, None, OUT_NONE)

    def forward_selected(self, tokens, rows):
        return self.forward_layout(tokens, None, OUT_SELECTED, rows)

    def forward_tree(self, trunk, branches, rows):
        tr = i32(trunk)
        lens = i32([len(b) for b in branches])
        flat = i32(np.concatenate([i32(b) for b in branches]))
        r = i32(rows)
        out = np.empty(len(branches) * len(r), np.float32)
        rc = lib().orc_forward_tree(self._h, ip(tr), len(tr), ip(flat), ip(lens), len(branches), ip(r), len(r),
                                    fp(out), out.size)
        if rc != 0:
            raise ValueError("oracle tree forward rejected its arguments")
        return [out[b * len(r):(b + 1) * len(r)].copy() for b in range(len(branches))]

    def forward_branches(self, branches, rows):
        return self.forward_tree([], branches, rows)

    def forward_capture(self, tokens):
        """ForwardAsync(tokens, capture, options) (MinistralModel.cs:157-160): last-token
        logits and every observed tap, as [(name, array rows x columns)] in order."""
        tok = i32(tokens)
        taps = []

        def observe(_user, name, values, rows, cols):
            taps.append((name.decode(), np.ctypeslib.as_array(values, shape=(rows * cols,)).reshape(rows, cols).copy()))

        cb = SINK(observe)
        out = np.empty(self.config.vocab, np.float32)
        if lib().orc_forward_capture(self._h, ip(tok), len(tok), cb, None, fp(out), out.size) != 0:
            raise ValueError("oracle forward rejected its arguments")
        return out, taps
