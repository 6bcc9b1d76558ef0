"""Host-side mirror of the reference's MinistralModel API over libjev.

Method names and argument meanings follow src/Jevstral/Model/MinistralModel.cs;
errors surface as the exceptions the reference throws (ArgumentException ->
ArgumentError/ValueError, InvalidDataException -> DataError,
OperationCanceledException -> CancelledError).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, fields
from typing import Optional, Sequence

import numpy as np

from . import _lib as L


@dataclass
class ModelConfig:
    """ModelConfig (ModelConfig.cs:12-118); defaults are Ministral-3 3B."""
    n_layers: int = 26
    hidden: int = 3072
    n_heads: int = 32
    n_kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 9216
    vocab: int = 131072
    rms_eps: float = 1e-5
    rope_freq_base: float = 1e6
    rope_dim: int = 128
    rope_scale_factor: float = 1.0
    rope_scaling_yarn: int = 0
    rope_original_context: int = 0
    yarn_beta_fast: float = 32.0
    yarn_beta_slow: float = 1.0
    yarn_ext_factor: float = 1.0
    yarn_mscale: float = 0.0
    yarn_mscale_all_dim: float = 0.0
    rope_attn_factor: float = 1.0
    attention_temperature_scale: float = 0.0
    initial_kv_capacity: int = 512
    # general.architecture (ModelConfig.cs:14); host-side only, part of a
    # prefix snapshot's fingerprint
    architecture: str = "mistral3"

    @property
    def qdim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kvdim(self) -> int:
        return self.n_kv_heads * self.head_dim

    def to_c(self) -> L.Config:
        c = L.Config()
        for f in fields(self):
            if f.name != "architecture":
                setattr(c, f.name, getattr(self, f.name))
        return c


MINISTRAL_3B = ModelConfig()


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _ptr(a: Optional[np.ndarray], ctype):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctype))


class TokenLayout:
    """TokenLayout (MinistralModel.cs:703-781) with shared_lo (0 in the reference's layouts)."""

    def __init__(self, slot, position, shared_hi, segment, outputs, end, shared_lo=None):
        self.slot = _i32(slot)
        self.position = _i32(position)
        self.shared_hi = _i32(shared_hi)
        self.segment = _i32(segment)
        self.shared_lo = _i32(shared_lo if shared_lo is not None else np.zeros(len(self.slot), np.int32))
        self.outputs = _i32(outputs)
        self.end = int(end)

    @staticmethod
    def tree(start_pos: int, trunk: int, offsets: Sequence[int], tokens: int) -> "TokenLayout":
        """TokenLayout.Tree (MinistralModel.cs:720-745)."""
        slot = np.arange(start_pos, start_pos + tokens, dtype=np.int32)
        pos = np.empty(tokens, np.int32)
        shared = np.empty(tokens, np.int32)
        seg = np.empty(tokens, np.int32)
        branch = -1
        for t in range(tokens):
            while branch + 1 < len(offsets) and t >= offsets[branch + 1]:
                branch += 1
            if t < trunk or branch < 0:
                pos[t], shared[t], seg[t] = start_pos + t, start_pos, start_pos
            else:
                pos[t] = start_pos + trunk + (t - offsets[branch])
                shared[t] = start_pos + trunk
                seg[t] = start_pos + offsets[branch]
        outputs = [(offsets[b + 1] if b + 1 < len(offsets) else tokens) - 1 for b in range(len(offsets))]
        return TokenLayout(slot, pos, shared, seg, outputs, start_pos + tokens)

    @staticmethod
    def rows(shared: int, row_base, row_length, row_tokens) -> "TokenLayout":
        """TokenLayout.Rows (MinistralModel.cs:758-780)."""
        slot, pos, sh, seg, outputs = [], [], [], [], []
        end = shared
        for r, n in enumerate(row_tokens):
            for i in range(n):
                s = row_base[r] + row_length[r] + i
                slot.append(s)
                pos.append(shared + row_length[r] + i)
                sh.append(shared)
                seg.append(row_base[r])
                end = max(end, s + 1)
            outputs.append(len(slot) - 1)
        return TokenLayout(slot, pos, sh, seg, outputs, end)

    @staticmethod
    def forest(trees: Sequence[tuple]) -> "TokenLayout":
        """Independent trees laid end to end in one cache, each (trunk length,
        [branch lengths]) as TokenLayout.Tree with its own first slot: tree d
        owns slots [b_d, b_d + its tokens); its trunk is causal from position
        0, a branch sees its tree's trunk (shared_lo .. shared_hi) and itself
        (positions continue after the trunk); the outputs are the branches'
        last tokens, in tree order.  The reference's layouts are the case of
        one tree (shared_lo = 0): this is the batch of independent decisions."""
        slot, pos, lo, hi, seg, outputs = [], [], [], [], [], []
        b0 = 0
        for trunk, branch_lengths in trees:
            for t in range(trunk):
                slot.append(b0 + t)
                pos.append(t)
                lo.append(b0)
                hi.append(b0)
                seg.append(b0)
            s0 = b0 + trunk
            for bl in branch_lengths:
                if bl <= 0:
                    raise L.ArgumentError(L.JEV_EINVAL, "Branch is empty.")
                for i in range(bl):
                    slot.append(s0 + i)
                    pos.append(trunk + i)
                    lo.append(b0)
                    hi.append(b0 + trunk)
                    seg.append(s0)
                outputs.append(len(slot) - 1)
                s0 += bl
            b0 = s0
        return TokenLayout(slot, pos, hi, seg, outputs, b0, shared_lo=lo)

    def with_outputs(self, outputs) -> "TokenLayout":
        return TokenLayout(self.slot, self.position, self.shared_hi, self.segment, outputs, self.end, self.shared_lo)

    def to_c(self) -> L.Layout:
        c = L.Layout()
        c.slot = _ptr(self.slot, ctypes.c_int32)
        c.position = _ptr(self.position, ctypes.c_int32)
        c.shared_lo = _ptr(self.shared_lo, ctypes.c_int32)
        c.shared_hi = _ptr(self.shared_hi, ctypes.c_int32)
        c.segment = _ptr(self.segment, ctypes.c_int32)
        c.outputs = _ptr(self.outputs, ctypes.c_int32)
        c.n_outputs = len(self.outputs)
        c.end = self.end
        return c


class DeviceSnapshot:
    """A KV snapshot resident in HBM (jev_kv_snapshot_device); restore it with
    MinistralModel.kv_restore, read it out with to_host (KvCache.Snapshot's
    flat layout, what SHKV files hold)."""

    def __init__(self, handle: ctypes.c_void_p, config: ModelConfig):
        self.handle = handle
        self._lib = L.lib()
        n = ctypes.c_int32()
        L.check(self._lib.jev_snapshot_length(handle, ctypes.byref(n)))
        self.length = int(n.value)
        self.floats = 2 * config.n_layers * config.n_kv_heads * self.length * config.head_dim

    def to_host(self) -> np.ndarray:
        out = np.empty(self.floats, np.float32)
        L.check(self._lib.jev_snapshot_read(self.handle, _ptr(out, ctypes.c_float), out.size))
        return out

    def close(self) -> None:
        if getattr(self, "handle", None) and self.handle.value:
            self._lib.jev_snapshot_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MinistralModel:
    """One libjev context: device weights, the HBM KV cache and a stream.

    Not thread-safe (MinistralModel.cs:21-22); `cancel` is the only call that
    may come from another thread.
    """

    def __init__(self, config: ModelConfig, device: int = 0):
        self.config = config
        # MinistralModel.ModelPath (MinistralModel.cs:51): the GGUF file the
        # weights came from, None for weights bound from memory
        self.model_path: Optional[str] = None
        self._lib = L.lib()
        h = ctypes.c_void_p()
        L.check(self._lib.jev_create(ctypes.byref(config.to_c()), device, ctypes.byref(h)))
        self._h = h

    # ------------------------------------------------------------ lifecycle
    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            self._lib.jev_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def bind(self, slot: int, layer: int, ggml_type: int, rows: int, cols: int, data: np.ndarray) -> None:
        """WeightMatrix.From / VectorParameter.From for one GGUF tensor's bytes."""
        buf = np.ascontiguousarray(data).view(np.uint8)
        L.check(self._lib.jev_bind_tensor(self._h, slot, layer, ggml_type, rows, cols,
                                          buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes))

    def finalize(self) -> None:
        L.check(self._lib.jev_finalize(self._h))

    # ------------------------------------------------------------ KvCache
    @property
    def cached_token_count(self) -> int:
        n = ctypes.c_int32()
        L.check(self._lib.jev_kv_length(self._h, ctypes.byref(n)))
        return n.value

    @property
    def kv_capacity(self) -> int:
        n = ctypes.c_int32()
        L.check(self._lib.jev_kv_capacity(self._h, ctypes.byref(n)))
        return n.value

    def kv_reserve(self, required: int) -> None:
        L.check(self._lib.jev_kv_reserve(self._h, required))

    def kv_truncate(self, length: int) -> None:
        L.check(self._lib.jev_kv_truncate(self._h, length))

    def reset_kv_cache(self) -> None:
        L.check(self._lib.jev_kv_reset(self._h))

    def kv_snapshot(self, length: int) -> np.ndarray:
        c = self.config
        n = 2 * c.n_layers * c.n_kv_heads * length * c.head_dim
        out = np.empty(n, np.float32)
        L.check(self._lib.jev_kv_snapshot(self._h, length, _ptr(out, ctypes.c_float), n))
        return out

    def kv_restore(self, snapshot, length: Optional[int] = None) -> None:
        """KvCache.Restore (KvCache.cs:115-136) from a flat host array (length
        positions) or from a DeviceSnapshot (its own length)."""
        if isinstance(snapshot, DeviceSnapshot):
            if length is not None and length != snapshot.length:
                raise L.ArgumentError(L.JEV_EINVAL, f"the snapshot holds {snapshot.length} positions, not {length}")
            L.check(self._lib.jev_kv_restore_device(self._h, snapshot.handle))
            return
        s = np.ascontiguousarray(snapshot, dtype=np.float32)
        L.check(self._lib.jev_kv_restore(self._h, _ptr(s, ctypes.c_float), s.size, length))

    def kv_snapshot_device(self, length: int) -> "DeviceSnapshot":
        """KvCache.Snapshot kept in HBM: a copy inside device memory."""
        h = ctypes.c_void_p()
        L.check(self._lib.jev_kv_snapshot_device(self._h, length, ctypes.byref(h)))
        return DeviceSnapshot(h, self.config)

    # ------------------------------------------------------------ forward
    def forward_layout(self, tokens, layout: Optional[TokenLayout], mode: int, rows=None) -> np.ndarray:
        """The private ForwardAsync (MinistralModel.cs:301-435)."""
        tok = _i32(tokens)
        r = _i32(rows) if rows is not None else None
        n_out = 1 if layout is None else len(layout.outputs)
        if mode == L.OUT_NONE:
            size = 0
        elif mode == L.OUT_LAST_FULL:
            size = self.config.vocab
        elif mode == L.OUT_SELECTED:
            size = n_out * len(r)
        else:
            size = n_out * self.config.vocab
        out = np.empty(max(size, 1), np.float32)
        lay = layout.to_c() if layout is not None else None
        L.check(self._lib.jev_forward(self._h, _ptr(tok, ctypes.c_int32), len(tok),
                                      ctypes.byref(lay) if lay is not None else None, mode,
                                      _ptr(r, ctypes.c_int32), 0 if r is None else len(r),
                                      _ptr(out, ctypes.c_float), out.size))
        return out[:size]

    def forward(self, tokens) -> np.ndarray:
        """ForwardAsync(tokens): logits of the final position (MinistralModel.cs:139)."""
        return self.forward_layout(tokens, None, L.OUT_LAST_FULL)

    def prefill(self, tokens) -> None:
        """PrefillAsync (MinistralModel.cs:148-149)."""
        self.forward_layout(tokens, None, L.OUT_NONE)

    def forward_selected(self, tokens, vocab_rows) -> np.ndarray:
        """ForwardSelectedAsync (MinistralModel.cs:165-172)."""
        return self.forward_layout(tokens, None, L.OUT_SELECTED, vocab_rows)

    def forward_tree(self, trunk, branches: Sequence[Sequence[int]], vocab_rows) -> list:
        """ForwardTreeAsync (MinistralModel.cs:198-219)."""
        if len(branches) == 0:
            raise L.ArgumentError(L.JEV_EINVAL, "No branches to forward.")
        tr = _i32(trunk)
        lens = _i32([len(b) for b in branches])
        flat = _i32(np.concatenate([_i32(b) for b in branches])) if lens.sum() > 0 else _i32([0])
        r = _i32(vocab_rows)
        out = np.empty(len(branches) * len(r), np.float32)
        L.check(self._lib.jev_forward_tree(self._h, _ptr(tr, ctypes.c_int32), len(tr), _ptr(flat, ctypes.c_int32),
                                           _ptr(lens, ctypes.c_int32), len(branches), _ptr(r, ctypes.c_int32), len(r),
                                           _ptr(out, ctypes.c_float), out.size))
        return [out[b * len(r):(b + 1) * len(r)].copy() for b in range(len(branches))]

    def forward_branches(self, branches, vocab_rows) -> list:
        """ForwardBranchesAsync (MinistralModel.cs:187-189)."""
        return self.forward_tree([], branches, vocab_rows)

    def forward_tree_logits(self, trunk, branches) -> list:
        """ForwardTreeLogitsAsync (MinistralModel.cs:227-255)."""
        offsets, total = [], len(trunk)
        for b in branches:
            if len(b) == 0:
                raise L.ArgumentError(L.JEV_EINVAL, "Branch is empty.")
            offsets.append(total)
            total += len(b)
        tokens = np.concatenate([_i32(trunk)] + [_i32(b) for b in branches])
        tree = TokenLayout.tree(self.cached_token_count, len(trunk), offsets, total)
        outs = list(range(len(trunk), total))
        flat = self.forward_layout(tokens, tree.with_outputs(outs), L.OUT_FULL).reshape(len(outs), self.config.vocab)
        res, k = [], 0
        for b in branches:
            res.append([flat[k + i].copy() for i in range(len(b))])
            k += len(b)
        return res

    def forward_rows(self, shared: int, row_base, row_length, row_tokens, vocab_rows=None) -> list:
        """ForwardRowsAsync (MinistralModel.cs:282-294)."""
        counts = [len(r) for r in row_tokens]
        if any(c == 0 for c in counts):
            raise L.ArgumentError(L.JEV_EINVAL, "Every row needs at least one token.")
        tokens = np.concatenate([_i32(r) for r in row_tokens])
        lay = TokenLayout.rows(shared, list(row_base), list(row_length), counts)
        if vocab_rows is None:
            flat = self.forward_layout(tokens, lay, L.OUT_FULL).reshape(len(counts), self.config.vocab)
            return [flat[i].copy() for i in range(len(counts))]
        r = _i32(vocab_rows)
        flat = self.forward_layout(tokens, lay, L.OUT_SELECTED, r).reshape(len(counts), len(r))
        return [flat[i].copy() for i in range(len(counts))]

    def decode_greedy(self, first: int, steps: int) -> np.ndarray:
        """Greedy decode: ForwardAsync([next]) + ArgMax per step (Benchmark.cs:411-422)."""
        out = np.empty(steps, np.int32)
        L.check(self._lib.jev_decode_greedy(self._h, first, steps, _ptr(out, ctypes.c_int32), out.size))
        return out

    def decode_rows_greedy(self, shared: int, row_base, row_length, first, steps: int) -> np.ndarray:
        """ReasoningDecider's batched greedy loop (ReasoningDecider.cs:157-178) as a
        replayed device graph: every row runs `steps` one-token passes fed with
        its own argmax.  Returns the tokens as [steps][rows]."""
        base, length, fst = _i32(row_base), _i32(row_length), _i32(first)
        n = len(base)
        if len(length) != n or len(fst) != n:
            raise L.ArgumentError(L.JEV_EINVAL, "row_base, row_length and first must have one entry per row")
        out = np.empty((steps, n), np.int32)
        L.check(self._lib.jev_decode_rows_greedy(self._h, shared, n, _ptr(base, ctypes.c_int32),
                                                 _ptr(length, ctypes.c_int32), _ptr(fst, ctypes.c_int32), steps,
                                                 _ptr(out, ctypes.c_int32), out.size))
        return out

    def forward_capture(self, tokens):
        """ForwardAsync(tokens, capture, options) (MinistralModel.cs:157-160): the last
        token's logits and every tensor an IActivationSink observes, as
        [(name, array rows x columns)] in the reference's order."""
        tok = _i32(tokens)
        taps = []

        def observe(_user, name, values, rows, cols):
            taps.append((name.decode(), np.ctypeslib.as_array(values, shape=(rows * cols,)).reshape(rows, cols).copy()))

        sink = L.SINK(observe)
        out = np.empty(self.config.vocab, np.float32)
        L.check(self._lib.jev_capture(self._h, _ptr(tok, ctypes.c_int32), len(tok), sink, None,
                                      _ptr(out, ctypes.c_float), out.size))
        return out, taps

    def cancel(self) -> None:
        self._lib.jev_cancel(self._h)


def margins(verdicts, n_yes: int, n_no: int, temperature: float = 1.0):
    """JevstralDecider margins z_i = max(yes) - max(no) and softmax(z / T) (JevstralDecider.cs:306-313)."""
    v = np.ascontiguousarray(np.asarray(verdicts, np.float32).reshape(len(verdicts), n_yes + n_no))
    m = np.empty(len(v), np.float32)
    p = np.empty(len(v), np.float32)
    L.check(L.lib().jev_margins(_ptr(v, ctypes.c_float), len(v), n_yes, n_no, temperature,
                                _ptr(m, ctypes.c_float), _ptr(p, ctypes.c_float)))
    return m, p


def rope_table(config: ModelConfig):
    """The Rope ctor's frequency table and magnitude scale (Rope.cs:33-106), as the library uploads them."""
    n = config.rope_dim // 2
    f = np.empty(n, np.float32)
    m = ctypes.c_float()
    L.check(L.lib().jev_rope_table(ctypes.byref(config.to_c()), _ptr(f, ctypes.c_float), n, ctypes.byref(m)))
    return f, float(m.value)
