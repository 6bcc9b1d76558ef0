"""Shared helpers for the parity tests (test infrastructure)."""
import base64
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def quant_fixtures():
    with open(os.path.join(GOLDEN, "quantization_q.json")) as f:
        data = json.load(f)
    out = {}
    for c in data["cases"]:
        entry = {}
        for kind in ("quantized", "synthetic"):
            if kind in c:
                raw = np.frombuffer(base64.b64decode(c[kind]["bytes"]), np.uint8)
                entry[kind] = (raw, np.asarray(c[kind]["expected"], np.float32))
        out[c["type"]] = (c["ggml_type"], entry)
    return out


def worst_close(expected, actual) -> float:
    """Numeric.Close's measure (tests/Jevstral.Tests/Numeric.cs:16-41): |a - e| / max(1, |e|)."""
    e = np.asarray(expected, np.float64).ravel()
    a = np.asarray(actual, np.float64).ravel()
    return float(np.max(np.abs(a - e) / np.maximum(1.0, np.abs(e)))) if e.size else 0.0


def rel_l2(expected, actual) -> float:
    e = np.asarray(expected, np.float64).ravel()
    a = np.asarray(actual, np.float64).ravel()
    return float(np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30))


# Small model used by the CPU and GPU parity tests: every kernel shape rule
# (128-wide heads, GQA group 2, two K blocks of 32 per tile, ...) is exercised.
def tiny_config(**kw):
    from jev import ModelConfig
    base = dict(n_layers=2, hidden=256, n_heads=4, n_kv_heads=2, head_dim=128, ffn=512, vocab=2048,
                initial_kv_capacity=64)
    base.update(kw)
    return ModelConfig(**base)


LAYER_TAPS = ("attn_norm", "q_rope", "k_rope", "v", "attn_weighted", "attn_out", "post_attn", "ffn_norm", "ffn_out",
              "output")


def capture_names(n_layers):
    """The names ForwardAsync(tokens, capture, options) observes, in order
    (MinistralModel.cs:331-357 with AttentionAsync's taps at :459, :470, :474,
    :549, then :418-422)."""
    names = ["embeddings"]
    for l in range(n_layers):
        names += [f"blk.{l}.{t}" for t in LAYER_TAPS]
    return names + ["final_norm", "logits"]
