"""An independent float64 numpy statement of the Ministral-3 forward pass
(test infrastructure).  Written from the model's definition -- RMSNorm ->
GQA with adjacent-pair RoPE -> residual -> RMSNorm -> SwiGLU -> residual, tied
head -- with attention visibility given as an explicit boolean mask, the way
the reference's research path states tree masks (tools/decision/engine.py
margins_qcache).  It shares no code with the oracle: only the dequantized
weights (pinned bit-exactly by the golden fixtures) come from it.
"""
import numpy as np

from oracle import oracle


def dequantized(synth):
    W = {}
    for name, t in synth.tensors.items():
        if t.ggml_type == 0:
            W[name] = t.data.view(np.float32).astype(np.float64)
        else:
            W[name] = oracle.dequantize(t.ggml_type, t.data, t.rows * t.cols).reshape(t.rows, t.cols).astype(np.float64)
    return W


def rmsnorm(x, w, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * w


def rope(x, pos, n_heads, cfg):
    hd = cfg.head_dim
    freqs = 1.0 / np.power(np.float64(cfg.rope_freq_base), 2 * np.arange(cfg.rope_dim // 2) / cfg.rope_dim)
    th = np.float32(pos)[:, None].astype(np.float32) * freqs.astype(np.float32)[None, :]  # float angle
    th = th.astype(np.float64)
    c, s = np.cos(th), np.sin(th)
    x = x.reshape(len(pos), n_heads, hd).copy()
    x0, x1 = x[:, :, 0:cfg.rope_dim:2].copy(), x[:, :, 1:cfg.rope_dim:2].copy()
    x[:, :, 0:cfg.rope_dim:2] = x0 * c[:, None, :] - x1 * s[:, None, :]
    x[:, :, 1:cfg.rope_dim:2] = x0 * s[:, None, :] + x1 * c[:, None, :]
    return x.reshape(len(pos), n_heads * hd)


def forward(cfg, W, tokens, positions, mask, out_rows):
    """tokens [T], positions [T], mask [T, T] (query, key) -> normalised final
    states at out_rows, and the head logits for them."""
    T = len(tokens)
    hd, H, KV = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    g = H // KV
    h = W["token_embd.weight"][tokens].copy()
    for l in range(cfg.n_layers):
        p = f"blk.{l}."
        x = rmsnorm(h, W[p + "attn_norm.weight"], cfg.rms_eps)
        q = rope(x @ W[p + "attn_q.weight"].T, positions, H, cfg).reshape(T, H, hd)
        k = rope(x @ W[p + "attn_k.weight"].T, positions, KV, cfg).reshape(T, KV, hd)
        v = (x @ W[p + "attn_v.weight"].T).reshape(T, KV, hd)
        ctx = np.empty((T, H, hd))
        for head in range(H):
            s = q[:, head, :] @ k[:, head // g, :].T / np.sqrt(hd)
            s = np.where(mask, s, -np.inf)
            s = np.exp(s - s.max(-1, keepdims=True))
            s /= s.sum(-1, keepdims=True)
            ctx[:, head, :] = s @ v[:, head // g, :]
        h = h + ctx.reshape(T, H * hd) @ W[p + "attn_output.weight"].T
        x = rmsnorm(h, W[p + "ffn_norm.weight"], cfg.rms_eps)
        gate = x @ W[p + "ffn_gate.weight"].T
        up = x @ W[p + "ffn_up.weight"].T
        h = h + (gate / (1 + np.exp(-gate)) * up) @ W[p + "ffn_down.weight"].T
    hn = rmsnorm(h[out_rows], W["output_norm.weight"], cfg.rms_eps)
    return hn @ W["token_embd.weight"].T


def causal_mask(T):
    return np.tril(np.ones((T, T), bool))


def tree_mask(trunk, lens):
    """Trunk causal; each branch sees the trunk and itself causally, never another branch."""
    T = trunk + sum(lens)
    m = np.zeros((T, T), bool)
    m[:trunk, :trunk] = np.tril(np.ones((trunk, trunk), bool))
    o = trunk
    for n in lens:
        m[o:o + n, :trunk] = True
        m[o:o + n, o:o + n] = np.tril(np.ones((n, n), bool))
        o += n
    pos = np.concatenate([np.arange(trunk)] + [trunk + np.arange(n) for n in lens])
    return m, pos
