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


def yarn_active(cfg) -> bool:
    """ModelConfig.YarnActive (ModelConfig.cs:54-56)."""
    return bool(cfg.rope_scaling_yarn) and cfg.rope_original_context > 0 and cfg.yarn_ext_factor != 0 \
        and cfg.rope_scale_factor > 1


def rope_tables(cfg):
    """Rotary frequencies and magnitude scale in float64, from YaRN's definition
    (Peng et al. 2023, "YaRN: Efficient Context Window Extension of Large Language
    Models", sec. 3.2-3.4) in the form ggml implements it.

    Pair i turns at theta_i = base^(-2i/d).  Over the original window of L
    tokens it makes r(i) = L * theta_i / (2 pi) turns.  Pairs that turn at
    least beta_fast times keep theta_i (extrapolation), pairs that turn at most
    beta_slow times take theta_i / s (interpolation), and the pairs between
    blend the two on a ramp that is linear in the pair index, between
    floor(i_fast) and ceil(i_slow), where r(i_fast) = beta_fast and
    r(i_slow) = beta_slow (found here by root-finding on r, not by the closed
    form).  ext_factor scales the extrapolated share.  The attention
    magnitude factor is 1 + 0.1 m ln s (sec. 3.4), taken as the ratio of the
    "mscale" and "mscale_all_dim" variants when the latter is stored, times
    the checkpoint's attention factor.  Without YaRN every pair is theta_i / s
    and the magnitude is the attention factor alone."""
    from scipy.optimize import brentq

    d, base, s = cfg.rope_dim, np.float64(cfg.rope_freq_base), np.float64(cfg.rope_scale_factor)
    i = np.arange(d // 2, dtype=np.float64)
    theta = base ** (-2.0 * i / d)
    if not yarn_active(cfg):
        return theta / s, np.float64(cfg.rope_attn_factor)
    L = np.float64(cfg.rope_original_context)

    def log_turns(x):  # ln r(x), so the bracket below never overflows
        return np.log(L) - 2.0 * x / d * np.log(base) - np.log(2.0 * np.pi)

    if cfg.yarn_beta_fast == 0 and cfg.yarn_beta_slow == 0:
        low, high = np.float64(np.finfo(np.float32).max), d / 2.0 - 1.0
    else:
        root = lambda beta: brentq(lambda x: log_turns(x) - np.log(beta), -1e4, 1e4, xtol=1e-12)
        low = max(0.0, np.floor(root(np.float64(cfg.yarn_beta_fast))))
        high = min(d / 2.0 - 1.0, np.ceil(root(np.float64(cfg.yarn_beta_slow))))
    ramp = np.clip((i - low) / max(0.001, high - low), 0.0, 1.0)
    mix = (1.0 - ramp) * cfg.yarn_ext_factor
    freqs = theta / s * (1.0 - mix) + theta * mix

    def magnitude(m):
        return 1.0 if s <= 1 else 1.0 + 0.1 * m * np.log(s)

    m = cfg.yarn_mscale if cfg.yarn_mscale != 0 else 1.0
    ratio = magnitude(m) / magnitude(cfg.yarn_mscale_all_dim) if cfg.yarn_mscale_all_dim != 0 else magnitude(1.0)
    return freqs, np.float64(ratio * cfg.rope_attn_factor)


def position_scale(cfg, pos):
    """Llama-4 attention temperature on the queries: 1 + beta ln(1 + floor(pos / n_orig))."""
    pos = np.asarray(pos, np.float64)
    if cfg.rope_original_context <= 0 or cfg.attention_temperature_scale == 0:
        return np.ones_like(pos)
    return 1.0 + np.float64(np.float32(cfg.attention_temperature_scale)) * np.log1p(
        np.floor(pos / cfg.rope_original_context))


def rope(x, pos, n_heads, cfg):
    hd = cfg.head_dim
    freqs, mscale = rope_tables(cfg)
    th = np.float32(pos)[:, None].astype(np.float32) * freqs.astype(np.float32)[None, :]  # float angle
    th = th.astype(np.float64)
    c, s = np.cos(th) * mscale, np.sin(th) * mscale
    x = x.reshape(len(pos), n_heads, hd).copy()
    x0, x1 = x[:, :, 0:cfg.rope_dim:2].copy(), x[:, :, 1:cfg.rope_dim:2].copy()
    x[:, :, 0:cfg.rope_dim:2] = x0 * c[:, None, :] - x1 * s[:, None, :]
    x[:, :, 1:cfg.rope_dim:2] = x0 * s[:, None, :] + x1 * c[:, None, :]
    return x.reshape(len(pos), n_heads * hd)


def forward(cfg, W, tokens, positions, mask, out_rows, taps=None):
    """tokens [T], positions [T], mask [T, T] (query, key) -> normalised final
    states at out_rows, and the head logits for them.  `taps` (a dict) receives
    the intermediate tensors under the names the reference's activation sink
    uses (MinistralModel.cs:331-357, :418-422), for a causal call."""
    T = len(tokens)
    hd, H, KV = cfg.head_dim, cfg.n_heads, cfg.n_kv_heads
    g = H // KV
    tap = (lambda name, v: taps.__setitem__(name, np.array(v))) if taps is not None else (lambda name, v: None)
    h = W["token_embd.weight"][tokens].copy()
    tap("embeddings", h)
    for l in range(cfg.n_layers):
        p = f"blk.{l}."
        x = rmsnorm(h, W[p + "attn_norm.weight"], cfg.rms_eps)
        tap(p + "attn_norm", x)
        q = rope(x @ W[p + "attn_q.weight"].T, positions, H, cfg) * position_scale(cfg, positions)[:, None]
        tap(p + "q_rope", q)
        q = q.reshape(T, H, hd)
        k = rope(x @ W[p + "attn_k.weight"].T, positions, KV, cfg)
        tap(p + "k_rope", k)
        k = k.reshape(T, KV, hd)
        v = x @ W[p + "attn_v.weight"].T
        tap(p + "v", v)
        v = v.reshape(T, KV, hd)
        ctx = np.empty((T, H, hd))
        for head in range(H):
            s = q[:, head, :] @ k[:, head // g, :].T / np.sqrt(hd)
            s = np.where(mask, s, -np.inf)
            s = np.exp(s - s.max(-1, keepdims=True))
            s /= s.sum(-1, keepdims=True)
            ctx[:, head, :] = s @ v[:, head // g, :]
        tap(p + "attn_weighted", ctx.reshape(T, H * hd))
        a = ctx.reshape(T, H * hd) @ W[p + "attn_output.weight"].T
        tap(p + "attn_out", a)
        h = h + a
        tap(p + "post_attn", h)
        x = rmsnorm(h, W[p + "ffn_norm.weight"], cfg.rms_eps)
        tap(p + "ffn_norm", x)
        gate = x @ W[p + "ffn_gate.weight"].T
        up = x @ W[p + "ffn_up.weight"].T
        f = (gate / (1 + np.exp(-gate)) * up) @ W[p + "ffn_down.weight"].T
        tap(p + "ffn_out", f)
        h = h + f
        tap(p + "output", h)
    hn = rmsnorm(h[out_rows], W["output_norm.weight"], cfg.rms_eps)
    logits = hn @ W["token_embd.weight"].T
    tap("final_norm", hn[-1:])
    tap("logits", logits[-1:])
    return logits


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
