"""The oracle's whole forward pass on a small synthetic model, pinned against
an independent float64 statement of the model, plus the reference's
model-level invariants (DeciderTests.cs:55-91, SystemPromptCacheTests.cs:42-68,
RopeAndCacheTests.cs:159-252) -- bitwise where the reference asserts bitwise.
"""
import numpy as np
import pytest

import jev
import npref
from helpers import rel_l2, tiny_config, worst_close
from oracle import oracle


@pytest.fixture(scope="module")
def synth():
    return jev.SynthModel(tiny_config(), jev.TYPE_Q8_0)


@pytest.fixture(scope="module")
def W(synth):
    return npref.dequantized(synth)


def open_oracle(synth):
    return oracle.OracleModel(synth.config).bind_synth(synth)


def test_causal_logits_match_float64_model(synth, W):
    cfg = synth.config
    tokens = jev.random_tokens(37, cfg.vocab, 11)
    m = open_oracle(synth)
    got = m.forward(tokens)
    ref = npref.forward(cfg, W, tokens, np.arange(37), npref.causal_mask(37), [36])[0]
    assert worst_close(ref, got) <= 1e-4
    assert m.cached_token_count == 37


def test_tree_selected_rows_match_float64_model(synth, W):
    cfg = synth.config
    trunk = jev.random_tokens(20, cfg.vocab, 1)
    branches = [jev.random_tokens(n, cfg.vocab, 10 + n) for n in (3, 5, 1)]
    rows = [5, 17, 2047]
    m = open_oracle(synth)
    got = m.forward_tree(trunk, branches, rows)
    mask, pos = npref.tree_mask(20, [3, 5, 1])
    toks = np.concatenate([trunk] + branches)
    ends = [20 + 3 - 1, 20 + 8 - 1, 20 + 9 - 1]
    ref = npref.forward(cfg, W, toks, pos, mask, ends)[:, rows]
    for b in range(3):
        assert worst_close(ref[b], got[b]) <= 1e-4


def test_tree_equals_each_branch_alone_bitwise(synth):
    # DeciderTests.BranchesMatchRunningEachContinuationAlone (DeciderTests.cs:55-91)
    cfg = synth.config
    prefix = jev.random_tokens(19, cfg.vocab, 2)
    branches = [jev.random_tokens(n, cfg.vocab, 30 + n) for n in (4, 6, 2)]
    rows = [13, 1956 % cfg.vocab, 263]
    m = open_oracle(synth)
    m.prefill(prefix)
    alone = []
    for b in branches:
        m.kv_truncate(len(prefix))
        alone.append(m.forward_selected(b, rows))
    m.reset_kv_cache()
    tree = m.forward_tree(prefix, branches, rows)
    m.reset_kv_cache()
    m.prefill(prefix)
    cached = m.forward_branches(branches, rows)
    for b in range(len(branches)):
        assert np.array_equal(alone[b], tree[b])
        assert np.array_equal(alone[b], cached[b])


def test_cached_prefix_equals_whole_prompt_bitwise(synth):
    # SystemPromptCacheTests.cs:42-68: cached == uncached logits over the whole vocabulary.
    cfg = synth.config
    tokens = jev.random_tokens(30, cfg.vocab, 4)
    m = open_oracle(synth)
    whole = m.forward(tokens)
    m.reset_kv_cache()
    m.prefill(tokens[:18])
    snap = m.kv_snapshot(18)
    m.reset_kv_cache()
    m.kv_restore(snap, 18)
    part = m.forward(tokens[18:])
    assert np.array_equal(whole, part)


def test_kv_snapshot_layout_and_growth(synth):
    # KvCache.Snapshot's flat layout: keys [l][h][0..len)[hd] then values;
    # growth past the initial capacity keeps the prefix (RopeAndCacheTests.cs:159-252).
    cfg = synth.config
    m = open_oracle(synth)
    tokens = jev.random_tokens(90, cfg.vocab, 5)  # initial capacity 64 -> grows to 128
    m.prefill(tokens[:50])
    m.prefill(tokens[50:])
    snap = m.kv_snapshot(90).reshape(2, cfg.n_layers, cfg.n_kv_heads, 90, cfg.head_dim)
    assert np.array_equal(snap[0, 1, 1, 77], m.kv_key(1, 1, 77))
    assert np.array_equal(snap[1, 0, 0, 3], m.kv_value(0, 0, 3))
    with pytest.raises(ValueError):
        m.kv_snapshot(91)


def test_one_token_path_close_to_panel_path(synth, W):
    # Decode steps (one token) use the row-wise dot, prefill the panel chain;
    # both agree with the float64 model.
    cfg = synth.config
    tokens = jev.random_tokens(12, cfg.vocab, 6)
    m = open_oracle(synth)
    m.prefill(tokens[:11])
    got = m.forward(tokens[11:])
    ref = npref.forward(cfg, W, tokens, np.arange(12), npref.causal_mask(12), [11])[0]
    assert worst_close(ref, got) <= 1e-4


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1])
def test_other_block_types_match_float64_model(t):
    synth = jev.SynthModel(tiny_config(n_layers=1), t)
    W = npref.dequantized(synth)
    tokens = jev.random_tokens(9, synth.config.vocab, 8)
    got = oracle.OracleModel(synth.config).bind_synth(synth).forward(tokens)
    ref = npref.forward(synth.config, W, tokens, np.arange(9), npref.causal_mask(9), [8])[0]
    assert worst_close(ref, got) <= 1e-4 and rel_l2(ref, got) <= 1e-5


def test_capture_taps_match_float64_model(synth, W):
    # ForwardAsync(tokens, capture, options): every tap the reference observes
    # (MinistralModel.cs:331-357, :418-422), in its order and shape, against the
    # same intermediate of the independent float64 model; and capturing changes
    # nothing (the logits equal a plain forward bit for bit).
    from helpers import capture_names
    cfg = synth.config
    tokens = jev.random_tokens(21, cfg.vocab, 17)
    m = open_oracle(synth)
    m.prefill(tokens[:5])  # a cached prefix: positions and slots start at 5
    logits, taps = m.forward_capture(tokens[5:])
    assert [n for n, _ in taps] == capture_names(cfg.n_layers)
    ref = {}
    npref.forward(cfg, W, tokens, np.arange(21), npref.causal_mask(21), [20], taps=ref)
    for name, got in taps:
        want = ref[name][5:] if ref[name].shape[0] == 21 else ref[name]
        assert got.shape == want.shape, name
        assert worst_close(want, got) <= 1e-4, name
    plain = open_oracle(synth)
    plain.prefill(tokens[:5])
    assert np.array_equal(plain.forward(tokens[5:]), logits)
    assert np.array_equal(taps[-1][1][0], logits)
