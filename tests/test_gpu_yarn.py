"""The GPU with YaRN RoPE and the Llama-4 attention temperature switched on,
the way the real checkpoint runs (VerdictScoreTests.cs:165-174: factor 16,
beta 32 / 1, temperature 0.1), on the tiny model with an original window of
64 tokens so that positions cross it several times.

Every kernel that rotates or scales runs here with mscale != 1 and the
temperature branch taken: the prefill RoPE/KV store (rope_store_kernel), the
RoPE fused into the one-token decode attention, and the graph-replayed greedy
decode.  Each is compared with the oracle, whose tables and forward pass are
pinned against the float64 YaRN statement in tests/test_rope_yarn.py.

Bars: logits Numeric.Close <= 1e-3, verdict z <= 2e-2 absolute, tree pass
bit-identical to each branch alone.
"""
import numpy as np
import pytest

import jev
from helpers import tiny_config, worst_close
from oracle import oracle

pytestmark = pytest.mark.gpu

ROWS = [13059 % 2048, 2649 % 2048, 77]


def yarn_tiny(**kw):
    base = dict(rope_scale_factor=16.0, rope_scaling_yarn=1, rope_original_context=64, yarn_beta_fast=32.0,
                yarn_beta_slow=1.0, yarn_mscale=2.0, yarn_mscale_all_dim=1.0, attention_temperature_scale=0.1,
                initial_kv_capacity=256)
    base.update(kw)
    return tiny_config(**base)


@pytest.fixture(scope="module", params=["mscale_2_over_1", "shieldstral_like"])
def synth(request):
    kw = {} if request.param == "mscale_2_over_1" else dict(yarn_mscale=1.0)
    return jev.SynthModel(yarn_tiny(**kw), jev.TYPE_Q8_0)


@pytest.fixture(scope="module")
def model(gpu, synth):
    m = synth.open(0)
    yield m
    m.close()


@pytest.fixture(scope="module")
def ref(synth):
    return oracle.OracleModel(synth.config).bind_synth(synth)


def fresh(m):
    m.reset_kv_cache()
    return m


def test_tables_are_the_ones_pinned_on_the_cpu(synth):
    f, m = jev.rope_table(synth.config)
    of, om = oracle.rope_freqs(synth.config)
    assert np.allclose(f, of, rtol=1e-6) and abs(m - om) <= 1e-6
    if synth.config.yarn_mscale == 2.0:
        assert m > 1.1  # the magnitude branch is live


def test_causal_prefill_crossing_the_window(model, ref):
    tokens = jev.random_tokens(200, 2048, 41)  # positions 0..199: temperature 1, 1.07, 1.11, 1.14
    g = fresh(model).forward(tokens)
    e = fresh(ref).forward(tokens)
    assert worst_close(e, g) <= 1e-3


def test_decode_steps_across_a_window_boundary(model, ref):
    # one-token passes: RoPE and the temperature run inside the decode attention kernel
    tokens = jev.random_tokens(140, 2048, 42)
    fresh(model).prefill(tokens[:120])
    fresh(ref).prefill(tokens[:120])
    for t in tokens[120:]:  # positions 120..139 cross 128
        assert worst_close(ref.forward([t]), model.forward([t])) <= 1e-3


def test_tree_verdicts_and_bitwise_contract(model, ref):
    trunk = jev.random_tokens(100, 2048, 43)
    branches = [jev.random_tokens(n, 2048, 44 + n) for n in (40, 3, 29, 1)]
    g = np.array(fresh(model).forward_tree(trunk, branches, ROWS))
    e = np.array(fresh(ref).forward_tree(trunk, branches, ROWS))
    assert worst_close(e, g) <= 1e-3
    assert np.max(np.abs((g[:, 0] - g[:, 1]) - (e[:, 0] - e[:, 1]))) <= 2e-2
    m = fresh(model)
    m.prefill(trunk)
    for b, br in enumerate(branches):
        m.kv_truncate(len(trunk))
        alone = m.forward_selected(br, ROWS)
        if len(br) >= 2:
            assert np.array_equal(alone, g[b]), b
        else:
            # one token alone takes the one-token (row-dot) path, as the reference
            # dispatches below PanelMinTokens = 2 (QuantMatMul.cs:51, :84): the
            # tolerance applies, not the bitwise contract
            assert worst_close(g[b], alone) <= 1e-3, b


def test_greedy_decode_graph_follows_oracle(model, ref):
    tokens = jev.random_tokens(120, 2048, 45)
    fresh(model).prefill(tokens)
    fresh(ref).prefill(tokens)
    out = model.decode_greedy(int(tokens[-1]), 12)  # positions 120..131
    nxt = int(tokens[-1])
    for tok in out:
        e = ref.forward([nxt])
        assert e[tok] >= e.max() - 2e-3
        nxt = int(tok)


def test_rows_of_one_token_across_the_window(model, ref):
    # Rows of one token each (RoPE, temperature and the KV store inside the
    # per-token decode attention) at positions on both sides of n_orig = 64
    # and past 128: each row's logits against the oracle's.
    shared = jev.random_tokens(50, 2048, 23)
    model.reset_kv_cache()
    ref.reset_kv_cache()
    model.prefill(shared)
    ref.prefill(shared)
    bases, lengths = [50, 70, 150], [3, 20, 90]
    prompts = [list(jev.random_tokens(n, 2048, 24 + n)) for n in lengths]
    model.forward_rows(50, bases, [0, 0, 0], prompts, ROWS)
    ref.forward_layout(np.concatenate(prompts).astype(np.int32), jev.TokenLayout.rows(50, bases, [0, 0, 0], lengths),
                       oracle.OUT_SELECTED, ROWS)
    step = [9, 400, 1999]
    g = np.array(model.forward_rows(50, bases, lengths, [[t] for t in step]))
    e = ref.forward_layout(step, jev.TokenLayout.rows(50, bases, lengths, [1, 1, 1]), oracle.OUT_FULL).reshape(3, -1)
    assert worst_close(e, g) <= 1e-3
