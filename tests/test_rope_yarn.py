"""YaRN RoPE and the Llama-4 attention temperature, pinned on the CPU.

The real checkpoint runs with YaRN (factor 16 over a 16384-token window,
beta 32 / 1) and an attention temperature of 0.1 (VerdictScoreTests.cs:165-174),
so these paths carry the model's definition:

* the frequency table and the magnitude scale of the oracle (Rope ctor,
  Rope.cs:33-106) and of libjev (the table jev_create uploads, read through the
  host-only jev_rope_table hook) against a float64 statement of YaRN from its
  published definition (tests/npref.py: correction dims by root-finding on the
  rotation count, not by the closed form), element by element, for the
  checkpoint's parameters and for variants that move every branch: a window
  whose fast bound clamps to 0, beta 0 / 0, a partial ext_factor, mscale !=
  mscale_all_dim, no stored log multiplier, an attention factor, and plain
  linear scaling;
* the paper's boundary property itself: pairs turning at least beta_fast times
  over the window keep their frequency, pairs turning at most beta_slow times
  are divided by the factor;
* the reference's own known answers (RopeAndCacheTests.cs:41-95);
* the whole oracle forward with YaRN, mscale != 1 and the temperature term on,
  at positions that cross the original window several times, against the
  independent float64 model (tests/npref.py) -- causal and tree.
"""
import numpy as np
import pytest

import jev
import npref
from helpers import tiny_config, worst_close
from oracle import oracle

SHIELDSTRAL = dict(rope_scale_factor=16.0, rope_scaling_yarn=1, rope_original_context=16384, yarn_beta_fast=32.0,
                   yarn_beta_slow=1.0, yarn_ext_factor=1.0, yarn_mscale=1.0, yarn_mscale_all_dim=1.0,
                   rope_attn_factor=1.0, attention_temperature_scale=0.1)

CASES = {
    "shieldstral": {},
    "window_64": dict(rope_original_context=64),  # fast bound below pair 0: clamps to 0
    "window_4096_base_1e4": dict(rope_original_context=4096, rope_freq_base=10000.0),
    "betas_zero": dict(yarn_beta_fast=0.0, yarn_beta_slow=0.0),
    "ext_half": dict(yarn_ext_factor=0.5),
    "mscale_2_over_1": dict(yarn_mscale=2.0, yarn_mscale_all_dim=1.0),
    "no_log_multiplier": dict(yarn_mscale=0.0, yarn_mscale_all_dim=0.0),
    "all_dim_only": dict(yarn_mscale=0.0, yarn_mscale_all_dim=0.5),
    "attn_factor": dict(rope_attn_factor=0.8, yarn_mscale=2.0),
    "rope_dim_64": dict(rope_dim=64),
    "linear_scaling": dict(rope_scaling_yarn=0, rope_scale_factor=2.0, rope_attn_factor=1.25),
    "plain": dict(rope_scaling_yarn=0, rope_scale_factor=1.0),
}


def config(**kw):
    base = dict(SHIELDSTRAL)
    base.update(kw)
    return jev.ModelConfig(n_layers=2, **base)


@pytest.mark.parametrize("case", sorted(CASES))
@pytest.mark.parametrize("impl", ["oracle", "libjev"])
def test_frequency_table_and_mscale_match_the_yarn_definition(case, impl):
    cfg = config(**CASES[case])
    want_f, want_m = npref.rope_tables(cfg)
    got_f, got_m = oracle.rope_freqs(cfg) if impl == "oracle" else jev.rope_table(cfg)
    assert len(got_f) == cfg.rope_dim // 2
    rel = np.abs(np.asarray(got_f, np.float64) - want_f) / want_f
    assert rel.max() <= 4e-6, (case, int(rel.argmax()), rel.max())
    assert abs(got_m - want_m) <= 1e-6 * abs(want_m), (case, got_m, want_m)


def test_the_checkpoint_ramp_has_an_interior():
    # factor 16 over 16384 tokens, beta 32 / 1: pairs 0..20 extrapolate, 37..63
    # interpolate and the 16 pairs between blend -- the ramp interior is where a
    # wrong correction dim would show.
    cfg = config()
    f, _ = jev.rope_table(cfg)
    theta = 1.0 / np.power(1e6, 2 * np.arange(64) / 128)
    ratio = np.asarray(f, np.float64) / theta
    assert np.allclose(ratio[:21], 1.0, rtol=4e-6)
    assert np.allclose(ratio[37:], 1 / 16, rtol=4e-6)
    interior = ratio[21:37]
    assert np.all((interior < 1.0 - 1e-3) & (interior > 1 / 16 + 1e-4))
    # linear in the pair index between low = 20 and high = 37
    mix = (interior - 1 / 16) / (1 - 1 / 16)
    assert np.allclose(mix, 1 - (np.arange(21, 37) - 20) / 17, atol=4e-6)


@pytest.mark.parametrize("window", [16384, 64, 4096])
def test_paper_boundaries_extrapolate_fast_pairs_and_interpolate_slow_ones(window):
    cfg = config(rope_original_context=window)
    f, _ = oracle.rope_freqs(cfg)
    theta = 1.0 / np.power(1e6, 2 * np.arange(64) / 128)
    turns = window * theta / (2 * np.pi)
    fast, slow = turns >= 32, turns <= 1
    assert np.allclose(f[fast], theta[fast], rtol=4e-6)
    assert np.allclose(f[slow], theta[slow] / 16, rtol=4e-6)
    assert np.all(np.diff(np.asarray(f, np.float64)) < 0)  # monotone (RopeAndCacheTests.cs:85-89)


def test_reference_known_answers():
    # RopeAndCacheTests.cs:41-95
    for impl in (oracle.rope_freqs, jev.rope_table):
        _, m = impl(config())
        assert abs(m - 1.0) <= 1e-6  # apply_scale false: the mscale terms cancel
        _, m = impl(config(yarn_mscale=0.0, yarn_mscale_all_dim=0.0))
        assert abs(m - (1 + 0.1 * np.log(16.0))) <= 1e-5
        yarn, _ = impl(config())
        plain, _ = impl(config(rope_scaling_yarn=0, rope_scale_factor=1.0))
        assert abs(yarn[0] - plain[0]) <= 1e-6
        assert abs(yarn[-1] - plain[-1] / 16) <= 1e-10


def test_position_scale_definition():
    # q *= 1 + beta ln(1 + floor(pos / n_orig)); exactly 1 inside the first window
    cfg = config(rope_original_context=64)
    s = npref.position_scale(cfg, [0, 63, 64, 127, 128, 200])
    assert np.array_equal(s[:2], [1.0, 1.0])
    assert np.allclose(s[2:], 1 + 0.1 * np.log([2, 2, 3, 4]), rtol=1e-7)


# ---------------------------------------------------------------- whole model

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


def test_oracle_forward_with_yarn_and_temperature_matches_float64_model(synth):
    cfg = synth.config
    W = npref.dequantized(synth)
    tokens = jev.random_tokens(200, cfg.vocab, 31)  # positions 0..199: windows 0..3
    m = oracle.OracleModel(cfg).bind_synth(synth)
    got = m.forward(tokens)
    ref = npref.forward(cfg, W, tokens, np.arange(200), npref.causal_mask(200), [199])[0]
    assert worst_close(ref, got) <= 1e-4
    # the temperature term matters at these positions: without it the logits move
    plain = jev.ModelConfig(**{**cfg.__dict__, "attention_temperature_scale": 0.0})
    off = npref.forward(plain, W, tokens, np.arange(200), npref.causal_mask(200), [199])[0]
    assert worst_close(ref, off) > 1e-3


def test_oracle_tree_with_yarn_matches_float64_model(synth):
    cfg = synth.config
    W = npref.dequantized(synth)
    trunk = jev.random_tokens(100, cfg.vocab, 32)
    lens = [40, 3, 29]
    branches = [jev.random_tokens(n, cfg.vocab, 33 + n) for n in lens]
    rows = [5, 17, 2047]
    got = oracle.OracleModel(cfg).bind_synth(synth).forward_tree(trunk, branches, rows)
    mask, pos = npref.tree_mask(100, lens)
    ends = list(np.cumsum(lens) + 100 - 1)
    ref = npref.forward(cfg, W, np.concatenate([trunk] + branches), pos, mask, ends)[:, rows]
    for b in range(len(lens)):
        assert worst_close(ref[b], got[b]) <= 1e-4
