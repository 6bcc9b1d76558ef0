"""The whole 3B shape on the GPU: 26 layers, d 3072, 32 / 8 heads, FFN 9216,
vocabulary 131072, synthetic Q8_0 weights (counter-based N(0, 0.02), the
ggml quantizer) -- the model every benchmark row runs.

* a short prompt and two decode steps against the oracle at the logits bar
  (Numeric.Close <= 1e-3);
* the reference's bitwise contracts at full size: the tree pass equals each
  branch run alone after the trunk and the branches off a cached trunk
  (DeciderTests.cs:55-91, with the benchmark tree's 9 x 48-token branches),
  and a restored prefix snapshot equals the whole prompt
  (SystemPromptCacheTests.cs:42-68).
"""
import os

import numpy as np
import pytest

import jev
from helpers import worst_close
from oracle import oracle

pytestmark = pytest.mark.gpu

VOCAB = 131072
ROWS = [jev.VERDICT_YES, jev.VERDICT_NO, 77]


@pytest.fixture(scope="module")
def synth():
    return jev.SynthModel(jev.ModelConfig(initial_kv_capacity=2048), jev.TYPE_Q8_0)


@pytest.fixture(scope="module")
def model(gpu, synth):
    m = synth.open(0)
    yield m
    m.close()


def test_full_shape_logits_and_decode_match_oracle(model, synth):
    tokens = jev.random_tokens(24, VOCAB, 5)
    model.reset_kv_cache()
    g = model.forward(tokens)
    oracle.set_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = oracle.OracleModel(synth.config).bind_synth(synth)
    try:
        assert worst_close(ref.forward(tokens), g) <= 1e-3
        for t in (7, 99_999):
            assert worst_close(ref.forward([t]), model.forward([t])) <= 1e-3
    finally:
        ref.close()


def test_full_shape_tree_equals_branches_alone_bitwise(model):
    trunk = jev.random_tokens(600, VOCAB, 6)
    branches = [jev.random_tokens(48, VOCAB, 60 + i) for i in range(9)]
    model.reset_kv_cache()
    model.prefill(trunk)
    alone = []
    for b in branches:
        model.kv_truncate(len(trunk))
        alone.append(model.forward_selected(b, ROWS))
    model.reset_kv_cache()
    tree = model.forward_tree(trunk, branches, ROWS)
    model.reset_kv_cache()
    model.prefill(trunk)
    cached = model.forward_branches(branches, ROWS)
    for i in range(len(branches)):
        assert np.array_equal(alone[i], tree[i]), i
        assert np.array_equal(alone[i], cached[i]), i


def test_full_shape_restored_prefix_equals_whole_prompt_bitwise(model):
    tokens = jev.random_tokens(300, VOCAB, 8)
    model.reset_kv_cache()
    whole = model.forward(tokens)
    model.reset_kv_cache()
    model.prefill(tokens[:170])
    snap = model.kv_snapshot(170)
    model.reset_kv_cache()
    model.kv_restore(snap, 170)
    assert np.array_equal(model.forward(tokens[170:]), whole)
