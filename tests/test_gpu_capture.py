"""jev_capture: ForwardAsync(tokens, capture, options) with an activation sink
(MinistralModel.cs:157-160, :331-357, :418-422; IActivationSink :787-790) on the
GPU.  Every tap arrives with the reference's name, in its order and shape, and
matches the same tensor of the oracle's capture (itself pinned against the
float64 model in tests/test_oracle_model.py) at the logits bar; capturing
changes no result bit; the cache advances as a plain forward's would."""
import numpy as np
import pytest

import jev
from helpers import capture_names, tiny_config, worst_close
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def synth():
    return jev.SynthModel(tiny_config(), jev.TYPE_Q8_0)


@pytest.fixture(scope="module")
def model(gpu, synth):
    m = synth.open(0)
    yield m
    m.close()


@pytest.fixture(scope="module")
def ref(synth):
    return oracle.OracleModel(synth.config).bind_synth(synth)


@pytest.mark.parametrize("prefix,n", [(0, 40), (37, 20), (70, 1), (130, 1)])
def test_capture_taps_match_the_oracle(model, ref, synth, prefix, n):
    tokens = jev.random_tokens(prefix + n, 2048, 100 + prefix + n)
    model.reset_kv_cache()
    ref.reset_kv_cache()
    if prefix:
        model.prefill(tokens[:prefix])
        ref.prefill(tokens[:prefix])
    logits, taps = model.forward_capture(tokens[prefix:])
    assert model.cached_token_count == prefix + n
    e_logits, e_taps = ref.forward_capture(tokens[prefix:])
    assert [name for name, _ in taps] == capture_names(synth.config.n_layers)
    for (name, got), (_, want) in zip(taps, e_taps):
        assert got.shape == want.shape, name
        assert worst_close(want, got) <= 1e-3, name
    assert worst_close(e_logits, logits) <= 1e-3
    assert np.array_equal(taps[-1][1][0], logits)
    # the same pass without a sink: the same bits
    model.reset_kv_cache()
    if prefix:
        model.prefill(tokens[:prefix])
    assert np.array_equal(model.forward(tokens[prefix:]), logits)
