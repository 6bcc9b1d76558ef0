"""ReasoningDecider's batched greedy decode on the GPU (ReasoningDecider.cs:134-174).

Rows of one cache, each prompt prefilled alone, then one row-sparse pass of
one token per running row per step.  Every row's tokens are checked by
teacher-forcing the oracle on that prompt alone: each chosen token must be the
oracle's argmax up to the logits tolerance (1e-3 relative, as everywhere).
"""
import numpy as np
import pytest

import jev
from helpers import tiny_config
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def synth():
    return jev.SynthModel(tiny_config(initial_kv_capacity=64), jev.TYPE_Q8_0)


def test_batched_greedy_rows_follow_the_oracle(gpu, synth):
    prompts = [list(jev.random_tokens(n, 2048, 40 + n)) for n in (9, 23, 14, 31)]
    with synth.open(0) as m:
        got = jev.batched_greedy(m, prompts, 6, max_rows=3)  # two batches; the cache grows past 64
    ref = oracle.OracleModel(synth.config).bind_synth(synth)
    for p, toks in zip(prompts, got):
        assert len(toks) == 6
        ref.reset_kv_cache()
        e = ref.forward(p)
        for i, t in enumerate(toks):
            assert e[t] >= e.max() - 2e-3 * max(1.0, abs(float(e.max()))), (len(p), i)
            e = ref.forward([t])


def test_a_stop_token_ends_its_row_only(gpu, synth):
    prompts = [list(jev.random_tokens(n, 2048, 60 + n)) for n in (12, 17)]
    with synth.open(0) as m:
        free = jev.batched_greedy(m, prompts, 5)
        stop = free[0][1]  # row 0's second token
        got = jev.batched_greedy(m, prompts, 5, stop_tokens=[stop])
    for f, g in zip(free, got):
        assert g == (f[:f.index(stop) + 1] if stop in f else f)
    assert len(got[0]) <= 2
