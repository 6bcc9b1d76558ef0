"""The whole 3B shape on the GPU: 26 layers, d 3072, 32 / 8 heads, FFN 9216,
vocabulary 131072, synthetic Q8_0 weights (counter-based N(0, 0.02), the
ggml quantizer) -- the model every benchmark row runs.

* a short prompt and two decode steps against the oracle at the logits bar
  (Numeric.Close <= 1e-3), and the benchmark's 256-token prefill (seed 11)
  with its full-vocabulary logits;
* the reference's bitwise contracts at full size: the tree pass equals each
  branch run alone after the trunk and the branches off a cached trunk
  (DeciderTests.cs:55-91, with the benchmark tree's 9 x 48-token branches),
  and a restored prefix snapshot equals the whole prompt
  (SystemPromptCacheTests.cs:42-68);
* the batched-decisions layout (independent trees, Q4_0) equals each tree
  run alone, bit for bit;
* Q5_1 greedy decode (one step replayed as a HIP graph): every chosen token
  is the oracle's argmax, teacher-forced, up to the logits bar.
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


def test_headline_prefill_logits_match_oracle(model, synth):
    # the benchmark's own workload: 256 uniform token ids (seed 11) through the
    # Q8_0 3B shape, final-position logits over the whole vocabulary
    # (MinistralModel.cs:411-424), at the logits bar (Numeric.Close <= 1e-3)
    tokens = jev.random_tokens(256, VOCAB, 11)
    model.reset_kv_cache()
    g = model.forward(tokens)
    oracle.set_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = oracle.OracleModel(synth.config).bind_synth(synth)
    try:
        e = ref.forward(tokens)
    finally:
        ref.close()
    assert g.shape == (VOCAB,)
    assert worst_close(e, g) <= 1e-3


def test_full_shape_tree_equals_branches_alone_bitwise(model):
    trunk = jev.random_tokens(600, VOCAB, 6)
    # seven 48-token branches and two short ones: a short branch alone runs the
    # small-batch GEMM (2..16 tokens), inside the tree the large-batch one
    branches = [jev.random_tokens(n, VOCAB, 60 + i) for i, n in enumerate([48] * 7 + [5, 16])]
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


def test_full_shape_q4_0_forest_equals_each_tree_alone_bitwise(gpu):
    synth = jev.SynthModel(jev.ModelConfig(initial_kv_capacity=512), jev.TYPE_Q4_0)
    trees = [(64, [16, 16, 16]), (40, [8, 24])]
    with synth.open(0) as m:
        tokens, alone = [], []
        for i, (trunk_n, bls) in enumerate(trees):
            trunk = list(jev.random_tokens(trunk_n, VOCAB, 500 + i))
            branches = [list(jev.random_tokens(n, VOCAB, 600 + 10 * i + j)) for j, n in enumerate(bls)]
            tokens += trunk + [t for b in branches for t in b]
            m.reset_kv_cache()
            alone += m.forward_tree(trunk, branches, ROWS)
        lay = jev.TokenLayout.forest(trees)
        m.reset_kv_cache()
        got = m.forward_layout(tokens, lay, jev.OUT_SELECTED, ROWS).reshape(len(lay.outputs), len(ROWS))
    for k in range(len(alone)):
        assert np.array_equal(got[k], alone[k]), k


def test_full_shape_q5_1_greedy_decode_follows_oracle(gpu):
    synth = jev.SynthModel(jev.ModelConfig(initial_kv_capacity=256), jev.TYPE_Q5_1)
    prompt = jev.random_tokens(32, VOCAB, 9)
    with synth.open(0) as m:
        m.prefill(prompt)
        out = m.decode_greedy(int(prompt[-1]), 4)
    oracle.set_threads(max(1, min(16, os.cpu_count() or 1)))
    ref = oracle.OracleModel(synth.config).bind_synth(synth)
    try:
        ref.prefill(prompt)
        nxt = int(prompt[-1])
        for tok in out:
            e = ref.forward([nxt])
            assert e[tok] >= e.max() - 1e-3 * max(1.0, abs(float(e.max())))
            nxt = int(tok)
    finally:
        ref.close()


def _cancel_while_running(m, run):
    import threading
    import time
    stop = threading.Event()

    def spam():
        while not stop.is_set():
            m.cancel()
            time.sleep(2e-4)

    t = threading.Thread(target=spam)
    t.start()
    try:
        return run()
    finally:
        stop.set()
        t.join()


def test_full_shape_cancel_reaches_a_prefill_and_a_decode_in_flight(model):
    """OperationCanceledException's contract (KernelTests.cs:206-219) at the 3B shape: another
    thread cancels a 4096-token prefill (~60 ms on the device) and a 64-step greedy decode while
    they run; each returns cancelled, the prefill leaves the cache length unchanged, the decode
    keeps the steps that ran, and the next call gives the same bits as an uncancelled run."""
    import time
    tokens = jev.random_tokens(4096, VOCAB, 31)
    model.reset_kv_cache()
    want = model.forward(tokens[:64])
    model.reset_kv_cache()
    t0 = time.perf_counter()
    with pytest.raises(jev.CancelledError):
        _cancel_while_running(model, lambda: model.prefill(tokens))
    took = time.perf_counter() - t0
    assert model.cached_token_count == 0
    assert np.array_equal(model.forward(tokens[:64]), want)
    model.reset_kv_cache()
    model.prefill(tokens[:32])
    with pytest.raises(jev.CancelledError):
        _cancel_while_running(model, lambda: model.decode_greedy(int(tokens[31]), 64))
    assert 32 <= model.cached_token_count < 32 + 64
    model.cancel()  # aimed at no call
    model.reset_kv_cache()
    assert np.array_equal(model.forward(tokens[:64]), want)
    print(f"cancelled 4096-token prefill returned after {took * 1e3:.1f} ms", flush=True)
