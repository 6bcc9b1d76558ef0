"""Prefix snapshots and the decider's cache reuse on the GPU: bit for bit.

SystemPromptCacheTests.CachedAndUncachedProduceIdenticalLogits
(SystemPromptCacheTests.cs:42-68): a restored system-prompt snapshot and a
cold whole-prompt pass give identical verdict logits -- here also through an
SHKV file loaded into a second context of the same GGUF file.
DeciderTests.ReusingTheQuestionPrefixIsBitIdentical and
InterleavedQuestionsAreRestoredFromTheirSnapshots (DeciderTests.cs:99-138):
a warm decider's margins equal a cold one's, bit for bit.
"""
import os

import numpy as np
import pytest

import jev
from helpers import tiny_config

pytestmark = pytest.mark.gpu

ROWS = [13059 % 2048, 2649 % 2048, 77]
YES, NO = [13059 % 2048, 77], [2649 % 2048]


@pytest.fixture(scope="module")
def synth():
    return jev.SynthModel(tiny_config(), jev.TYPE_Q8_0)


@pytest.fixture(scope="module")
def model(gpu, synth):
    m = synth.open(0)
    yield m
    m.close()


def _tok(n, seed):
    return list(jev.random_tokens(n, 2048, seed))


def test_restored_system_snapshot_gives_identical_logits(model):
    system = _tok(37, 1)
    cache = jev.SystemPromptCache.capture(model, system)
    assert model.cached_token_count == 37 and cache.byte_size == model.kv_snapshot(37).nbytes
    for n, seed in ((12, 2), (30, 3), (65, 4)):
        suffix = _tok(n, seed)
        model.reset_kv_cache()
        cold = model.forward_selected(system + suffix, ROWS)
        model.reset_kv_cache()
        cache.restore_into(model)
        warm = model.forward_selected(suffix, ROWS)
        assert np.array_equal(cold, warm), n


def test_shkv_file_restores_into_another_context_of_the_same_file(gpu, synth, tmp_path):
    p = str(tmp_path / "tiny.gguf")
    synth.write_gguf(p)
    system, suffix = _tok(40, 5), _tok(21, 6)
    cap = synth.config.initial_kv_capacity
    with jev.load_gguf(p, initial_kv_capacity=cap) as a:
        assert a.model_path == p and a.config.architecture == "mistral3"
        cold = a.forward_selected(system + suffix, ROWS)
        shkv = str(tmp_path / "system.shkv")
        jev.SystemPromptCache.capture(a, system).save(shkv)
    with jev.load_gguf(p, initial_kv_capacity=cap) as b:
        loaded = jev.SystemPromptCache.try_load(shkv, b)
        assert loaded is not None and loaded.token_count == 40
        loaded.restore_into(b)
        assert np.array_equal(b.forward_selected(suffix, ROWS), cold)
        st = os.stat(p)
        os.utime(p, ns=(st.st_atime_ns, st.st_mtime_ns + 10**9))  # the model file changed: a miss
        assert jev.SystemPromptCache.try_load(shkv, b) is None


SYSTEM_LEN = 24


def _prompt(question_seed, q_len, data_seed, d_len, system):
    question = system + _tok(q_len, question_seed) + [5]
    return question + _tok(d_len, data_seed), question


def _branches(seed, n):
    return [_tok(4 + i, seed + i) for i in range(n)]


def test_reusing_the_question_prefix_is_bit_identical(model):
    system = _tok(SYSTEM_LEN, 7)
    b = _branches(100, 2)
    warm = jev.TreeDecider(model, YES, NO, system_tokens=system)
    p1, q = _prompt(8, 30, 9, 50, system)
    warm.decide(p1, q, b)
    p2, q = _prompt(8, 30, 10, 61, system)
    reused = warm.decide(p2, q, b)
    cold = jev.TreeDecider(model, YES, NO, system_tokens=system).decide(p2, q, b)
    assert reused.cached_tokens > cold.cached_tokens == SYSTEM_LEN
    assert np.array_equal(reused.margins, cold.margins)
    assert np.array_equal(reused.probabilities, cold.probabilities)


def test_interleaved_questions_are_restored_from_their_snapshots(model):
    system = _tok(SYSTEM_LEN, 11)
    b1, b2 = _branches(200, 3), _branches(300, 2)
    warm = jev.TreeDecider(model, YES, NO, system_tokens=system)
    p, q = _prompt(12, 33, 13, 40, system)
    warm.decide(p, q, b1)
    p, q = _prompt(14, 26, 15, 45, system)
    warm.decide(p, q, b2)
    p, q = _prompt(12, 33, 16, 52, system)
    restored = warm.decide(p, q, b1)
    cold = jev.TreeDecider(model, YES, NO, system_tokens=system).decide(p, q, b1)
    assert warm.question_cache_hits == 1
    assert restored.cached_tokens == len(q) > cold.cached_tokens
    assert np.array_equal(restored.margins, cold.margins)


def test_device_snapshot_matches_the_host_snapshot_and_restores_bitwise(gpu, synth, model):
    """The HBM snapshot (jev_kv_snapshot_device) holds exactly KvCache.Snapshot's flat state, and a
    restore from it (a copy inside device memory, pair shadows rebuilt) continues bit for bit like
    the whole prompt -- also after the cache grew, and into a second context of the same model."""
    tokens = _tok(150, 31)
    model.reset_kv_cache()
    whole = model.forward(tokens)
    model.reset_kv_cache()
    model.prefill(tokens[:90])  # initial capacity 64: the arena grew to 128
    snap = model.kv_snapshot_device(90)
    assert snap.length == 90 and np.array_equal(snap.to_host(), model.kv_snapshot(90))
    model.reset_kv_cache()
    model.forward(_tok(200, 32))  # overwrite the arena and grow it again
    model.kv_restore(snap)
    assert model.cached_token_count == 90
    assert np.array_equal(model.forward(tokens[90:]), whole)
    with synth.open(0) as other:
        other.kv_restore(snap)
        assert np.array_equal(other.forward(tokens[90:]), whole)
    snap.close()


def test_device_snapshot_refuses_another_geometry(gpu, model):
    model.reset_kv_cache()
    model.prefill(_tok(20, 33))
    snap = model.kv_snapshot_device(20)
    other = jev.SynthModel(tiny_config(n_kv_heads=1, n_heads=2), jev.TYPE_Q8_0).open(0)
    try:
        with pytest.raises(jev.ArgumentError, match="KV heads"):
            other.kv_restore(snap)
        with pytest.raises(jev.ArgumentError):
            model.kv_snapshot_device(21)  # more than cached
    finally:
        other.close()
        snap.close()
