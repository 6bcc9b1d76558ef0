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


def _rows_stepwise(m, shared, bases, lengths, first, steps):
    """The loop jev_decode_rows_greedy replays, one forward_rows call per step."""
    lengths, nxt, out = list(lengths), list(first), []
    for _ in range(steps):
        logits = m.forward_rows(shared, bases, lengths, [[t] for t in nxt])
        lengths = [n + 1 for n in lengths]
        nxt = [jev.reasoning.index_of_max(z) for z in logits]
        out.append(nxt)
    return np.array(out, np.int32)


def test_rows_graph_is_the_step_by_step_loop_over_a_shared_prefix(gpu, synth):
    trunk = jev.random_tokens(21, 2048, 70)
    prompts = [list(jev.random_tokens(n, 2048, 71 + n)) for n in (5, 11, 2)]
    bases = [40, 80, 120]
    steps = 13
    with synth.open(0) as m:
        def start():
            m.reset_kv_cache()
            m.prefill(trunk)
            logits = m.forward_rows(len(trunk), bases, [0, 0, 0], prompts)
            return [jev.reasoning.index_of_max(z) for z in logits]
        first = start()
        g = m.decode_rows_greedy(len(trunk), bases, [len(p) for p in prompts], first, steps)
        assert m.cached_token_count >= bases[2] + len(prompts[2]) + steps
        assert start() == first
        s = _rows_stepwise(m, len(trunk), bases, [len(p) for p in prompts], first, steps)
    assert g.shape == (steps, 3)
    assert np.array_equal(g, s)
    # row 1 teacher-forced through the oracle on trunk + its prompt alone
    ref = oracle.OracleModel(synth.config).bind_synth(synth)
    e = ref.forward(list(trunk) + prompts[1])
    assert e[first[1]] >= e.max() - 2e-3 * max(1.0, abs(float(e.max())))
    for t_in, t_out in zip([first[1]] + list(g[:-1, 1]), g[:, 1]):
        e = ref.forward([int(t_in)])
        assert e[t_out] >= e.max() - 2e-3 * max(1.0, abs(float(e.max())))


def test_one_row_is_the_one_token_decode(gpu, synth):
    # a lone row takes the one-token path: the same kernels and keys as jev_decode_greedy
    tokens = jev.random_tokens(30, 2048, 75)
    with synth.open(0) as m:
        m.reset_kv_cache()
        m.prefill(tokens)
        want = m.decode_greedy(int(tokens[-1]), 9)
        m.reset_kv_cache()
        m.prefill(tokens)
        got = m.decode_rows_greedy(0, [0], [len(tokens)], [int(tokens[-1])], 9)
    assert np.array_equal(got[:, 0], want)


@pytest.mark.parametrize("chunk", [3, 32])
def test_graph_batches_give_the_step_by_step_tokens(gpu, synth, chunk):
    prompts = [list(jev.random_tokens(n, 2048, 80 + n)) for n in (6, 13, 9, 17)]
    with synth.open(0) as m:
        free = jev.batched_greedy(m, prompts, 10)
        assert jev.batched_greedy(m, prompts, 10, graph=True, chunk=chunk) == free
        # rows stop one after another until one runs alone
        stops = {free[0][2], free[1][4], free[2][5]} - set(free[3])
        want = jev.batched_greedy(m, prompts, 10, stop_tokens=stops)
        got = jev.batched_greedy(m, prompts, 10, stop_tokens=stops, graph=True, chunk=chunk)
    assert got == want


def test_rows_graph_rejects_rows_that_meet(gpu, synth):
    with synth.open(0) as m:
        m.reset_kv_cache()
        m.prefill(jev.random_tokens(8, 2048, 90))
        n = m.cached_token_count
        for shared, bases, lengths in [(8, [10, 20], [7, 2]),     # row 0 runs into row 1 within 4 steps
                                       (8, [4, 30], [0, 0]),      # row 0 inside the shared prefix
                                       (8, [30, 30], [0, 0])]:
            with pytest.raises(jev.ArgumentError):
                m.decode_rows_greedy(shared, bases, lengths, [1, 2], 4)
        with pytest.raises(jev.ArgumentError):
            m.decode_rows_greedy(8, [10, 40], [0, 0], [1, 5000], 4)  # outside the embedding table
        assert m.cached_token_count == n


def test_rows_over_a_long_prefix_run_in_token_groups_and_match_the_loop(gpu, synth):
    # 12 rows over a 22000-token shared prefix: 12 x 345 chunk partials exceed
    # one decode-attention launch's budget (4096), so every step runs the rows
    # in two token groups.  The graph (kernel choice fixed at capture) must
    # give the tokens of the step-by-step loop in which rows stop one after
    # another, and a row's tokens must not depend on the rows beside it (the
    # same row decoded in a pair, one launch group).
    trunk = jev.random_tokens(22000, 2048, 91)
    n_rows, steps = 12, 6
    prompts = [list(jev.random_tokens(3 + r, 2048, 92 + r)) for r in range(n_rows)]
    bases = [22016 + 64 * r for r in range(n_rows)]
    with synth.open(0) as m:
        def start(rows):
            m.reset_kv_cache()
            m.prefill(trunk)
            logits = m.forward_rows(len(trunk), [bases[r] for r in rows], [0] * len(rows), [prompts[r] for r in rows])
            return [jev.reasoning.index_of_max(z) for z in logits]

        first = start(range(n_rows))
        g = m.decode_rows_greedy(len(trunk), bases, [len(p) for p in prompts], first, steps)
        # step by step, rows 0..4 stopping after 1..5 steps
        assert start(range(n_rows)) == first
        lengths = [len(p) for p in prompts]
        live, nxt = list(range(n_rows)), list(first)
        loop = {r: [] for r in range(n_rows)}
        for step in range(steps):
            logits = m.forward_rows(len(trunk), [bases[r] for r in live], [lengths[r] for r in live],
                                    [[nxt[r]] for r in live])
            for r, z in zip(live, logits):
                lengths[r] += 1
                nxt[r] = jev.reasoning.index_of_max(z)
                loop[r].append(nxt[r])
            live = [r for r in live if not (r < 5 and len(loop[r]) == r + 1)]
            if len(live) < 2:
                break
        for r in range(n_rows):
            assert list(g[:len(loop[r]), r]) == loop[r], r
        # rows 3 and 9 alone as a pair
        pair = start([3, 9])
        assert pair == [first[3], first[9]]
        gp = m.decode_rows_greedy(len(trunk), [bases[3], bases[9]], [len(prompts[3]), len(prompts[9])], pair, steps)
    assert np.array_equal(gp[:, 0], g[:, 3]) and np.array_equal(gp[:, 1], g[:, 9])


def test_greedy_decodes_refuse_a_short_destination(gpu, synth):
    import ctypes
    with synth.open(0) as m:
        m.reset_kv_cache()
        m.prefill(jev.random_tokens(8, 2048, 93))
        n = m.cached_token_count
        L = jev.lib()
        out = np.zeros(5, np.int32)
        p = out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))
        assert L.jev_decode_greedy(m._h, 1, 6, p, out.size) == jev._lib.JEV_EINVAL
        rows = np.array([16, 32], np.int32)
        lens = np.zeros(2, np.int32)
        first = np.array([1, 2], np.int32)
        i32 = ctypes.POINTER(ctypes.c_int32)
        assert L.jev_decode_rows_greedy(m._h, 8, 2, rows.ctypes.data_as(i32), lens.ctypes.data_as(i32),
                                        first.ctypes.data_as(i32), 3, p, out.size) == jev._lib.JEV_EINVAL
        assert m.cached_token_count == n
        assert np.all(out == 0)


def test_step_stamps_time_every_step_and_change_no_token(gpu, synth):
    # jev_profile_enable mode 2: a timing event at every step boundary of a
    # greedy decode, the graphs kept; the tokens are those of the plain run
    import ctypes
    tokens = jev.random_tokens(40, 2048, 94)
    L = jev.lib()
    with synth.open(0) as m:
        m.reset_kv_cache()
        m.prefill(tokens)
        want = m.decode_greedy(int(tokens[-1]), 7)
        m.reset_kv_cache()
        m.prefill(tokens)
        jev._lib.check(L.jev_profile_enable(m._h, 2))
        got = m.decode_greedy(int(tokens[-1]), 7)
        ms = np.zeros(16, np.float32)
        n = ctypes.c_int32()
        jev._lib.check(L.jev_profile_steps(m._h, ms.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), ms.size,
                                           ctypes.byref(n)))
        jev._lib.check(L.jev_profile_enable(m._h, 0))
    assert np.array_equal(got, want)
    assert n.value == 7
    assert np.all(ms[:7] > 0) and np.all(ms[7:] == 0)
