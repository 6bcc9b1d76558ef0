"""ReasoningDecider's batched greedy decode (ReasoningDecider.cs:109-181) on the host.

The batching plan and the row bases against their closed forms, and the token
loop over a stand-in model whose next token is a fixed function of the row's
last token, so every row's sequence is known in advance.  The GPU test
(test_gpu_reasoning.py) runs the loop on the real kernels against the oracle.
"""
import numpy as np
import pytest

import jev
from jev import reasoning as R

V = 50


class RowsModel:
    """forward_rows logits: one-hot at (7 * last token + 3) % V per row; the
    calls are recorded."""

    def __init__(self):
        self.calls = []
        self.resets = 0

    def reset_kv_cache(self):
        self.resets += 1

    def forward_rows(self, shared, row_base, row_length, row_tokens, vocab_rows=None):
        assert shared == 0 and vocab_rows is None
        self.calls.append((list(row_base), list(row_length), [list(t) for t in row_tokens]))
        out = []
        for toks in row_tokens:
            z = np.zeros(V, np.float32)
            z[(7 * toks[-1] + 3) % V] = 1.0
            out.append(z)
        return out


class GraphRowsModel(RowsModel):
    """RowsModel plus decode_rows_greedy.  A pass of one token in total takes
    another next-token rule, as a lone row takes the one-token path on the
    device, so a loop that runs the last row with others where the step-by-step
    loop runs it alone gives other tokens."""

    def __init__(self):
        super().__init__()
        self.graph_calls = []

    @staticmethod
    def rule(t, alone):
        return (5 * t + 1) % V if alone else (7 * t + 3) % V

    def forward_rows(self, shared, row_base, row_length, row_tokens, vocab_rows=None):
        self.calls.append((list(row_base), list(row_length), [list(t) for t in row_tokens]))
        alone = sum(len(t) for t in row_tokens) == 1
        out = []
        for toks in row_tokens:
            z = np.zeros(V, np.float32)
            z[self.rule(toks[-1], alone)] = 1.0
            out.append(z)
        return out

    def decode_rows_greedy(self, shared, row_base, row_length, first, steps):
        assert shared == 0
        self.graph_calls.append((list(row_base), list(row_length), list(first), steps))
        out = np.empty((steps, len(first)), np.int32)
        t = list(first)
        for k in range(steps):
            t = [self.rule(x, len(first) == 1) for x in t]
            out[k] = t
        return out


def _expected(prompt, n, stops):
    seq, t = [], prompt[-1]
    for _ in range(n):
        t = (7 * t + 3) % V
        seq.append(t)
        if t in stops:
            break
    return seq


def test_plan_sorts_by_length_and_respects_both_budgets():
    lens = [50, 10, 30, 20, 40]
    assert R.plan_batches(lens, 100) == [[1, 3, 2, 4, 0]]
    assert R.plan_batches(lens, 100, max_rows=2) == [[1, 3], [2, 4], [0]]
    # need = len + 100 + 8; a batch closes before rows * widest would pass the budget
    assert R.plan_batches(lens, 100, kv_token_budget=3 * 138) == [[1, 3, 2], [4, 0]]
    assert R.plan_batches([5, 5, 5], 1, kv_token_budget=1) == [[0], [1], [2]]
    assert R.plan_batches([], 4) == []


def test_row_bases_lay_rows_end_to_end():
    assert R.row_bases([5, 9, 2], 10) == [0, 5 + 18, 5 + 18 + 9 + 18]
    assert R.row_bases([3], 1) == [0]


def test_decode_loop_feeds_active_rows_one_token_each():
    m = RowsModel()
    prompts = [[1, 2, 3], [4, 5], [6]]
    stops = {(7 * 5 + 3) % V}  # row 1 stops on its first token
    got = R.decode_batch(m, prompts, 4, stop_tokens=stops)
    assert got == [_expected(p, 4, stops) for p in prompts]
    assert got[1] == [(7 * 5 + 3) % V]
    bases = R.row_bases([3, 2, 1], 4)
    # one prefill per row (row length 0), then rows 0 and 2 (row 1 stopped) step by one token
    assert m.calls[:3] == [([bases[r]], [0], [prompts[r]]) for r in range(3)]
    assert [c[0] for c in m.calls[3:]] == [[bases[0], bases[2]]] * 3
    assert [c[1] for c in m.calls[3:]] == [[3, 1], [4, 2], [5, 3]]
    assert len(m.calls) == 3 + 3  # the last step's token is never fed


def test_batched_greedy_orders_results_and_resets_between_batches():
    m = RowsModel()
    prompts = [[9, 9, 9, 9], [1], [2, 2]]
    got = jev.batched_greedy(m, prompts, 3, max_rows=2)
    assert got == [_expected(p, 3, set()) for p in prompts]
    assert m.resets == 2 * 2  # each batch starts and ends with a reset


def test_rejections():
    with pytest.raises(jev.ArgumentError):
        R.decode_batch(RowsModel(), [[1], []], 2)
    with pytest.raises(jev.ArgumentError):
        R.decode_batch(RowsModel(), [[1]], 0)


def test_index_of_max_follows_index_of_max():
    assert R.index_of_max([1.0, 3.0, 3.0, 2.0]) == 1                 # lowest index on ties
    assert R.index_of_max([1.0, np.nan, 5.0, np.nan]) == 1           # the first NaN
    assert R.index_of_max([np.nan, np.nan]) == 0
    assert R.index_of_max([-0.0, 0.0, -1.0]) == 1                    # +0 above -0
    assert R.index_of_max([0.0, -0.0]) == 0
    assert R.index_of_max([-np.inf, -np.inf]) == 0
    assert R.index_of_max([-5.0, -0.0, -0.0]) == 1


@pytest.mark.parametrize("chunk", [1, 2, 3, 32])
@pytest.mark.parametrize("stop_on", [None, "first", "late", "all_but_one"])
def test_graph_chunks_give_the_step_by_step_tokens(chunk, stop_on):
    prompts = [[1, 2, 3], [4, 5], [6], [11, 12, 13, 14]]
    n = 9
    free = R.decode_batch(GraphRowsModel(), prompts, n)
    stops = set()
    if stop_on == "first":
        stops = {free[1][0]}
    elif stop_on == "late":
        stops = {free[2][4]}
    elif stop_on == "all_but_one":  # rows stop one by one; the last runs alone for a while
        stops = {free[0][1], free[1][2], free[2][3]} - set(free[3])
    want = R.decode_batch(GraphRowsModel(), prompts, n, stop_tokens=stops)
    m = GraphRowsModel()
    got = R.decode_batch(m, prompts, n, stop_tokens=stops, graph=True, chunk=chunk)
    assert got == want
    bases = R.row_bases([len(p) for p in prompts], n)
    for base, length, first, steps in m.graph_calls:
        assert 1 <= steps <= chunk
        for b, ln in zip(base, length):  # each row stays inside its own slots
            r = bases.index(b)
            assert len(prompts[r]) <= ln and ln + steps <= len(prompts[r]) + n - 1
    if stop_on == "all_but_one" and len(stops) == 3:
        assert any(len(c[0]) == 1 for c in m.graph_calls)  # the survivor ran alone


def test_graph_mode_rejects_a_zero_chunk():
    with pytest.raises(jev.ArgumentError):
        R.decode_batch(GraphRowsModel(), [[1], [2]], 3, graph=True, chunk=0)
