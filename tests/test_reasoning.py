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
