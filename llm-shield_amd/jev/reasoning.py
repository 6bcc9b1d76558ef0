"""ReasoningDecider's batched greedy decode (src/Jevstral/ReasoningDecider.cs:109-181) over libjev.

Many independent prompts decode together as rows of one KV cache
(TokenLayout.Rows): row r owns the slots from its base, each prompt is
prefilled on its own (one long GEMM), then every step feeds the last token of
every row still running as one row-sparse pass of 1 token per row, and takes
each row's argmax.  A row stops after emitting one of `stop_tokens`.
Prompt rendering, tokenization and the label scoring that follows the loop
are not part of this library.
"""
from __future__ import annotations

from typing import List, Sequence

import numpy as np

from . import _lib as L

MAX_ROWS = 12            # ReasoningDecider.MaxRows (ReasoningDecider.cs:43)
KV_TOKEN_BUDGET = 24_000  # ReasoningDecider.KvTokenBudget (:46)
ROW_SLACK = 8            # slots past prompt + max new tokens per row (:119, :139)


def plan_batches(lengths: Sequence[int], max_new_tokens: int, max_rows: int = MAX_ROWS,
                 kv_token_budget: int = KV_TOKEN_BUDGET) -> List[List[int]]:
    """DecideAsync's batching (ReasoningDecider.cs:113-130): prompts by
    ascending length (stable), a batch closed before it would exceed
    `max_rows` rows or (rows x widest row) > `kv_token_budget` slots."""
    order = sorted(range(len(lengths)), key=lambda i: lengths[i])
    batches, batch, widest = [], [], 0
    for i in order:
        need = lengths[i] + max_new_tokens + ROW_SLACK
        if batch and (len(batch) >= max_rows or (len(batch) + 1) * max(widest, need) > kv_token_budget):
            batches.append(batch)
            batch, widest = [], 0
        batch.append(i)
        widest = max(widest, need)
    if batch:
        batches.append(batch)
    return batches


def row_bases(lengths: Sequence[int], max_new_tokens: int) -> List[int]:
    """Row r's first slot (ReasoningDecider.cs:139): the rows laid end to end,
    each prompt + max new tokens + 8 slots wide."""
    bases = [0] * len(lengths)
    for r in range(1, len(lengths)):
        bases[r] = bases[r - 1] + lengths[r - 1] + max_new_tokens + ROW_SLACK
    return bases


def index_of_max(x) -> int:
    """Kernels.ArgMax (Kernels.cs:146), TensorPrimitives.IndexOfMax: the first
    NaN if there is one, else the largest value with +0 above -0, the lowest
    index on ties (the order the device argmax reduces in)."""
    x = np.asarray(x, np.float32).reshape(-1)
    nan = np.flatnonzero(np.isnan(x))
    if nan.size:
        return int(nan[0])
    top = np.flatnonzero(x == x.max())
    if x[top[0]] == 0:
        pos = top[~np.signbit(x[top])]
        if pos.size:
            return int(pos[0])
    return int(top[0])


_argmax = index_of_max


def decode_batch(model, prompts: Sequence[Sequence[int]], max_new_tokens: int,
                 stop_tokens: Sequence[int] = (), graph: bool = False, chunk: int = 32) -> List[List[int]]:
    """RunBatchAsync's token loop (ReasoningDecider.cs:134-174) for one batch.

    Returns each row's decoded tokens, a stop token included when one ended
    the row.  Leaves the rows in the cache (the caller may continue them).

    graph=True runs the loop as replayed device graphs of up to `chunk` steps
    (jev_decode_rows_greedy) and checks stop tokens between chunks; the
    tokens are the ones the step-by-step loop gives (see _decode_graph)."""
    if max_new_tokens < 1:
        raise L.ArgumentError(L.JEV_EINVAL, "max_new_tokens must be at least 1.")
    if any(len(p) == 0 for p in prompts):
        raise L.ArgumentError(L.JEV_EINVAL, "Every row needs at least one token.")
    rows = len(prompts)
    lengths = [len(p) for p in prompts]
    bases = row_bases(lengths, max_new_tokens)
    model.reset_kv_cache()
    stops = set(int(t) for t in stop_tokens)
    nxt, length = [0] * rows, [0] * rows
    for r, p in enumerate(prompts):  # one row at a time: a single long GEMM each
        logits = model.forward_rows(0, [bases[r]], [0], [list(p)])
        length[r] = lengths[r]
        nxt[r] = _argmax(logits[0])
    out: List[List[int]] = [[] for _ in range(rows)]
    done = [False] * rows
    if graph:
        for r in range(rows):
            out[r].append(nxt[r])
            done[r] = nxt[r] in stops
        _decode_graph(model, bases, length, nxt, out, done, stops, max_new_tokens, chunk)
        return out
    for step in range(max_new_tokens):
        active = []
        for r in range(rows):
            if done[r]:
                continue
            out[r].append(nxt[r])
            if nxt[r] in stops:
                done[r] = True
            else:
                active.append(r)
        if not active or step == max_new_tokens - 1:
            break
        logits = model.forward_rows(0, [bases[r] for r in active], [length[r] for r in active],
                                    [[nxt[r]] for r in active])
        for k, r in enumerate(active):
            length[r] += 1
            nxt[r] = _argmax(logits[k])
    return out


def _decode_graph(model, bases, length, nxt, out, done, stops, max_new_tokens: int, chunk: int) -> None:
    """The token loop in chunks of replayed steps.  Every row of a chunk runs
    every step, a stopped one too (its extra tokens are dropped and its slots
    beyond its length are never read).  The kernels are batch invariant, so a
    row's tokens do not depend on which other rows share its passes, except
    that one row alone takes the one-token path (QuantMatMul.cs:84, below
    PanelMinTokens): when the step-by-step loop would run the last surviving
    row alone, its tokens from that step on are dropped and it continues as
    a chunk of one row, rewriting those slots."""
    if chunk < 1:
        raise L.ArgumentError(L.JEV_EINVAL, "chunk must be at least 1.")
    rows = len(out)
    while True:
        active = [r for r in range(rows) if not done[r] and len(out[r]) < max_new_tokens]
        if not active:
            return
        n = min(chunk, max_new_tokens - len(out[active[0]]))
        toks = model.decode_rows_greedy(0, [bases[r] for r in active], [length[r] for r in active],
                                        [nxt[r] for r in active], n)
        alive = list(range(len(active)))
        for k in range(n):
            if len(active) >= 2 and len(alive) == 1:
                break  # the survivor runs alone from here: next chunk
            still = []
            for i in alive:
                r = active[i]
                t = int(toks[k, i])
                length[r] += 1
                nxt[r] = t
                out[r].append(t)
                if t in stops:
                    done[r] = True
                else:
                    still.append(i)
            alive = still
            if not alive:
                break


def batched_greedy(model, prompts: Sequence[Sequence[int]], max_new_tokens: int, stop_tokens: Sequence[int] = (),
                   max_rows: int = MAX_ROWS, kv_token_budget: int = KV_TOKEN_BUDGET, graph: bool = False,
                   chunk: int = 32) -> List[List[int]]:
    """Every prompt's greedy continuation, decoded in batches of rows
    (DecideAsync + RunBatchAsync); the cache is reset after each batch."""
    results: List[List[int]] = [[] for _ in prompts]
    for batch in plan_batches([len(p) for p in prompts], max_new_tokens, max_rows, kv_token_budget):
        got = decode_batch(model, [prompts[i] for i in batch], max_new_tokens, stop_tokens, graph, chunk)
        for i, toks in zip(batch, got):
            results[i] = toks
        model.reset_kv_cache()
    return results
