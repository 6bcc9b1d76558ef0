"""The benchmark workloads themselves, at full size, against the oracle and the
reference's bitwise contracts -- the exact inputs bench.py times.

* 4k-trunk tree decision (Q8_0): 4096 trunk tokens + 9 branches x 48 (token
  seed 23, verdict rows 13059 / 2649).  The tree pass equals every branch run
  alone after the trunk, bit for bit (DeciderTests.cs:55-91), and the 9 verdict
  log-odds z match the oracle within 2e-2 (the verdict rows within 1e-3).
* 64 batched Q4_0 decisions: 64 x (512 + 5 x 32) tokens in one tree-masked
  pass (token seed 47).  Every decision equals that decision run alone, bit for
  bit, and the first and last decisions' z match the oracle.
* Q5_1 decode: the 512-token prompt (seed 31), then one-token steps over 512 to
  528 cached keys (8 to 9 chunks merged in the O projection) against the
  oracle's logits, and the graph-replayed greedy loop teacher-forced against
  the oracle's argmax.

The oracle runs on the host cores; its trunk prefill goes in 512-token chunks
(cached-prefix continuation is bit-identical to one pass in the oracle) so
each step reports progress.
"""
import os
import sys
import time

import numpy as np
import pytest

import jev
from helpers import worst_close
from oracle import oracle

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

VOCAB = 131072
ROWS = [jev.VERDICT_YES, jev.VERDICT_NO]


def note(msg):
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def host_oracle(synth):
    oracle.set_threads(max(1, min(16, os.cpu_count() or 1)))
    return oracle.OracleModel(synth.config).bind_synth(synth)


def chunked_prefill(ref, tokens, chunk=512):
    for i in range(0, len(tokens), chunk):
        ref.prefill(tokens[i:i + chunk])
        note(f"oracle prefill {i + len(tokens[i:i + chunk])}/{len(tokens)}")


def z_of(v):
    v = np.asarray(v, np.float64).reshape(-1, 2)
    return v[:, 0] - v[:, 1]


def test_tree_decision_4k_trunk_9_branches(gpu):
    trunk_n, nb, bl = 4096, 9, 48
    synth = jev.SynthModel(jev.ModelConfig(initial_kv_capacity=trunk_n + nb * bl), jev.TYPE_Q8_0)
    toks = jev.random_tokens(trunk_n + nb * bl, VOCAB, 23)
    trunk = toks[:trunk_n]
    branches = [toks[trunk_n + b * bl: trunk_n + (b + 1) * bl] for b in range(nb)]
    lay = jev.TokenLayout.tree(0, trunk_n, [trunk_n + b * bl for b in range(nb)], len(toks))
    with synth.open(0) as m:
        tree = m.forward_layout(toks, lay, jev.OUT_SELECTED, ROWS).reshape(nb, 2)
        m.reset_kv_cache()
        m.prefill(trunk)
        alone = []
        for b in branches:
            m.kv_truncate(trunk_n)
            alone.append(m.forward_selected(b, ROWS))
    note("GPU tree pass and branches alone done")
    for b in range(nb):
        assert np.array_equal(tree[b], alone[b]), b
    ref = host_oracle(synth)
    try:
        chunked_prefill(ref, trunk)
        e = np.array(ref.forward_branches(branches, ROWS))
    finally:
        ref.close()
    note(f"z gpu {np.round(z_of(tree), 4).tolist()} oracle {np.round(z_of(e), 4).tolist()}")
    assert worst_close(e, tree) <= 1e-3
    assert np.max(np.abs(z_of(tree) - z_of(e))) <= 2e-2


def test_batched_q4_0_decisions(gpu):
    nd, trunk_n, nb, bl = 64, 512, 5, 32
    per = trunk_n + nb * bl
    synth = jev.SynthModel(jev.ModelConfig(initial_kv_capacity=nd * per), jev.TYPE_Q4_0)
    toks = jev.random_tokens(nd * per, VOCAB, 47)
    lay = jev.TokenLayout.forest([(trunk_n, [bl] * nb)] * nd)

    def decision(d):
        t = toks[d * per:(d + 1) * per]
        return t[:trunk_n], [t[trunk_n + b * bl: trunk_n + (b + 1) * bl] for b in range(nb)]

    with synth.open(0) as m:
        got = m.forward_layout(toks, lay, jev.OUT_SELECTED, ROWS).reshape(nd, nb, 2)
        note("GPU forest pass done")
        for d in range(nd):
            trunk, branches = decision(d)
            m.reset_kv_cache()
            alone = np.array(m.forward_tree(trunk, branches, ROWS))
            assert np.array_equal(got[d], alone), d
    note("64 decisions alone done")
    ref = host_oracle(synth)
    try:
        for d in (0, nd - 1):
            trunk, branches = decision(d)
            ref.reset_kv_cache()
            e = np.array(ref.forward_tree(trunk, branches, ROWS))
            note(f"decision {d}: z gpu {np.round(z_of(got[d]), 4).tolist()} oracle {np.round(z_of(e), 4).tolist()}")
            assert worst_close(e, got[d]) <= 1e-3
            assert np.max(np.abs(z_of(got[d]) - z_of(e))) <= 2e-2
    finally:
        ref.close()


def test_q5_1_decode_after_a_512_token_prompt(gpu):
    synth = jev.SynthModel(jev.ModelConfig(initial_kv_capacity=1024), jev.TYPE_Q5_1)
    prompt = jev.random_tokens(512, VOCAB, 31)
    steps = 16
    ref = host_oracle(synth)
    try:
        with synth.open(0) as m:
            m.prefill(prompt)
            greedy = m.decode_greedy(int(prompt[-1]), steps)
            m.reset_kv_cache()
            first = m.forward(prompt)
            assert worst_close(ref.forward(prompt), first) <= 1e-3
            note("512-token Q5_1 prefill logits match the oracle")
            # teacher-forced one-token passes: the GPU's logits against the oracle's
            # at every step, feeding the GPU's greedy choices to both
            nxt = int(prompt[-1])
            for i, tok in enumerate(greedy):
                g = m.forward([nxt])
                e = ref.forward([nxt])
                assert worst_close(e, g) <= 1e-3, i
                assert int(np.argmax(g)) == int(tok), i  # the graph replays the same step
                assert e[tok] >= e.max() - 1e-3 * max(1.0, abs(float(e.max()))), i
                nxt = int(tok)
            note(f"{steps} decode steps over {len(prompt)}..{len(prompt) + steps} keys match the oracle")
    finally:
        ref.close()


def test_q5_1_rows_of_one_token_after_prompts_alone(gpu):
    # The reasoning decider's rows (ReasoningDecider.cs:134-174) at full shape:
    # prompts of 64, 150, 256 and 300 tokens, each prefilled alone into its
    # row, then one-token steps of all four rows (2 to 5 chunks of 64 keys per
    # token, merged per token) against the oracle's full-vocabulary logits.
    synth = jev.SynthModel(jev.ModelConfig(initial_kv_capacity=1024), jev.TYPE_Q5_1)
    lengths = [64, 150, 256, 300]
    prompts = [list(jev.random_tokens(n, VOCAB, 80 + i)) for i, n in enumerate(lengths)]
    steps = 2
    bases = jev.row_bases(lengths, steps + 1)
    ref = host_oracle(synth)
    try:
        with synth.open(0) as m:
            nxt = []
            for r, p in enumerate(prompts):
                z = m.forward_rows(0, [bases[r]], [0], [p])[0]
                e = ref.forward_layout(p, jev.TokenLayout.rows(0, [bases[r]], [0], [len(p)]), oracle.OUT_FULL)
                assert worst_close(e, z) <= 1e-3, r
                nxt.append(jev.index_of_max(z))
            note("four prompts prefilled alone into their rows match the oracle")
            lens = list(lengths)
            for i in range(steps):
                g = np.array(m.forward_rows(0, bases, lens, [[t] for t in nxt]))
                lay = jev.TokenLayout.rows(0, bases, lens, [1] * len(lens))
                e = ref.forward_layout(nxt, lay, oracle.OUT_FULL).reshape(len(lens), -1)
                assert worst_close(e, g) <= 1e-3, i
                lens = [n + 1 for n in lens]
                nxt = [jev.index_of_max(z) for z in g]
            note(f"{steps} one-token steps of {len(lens)} rows match the oracle")
    finally:
        ref.close()


def test_q5_1_rows_graph_is_the_step_by_step_loop(gpu):
    # The reasoning decider's rows at full shape, as bench.py runs them (12 rows,
    # each prompt prefilled alone): the replayed rows graph gives the tokens of
    # one forward_rows call per step, bit for bit.
    synth = jev.SynthModel(jev.ModelConfig(initial_kv_capacity=2048), jev.TYPE_Q5_1)
    n_rows, plen, steps = 12, 64, 6
    prompts = [list(jev.random_tokens(plen, VOCAB, 50 + r)) for r in range(n_rows)]
    bases = jev.row_bases([plen] * n_rows, steps + 1)
    with synth.open(0) as m:
        def start():
            m.reset_kv_cache()
            return [jev.index_of_max(m.forward_rows(0, [bases[r]], [0], [prompts[r]])[0]) for r in range(n_rows)]
        first = start()
        graph = m.decode_rows_greedy(0, bases, [plen] * n_rows, first, steps)
        assert start() == first
        lengths, nxt, loop = [plen] * n_rows, list(first), []
        for _ in range(steps):
            z = m.forward_rows(0, bases, lengths, [[t] for t in nxt])
            lengths = [n + 1 for n in lengths]
            nxt = [jev.index_of_max(v) for v in z]
            loop.append(nxt)
    assert np.array_equal(graph, np.array(loop, np.int32))
    note(f"{n_rows} rows x {steps} steps: graph == step-by-step loop")
