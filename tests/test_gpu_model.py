"""GPU parity of the whole token loop against the oracle, and the reference's
bitwise contracts run on the GPU.

Bars (the task's tolerances against the managed CPU path):
  logits            Numeric.Close <= 1e-3 (|g - e| / max(1, |e|))
  verdict z         <= 2e-2 absolute
  tree pass         bit-identical to each branch run alone after the prefix
                    (DeciderTests.cs:55-91), and to branches off a cached prefix
  cached prefix     bit-identical to the whole prompt (SystemPromptCacheTests.cs:42-68)
"""
import numpy as np
import pytest

import jev
from helpers import rel_l2, tiny_config, worst_close
from jev._lib import SLOT_OUTPUT
from oracle import oracle

pytestmark = pytest.mark.gpu

ROWS = [13059 % 2048, 2649 % 2048, 77]


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


def fresh(m):
    m.reset_kv_cache()
    return m


@pytest.mark.parametrize("n", [2, 37, 64, 65, 200])
def test_causal_prefill_logits(model, ref, n):
    tokens = jev.random_tokens(n, 2048, n)
    g = fresh(model).forward(tokens)
    e = fresh(ref).forward(tokens)
    assert worst_close(e, g) <= 1e-3 and rel_l2(e, g) <= 1e-4
    assert model.cached_token_count == n


def test_prefill_then_decode_steps(model, ref):
    tokens = jev.random_tokens(50, 2048, 3)
    fresh(model).prefill(tokens[:45])
    fresh(ref).prefill(tokens[:45])
    for t in tokens[45:]:
        g = model.forward([t])
        e = ref.forward([t])
        assert worst_close(e, g) <= 1e-3
    assert model.cached_token_count == 50


@pytest.mark.parametrize("ctx", [30, 600])
def test_single_token_passes_match_oracle(model, ref, ctx):
    # One-token passes: the O projection forms the attention output from the
    # decode attention's 64-key chunks while staging its input (600 keys: 10
    # chunks, more than one group of eight loads in flight).
    tokens = jev.random_tokens(ctx + 3, 2048, 70 + ctx)
    fresh(model).prefill(tokens[:ctx])
    fresh(ref).prefill(tokens[:ctx])
    for t in tokens[ctx:]:
        assert worst_close(ref.forward([t]), model.forward([t])) <= 1e-3
    # a one-token branch after the prefix: the same path under a tree layout
    g = model.forward_branches([[int(tokens[1])]], ROWS)
    e = ref.forward_branches([[int(tokens[1])]], ROWS)
    assert worst_close(np.array(e), np.array(g)) <= 1e-3


def test_tree_verdicts_match_oracle(model, ref):
    trunk = jev.random_tokens(100, 2048, 5)
    branches = [jev.random_tokens(n, 2048, 50 + n) for n in (48, 17, 1, 64, 70)]
    g = np.array(fresh(model).forward_tree(trunk, branches, ROWS))
    e = np.array(fresh(ref).forward_tree(trunk, branches, ROWS))
    assert worst_close(e, g) <= 1e-3
    zg, ze = g[:, 0] - g[:, 1], e[:, 0] - e[:, 1]
    assert np.max(np.abs(zg - ze)) <= 2e-2
    mg, pg = jev.margins(g[:, :2], 1, 1)
    me, pe = oracle.margins(e[:, :2], 1, 1)
    assert np.max(np.abs(mg - me)) <= 2e-2


def test_tree_equals_branches_alone_bitwise(model):
    prefix = jev.random_tokens(150, 2048, 8)
    branches = [jev.random_tokens(n, 2048, 80 + n) for n in (48, 20, 2, 66)]
    m = fresh(model)
    m.prefill(prefix)
    alone = []
    for b in branches:
        m.kv_truncate(len(prefix))
        alone.append(m.forward_selected(b, ROWS))
    tree = fresh(m).forward_tree(prefix, branches, ROWS)
    fresh(m).prefill(prefix)
    cached = m.forward_branches(branches, ROWS)
    for b in range(len(branches)):
        assert np.array_equal(alone[b], tree[b]), b
        assert np.array_equal(alone[b], cached[b]), b


@pytest.mark.parametrize("t", [jev.TYPE_Q5_1, jev.TYPE_Q4_0])
def test_tree_equals_branches_alone_bitwise_other_types(gpu, t):
    # Branches of 2..16 tokens alone take the small-batch GEMM (which, for
    # Q5_1, also forms the down projection's block sums); in the tree they
    # take the wide one and the block-sum kernel.  The bits must agree.
    synth = jev.SynthModel(tiny_config(), t)
    prefix = jev.random_tokens(90, 2048, 28)
    branches = [jev.random_tokens(n, 2048, 60 + n) for n in (30, 2, 9, 16)]
    with synth.open(0) as m:
        m.prefill(prefix)
        alone = []
        for b in branches:
            m.kv_truncate(len(prefix))
            alone.append(m.forward_selected(b, ROWS))
        tree = fresh(m).forward_tree(prefix, branches, ROWS)
    for b in range(len(branches)):
        assert np.array_equal(alone[b], tree[b]), b


@pytest.mark.parametrize("trunk", [2100, 4100])
def test_tree_equals_branches_alone_across_attention_grids(model, trunk):
    # The attention grid has one workgroup per 32-token tile and KV head; grids
    # smaller than the GPU split the 128 output dims over 2 (up to 255
    # workgroups) or 4 (up to 64) workgroups.  With this model's 2 KV heads a
    # 4100-token tree pass computes all dims per workgroup, a 2100-token one
    # splits them in two, the short branches alone in four.  The bits must not
    # change.
    prefix = jev.random_tokens(trunk, 2048, 21)
    branches = [jev.random_tokens(n, 2048, 90 + n) for n in (40, 3)]
    m = fresh(model)
    m.prefill(prefix)
    alone = []
    for b in branches:
        m.kv_truncate(len(prefix))
        alone.append(m.forward_selected(b, ROWS))
    tree = fresh(m).forward_tree(prefix, branches, ROWS)
    for b in range(len(branches)):
        assert np.array_equal(alone[b], tree[b]), b


def test_forest_equals_each_tree_alone_bitwise(model):
    # Independent decisions in one pass (TokenLayout.forest: each tree its own
    # shared range): every branch's verdict rows equal that tree run alone.
    trees = [(40, [5, 9]), (17, [3]), (64, [1, 20, 7])]
    tokens, alone = [], []
    for i, (trunk_n, bls) in enumerate(trees):
        trunk = list(jev.random_tokens(trunk_n, 2048, 300 + i))
        branches = [list(jev.random_tokens(n, 2048, 400 + 10 * i + j)) for j, n in enumerate(bls)]
        tokens += trunk + [t for b in branches for t in b]
        alone += fresh(model).forward_tree(trunk, branches, ROWS)
    lay = jev.TokenLayout.forest(trees)
    got = fresh(model).forward_layout(tokens, lay, jev.OUT_SELECTED, ROWS).reshape(len(lay.outputs), len(ROWS))
    for k in range(len(alone)):
        assert np.array_equal(got[k], alone[k]), k


def test_cached_prefix_equals_whole_prompt_bitwise(model):
    tokens = jev.random_tokens(120, 2048, 9)
    m = fresh(model)
    whole = m.forward(tokens)
    fresh(m).prefill(tokens[:70])
    snap = m.kv_snapshot(70)
    fresh(m).kv_restore(snap, 70)
    part = m.forward(tokens[70:])
    assert np.array_equal(whole, part)


def test_kv_snapshot_matches_oracle_cache(model, ref):
    tokens = jev.random_tokens(90, 2048, 10)  # initial capacity 64: grows once
    fresh(model).prefill(tokens[:40])
    model.prefill(tokens[40:])
    fresh(ref).prefill(tokens)
    g = model.kv_snapshot(90)
    e = ref.kv_snapshot(90)
    assert worst_close(e, g) <= 1e-3
    assert model.kv_capacity >= 90


def test_forward_tree_logits_full_vocab(model, ref):
    trunk = jev.random_tokens(10, 2048, 12)
    branches = [jev.random_tokens(3, 2048, 13), jev.random_tokens(2, 2048, 14)]
    g = fresh(model).forward_tree_logits(trunk, branches)
    lay_ref = fresh(ref)
    # oracle: the same layout through forward_layout
    offsets, total = [10, 13], 15
    tree = jev.TokenLayout.tree(0, 10, offsets, total).with_outputs(list(range(10, 15)))
    flat = lay_ref.forward_layout(np.concatenate([trunk] + branches), tree, oracle.OUT_FULL).reshape(5, 2048)
    got = np.array([x for b in g for x in b])
    assert worst_close(flat, got) <= 1e-3


def test_rows_layout_batched_decode(model, ref):
    # ForwardRowsAsync: independent rows after a shared prefix, one token each.
    shared = jev.random_tokens(20, 2048, 15)
    fresh(model).prefill(shared)
    fresh(ref).prefill(shared)
    rows_tok = [[5], [9], [1000]]
    g = model.forward_rows(20, [64, 96, 128], [0, 0, 0], rows_tok, ROWS)
    lay = jev.TokenLayout.rows(20, [64, 96, 128], [0, 0, 0], [1, 1, 1])
    e = ref.forward_layout([5, 9, 1000], lay, oracle.OUT_SELECTED, ROWS).reshape(3, len(ROWS))
    assert worst_close(e, np.array(g)) <= 1e-3


def test_rows_of_one_token_over_several_key_chunks(model, ref):
    # Rows of different lengths after a 150-token prefix, then one token per
    # row: 156, 211 and 261 visible keys, i.e. 3, 4 and 5 chunks of 64 merged
    # per token (the per-token decode attention and its chunk combine).
    shared = jev.random_tokens(150, 2048, 17)
    fresh(model).prefill(shared)
    fresh(ref).prefill(shared)
    bases, lengths = [150, 160, 230], [5, 60, 110]
    prompts = [list(jev.random_tokens(n, 2048, 18 + n)) for n in lengths]
    model.forward_rows(150, bases, [0, 0, 0], prompts, ROWS)
    lay = jev.TokenLayout.rows(150, bases, [0, 0, 0], lengths)
    ref.forward_layout(np.concatenate(prompts).astype(np.int32), lay, oracle.OUT_SELECTED, ROWS)
    step = [7, 11, 1500]
    g = model.forward_rows(150, bases, lengths, [[t] for t in step])
    lay = jev.TokenLayout.rows(150, bases, lengths, [1, 1, 1])
    e = ref.forward_layout(step, lay, oracle.OUT_FULL).reshape(3, -1)
    assert worst_close(e, np.array(g)) <= 1e-3


def test_single_token_tiles_that_see_each_other(model, ref):
    # A one-token trunk and one-token branches: every attention tile is one
    # token, but the branches see the trunk token written by the same pass,
    # so its key must be stored before any token's attention runs.
    prefix = jev.random_tokens(40, 2048, 19)
    fresh(model).prefill(prefix)
    fresh(ref).prefill(prefix)
    lay = jev.TokenLayout.tree(40, 1, [1, 2, 3], 4)
    toks = [5, 900, 77, 1234]
    g = model.forward_layout(toks, lay, jev.OUT_FULL).reshape(3, -1)
    e = ref.forward_layout(toks, lay, oracle.OUT_FULL).reshape(3, -1)
    assert worst_close(e, g) <= 1e-3


def test_greedy_decode_follows_oracle(model, ref):
    tokens = jev.random_tokens(30, 2048, 16)
    fresh(model).prefill(tokens)
    fresh(ref).prefill(tokens)
    out = model.decode_greedy(int(tokens[-1]), 8)
    # teacher-force the oracle on the GPU's choices: each must be the oracle's
    # argmax up to the logits tolerance
    nxt = int(tokens[-1])
    for tok in out:
        e = ref.forward([nxt])
        assert e[tok] >= e.max() - 2e-3
        nxt = int(tok)


@pytest.mark.parametrize("t", [jev.TYPE_Q4_0, jev.TYPE_Q5_1])
def test_other_block_types(gpu, t):
    synth = jev.SynthModel(tiny_config(), t)
    m = synth.open(0)
    r = oracle.OracleModel(synth.config).bind_synth(synth)
    tokens = jev.random_tokens(70, 2048, 17)
    assert worst_close(r.forward(tokens), m.forward(tokens)) <= 1e-3
    trunk, branches = tokens[:40], [jev.random_tokens(n, 2048, n) for n in (5, 9)]
    g = np.array(fresh(m).forward_tree(trunk, branches, ROWS))
    e = np.array(fresh(r).forward_tree(trunk, branches, ROWS))
    assert np.max(np.abs((g[:, 0] - g[:, 1]) - (e[:, 0] - e[:, 1]))) <= 2e-2
    fresh(m).prefill(tokens[:60])
    fresh(r).prefill(tokens[:60])
    assert worst_close(r.forward(tokens[60:61]), m.forward(tokens[60:61])) <= 1e-3
    m.close()


@pytest.mark.parametrize("t", [jev.TYPE_Q8_0, jev.TYPE_Q4_0, jev.TYPE_Q5_1])
@pytest.mark.parametrize("n", [70, 600])
def test_projection_segments_off_the_wide_tile_grid(gpu, t, n):
    # 3 query heads over 1 KV head: the fused QKV segments (384, 128, 128 rows)
    # do not split on 256-row boundaries, so the projections take the
    # dequant-in-LDS GEMM (small and large batch shapes) instead of B-direct.
    cfg = tiny_config(n_heads=3, n_kv_heads=1, initial_kv_capacity=1024)
    synth = jev.SynthModel(cfg, t)
    m = synth.open(0)
    r = oracle.OracleModel(cfg).bind_synth(synth)
    tokens = jev.random_tokens(n, 2048, n + t)
    assert worst_close(r.forward(tokens), m.forward(tokens)) <= 1e-3
    m.close()


@pytest.mark.parametrize("heads,kv", [(6, 1), (10, 2)])
@pytest.mark.parametrize("n", [70, 300])
def test_query_groups_wider_than_four_heads(gpu, heads, kv, n):
    # An attention workgroup serves four query heads of one KV head; a group of
    # 5 or 6 heads takes two workgroups per KV head, the second with waves past
    # the group's last head (they compute a clamped head and store nothing).
    cfg = tiny_config(n_heads=heads, n_kv_heads=kv, initial_kv_capacity=1024)
    synth = jev.SynthModel(cfg, jev.TYPE_Q8_0)
    m = synth.open(0)
    r = oracle.OracleModel(cfg).bind_synth(synth)
    tokens = jev.random_tokens(n, 2048, n + heads)
    assert worst_close(r.forward(tokens), m.forward(tokens)) <= 1e-3
    m.reset_kv_cache()
    r.reset_kv_cache()
    trunk = jev.random_tokens(n // 2, 2048, 3)
    branches = [jev.random_tokens(k, 2048, 40 + k) for k in (9, 33, 70)]
    rows = [5, 1999]
    got = np.array(m.forward_tree(trunk, branches, rows))
    exp = np.array(r.forward_tree(trunk, branches, rows))
    assert worst_close(exp, got) <= 1e-3
    m.close()


# ---------------------------------------------------------------- error paths

def test_errors_match_reference_exceptions(model):
    m = fresh(model)
    with pytest.raises(jev.ArgumentError):
        m.forward([])
    with pytest.raises(jev.ArgumentError):
        m.forward([2048])  # outside the embedding table
    with pytest.raises(jev.ArgumentError):
        m.forward_branches([[1], []], ROWS)
    with pytest.raises(jev.ArgumentError):
        m.forward_selected([1, 2], [5000])
    with pytest.raises(jev.ArgumentError):
        m.kv_snapshot(5)
    assert m.cached_token_count == 0
    # RopeAndCacheTests.RestoreRejectsAMissizedSnapshot / SnapshotRejectsMoreThanIsCached
    m.forward([1, 2])
    snap = m.kv_snapshot(2)
    with pytest.raises(jev.ArgumentError):
        m.kv_restore(snap, 3)
    with pytest.raises(jev.ArgumentError):
        m.kv_snapshot(3)
    assert m.cached_token_count == 2


def test_cancel_aimed_at_no_call_does_not_reach_the_next_one(model):
    # A token cancelled between calls cancels nothing the library runs: the
    # next call (any entry point) completes.
    m = fresh(model)
    m.cancel()
    m.forward([1, 2, 3])
    assert m.cached_token_count == 3
    m.cancel()
    m.decode_greedy(5, 2)
    assert m.cached_token_count == 5
    m.cancel()
    m.forward_branches([[7], [8, 9]], ROWS)


def cancel_while_running(m, run):
    """Runs `run()` while another thread cancels m's call in flight every 0.2 ms
    until it returns (ctypes releases the GIL during the library call)."""
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


def test_cancel_in_flight_leaves_the_cache_and_the_next_call_intact(model):
    tokens = jev.random_tokens(4000, 2048, 23)
    want = fresh(model).forward(tokens[:500])
    m = fresh(model)
    # the tiny model's prefill is short, so a cancel thread can miss it: a
    # call that completed uncancelled is rolled back and tried again
    for attempt in range(5):
        m.reset_kv_cache()
        m.prefill(tokens[:100])
        try:
            cancel_while_running(m, lambda: m.prefill(tokens[100:]))
        except jev.CancelledError:
            break
    else:
        pytest.fail("no cancel reached the prefill in flight in 5 attempts")
    assert m.cached_token_count == 100
    got = m.forward(tokens[100:500])  # continues the 100 cached tokens
    assert np.array_equal(got, want)


def test_finalize_requires_every_tensor(gpu, synth):
    m = jev.MinistralModel(synth.config)
    with pytest.raises(jev.JevError):
        m.forward([1])
    with pytest.raises(jev.DataError):
        m.finalize()
    t = synth.tensors["token_embd.weight"]
    with pytest.raises(jev.DataError):
        m.bind(t.slot, t.layer, t.ggml_type, t.rows, t.cols, t.data[:-1])  # truncated
    m.close()


@pytest.mark.parametrize("name", ["output_norm.weight", "blk.1.attn_norm.weight", "blk.0.ffn_norm.weight"])
def test_finalize_rejects_a_short_norm(gpu, synth, name):
    """A norm shorter than `hidden` would be read past its end by the norm kernel: finalize
    refuses it by name (InvalidDataException's role) before any kernel runs."""
    m = jev.MinistralModel(synth.config)
    for n, t in synth.tensors.items():
        if n == name:
            short = t.data[: (t.cols - 32) * 4]
            m.bind(t.slot, t.layer, t.ggml_type, 1, t.cols - 32, short)
        else:
            m.bind(t.slot, t.layer, t.ggml_type, t.rows, t.cols, t.data)
    with pytest.raises(jev.DataError, match=name.replace(".weight", "")):
        m.finalize()
    m.close()


def test_finalize_rejects_an_embedding_table_shorter_than_the_vocabulary(gpu, synth):
    """With an untied output head, greedy decoding still feeds argmax ids (< vocab) to the
    embedding gather, so token_embd must hold every vocabulary row."""
    c = synth.config
    m = jev.MinistralModel(c)
    for n, t in synth.tensors.items():
        if n == "token_embd.weight":
            keep = c.vocab - 16
            m.bind(t.slot, t.layer, t.ggml_type, keep, t.cols, t.data[: keep * (t.data.size // t.rows)])
            m.bind(SLOT_OUTPUT, 0, t.ggml_type, t.rows, t.cols, t.data)
        else:
            m.bind(t.slot, t.layer, t.ggml_type, t.rows, t.cols, t.data)
    with pytest.raises(jev.DataError, match="token_embd"):
        m.finalize()
    m.close()


def test_gguf_file_loads_the_same_model_bitwise(gpu, synth, model, tmp_path):
    """The unchanged loading path: GGUF file -> GgufFile -> jev_bind_tensor from the mapping."""
    p = tmp_path / "synth.gguf"
    synth.write_gguf(str(p))
    toks = jev.random_tokens(45, synth.config.vocab, 21)
    want = fresh(model).forward(toks)
    with jev.load_gguf(str(p), initial_kv_capacity=synth.config.initial_kv_capacity) as m:
        assert m.config.vocab == synth.config.vocab and m.config.n_layers == synth.config.n_layers
        got = m.forward(toks)
    assert np.array_equal(got, want)


def test_gguf_missing_tensor_is_reported_by_name(gpu, synth, tmp_path):
    from jev import gguf as G
    p = tmp_path / "partial.gguf"
    ts = [G.WriterTensor(n, (t.cols,) if t.rows == 1 else (t.cols, t.rows), t.ggml_type, t.data)
          for n, t in synth.tensors.items() if n != "blk.1.ffn_up.weight"]
    G.write_gguf(str(p), G.ministral_metadata(synth.config, synth.ggml_type), ts)
    with pytest.raises(KeyError, match="blk.1.ffn_up.weight"):
        jev.load_gguf(str(p))


def test_cache_growth_keeps_the_prefix_bitwise(gpu, synth):
    """KvCache.EnsureCapacity (KvCache.cs:48-70): growing a populated cache copies its rows (and the
    pair shadows the tree attention stages from), so continuing after growth equals the whole prompt."""
    tokens = jev.random_tokens(150, 2048, 12)
    with synth.bind(jev.MinistralModel(synth.config)) as m:
        whole = m.forward(tokens)
    with synth.bind(jev.MinistralModel(synth.config)) as m:
        assert m.kv_capacity == synth.config.initial_kv_capacity == 64
        m.prefill(tokens[:60])
        part = m.forward(tokens[60:])  # 150 positions: 64 -> 128 -> 256
        assert m.kv_capacity == 256
    assert np.array_equal(whole, part)
